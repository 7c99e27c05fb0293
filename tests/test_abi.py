"""CPU tests of the C-ABI boundary: the library loads without a GPU, exports
every extern "C" symbol declared in include/megakernel.h, the ctypes mirror of
MegaLaunchArgs matches the C struct, the workspace layout is sane, and bad
shapes are rejected.  No compute is launched here."""
import ctypes
import os
import re

import numpy as np
import pytest

import mini_mega_amd as mm
from mini_mega_amd import _lib
from mini_mega_amd.inputs import paired_to_torch_rows, unpack_tiles

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def _declared_c_symbols():
    text = open(os.path.join(ROOT, "include", "megakernel.h")).read()
    block = text[text.index('extern "C" {'):]
    return sorted(set(re.findall(r"\b(mm_[a-z_0-9]+)\s*\(", block)))


def test_library_exports_every_declared_symbol():
    L = mm.lib()
    syms = _declared_c_symbols()
    assert len(syms) >= 18
    for s in syms:
        assert hasattr(L, s), f"{s} not exported"
    assert set(syms) == set(_lib.EXPORTS)


def test_args_mirror_matches_c_struct():
    L = mm.lib()
    assert L.mm_abi_version() == 4
    assert L.mm_args_size() == ctypes.sizeof(mm.MegaLaunchArgs)
    for name, *_ in mm.MegaLaunchArgs._fields_:
        assert L.mm_args_offset(name.encode()) == getattr(mm.MegaLaunchArgs, name).offset
    assert L.mm_args_offset(b"no_such_field") == -1


@pytest.mark.parametrize("T", [32, 512, 2048, 8192])
def test_layout_regions_aligned_and_disjoint(T):
    E, K, H, I = 256, 8, 6144, 2048
    L = mm.layout(T, K, E, H, I)
    names = ["status", "chunk_hist", "counts", "offsets", "items", "perm", "pair_pos", "xq",
             "xq_sf", "ffn", "ffn_sf", "l2", "total"]
    offs = [getattr(L, n) for n in names]
    assert all(o % 256 == 0 for o in offs)
    assert offs == sorted(offs)
    P = T * K
    assert L.l2 + P * H * 2 <= L.total
    assert L.ffn_sf - L.ffn >= P * I
    assert L.max_items >= (P + L.m_tile - 1) // L.m_tile + E - 1


@pytest.mark.parametrize("dims", [(32, 8, 256, 100, 2048), (32, 8, 256, 6144, 200),
                                  (32, 0, 256, 6144, 2048), (32, 8, 2000, 6144, 2048),
                                  (0, 8, 256, 6144, 2048),
                                  # past the 32-bit activation row offsets: T*K*I > 2^32,
                                  # T*H > 2^32
                                  (262145, 8, 256, 6144, 2048), (699051, 1, 256, 6144, 128)])
def test_layout_rejects_bad_dims(dims):
    with pytest.raises(mm.MegaError):
        mm.layout(*dims)


def test_capacity_limit_is_inclusive():
    """T*K*I = 2^32 exactly (the last row's offsets still fit) is laid out;
    one token more is rejected by the layout and by a launch alike."""
    L = mm.layout(262144, 8, 256, 6144, 2048)
    assert L.max_pairs == 262144 * 8
    a = mm.MegaLaunchArgs(tokens=4, max_tokens=262145, rwk=1, self=1, topk_idx=1, w1=1, w2=1)
    assert mm.lib().mm_launch_full(ctypes.byref(a), None) == 2  # kErrBadDims


def test_launch_rejects_null_workspace_without_touching_gpu():
    L = mm.lib()
    a = mm.MegaLaunchArgs(tokens=4, max_tokens=4)
    assert L.mm_launch_full(ctypes.byref(a), None) == 1  # kErrNullPointer
    a = mm.MegaLaunchArgs(tokens=8, max_tokens=4, rwk=1, self=1, topk_idx=1, w1=1, w2=1)
    assert L.mm_launch_full(ctypes.byref(a), None) == 4  # kErrTooManyTokens
    a = mm.MegaLaunchArgs(tokens=4, max_tokens=4, rwk=1, self=1, topk_idx=1, w1=1, w2=1,
                          workspace_bytes=16)
    assert L.mm_launch_full(ctypes.byref(a), None) == 3  # kErrWorkspace
    # the L1 output's quantisation must follow the scale mode
    a = mm.MegaLaunchArgs(tokens=4, max_tokens=4, rwk=1, self=1, topk_idx=1, w1=1, w2=1,
                          ffn_ue8m0=1)
    assert L.mm_launch_full(ctypes.byref(a), None) == 6  # kErrUnsupported
    a = mm.MegaLaunchArgs(tokens=4, max_tokens=4, rwk=1, self=1, topk_idx=1, w1=1, w2=1,
                          x_sf=1, w1_sf=1, w2_sf=1, ffn_ue8m0=0)
    assert L.mm_launch_full(ctypes.byref(a), None) == 6  # kErrUnsupported


def _pack_numpy(w):
    """Tile layout written from the byte formula in mm_device.h (tile_byte)."""
    n, k = w.shape
    out = np.zeros(n * k, np.uint8)
    r = np.arange(n)[:, None]
    c = np.arange(k)[None, :]
    nt, kt, rr, kk = r // 16, c // 128, r % 16, c % 128
    off = (nt * (k // 128) + kt) * 2048 + ((kk % 32) // 16) * 1024 + (rr + 16 * (kk // 32)) * 16 \
        + kk % 16
    out[off.ravel()] = w.ravel()
    return out


def test_unpack_inverts_tile_formula():
    w = np.random.default_rng(0).integers(0, 256, size=(64, 384)).astype(np.uint8)
    assert np.array_equal(unpack_tiles(_pack_numpy(w), 64, 384), w)


@pytest.mark.parametrize("I", [128, 2048])
def test_paired_row_map_is_reference_pairing(I):
    """Paired row rho (gate of h at (h/G)*2G + h%G, up at +G; src/bench_check.cuh:
    444-445) maps to torch row h (gate) or I + h (up)."""
    G = mm.pairing_block(I)
    m = paired_to_torch_rows(I)
    assert sorted(m.tolist()) == list(range(2 * I))
    for h in sorted({0, 1, G - 1, min(G, I - 1), I - 1}):
        assert m[(h // G) * 2 * G + h % G] == h
        assert m[(h // G) * 2 * G + h % G + G] == I + h


def test_xcd_ranges_partition_units_and_balance_cost():
    """The XCD unit ranges the routing scan computes (restated in moe_case.xcd_cuts):
    a partition of the units into 8 contiguous ranges, each within its share of
    the grid, with modelled costs equal to within one expert's units."""
    import moe_case as mc
    rng = np.random.default_rng(7)
    for E, mean, m_tile, nb in ((8, 20, 64, 16), (256, 16, 256, 24), (256, 256, 256, 16),
                                (256, 64, 128, 24)):
        counts = rng.poisson(mean, size=E)
        counts[rng.integers(0, E)] *= 6   # one hot expert
        nm = -(-counts // m_tile)
        max_items = int(counts.sum() // m_tile + E)
        cuts = mc.xcd_cuts(counts, m_tile, nb, max_items)
        units = nb * int(nm.sum())
        assert cuts[0] == 0 and cuts[-1] == units and np.all(np.diff(cuts) >= 0)
        assert np.all(np.diff(cuts) <= (nb * max_items + 8) // 8)
        sz = np.where(nm > 0, -(-counts // np.maximum(nm, 1)), 0)
        uc = np.maximum(9, 2 + np.minimum((sz + 15) // 16, 16))
        cost = np.repeat(uc, nb * nm)
        per = np.array([cost[a:b].sum() for a, b in zip(cuts[:-1], cuts[1:])])
        assert per.max() - per.min() <= 2 * 18 + 1, per


def test_tail_ticket_orders_put_costly_units_first():
    """L1's tail-queue ticket order (restated in moe_case.tail_orders): per XCD
    a permutation of its last min(range, 32) units whose token tiles never
    rise along the tickets, ties in unit order, when some item holds more than
    128 rows; the identity otherwise.  Unit tiles are checked against a direct
    walk of the item table (block-major units)."""
    import moe_case as mc
    rng = np.random.default_rng(11)
    for E, mean, m_tile, nb in ((8, 20, 64, 16), (256, 64, 256, 16), (256, 260, 256, 24),
                                (64, 40, 128, 24)):
        counts = rng.poisson(mean, size=E)
        counts[rng.integers(0, E, size=3)] *= 9   # hot experts split into several items
        counts[rng.integers(0, E)] = 0
        max_items = int(counts.sum() // m_tile + E)
        tiles = mc.unit_tiles(counts, m_tile, nb)
        # direct: unit u of expert e's range is item (u - first) % nm's block
        direct = []
        for cnt in counts.tolist():
            nm, sz = mc.item_split(cnt, m_tile)
            rows = [min(cnt, (j + 1) * sz) - j * sz for j in range(nm)]
            for lu in range(nb * nm):
                direct.append(min((rows[lu % nm] + 15) // 16, 16))
        assert tiles.tolist() == direct
        cuts = mc.xcd_cuts(counts, m_tile, nb, max_items)
        ordered = max(mc.item_split(int(c), m_tile)[1] for c in counts) > 128
        for x, order in enumerate(mc.tail_orders(counts, m_tile, nb, cuts)):
            t = min(int(cuts[x + 1] - cuts[x]), 32)
            assert sorted(order.tolist()) == list(range(t))
            if not ordered:
                assert order.tolist() == list(range(t))
                continue
            seq = tiles[int(cuts[x + 1]) - t + order.astype(np.int64)]
            assert np.all(np.diff(seq) <= 0), seq
            for a, b in zip(order[:-1], order[1:]):
                if seq[list(order).index(a)] == seq[list(order).index(b)]:
                    assert a < b
