"""CPU tests that pin the oracle (oracle/moe_oracle.c) before it is trusted.

Each check compares against something independent of the oracle's own code:
torch's float8_e4m3fn / bfloat16 casts, closed forms, brute force on tiny
inputs, fp64 GEMMs, the reference's TK_INFO fixtures, or invariants a wrong
term / sign / index / transposition would break.
"""
import numpy as np
import pytest
import torch

from oracle import oracle as orc

rng = np.random.default_rng(1234)


# ------------------------------------------------------------------ codecs --
def test_e4m3_decode_matches_torch_all_256():
    table = orc.e4m3_decode_table()
    ref = torch.arange(256, dtype=torch.int32).to(torch.uint8).view(torch.float8_e4m3fn).float()
    ref = ref.numpy()
    nan = np.isnan(ref)
    assert np.array_equal(np.isnan(table), nan)
    assert nan.sum() == 2  # 0x7F / 0xFF
    assert np.array_equal(table[~nan], ref[~nan])
    assert table[0x7E] == 448.0 and table[0x01] == 2.0 ** -9 and table[0x80] == 0.0


def _edge_values():
    t = orc.e4m3_decode_table()
    fin = t[np.isfinite(t)]
    mids = []
    s = np.sort(np.unique(fin))
    mids = (s[1:] + s[:-1]) / 2  # exact ties
    nudge = np.concatenate([np.nextafter(mids.astype(np.float32), np.float32(np.inf)),
                            np.nextafter(mids.astype(np.float32), np.float32(-np.inf))])
    rand = rng.standard_normal(4000).astype(np.float32) * np.float32(50.0)
    small = rng.standard_normal(2000).astype(np.float32) * np.float32(0.01)
    return np.concatenate([fin, mids, nudge, rand, small, [0.0, -0.0, 447.9, 448.0]]).astype(
        np.float32)


def test_e4m3_quantize_matches_torch_rne_on_clamped_values():
    v = _edge_values()
    got = orc.e4m3_quantize(v)
    ref = torch.from_numpy(np.clip(v, -448, 448)).to(torch.float8_e4m3fn).view(torch.uint8)
    assert np.array_equal(got, ref.numpy())


def test_e4m3_quantize_saturates_and_nan():
    got = orc.e4m3_quantize(np.array([448.0, 464.0, 480.0, 1e9, np.inf, -1e9, -np.inf],
                                     np.float32))
    assert list(got) == [0x7E, 0x7E, 0x7E, 0x7E, 0x7E, 0xFE, 0xFE]
    assert orc.e4m3_quantize(np.array([np.nan], np.float32))[0] == 0x7F


def test_bf16_rne_matches_torch():
    v = np.concatenate([rng.standard_normal(20000).astype(np.float32) * 1000,
                        np.array([1.0 + 2 ** -8, 1.0 + 3 * 2 ** -8, -1.0 - 2 ** -8, 3.4e38,
                                  np.inf, -np.inf, 1e-40], np.float32)]).astype(np.float32)
    got = orc.f32_to_bf16(v)
    ref = torch.from_numpy(v).to(torch.bfloat16).view(torch.int16).numpy().view(np.uint16)
    assert np.array_equal(got, ref)


# ------------------------------------------------------------------- UE8M0 --
def test_ceil_ue8m0_closed_form():
    for e in range(-20, 20):
        assert orc.ceil_ue8m0(2.0 ** e) == 127 + e          # exact powers map to themselves
        assert orc.ceil_ue8m0(2.0 ** e * 1.0001) == 128 + e  # anything above rounds up
        assert orc.ceil_ue8m0(2.0 ** e * 0.9999) == 127 + e


@pytest.mark.parametrize("scale", [1e-3, 1.0, 37.0, 1e4])
def test_quant_rows_ue8m0_invariants(scale):
    x = (rng.standard_normal((16, 512)) * scale).astype(np.float32)
    q, sf = orc.quant_rows_ue8m0(x)
    table = orc.e4m3_decode_table()
    s = np.ldexp(1.0, sf.astype(np.int32) - 127)
    amax = np.abs(x).reshape(16, 4, 128).max(axis=2)
    # ceil-to-power-of-two of amax/448: amax/s in (224, 448]
    assert np.all(amax / s <= 448.0) and np.all(amax / s > 224.0)
    deq = table[q].reshape(16, 4, 128) * s[:, :, None]
    err = np.abs(deq - x.reshape(16, 4, 128))
    # e4m3 half-ulp: 2^-4 relative for normals, 2^-10 * s absolute for subnormals
    assert np.all(err <= np.maximum(np.abs(x.reshape(16, 4, 128)) * 2.0 ** -4,
                                    s[:, :, None] * 2.0 ** -10) + 1e-30)


def _torch_per_block_cast_ue8m0(w: np.ndarray, gran: int = 128):
    """utils/math.py:13-16,62-72 (ceil_to_ue8m0, per_block_cast_to_fp8 with
    use_ue8m0=True) in torch float32 on the CPU, for shapes that are multiples
    of gran (no padding): fp8 bytes and UE8M0 exponent bytes [rows/g][cols/g]."""
    x = torch.from_numpy(np.ascontiguousarray(w, np.float32))
    m, n = x.shape
    xv = x.view(m // gran, gran, n // gran, gran)
    amax = xv.abs().float().amax(dim=(1, 3), keepdim=True).clamp(1e-4)
    sf = amax / 448.0
    bits = sf.abs().float().view(torch.int32)
    exp = ((bits >> 23) & 0xFF) + (bits & 0x7FFFFF).bool().int()
    sf = (exp.clamp(1, 254) << 23).view(torch.float32)
    q = (xv * (1.0 / sf)).to(torch.float8_e4m3fn).view(m, n)
    return q.view(torch.uint8).numpy(), ((sf.view(torch.int32) >> 23) & 0xFF).to(
        torch.uint8).view(m // gran, n // gran).numpy()


@pytest.mark.parametrize("scale", [1e-3, 0.02, 5.0])
def test_quant_blocks_ue8m0_equals_torch_recipe(scale, mutation):
    """The block cast's bytes and scales against a torch restatement of
    per_block_cast_to_fp8 (utils/math.py:62-72), bit for bit, with a hot block,
    an all-zero block (amax clamps to 1e-4) and a tiny one; a planted mistake
    (the scale multiplied instead of divided) must fail it."""
    w = (rng.standard_normal((384, 256)) * scale).astype(np.float32)
    w[:128, :128] *= 64.0
    w[128:256, 128:] = 0.0
    w[256:, :128] *= 1e-6
    tq, tsf = _torch_per_block_cast_ue8m0(w)
    q, sf = orc.quant_blocks_ue8m0(w)
    assert np.array_equal(sf, tsf)
    assert np.array_equal(q, tq)
    mutation(4)
    bq, bsf = orc.quant_blocks_ue8m0(w)
    assert np.array_equal(bsf, tsf) and not np.array_equal(bq, tq)


def test_quant_blocks_ue8m0_scale_per_block():
    w = (rng.standard_normal((256, 384)) * 0.02).astype(np.float32)
    w[:128, :128] *= 100.0  # one hot block: its scale must differ from its neighbours'
    q, sf = orc.quant_blocks_ue8m0(w)
    assert sf.shape == (2, 3)
    assert sf[0, 0] > sf[0, 1] and sf[0, 0] > sf[1, 0]
    amax = np.abs(w.reshape(2, 128, 3, 128)).max(axis=(1, 3))
    s = np.ldexp(1.0, sf.astype(np.int32) - 127)
    assert np.all(amax / s <= 448.0) and np.all(amax / s > 224.0)


# ----------------------------------------------------------------- routing --
def _route_bruteforce(idx, E, cap):
    T, K = idx.shape
    flat = idx.ravel()
    pos = np.full(flat.size, -1, np.int64)
    perm, counts = [], np.zeros(E, np.int64)
    for e in range(E):
        members = [p for p in range(flat.size) if flat[p] == e][:cap]
        counts[e] = len(members)
        for p in members:
            pos[p] = len(perm)
            perm.append(p)
    return counts, np.array(perm, np.int64), pos


@pytest.mark.parametrize("T,K,E,cap", [(7, 3, 5, 100), (33, 4, 16, 100), (40, 8, 16, 9),
                                       (1, 1, 1, 100)])
def test_route_matches_bruteforce(T, K, E, cap):
    idx = rng.integers(-2, E + 2, size=(T, K)).astype(np.int64)  # includes invalid ids
    counts, offsets, perm, pair_pos = orc.route(idx, E, cap)
    bc, bperm, bpos = _route_bruteforce(idx, E, cap)
    assert np.array_equal(counts, bc)
    assert np.array_equal(offsets, np.concatenate([[0], np.cumsum(bc)]))
    assert np.array_equal(perm, bperm)
    assert np.array_equal(pair_pos, bpos)


def _tk_launches(name="tk_info_anchors.log"):
    """Per-expert counts [256] of each TK_INFO launch in a committed fixture
    (32 ranks x 8 local experts)."""
    import os
    import re
    path = os.path.join(os.path.dirname(__file__), "golden", name)
    data = {}
    for line in open(path):
        m = re.search(r"\[TK_INFO\] rank=(\d+) launch=(\d+) n=8 : (.*)", line)
        if m is None:
            continue
        data.setdefault(int(m.group(2)), {})[int(m.group(1))] = list(map(int, m.group(3).split()))
    out = {}
    for launch, ranks in data.items():
        assert len(ranks) == 32
        out[launch] = np.array([ranks[r] for r in range(32)], np.int32).ravel()
    return out


@pytest.mark.parametrize("launch", [804900, 809200, 853000])
def test_tk_fixture_routes_reproduce_counts(launch):
    """test/mega_common.cuh:460-482 + route_count_deviation (:485-495): routes
    rebuilt from a TK_INFO launch hit the logged per-expert counts exactly."""
    per_expert = _tk_launches()[launch]
    total = int(per_expert.sum())
    assert total % (32 * 8) == 0
    tokens = total // (32 * 8)
    idx = orc.routes_from_counts(per_expert, 32, 8, tokens, 8)
    counts, offsets, perm, pair_pos = orc.route(idx, 256)
    assert np.array_equal(counts, per_expert)
    for row in idx:
        assert len(set(row.tolist())) == 8  # duplicate free per token


@pytest.mark.parametrize("launch", [45400, 84900, 151000])
def test_real_decode_fixture_routes_reproduce_counts(launch):
    """The same for launches of the reference's real GLM-5.2 decode corpus
    (test/76.real_decode/dataset.tk_info; committed excerpt): the most skewed
    launch puts 398 of 4096 pairs on one expert and leaves 140 experts empty."""
    per_expert = _tk_launches("tk_real_decode.log")[launch]
    total = int(per_expert.sum())
    assert total % (32 * 8) == 0
    idx = orc.routes_from_counts(per_expert, 32, 8, total // (32 * 8), 8)
    counts, *_ = orc.route(idx, 256)
    assert np.array_equal(counts, per_expert)
    for row in idx:
        assert len(set(row.tolist())) == 8


def test_balanced_routes_exactly_16_per_expert():
    """make_routes(Balanced) (src/bench_check.cuh:52-55): every expert gets
    exactly TPR*R*8/E pairs at TPR 16, R 32."""
    idx = orc.balanced_routes(32, 16, 8, 8)
    counts, *_ = orc.route(idx, 256)
    assert np.all(counts == 16)


# ---------------------------------------------------------------- L1 / L2 --
def _rand_fp8(shape, scale):
    v = (rng.standard_normal(shape) * scale).astype(np.float32)
    return orc.e4m3_quantize(np.clip(v, -448, 448)).reshape(shape)


def test_l1_matches_fp64_gemm_and_pairing():
    H, I, G, rows = 256, 256, 256, 5
    x = _rand_fp8((rows, H), 1.0)
    w = _rand_fp8((2 * I, H), 0.05)
    t = orc.e4m3_decode_table().astype(np.float64)
    xd, wd = t[x], t[w]
    h_idx = np.arange(I)
    grow = (h_idx // G) * 2 * G + h_idx % G
    g = xd @ wd[grow].T
    u = xd @ wd[grow + G].T
    want = g / (1 + np.exp(-g)) * u
    got = orc.l1_rows(x, None, w, None, G)
    assert np.allclose(got, want, rtol=1e-4, atol=1e-4)
    # gate/up swapped would give silu(u)*g: must be far from the oracle
    swapped = u / (1 + np.exp(-u)) * g
    assert not np.allclose(got, swapped, rtol=1e-2, atol=1e-2)


def test_l1_pairing_block_128():
    """I = 128 uses pairing block G = 128: gate rows 0..127, up rows 128..255."""
    H, I, G = 256, 128, 128
    x = _rand_fp8((3, H), 1.0)
    w = np.zeros((2 * I, H), np.uint8)
    w[5, :] = 0x38  # 1.0 on gate row of h=5
    w[128 + 5, :] = 0x40  # 2.0 on up row of h=5
    got = orc.l1_rows(x, None, w, None, G)
    t = orc.e4m3_decode_table().astype(np.float64)
    g = t[x].sum(axis=1)
    want = g / (1 + np.exp(-g)) * (2 * g)
    assert np.allclose(got[:, 5], want, rtol=1e-5)
    assert np.all(got[:, np.arange(I) != 5] == 0)


def test_scaled_with_unit_scales_equals_unscaled_bitwise():
    H, I, G, rows = 256, 128, 128, 4
    x = _rand_fp8((rows, H), 1.0)
    w1 = _rand_fp8((2 * I, H), 0.05)
    w2 = _rand_fp8((H, I), 0.05)
    one_x = np.full((rows, H // 128), 127, np.uint8)
    one_w1 = np.full((2 * I // 128, H // 128), 127, np.uint8)
    one_w2 = np.full((H // 128, I // 128), 127, np.uint8)
    a = orc.l1_rows(x, None, w1, None, G)
    b = orc.l1_rows(x, one_x, w1, one_w1, G)
    assert np.array_equal(a.view(np.uint32), b.view(np.uint32))
    f = orc.quant_ffn(a, False)[0]
    one_f = np.full((rows, I // 128), 127, np.uint8)
    assert np.array_equal(orc.l2_rows(f, None, w2, None).view(np.uint32),
                          orc.l2_rows(f, one_f, w2, one_w2).view(np.uint32))


def test_l2_scale_is_exact_power_of_two_linearity():
    H, I, rows = 256, 256, 3
    f = _rand_fp8((rows, I), 1.0)
    w2 = _rand_fp8((H, I), 0.05)
    s = np.full((H // 128, I // 128), 127, np.uint8)
    base = orc.l2_rows(f, None, w2, s)
    s2 = s.copy()
    s2[1, :] += 3  # output rows 128..255 scaled by 8 exactly
    scaled = orc.l2_rows(f, None, w2, s2)
    assert np.array_equal(scaled[:, :128], base[:, :128])
    assert np.array_equal(scaled[:, 128:], base[:, 128:] * 8)
    t = orc.e4m3_decode_table().astype(np.float64)
    assert np.allclose(base, t[f] @ t[w2].T, rtol=1e-4, atol=1e-4)


def test_reduce_order_and_invalid_pairs():
    T, K, H = 4, 3, 256
    l2 = orc.f32_to_bf16(rng.standard_normal(6 * H).astype(np.float32)).reshape(6, H)
    pair_pos = np.array([[0, 1, -1], [2, -1, 3], [-1, -1, -1], [4, 5, 0]], np.int32)
    w = rng.random((T, K)).astype(np.float32)
    y, yb = orc.reduce(l2, pair_pos, w, T, K)
    vals = np.array([orc.lib().orc_bf16_to_f32(int(b)) for b in l2.ravel()],
                    np.float32).reshape(6, H)
    for t in range(T):
        acc = np.zeros(H, np.float32)
        for k in range(K):
            if pair_pos[t, k] >= 0:
                acc = (acc + (vals[pair_pos[t, k]] * w[t, k]).astype(np.float32)).astype(np.float32)
        assert np.array_equal(y[t], acc)
    assert np.all(y[2] == 0)


# ------------------------------------------------------- check.cu closed form --
@pytest.mark.parametrize("ranks,tpr,H,K", [(4, 3, 384, 8), (32, 2, 256, 8), (3, 5, 128, 4)])
def test_checkcu_inputs_equal_fill_inputs(ranks, tpr, H, K, mutation):
    """The check.cu inputs against a numpy evaluation of fill_inputs
    (test/mega_common.cuh:166-175) for every rank: x bytes (r*37 + t*7 +
    c*3) & 0x3f with t rank-local, weights 1 + 0.25 r + 0.01 (i % 7) with
    i = t*topk + k, in float32 left to right as the C++ does.  Planted
    mistakes (the global token in x, the rank term dropped) must fail it."""
    r = np.arange(ranks)[:, None, None]
    t = np.arange(tpr)[None, :, None]
    c = np.arange(H)[None, None, :]
    want_x = ((r * 37 + t * 7 + c * 3) & 0x3F).astype(np.uint8).reshape(ranks * tpr, H)
    i = (np.arange(tpr)[:, None] * K + np.arange(K)[None, :])
    want_w = np.empty((ranks, tpr, K), np.float32)
    for rr in range(ranks):
        want_w[rr] = (np.float32(1.0) + np.float32(rr) * np.float32(0.25)) + \
            (i % 7).astype(np.float32) * np.float32(0.01)
    want_w = want_w.reshape(ranks * tpr, K)
    x, w = orc.checkcu_inputs(ranks, tpr, H, K)
    assert np.array_equal(x, want_x)
    assert np.array_equal(w.view(np.uint32), want_w.view(np.uint32))
    mutation(5)
    bx, _ = orc.checkcu_inputs(ranks, tpr, H, K)
    assert not np.array_equal(bx, want_x)
    mutation(6)
    _, bw = orc.checkcu_inputs(ranks, tpr, H, K)
    assert not np.array_equal(bw, want_w)


def test_checkcu_inputs_saturate_every_ffn_byte():
    """check.cu inputs are all-positive with g, u ~ 4e5..9e5, so every L1
    output saturates to 448 = 0x7E; and g == u because 131*256 = 0 mod 64."""
    H, I, G = 6144, 2048, 256
    x, w = orc.checkcu_inputs(2, 2, H, 8)
    w1e = orc.wprobe_matrix(17, 0, 2 * I, H)
    assert np.array_equal(w1e[:256], w1e[256:512])  # gate rows == up rows (period 64)
    h = orc.l1_rows(x[:2], None, w1e, None, G)[:, :64]
    assert np.all(h > 448.0)
    q, _ = orc.quant_ffn(np.ascontiguousarray(h), False)
    assert np.all(q == 0x7E)
    assert np.allclose(w[0], 1.0 + 0.01 * (np.arange(8) % 7))


def test_layer_chain_small_against_fp64_model():
    """Full chain on a tiny layer vs a float64 numpy restatement of
    torch/tests/test_fp8_mega_moe.py:28-48 (reference())."""
    E, K, H, I, T = 4, 2, 256, 128, 9
    G = 128
    x = _rand_fp8((T, H), 1.0)
    w1 = np.stack([_rand_fp8((2 * I, H), 0.05) for _ in range(E)])
    w2 = np.stack([_rand_fp8((H, I), 0.05) for _ in range(E)])
    idx = np.stack([rng.permutation(E)[:K] for _ in range(T)]).astype(np.int64)
    idx[3, 1] = -1
    wts = rng.random((T, K)).astype(np.float32)
    ref = orc.layer(x, None, w1, None, w2, None, idx, wts, E=E, G=G, scaled=False)
    t = orc.e4m3_decode_table().astype(np.float64)
    y = np.zeros((T, H))
    for tok in range(T):
        for k in range(K):
            e = idx[tok, k]
            if e < 0:
                continue
            wl = t[w1[e]]
            h_idx = np.arange(I)
            g = t[x[tok]] @ wl[(h_idx // G) * 2 * G + h_idx % G].T
            u = t[x[tok]] @ wl[(h_idx // G) * 2 * G + h_idx % G + G].T
            h = np.clip(g / (1 + np.exp(-g)) * u, -448, 448)
            hq = torch.from_numpy(h.astype(np.float32)).to(torch.float8_e4m3fn).float().numpy()
            o = hq.astype(np.float64) @ t[w2[e]].T
            ob = torch.from_numpy(o.astype(np.float32)).to(torch.bfloat16).float().numpy()
            y[tok] += ob * wts[tok, k]
    rms = np.sqrt(np.mean(y ** 2))
    assert np.abs(ref["y"] - y).max() <= 2e-2 * rms


# ------------------------------------------------ block-scaled (UE8M0) path --
# The scaled oracle (x_sf per token per 128 columns, w1_sf / w2_sf per 128x128
# block of the paired / plain weight matrix, ffn requantised per 128 columns)
# checked against float64 dequantise-then-GEMM restatements of
# torch/tests/test_fp8_mega_moe.py:28-48 with the casts of
# torch/mxmegakernel/utils/math.py:13-72.  Every scale below is a random
# non-unit power of two; gate and up rows of one hidden column sit in
# different 128-row blocks, so a wrong block index changes the result by a
# power of two, far outside the tolerances.

def _dec64():
    return orc.e4m3_decode_table().astype(np.float64)


def _scale_of(sf):
    return np.ldexp(1.0, sf.astype(np.int32) - 127)


def _deq_rows(q, sf):
    """[rows][K] bytes with per-row per-128 scales [rows][K/128] -> float64."""
    return _dec64()[q] * np.repeat(_scale_of(sf), 128, axis=1)


def _deq_blocks(q, sf):
    """[N][K] bytes with 128x128 block scales [N/128][K/128] -> float64."""
    s = _scale_of(sf)
    return _dec64()[q] * np.repeat(np.repeat(s, 128, axis=0), 128, axis=1)


def _paired_rows(I, G):
    h = np.arange(I)
    grow = (h // G) * 2 * G + h % G
    return grow, grow + G


def _silu64(g):
    return g / (1.0 + np.exp(-np.clip(g, -700.0, 700.0)))


def _l1_model(xq, xsf, w1q, w1sf, G, up_block_of=None):
    """h = silu(g) * u in float64, with g, u and the sums of |terms| that bound
    their accumulation error.  up_block_of (a planted mistake, used only to
    show the comparison's sensitivity) maps each up row to the 128-row block
    whose scale it is given."""
    I = w1q.shape[0] // 2
    xd = _deq_rows(xq, xsf)
    wd = _deq_blocks(w1q, w1sf)
    grow, urow = _paired_rows(I, G)
    if up_block_of is not None:
        raw = _dec64()[w1q]
        s = _scale_of(w1sf)
        wu = raw[urow] * np.repeat(s[up_block_of(urow)], 128, axis=1)
    else:
        wu = wd[urow]
    g = xd @ wd[grow].T
    u = xd @ wu.T
    return (_silu64(g) * u, dict(g=g, u=u, ag=np.abs(xd) @ np.abs(wd[grow]).T,
                                 au=np.abs(xd) @ np.abs(wu).T))


def _scaled_l1_case(rows, H, I, seed):
    r = np.random.default_rng(seed)
    xq = _rand_fp8((rows, H), 1.0)
    w1q = _rand_fp8((2 * I, H), 0.05)
    xsf = r.integers(121, 134, size=(rows, H // 128)).astype(np.uint8)
    w1sf = r.integers(116, 138, size=(2 * I // 128, H // 128)).astype(np.uint8)
    return xq, xsf, w1q, w1sf


@pytest.fixture
def mutation():
    """Sets an oracle mutation for one test and always restores the faithful
    oracle afterwards."""
    yield orc.set_mutation
    orc.set_mutation(0)


def _l1_within_bound(got, want, m, H):
    # sequential fp32 sums of H terms: |err(g)| <= H * 2^-24 * sum|terms|
    # (likewise u); h = silu(g) * u moves by at most 1.1 |u| err(g) +
    # |silu(g)| err(u) (|silu'| <= 1.1), plus the final fp32 roundings
    c = H * 2.0 ** -24
    bound = 1.1 * np.abs(m["u"]) * c * m["ag"] + np.abs(_silu64(m["g"])) * c * m["au"]
    return np.abs(got - want) <= bound + 4 * 2.0 ** -24 * np.abs(want)


@pytest.mark.parametrize("H,I,G", [(384, 256, 256), (256, 512, 256), (512, 128, 128)])
def test_l1_scaled_matches_fp64_dequant_gemm(H, I, G, mutation):
    rows = 6
    xq, xsf, w1q, w1sf = _scaled_l1_case(rows, H, I, seed=H + I)
    want, m = _l1_model(xq, xsf, w1q, w1sf, G)
    got = orc.l1_rows(xq, xsf, w1q, w1sf, G).astype(np.float64)
    ok = _l1_within_bound(got, want, m, H)
    assert ok.all(), f"max |d| {np.abs(got - want).max():.3e}"
    # the pin catches an oracle whose up rows take their gate rows' scale block
    mutation(1)
    bad = orc.l1_rows(xq, xsf, w1q, w1sf, G).astype(np.float64)
    assert np.mean(~_l1_within_bound(bad, want, m, H)) > 0.5


def test_l1_scaled_row_and_block_scales_are_independent():
    """One x row's block scaled by 2^3 scales exactly that row's g and u
    contributions from those 128 columns; one W1 block scaled by 2^-2 scales
    exactly the rows of that block (power-of-two scales are exact)."""
    H, I, G = 256, 256, 256
    xq = _rand_fp8((3, H), 1.0)
    w1q = _rand_fp8((2 * I, H), 0.05)
    xsf = np.full((3, H // 128), 127, np.uint8)
    w1sf = np.full((2 * I // 128, H // 128), 127, np.uint8)
    base = orc.l1_rows(xq, xsf, w1q, w1sf, G)
    # gate rows 0..127 (block 0) get 2^-2 on both k-blocks: g of h = 0..127
    # scales by 1/4 exactly, so h = silu(g/4) * u, which the model reproduces
    w1sf2 = w1sf.copy()
    w1sf2[0, :] = 125
    got = orc.l1_rows(xq, xsf, w1q, w1sf2, G).astype(np.float64)
    want, _ = _l1_model(xq, xsf, w1q, w1sf2, G)
    assert np.allclose(got, want, rtol=1e-5, atol=1e-6)
    assert np.array_equal(got[:, 128:], base[:, 128:].astype(np.float64))
    assert not np.allclose(got[:, :128], base[:, :128], rtol=1e-3)


@pytest.mark.parametrize("H,I", [(384, 256), (256, 512)])
def test_l2_scaled_matches_fp64_dequant_gemm(H, I, mutation):
    rows = 5
    r = np.random.default_rng(H * I)
    fq = _rand_fp8((rows, I), 1.0)
    fsf = r.integers(118, 136, size=(rows, I // 128)).astype(np.uint8)
    w2q = _rand_fp8((H, I), 0.05)
    w2sf = r.integers(116, 138, size=(H // 128, I // 128)).astype(np.uint8)
    fd, wd = _deq_rows(fq, fsf), _deq_blocks(w2q, w2sf)
    want = fd @ wd.T
    terms = np.abs(fd) @ np.abs(wd).T     # sequential fp32: |err| <= I 2^-24 terms
    got = orc.l2_rows(fq, fsf, w2q, w2sf).astype(np.float64)
    assert np.all(np.abs(got - want) <= I * 2.0 ** -24 * terms)
    # the pin catches ffn scales taken from the neighbouring 128-column block
    mutation(3)
    bad = orc.l2_rows(fq, fsf, w2q, w2sf).astype(np.float64)
    assert np.mean(np.abs(bad - want) > I * 2.0 ** -24 * terms) > 0.5


def test_l2_scaled_block_index_not_transposed(mutation):
    """Square 2x2 block grid with distinct scales: W2 block (n/128, k/128)
    versus its transpose (k/128, n/128) differ on the off-diagonal blocks."""
    H = I = 256
    fq = _rand_fp8((4, I), 1.0)
    fsf = np.full((4, 2), 127, np.uint8)
    w2q = _rand_fp8((H, I), 0.05)
    w2sf = np.array([[127, 131], [123, 127]], np.uint8)   # 2^0, 2^4 / 2^-4, 2^0
    fd, wd = _deq_rows(fq, fsf), _deq_blocks(w2q, w2sf)
    want = fd @ wd.T
    terms = np.abs(fd) @ np.abs(wd).T
    got = orc.l2_rows(fq, fsf, w2q, w2sf).astype(np.float64)
    assert np.all(np.abs(got - want) <= I * 2.0 ** -24 * terms)
    mutation(2)
    bad = orc.l2_rows(fq, fsf, w2q, w2sf).astype(np.float64)
    assert np.abs(bad - want).max() > 1e-2 * np.abs(want).max()


def _torch_per_token_cast_ue8m0(h: np.ndarray):
    """utils/math.py:13-16,23-47 (ceil_to_ue8m0, per_token_cast_to_fp8 with
    use_ue8m0=True, gran 128) in torch float32 on the CPU: returns fp8 bytes
    and UE8M0 exponent bytes."""
    x = torch.from_numpy(np.ascontiguousarray(h, np.float32))
    m, n = x.shape
    xv = x.view(m, n // 128, 128)
    amax = xv.abs().float().amax(dim=2).clamp(1e-4)
    sf = amax / 448.0
    bits = sf.abs().float().view(torch.int32)
    exp = ((bits >> 23) & 0xFF) + (bits & 0x7FFFFF).bool().int()
    sf = (exp.clamp(1, 254) << 23).view(torch.float32)
    q = (xv * (1.0 / sf.unsqueeze(2))).to(torch.float8_e4m3fn).view(m, n)
    return q.view(torch.uint8).numpy(), ((sf.view(torch.int32) >> 23) & 0xFF).to(
        torch.uint8).numpy()


@pytest.mark.parametrize("scale", [1e-3, 0.7, 300.0])
def test_quant_ffn_scaled_equals_torch_recipe(scale):
    h = (rng.standard_normal((12, 512)) * scale).astype(np.float32)
    h[3, :128] = 0.0                      # an all-zero block: amax clamps to 1e-4
    h[5, 128:256] *= 1e-6                 # a tiny block next to normal ones
    q, sf = orc.quant_ffn(h, True)
    tq, tsf = _torch_per_token_cast_ue8m0(h)
    assert np.array_equal(sf, tsf)
    assert np.array_equal(q, tq)


def _chain_model(x, xsf, w1, w1sf, w2, w2sf, idx, wts, G, ffn_override=None):
    """Whole scaled layer in float64 / torch casts, the reference() of
    torch/tests/test_fp8_mega_moe.py:28-48 with block-scaled operands: per
    (token, k) h = silu(x W1g^T) * (x W1u^T), per_token_cast_to_fp8(h, ue8m0),
    out = bf16(deq(ffn) W2^T), y += out * w.  ffn_override[(t, k)] = (q, sf)
    feeds given ffn bytes to L2 instead (a staged check)."""
    T, K = idx.shape
    E = w1.shape[0]
    H = x.shape[1]
    y = np.zeros((T, H), np.float64)
    ffn = {}
    for t in range(T):
        for k in range(K):
            e = int(idx[t, k])
            if not (0 <= e < E):
                continue
            if ffn_override is not None:
                q, sf = ffn_override[(t, k)]
            else:
                h, _ = _l1_model(x[t:t + 1], xsf[t:t + 1], w1[e], w1sf[e], G)
                q, sf = _torch_per_token_cast_ue8m0(h.astype(np.float32))
            ffn[(t, k)] = (q, sf)
            o = _deq_rows(q, sf) @ _deq_blocks(w2[e], w2sf[e]).T
            ob = torch.from_numpy(o.astype(np.float32)).to(torch.bfloat16).float().numpy()
            y[t] += ob[0].astype(np.float64) * float(wts[t, k])
    return y, ffn


def test_layer_scaled_chain_against_fp64_model(mutation):
    """The scaled oracle chain (routing, L1 with x_sf / w1_sf, UE8M0 ffn
    requant, L2 with ffn / w2 scales, bf16, reduce) against the float64
    reference() model: ffn bytes and scales (almost all equal: the model sums
    in float64, the oracle in sequential fp32), the staged L2 + reduce on the
    oracle's own ffn (bf16 rows within one ulp), and y at the end-to-end bar."""
    E, K, H, I, T, G = 4, 2, 256, 256, 10, 256
    r = np.random.default_rng(77)
    x = _rand_fp8((T, H), 1.0)
    xsf = r.integers(122, 132, size=(T, H // 128)).astype(np.uint8)
    w1 = np.stack([_rand_fp8((2 * I, H), 0.05) for _ in range(E)])
    w1sf = r.integers(118, 136, size=(E, 2 * I // 128, H // 128)).astype(np.uint8)
    w2 = np.stack([_rand_fp8((H, I), 0.05) for _ in range(E)])
    w2sf = r.integers(118, 136, size=(E, H // 128, I // 128)).astype(np.uint8)
    idx = np.stack([r.permutation(E)[:K] for _ in range(T)]).astype(np.int64)
    idx[2, 1] = E + 1                      # an invalid id: no contribution
    wts = r.random((T, K)).astype(np.float32)
    ref = orc.layer(x, xsf, w1, w1sf, w2, w2sf, idx, wts, E=E, G=G, scaled=True)
    y_model, ffn_model = _chain_model(x, xsf, w1, w1sf, w2, w2sf, idx, wts, G)
    # ffn: slot of pair (t, k) is pair_pos[t*K + k]
    flips = total = sf_diff = 0
    override = {}
    for (t, k), (q, sf) in ffn_model.items():
        s = int(ref["pair_pos"][t * K + k])
        assert s >= 0
        oq, osf = ref["ffn"][s], ref["ffn_sf"][s]
        flips += int(np.sum(oq != q[0]))
        total += q.size
        sf_diff += int(np.sum(osf != sf[0]))
        override[(t, k)] = (oq[None, :], osf[None, :])
    assert sf_diff == 0, "ffn block scales differ from the torch recipe"
    assert flips <= max(1, total // 500), f"{flips} of {total} ffn bytes differ"
    # staged: L2 + reduce on the oracle's own ffn
    y_staged, _ = _chain_model(x, xsf, w1, w1sf, w2, w2sf, idx, wts, G, ffn_override=override)
    rms = float(np.sqrt(np.mean(y_staged ** 2)))
    assert np.abs(ref["y"] - y_staged).max() <= 2 ** -7 * rms
    # end to end
    rms = float(np.sqrt(np.mean(y_model ** 2)))
    err = float(np.abs(ref["y"] - y_model).max())
    cos = float((ref["y"] * y_model).sum() / (np.linalg.norm(ref["y"]) * np.linalg.norm(y_model)))
    assert err <= 2e-2 * rms and cos >= 0.9995, (err / rms, cos)
    # the end-to-end bar rejects an oracle with any of the planted scale slips
    for m in (1, 2, 3):
        mutation(m)
        bad = orc.layer(x, xsf, w1, w1sf, w2, w2sf, idx, wts, E=E, G=G, scaled=True)["y"]
        assert np.abs(bad - y_model).max() > 2e-2 * rms, f"mutation {m} not detected"
