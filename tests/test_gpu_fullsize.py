"""Full-output end-to-end parity at the benchmark's full sizes: every T x H output
of the layer against the oracle's whole chain (route -> L1 -> UE8M0 requant ->
L2 -> bf16 -> reduce over all 256 experts), plus the share of L1 output bytes
and L2 bf16 outputs that differ from the oracle's over ALL routed slots.
T=8192 runs the oracle 1024 tokens at a time and compares every token.
Each assertion message carries the margins against the bars."""
import sys
import time

import numpy as np
import pytest
import torch

import mini_mega_amd as mm
from oracle import oracle as orc

import moe_case as mc

pytestmark = pytest.mark.gpu

E, K, H, I = 256, 8, 6144, 2048


def _say(msg):
    print(f"[case] {msg}", flush=True)
    sys.stdout.flush()


@pytest.fixture(scope="module", autouse=True)
def _gpu():
    assert torch.cuda.is_available(), "GPU tests need an MI355X"
    torch.cuda.set_device(0)
    mm.lib()
    yield


@pytest.mark.timeout(900)
@pytest.mark.parametrize("T,zipf,chunk", [(512, None, None), (2048, None, None),
                                          (2048, 1.1, None), (8192, None, 1024)])
def test_full_output_end_to_end(T, zipf, chunk):
    """chunk: the oracle runs the layer over `chunk` tokens at a time (each
    token's output and each pair's ffn / L2 row depend only on that token),
    so T=8192 compares every token, every expert's every item and token tile,
    with a progress line per chunk."""
    t0 = time.time()
    _say(f"full output T={T} zipf={zipf} (oracle chunks of {chunk or T} tokens)")
    c = mc.normal_case(E, K, H, I, T, seed=T + 1, scaled=True, zipf=zipf)
    r = mc.run_layer(c)
    mc.check_routing(c, r)
    w1, w2 = mc.logical_weights(c)
    s1 = np.ascontiguousarray(c.s1.cpu().numpy())
    s2 = np.ascontiguousarray(c.s2.cpu().numpy())
    slots = int(r.offsets[-1])
    ffn_d = r.buf.ffn(slots).cpu().numpy()
    sf_d = r.buf.ffn_sf(slots).cpu().numpy()
    l2_d = r.buf.l2_out(slots).cpu().numpy().view(np.uint16)
    step = chunk or T
    y_ref = np.empty((T, H), np.float32)
    n_ffn = n_sf = n_l2 = 0
    for t0c in range(0, T, step):
        tok = np.arange(t0c, min(T, t0c + step))
        ref = orc.layer(np.ascontiguousarray(c.x[tok]), np.ascontiguousarray(c.xsf[tok]), w1, s1,
                        w2, s2, np.ascontiguousarray(c.idx[tok]),
                        np.ascontiguousarray(c.wts[tok]), E=E, G=c.G, scaled=True, nthreads=16)
        y_ref[tok] = ref["y"]
        # the chunk's pairs: device slots (full-layer order) vs the oracle's own
        pos = r.pair_pos.reshape(T, K)[tok].ravel()
        rpos = ref["pair_pos"]
        ok = pos >= 0
        assert np.array_equal(ok, rpos >= 0)
        pos, rpos = pos[ok], rpos[ok]
        n_ffn += int(np.count_nonzero(ffn_d[pos] != ref["ffn"][rpos]))
        n_sf += int(np.count_nonzero(sf_d[pos] != ref["ffn_sf"][rpos]))
        n_l2 += int(np.count_nonzero(l2_d[pos] != ref["l2"][rpos]))
        if chunk:
            _say(f"  tokens {tok[0]}..{tok[-1]} compared ({time.time() - t0:.0f} s)")
        del ref
    ffn_flips = n_ffn / float(ffn_d.size)
    sf_flips = n_sf / float(sf_d.size)
    l2_flips = n_l2 / float(l2_d.size)
    del w1, w2
    msg = (f"T={T} zipf={zipf}: ffn byte flips={ffn_flips:.2e} (bar {mc.FLIP_MAX:.0e}) "
           f"ffn scale diffs={sf_flips:.2e} l2 bf16 diffs={l2_flips:.2e}")
    _say(f"  {msg} ({time.time() - t0:.0f} s)")
    assert ffn_flips <= mc.FLIP_MAX, msg
    g = mc.e2e_gate(r.y, r.y32, y_ref, what=f"T={T} zipf={zipf} full output")
    _say(f"  {g['msg']}")
