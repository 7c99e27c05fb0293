"""Full-output end-to-end parity at the benchmark's full sizes: every T x H output
of the layer against the oracle's whole chain (route -> L1 -> UE8M0 requant ->
L2 -> bf16 -> reduce over all 256 experts), plus the share of L1 output bytes
and L2 bf16 outputs that differ from the oracle's over ALL routed slots.
T=8192 compares the first 1024 tokens' full rows (every expert they reach)."""
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


@pytest.mark.parametrize("T,zipf,ntok", [(512, None, None), (2048, None, None),
                                         (2048, 1.1, None), (8192, None, 1024)])
def test_full_output_end_to_end(T, zipf, ntok):
    t0 = time.time()
    _say(f"full output T={T} zipf={zipf} tokens={ntok or T}")
    c = mc.normal_case(E, K, H, I, T, seed=T + 1, scaled=True, zipf=zipf)
    r = mc.run_layer(c)
    mc.check_routing(c, r)
    w1, w2 = mc.logical_weights(c)
    s1 = np.ascontiguousarray(c.s1.cpu().numpy())
    s2 = np.ascontiguousarray(c.s2.cpu().numpy())
    tok = np.arange(ntok or T)
    if ntok is None:
        ref = orc.layer(c.x, c.xsf, w1, s1, w2, s2, c.idx, c.wts, E=E, G=c.G, scaled=True,
                        nthreads=16)
        slots = int(r.offsets[-1])
        ffn_d = r.buf.ffn(slots).cpu().numpy()
        l2_d = r.buf.l2_out(slots).cpu().numpy().view(np.uint16)
        ffn_flips = float(np.mean(ffn_d != ref["ffn"]))
        sf_flips = float(np.mean(r.buf.ffn_sf(slots).cpu().numpy() != ref["ffn_sf"]))
        l2_flips = float(np.mean(l2_d != ref["l2"]))
    else:
        sub = np.ascontiguousarray(c.idx[tok])
        ref = orc.layer(np.ascontiguousarray(c.x[tok]), np.ascontiguousarray(c.xsf[tok]), w1, s1,
                        w2, s2, sub, np.ascontiguousarray(c.wts[tok]), E=E, G=c.G, scaled=True,
                        nthreads=16)
        # slots of the sub-problem's pairs in the device's full-layer order
        pos = r.pair_pos.reshape(T, K)[tok].ravel()
        rpos = ref["pair_pos"]
        ffn_all = r.buf.ffn(int(r.offsets[-1])).cpu().numpy()
        ffn_flips = float(np.mean(ffn_all[pos] != ref["ffn"][rpos]))
        sf_flips = float(np.mean(r.buf.ffn_sf(int(r.offsets[-1])).cpu().numpy()[pos]
                                 != ref["ffn_sf"][rpos]))
        l2_all = r.buf.l2_out(int(r.offsets[-1])).cpu().numpy().view(np.uint16)
        l2_flips = float(np.mean(l2_all[pos] != ref["l2"][rpos]))
    err, rms, cos = mc.e2e_metrics(r.y[tok], ref["y"])
    del w1, w2
    _say(f"  T={T} zipf={zipf}: max|d|/rms={err / rms:.4f} cos={cos:.7f} "
         f"ffn byte flips={ffn_flips:.2e} ffn scale diffs={sf_flips:.2e} "
         f"l2 bf16 diffs={l2_flips:.2e} ({time.time() - t0:.0f} s)")
    assert ffn_flips <= mc.FLIP_MAX, f"ffn bytes differ at {ffn_flips:.2e}"
    assert err <= mc.E2E_ABS_FRAC * rms and cos >= mc.E2E_COS, (err / rms, cos)
