"""The opt-in fp8 MFMA path (MegaLaunchArgs::mfma_fp8: both GEMMs on gfx950's
block-scaled v_mfma_scale_f32_16x16x128_f8f6f4, the reference's own fp8 MMA
arithmetic class, src/compute.cuh:414-417,593-596) against the oracle, at the
reference's staged check.cu tolerances (test/check.cu:397-507): routing
bit-exact, L1 within the tolerance or the interval of the fp8 MFMA's
truncating sum (|error| <= 2^-15 sum|terms|), L2 fed with the device's ffn
within rel 1e-2 / abs 1e-3 rms, REDUCE bit-exact, and the whole layer at
cos >= 0.9995.  Its max|d| is printed, not gated: the fp8 MFMA's sums put it
outside the 2e-2 rms(y) bar that the default bf16 path meets (the MFMA
precision tests measure why).  Bad option combinations are rejected."""
import ctypes
import sys

import numpy as np
import pytest
import torch

import mini_mega_amd as mm

import moe_case as mc

pytestmark = pytest.mark.gpu

F8_EPS = 2.0 ** -15       # fp8 MFMA sum error bound, in units of sum|terms|
F8_FLIP_MAX = 1e-2        # share of L1 bytes allowed to differ from the oracle's


def _say(msg):
    print(f"[case] {msg}", flush=True)
    sys.stdout.flush()


@pytest.fixture(scope="module", autouse=True)
def _gpu():
    assert torch.cuda.is_available(), "GPU tests need an MI355X"
    torch.cuda.set_device(0)
    mm.lib()
    yield


def _run_f8(c):
    buf = mm.get_symm_buffer_for_mega_moe(None, c.E, c.T, c.K, c.H, c.I, expert_window=c.win)
    buf.mfma_fp8 = True
    return mc.run_layer(c, buf=buf)


@pytest.mark.timeout(600)
@pytest.mark.parametrize("E,K,H,I,T,zipf,win,scaled", [
    (32, 8, 1024, 512, 300, None, 0, True),
    (16, 4, 512, 256, 777, 1.1, 64, True),
    (32, 8, 1024, 768, 200, None, 128, False),
    (8, 8, 768, 512, 1200, None, 0, True),     # 15-tile items: one activation stage
    (256, 8, 6144, 2048, 512, None, 0, True),
    (256, 8, 6144, 2048, 2048, 1.1, 0, True),    # skewed: hot experts in several items
    (256, 8, 6144, 2048, 8192, None, 0, True),
])
def test_fp8_mfma_layer_at_checkcu_tolerances(E, K, H, I, T, zipf, win, scaled):
    _say(f"fp8 MFMA E={E} K={K} H={H} I={I} T={T} zipf={zipf} win={win} scaled={scaled}")
    c = mc.normal_case(E, K, H, I, T, seed=T + 7, scaled=scaled, zipf=zipf, win=win)
    r = _run_f8(c)
    mc.check_routing(c, r)
    nz = np.nonzero(r.counts)[0]
    order = nz[np.argsort(r.counts[nz], kind="stable")]
    for e in {int(order[-1]), int(order[0])}:
        flips = mc.check_l1(c, r, e, max_rows=None if E < 256 else 64, eps=F8_EPS,
                            flip_max=F8_FLIP_MAX)
        mc.check_l2(c, r, e, max_rows=None if E < 256 else 64)
        _say(f"  expert {e} ({int(r.counts[e])} rows): L1 bytes differing {flips:.2e}")
    mc.check_reduce(c, r)
    tok = np.arange(T) if T <= 1200 else np.array([0, 1, T // 3, T // 2, T - 1])
    from oracle import oracle as orc
    sub = c.idx[tok]
    experts = np.unique(sub[(sub >= 0) & (sub < c.E)])
    remap = {int(e): i for i, e in enumerate(experts)}
    idx2 = np.vectorize(lambda v: remap.get(int(v), -1))(sub).astype(np.int64)
    w1 = np.stack([c.w1_logical(int(e)) for e in experts])
    w2 = np.stack([c.w2_logical(int(e)) for e in experts])
    s1 = None if c.s1 is None else np.ascontiguousarray(c.s1[torch.from_numpy(experts)].cpu().numpy())
    s2 = None if c.s2 is None else np.ascontiguousarray(c.s2[torch.from_numpy(experts)].cpu().numpy())
    xs = np.ascontiguousarray(c.x[tok])
    xsf = None if c.xsf is None else np.ascontiguousarray(c.xsf[tok])
    ref = orc.layer(xs, xsf, w1, s1, w2, s2, idx2, np.ascontiguousarray(c.wts[tok]),
                    E=len(experts), G=c.G, scaled=c.scaled, nthreads=16)
    err, rms, cos = mc.e2e_metrics(r.y32[tok], ref["y"])
    _say(f"  fp8 MFMA end to end ({len(tok)} tokens): fp32 y max|d|/rms={err / rms:.4f} "
         f"(not gated; the default path's bar is {mc.E2E_ABS_FRAC}) cos={cos:.7f}")
    assert cos >= mc.E2E_COS, f"cos {cos:.7f}"


def test_fp8_mfma_rejects_decode_windows_and_fused_launch():
    """mfma_fp8 runs on the LDS-staged kernels in two launches: windows of 16 /
    32 rows or fuse_l1l2 are rejected with kErrUnsupported (6)."""
    _say("fp8 MFMA option checks")
    E, K, H, I, T = 16, 4, 512, 256, 64
    c = mc.normal_case(E, K, H, I, T, seed=3, scaled=True)
    sp = torch.cuda.current_stream().cuda_stream
    for win, fuse in ((16, False), (32, False), (0, True)):
        buf = mm.get_symm_buffer_for_mega_moe(None, E, T, K, H, I, expert_window=win)
        buf.mfma_fp8 = True
        buf.fuse_l1l2 = fuse
        y = torch.empty((T, H), dtype=torch.bfloat16, device="cuda")
        a = buf.make_args(T, (c.w1, c.s1), (c.w2, c.s2), y_bf16=y)
        assert mm.lib().mm_launch_full(ctypes.byref(a), sp) == 6, (win, fuse)
    torch.cuda.synchronize()
