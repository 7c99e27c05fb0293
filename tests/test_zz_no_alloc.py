"""The allocation-free entry point mm_launch_full_noalloc (workspace in the
library's fixed per-GPU scratch array) against mm_launch_full with a
caller-owned workspace, through the C ABI: two calls in a row, the second with
a smaller input, each bit-identical to the existing entry point's output;
sizes past the scratch are rejected with kErrScratch."""
import ctypes
import sys

import numpy as np
import pytest
import torch

import mini_mega_amd as mm

import moe_case as mc

pytestmark = pytest.mark.gpu


def _say(msg):
    print(f"[case] {msg}", flush=True)
    sys.stdout.flush()


@pytest.fixture(scope="module", autouse=True)
def _gpu():
    assert torch.cuda.is_available(), "GPU tests need an MI355X"
    torch.cuda.set_device(0)
    mm.lib()
    yield


def _both(c, buf):
    """Runs case c through mm_launch_full (buf's workspace) and through
    mm_launch_full_noalloc on the same input views; returns both outputs."""
    L = mm.lib()
    sp = torch.cuda.current_stream().cuda_stream
    buf.x.view(torch.uint8)[:c.T].copy_(torch.from_numpy(c.x))
    if c.xsf is not None:
        buf.x_sf[:c.T].copy_(torch.from_numpy(c.xsf))
    buf.topk_idx[:c.T].copy_(torch.from_numpy(c.idx))
    buf.topk_weights[:c.T].copy_(torch.from_numpy(c.wts))
    outs = []
    for fn in (L.mm_launch_full, L.mm_launch_full_noalloc):
        y = torch.full((c.T, c.H), 3.0, dtype=torch.bfloat16, device="cuda")
        y32 = torch.full((c.T, c.H), 5.0, dtype=torch.float32, device="cuda")
        a = buf.make_args(c.T, (c.w1, c.s1), (c.w2, c.s2), y_bf16=y, y_fp32=y32)
        if fn is L.mm_launch_full_noalloc:
            a.rwk = None                    # ignored: the scratch replaces it
            a.workspace_bytes = 0
        assert fn(ctypes.byref(a), sp) == 0
        torch.cuda.synchronize()
        outs.append((y, y32))
    return outs


@pytest.mark.parametrize("sizes", [((32, 8, 1024, 512), (200, 37)),
                                   ((256, 8, 6144, 2048), (512, 96))])
def test_noalloc_matches_full_twice(sizes):
    (E, K, H, I), (T1, T2) = sizes
    buf = mm.get_symm_buffer_for_mega_moe(None, E, T1, K, H, I)
    for T, seed in ((T1, 11), (T2, 12)):
        _say(f"noalloc E={E} H={H} I={I} T={T} (buffer for {T1})")
        c = mc.normal_case(E, K, H, I, T, seed=seed, scaled=True)
        (y, y32), (z, z32) = _both(c, buf)
        assert torch.equal(y, z), f"bf16 y differs at T={T}"
        assert torch.equal(y32.view(torch.int32), z32.view(torch.int32)), f"fp32 y differs at T={T}"
        assert float(y.float().abs().max()) > 0


def test_noalloc_rejects_sizes_past_the_scratch():
    _say("noalloc size limit")
    L = mm.lib()
    limit = int(L.mm_noalloc_scratch_bytes())
    assert limit == 64 << 20
    E, K, H, I = 256, 8, 6144, 2048
    big = 4096
    assert int(mm.layout(big, K, E, H, I).total) > limit
    buf = mm.get_symm_buffer_for_mega_moe(None, E, 16, K, H, I)
    a = buf.make_args(16, buf.x, buf.x)
    a.max_tokens = big
    assert L.mm_launch_full_noalloc(ctypes.byref(a),
                                    torch.cuda.current_stream().cuda_stream) == 8
    torch.cuda.synchronize()
