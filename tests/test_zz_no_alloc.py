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


def _noalloc_args(buf, c, y, skip_prologue=0, T=None):
    a = buf.make_args(c.T if T is None else T, (c.w1, c.s1), (c.w2, c.s2), y_bf16=y,
                      skip_prologue=skip_prologue)
    a.rwk = None
    a.workspace_bytes = 0
    return a


def test_noalloc_skip_prologue_needs_the_routed_shape():
    """skip_prologue reuses the scratch's routing only when the last routed
    call on this GPU had the same shape (E, topk, H, I, max_tokens, win_cap,
    tokens); otherwise the call is rejected with kErrUnsupported (6) before
    any launch.  With the same shape it equals mm_launch_full."""
    _say("noalloc skip_prologue routing-shape check")
    L = mm.lib()
    sp = torch.cuda.current_stream().cuda_stream
    E, K, H, I, T1 = 32, 8, 1024, 512, 200
    buf = mm.get_symm_buffer_for_mega_moe(None, E, T1, K, H, I)
    c = mc.normal_case(E, K, H, I, T1, seed=21, scaled=True)
    (y, _), (z, _) = _both(c, buf)          # the noalloc call routes T1 tokens
    assert torch.equal(y, z)
    w = torch.full_like(y, 7.0)
    # another token count: rejected, nothing launched (w untouched)
    assert L.mm_launch_full_noalloc(ctypes.byref(_noalloc_args(buf, c, w, 1, T=37)), sp) == 6
    torch.cuda.synchronize()
    assert bool((w == 7.0).all())
    # the routed shape: reuses the routing, equal output
    assert L.mm_launch_full_noalloc(ctypes.byref(_noalloc_args(buf, c, w, 1)), sp) == 0
    torch.cuda.synchronize()
    assert torch.equal(w, y)
    # a routed call of another layer shape, then skip_prologue of the first: rejected
    E2, H2, I2, T2 = 16, 512, 256, 64
    buf2 = mm.get_symm_buffer_for_mega_moe(None, E2, T2, K, H2, I2)
    c2 = mc.normal_case(E2, K, H2, I2, T2, seed=22, scaled=True)
    (y2, _), (z2, _) = _both(c2, buf2)
    assert torch.equal(y2, z2)
    w.fill_(7.0)
    assert L.mm_launch_full_noalloc(ctypes.byref(_noalloc_args(buf, c, w, 1)), sp) == 6
    torch.cuda.synchronize()
    assert bool((w == 7.0).all())


def test_noalloc_allocates_nothing_and_replays_in_a_graph():
    """An eager mm_launch_full_noalloc leaves the device's free memory
    unchanged; two calls captured in a graph (global capture mode, under which
    a device allocation fails) replay three times, with eager launches of
    another shape on the same scratch in between, each replay equal to
    mm_launch_full."""
    _say("noalloc: no allocation, graph capture and replay")
    L = mm.lib()
    E, K, H, I, T = 32, 8, 1024, 512, 160
    buf = mm.get_symm_buffer_for_mega_moe(None, E, T, K, H, I)
    c = mc.normal_case(E, K, H, I, T, seed=31, scaled=True)
    (y, _), (z, _) = _both(c, buf)
    assert torch.equal(y, z)
    w = torch.empty_like(y)
    a = _noalloc_args(buf, c, w)
    torch.cuda.synchronize()
    free0, _ = torch.cuda.mem_get_info()
    assert L.mm_launch_full_noalloc(ctypes.byref(a), torch.cuda.current_stream().cuda_stream) == 0
    torch.cuda.synchronize()
    free1, _ = torch.cuda.mem_get_info()
    assert free1 == free0, f"free device memory moved by {free0 - free1} bytes"
    assert torch.equal(w, y)
    # other work between the replays: a routed noalloc call of another shape
    E2, H2, I2, T2 = 16, 512, 256, 64
    buf2 = mm.get_symm_buffer_for_mega_moe(None, E2, T2, K, H2, I2)
    c2 = mc.normal_case(E2, K, H2, I2, T2, seed=32, scaled=True)
    (y2, _), _ = _both(c2, buf2)
    ys = [torch.empty_like(y) for _ in range(2)]
    args = [_noalloc_args(buf, c, yy) for yy in ys]
    torch.cuda.synchronize()
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        g = torch.cuda.CUDAGraph()
        with torch.cuda.graph(g, stream=s):
            for aa in args:
                assert L.mm_launch_full_noalloc(ctypes.byref(aa), s.cuda_stream) == 0
    torch.cuda.current_stream().wait_stream(s)
    for rep in range(3):
        for yy in ys:
            yy.zero_()
        torch.cuda.synchronize()
        g.replay()
        torch.cuda.synchronize()
        for i, yy in enumerate(ys):
            assert torch.equal(yy, y), f"replay {rep} node {i} differs"
        w2 = torch.empty_like(y2)
        assert L.mm_launch_full_noalloc(ctypes.byref(_noalloc_args(buf2, c2, w2)),
                                        torch.cuda.current_stream().cuda_stream) == 0
        torch.cuda.synchronize()
        assert torch.equal(w2, y2)
