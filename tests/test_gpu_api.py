"""GPU tests of the operator API around the layer: the split compute / reduce
pair, the reference's launch-time switches, skip_prologue (alone and as graph
nodes), empty batches, output checks and the device status words.  Every
result is compared bit for bit with the plain full-layer launch of the same
inputs, which the parity tests check against the oracle."""
import ctypes
import sys

import numpy as np
import pytest
import torch

import mini_mega_amd as mm
from mini_mega_amd import inputs

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


def _stream():
    return torch.cuda.current_stream().cuda_stream


def _load(buf, c):
    buf.x.view(torch.uint8)[:c.T].copy_(torch.from_numpy(c.x))
    if c.xsf is not None:
        buf.x_sf[:c.T].copy_(torch.from_numpy(c.xsf))
    buf.topk_idx[:c.T].copy_(torch.from_numpy(c.idx))
    buf.topk_weights[:c.T].copy_(torch.from_numpy(c.wts))


def _full(buf, c):
    y = torch.empty((c.T, c.H), dtype=torch.bfloat16, device="cuda")
    mm.fp8_mega_moe(y, (c.w1, c.s1), (c.w2, c.s2), buf)
    torch.cuda.synchronize()
    return y.clone()


def test_split_compute_reduce_equals_full_layer():
    """fp8_mega_moe_compute, an unrelated kernel, then fp8_mega_moe_reduce give
    the full layer's output bit for bit (reference mega/__init__.py:658-712,
    torch/csrc/apis/mega.hpp:332-366)."""
    _say("split compute / reduce")
    E, K, H, I, T = 32, 8, 1024, 512, 200
    c = mc.normal_case(E, K, H, I, T, seed=91, scaled=True)
    buf = mm.get_symm_buffer_for_mega_moe(None, E, T, K, H, I)
    _load(buf, c)
    y_full = _full(buf, c)
    # unrelated work between the two halves, on the same stream
    a = torch.randn(512, 512, device="cuda")
    mm.fp8_mega_moe_compute((c.w1, c.s1), (c.w2, c.s2), buf, T)
    _ = a @ a
    y = torch.empty((T, H), dtype=torch.bfloat16, device="cuda")
    y.fill_(7.0)
    mm.fp8_mega_moe_reduce(y, buf)
    torch.cuda.synchronize()
    assert torch.equal(y, y_full)
    # a prefix of the tokens reduces to the prefix of the output
    y5 = torch.empty((5, H), dtype=torch.bfloat16, device="cuda")
    mm.fp8_mega_moe_reduce(y5, buf)
    torch.cuda.synchronize()
    assert torch.equal(y5, y_full[:5])


def test_reference_env_switches_skip_the_reduce(monkeypatch):
    """The reference's launch-time switches (src/megakernel.cu:137-139,255-258):
    MX_SKIP_REDUCE=1 makes launch_full run the compute only, MX_SKIP_COMBINE=1
    makes launch_reduce a no-op; without them the reduce of that computed
    routing gives the full layer's output."""
    _say("MX_SKIP_REDUCE / MX_SKIP_COMBINE")
    L = mm.lib()
    E, K, H, I, T = 32, 8, 1024, 512, 96
    c = mc.normal_case(E, K, H, I, T, seed=93, scaled=True)
    buf = mm.get_symm_buffer_for_mega_moe(None, E, T, K, H, I)
    _load(buf, c)
    y_full = _full(buf, c)
    y = torch.full((T, H), 7.0, dtype=torch.bfloat16, device="cuda")
    a = buf.make_args(T, (c.w1, c.s1), (c.w2, c.s2), y_bf16=y)
    monkeypatch.setenv("MX_SKIP_REDUCE", "1")
    assert L.mm_launch_full(ctypes.byref(a), _stream()) == 0
    torch.cuda.synchronize()
    assert bool((y == 7.0).all()), "launch_full reduced under MX_SKIP_REDUCE=1"
    monkeypatch.delenv("MX_SKIP_REDUCE")
    monkeypatch.setenv("MX_SKIP_COMBINE", "1")
    assert L.mm_launch_reduce(ctypes.byref(a), _stream()) == 0
    torch.cuda.synchronize()
    assert bool((y == 7.0).all()), "launch_reduce wrote y under MX_SKIP_COMBINE=1"
    monkeypatch.setenv("MX_SKIP_COMBINE", "0")
    assert L.mm_launch_reduce(ctypes.byref(a), _stream()) == 0
    torch.cuda.synchronize()
    assert torch.equal(y, y_full)


def test_split_reduce_rejects_bad_calls():
    _say("split reduce argument checks")
    E, K, H, I, T = 8, 2, 256, 128, 16
    c = mc.normal_case(E, K, H, I, T, seed=92, scaled=True)
    buf = mm.get_symm_buffer_for_mega_moe(None, E, T, K, H, I)
    _load(buf, c)
    y = torch.empty((T, H), dtype=torch.bfloat16, device="cuda")
    with pytest.raises(RuntimeError):
        mm.fp8_mega_moe_reduce(y, buf)            # no compute yet
    mm.fp8_mega_moe_compute((c.w1, c.s1), (c.w2, c.s2), buf, 10)
    with pytest.raises(ValueError):
        mm.fp8_mega_moe_reduce(y, buf)            # 16 > the 10 computed tokens
    with pytest.raises(ValueError):
        mm.fp8_mega_moe_reduce(torch.empty((10, H + 128), dtype=torch.bfloat16,
                                           device="cuda"), buf)
    with pytest.raises(TypeError):
        mm.fp8_mega_moe_reduce(torch.empty((10, H), dtype=torch.float32, device="cuda"), buf)
    with pytest.raises(ValueError):
        mm.fp8_mega_moe(torch.empty((T, H // 2), dtype=torch.bfloat16, device="cuda"),
                        (c.w1, c.s1), (c.w2, c.s2), buf)
    with pytest.raises(ValueError):
        mm.fp8_mega_moe(torch.empty((T, H), dtype=torch.bfloat16), (c.w1, c.s1),
                        (c.w2, c.s2), buf)    # host tensor
    with pytest.raises(ValueError):
        mm.fp8_mega_moe_compute((c.w1, c.s1), (c.w2, c.s2), buf, 12, skip_prologue=1)
    torch.cuda.synchronize()


def test_skip_prologue_bf16_input_refolds_x():
    """A bf16xfp8 buffer, two launches with the same routing and different x,
    the second with skip_prologue=1: only the routing is reused, x is folded
    again, so the output equals a fresh launch on the new x."""
    _say("skip_prologue with a new bf16 x")
    E, K, H, I, T = 16, 4, 512, 256, 64
    xb1, _, _ = inputs.make_x(T, H, seed=5, scaled=True)
    xb2, _, _ = inputs.make_x(T, H, seed=6, scaled=True)
    (w1, s1), (w2, s2) = inputs.make_weights_normal(E, H, I, seed=7)
    idx, wts = inputs.route(T, E, K, seed=8)

    def buffer():
        b = mm.get_symm_buffer_for_mega_moe(None, E, T, K, H, I, mma_type="bf16xfp8")
        b.topk_idx[:T].copy_(torch.from_numpy(idx))
        b.topk_weights[:T].copy_(torch.from_numpy(wts))
        return b

    fresh = buffer()
    fresh.x[:T].copy_(xb2)
    y_want = torch.empty((T, H), dtype=torch.bfloat16, device="cuda")
    mm.bf16_fp8_mega_moe(y_want, (w1, s1), (w2, s2), fresh)

    buf = buffer()
    buf.x[:T].copy_(xb1)
    y1 = torch.empty((T, H), dtype=torch.bfloat16, device="cuda")
    mm.bf16_fp8_mega_moe(y1, (w1, s1), (w2, s2), buf)
    buf.x[:T].copy_(xb2)
    mm.fp8_mega_moe_compute((w1, s1), (w2, s2), buf, T, skip_prologue=1)
    y2 = torch.empty((T, H), dtype=torch.bfloat16, device="cuda")
    mm.fp8_mega_moe_reduce(y2, buf)
    torch.cuda.synchronize()
    assert not torch.equal(y1, y_want)
    assert torch.equal(y2, y_want)


def test_graph_with_skip_prologue_nodes_matches_eager():
    """A graph of N launches whose nodes 2..N reuse the first node's routing
    (skip_prologue=1, the reference's non-first graph nodes,
    src/megakernel.h:106, test/check.cu:533-745), replayed three times with
    eager launches in between: every output equals the eager launch."""
    _say("graph with skip_prologue nodes")
    E, K, H, I, T = 32, 8, 1024, 512, 128
    c = mc.normal_case(E, K, H, I, T, seed=93, scaled=True)
    buf = mm.get_symm_buffer_for_mega_moe(None, E, T, K, H, I)
    _load(buf, c)
    y_eager = _full(buf, c)
    L = mm.lib()
    ys = [torch.empty((T, H), dtype=torch.bfloat16, device="cuda") for _ in range(4)]
    args = [buf.make_args(T, (c.w1, c.s1), (c.w2, c.s2), y_bf16=y, skip_prologue=int(i > 0))
            for i, y in enumerate(ys)]
    torch.cuda.synchronize()
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        g = torch.cuda.CUDAGraph()
        with torch.cuda.graph(g, stream=s):
            for a in args:
                rc = L.mm_launch_full(ctypes.byref(a), s.cuda_stream)
                assert rc == 0
    torch.cuda.current_stream().wait_stream(s)
    for rep in range(3):
        for y in ys:
            y.zero_()
        torch.cuda.synchronize()
        g.replay()
        torch.cuda.synchronize()
        for i, y in enumerate(ys):
            assert torch.equal(y, y_eager), f"replay {rep} node {i} differs"
        assert torch.equal(_full(buf, c), y_eager)


def test_empty_batch_on_fresh_buffer():
    """T=0 on a buffer that has never run, with only the bf16 output: the
    launch succeeds (reference fp8_mega_moe with num_tokens = 0), also through
    the C ABI with both outputs null."""
    _say("empty batch on a fresh buffer")
    E, K, H, I = 16, 4, 512, 256
    buf = mm.get_symm_buffer_for_mega_moe(None, E, 32, K, H, I)
    assert buf.write_fp32_y is False
    (w1, s1), (w2, s2) = inputs.make_weights_normal(E, H, I, seed=9)
    y0 = torch.empty((0, H), dtype=torch.bfloat16, device="cuda")
    mm.fp8_mega_moe(y0, (w1, s1), (w2, s2), buf)
    a = buf.make_args(0, (w1, s1), (w2, s2))
    a.y = None
    a.y_bf16 = None
    assert mm.lib().mm_launch_full(ctypes.byref(a), _stream()) == 0
    torch.cuda.synchronize()
    assert int(buf.counts().abs().sum()) == 0
    st = buf.device_status()
    assert st["error"] == 0 and st["slots"] == 0 and st["items"] == 0


def test_device_status_words():
    """The status words read through the C ABI after a launch: routed slots,
    work items, pairs dropped by the slot capacity, invalid expert ids."""
    _say("device status words")
    E, K, H, I, T, cap = 32, 8, 1024, 512, 200, 30
    c = mc.normal_case(E, K, H, I, T, seed=51, scaled=True)
    idx = c.idx.copy()
    idx[3, 0], idx[7, 5], idx[100, 2] = -1, E + 3, E
    import dataclasses
    c = dataclasses.replace(c, idx=idx, cap=cap)
    r = mc.run_layer(c)
    st = r.buf.device_status()
    from oracle import oracle as orc
    counts, offsets, perm, pair_pos = orc.route(idx, E, cap)
    valid = int(((idx >= 0) & (idx < E)).sum())
    assert st["error"] == 0
    assert st["slots"] == int(offsets[-1])
    assert st["invalid_ids"] == 3
    assert st["dropped_by_capacity"] == valid - int(offsets[-1]) > 0
    assert st["items"] == int(r.status[1])


def _outputs(buf, c, y):
    slots = int(buf.offsets()[-1])
    return (y.view(torch.int16).cpu().numpy(), buf.ffn(max(slots, 1)).cpu().numpy()[:slots],
            buf.l2_out(max(slots, 1)).cpu().numpy()[:slots])


@pytest.mark.parametrize("E,K,H,I,T,zipf,win,scaled", [
    (32, 8, 1024, 512, 300, None, 0, True),
    (64, 4, 2048, 768, 200, 1.1, 64, True),
    (32, 8, 1024, 512, 300, None, 128, False),
    (256, 8, 6144, 2048, 512, None, 0, True),
    (256, 8, 6144, 2048, 2048, 1.1, 0, True),
    (256, 8, 6144, 2048, 8192, None, 0, True),
])
def test_fused_l1l2_matches_two_launches(E, K, H, I, T, zipf, win, scaled):
    """fuse_l1l2 (L1 and L2 in one launch, per-item ready counters): y, the
    ffn bytes and the L2 rows are bit-identical to the two stream-ordered
    launches, on small and full-size layers, skewed routing, fixed windows and
    the raw (unscaled) path; no wait times out.  Then a launch reusing the
    routing (skip_prologue, ready counters zeroed by the host path) and a
    graph of two fused launches replayed twice give the same outputs."""
    _say(f"fused L1->L2 E={E} T={T} zipf={zipf} win={win} scaled={scaled}")
    c = mc.normal_case(E, K, H, I, T, seed=T + 7, scaled=scaled, zipf=zipf, win=win)
    buf = mm.get_symm_buffer_for_mega_moe(None, E, T, K, H, I, expert_window=win)
    _load(buf, c)
    l1 = (c.w1, c.s1) if scaled else c.w1
    l2 = (c.w2, c.s2) if scaled else c.w2
    y = torch.empty((T, H), dtype=torch.bfloat16, device="cuda")
    mm.fp8_mega_moe(y, l1, l2, buf)
    torch.cuda.synchronize()
    want = _outputs(buf, c, y)
    buf.fuse_l1l2 = True
    for rep in range(2):
        y.zero_()
        buf.workspace[int(buf.layout.ffn):].zero_()
        mm.fp8_mega_moe(y, l1, l2, buf)
        torch.cuda.synchronize()
        got = _outputs(buf, c, y)
        for g, w, name in zip(got, want, ("y", "ffn", "l2")):
            assert np.array_equal(g, w), f"fused launch {rep}: {name} differs"
        assert buf.device_status()["error"] == 0
    # routing reused: the host zeroes the ready counters itself
    y.zero_()
    a = buf.make_args(T, l1, l2, y_bf16=y, skip_prologue=1)
    assert mm.lib().mm_launch_full(ctypes.byref(a), _stream()) == 0
    torch.cuda.synchronize()
    assert np.array_equal(_outputs(buf, c, y)[0], want[0]), "fused skip_prologue differs"
    assert buf.device_status()["error"] == 0
    # two fused launches as one graph, replayed twice
    ys = [torch.empty((T, H), dtype=torch.bfloat16, device="cuda") for _ in range(2)]
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        g = torch.cuda.CUDAGraph()
        with torch.cuda.graph(g, stream=s):
            for yy in ys:
                mm.fp8_mega_moe(yy, l1, l2, buf)
    torch.cuda.current_stream().wait_stream(s)
    for rep in range(2):
        for yy in ys:
            yy.zero_()
        torch.cuda.synchronize()
        g.replay()
        torch.cuda.synchronize()
        for yy in ys:
            assert np.array_equal(yy.view(torch.int16).cpu().numpy(), want[0]), \
                f"fused graph replay {rep} differs"
    buf.destroy()


@pytest.mark.parametrize("E,K,H,I,T,zipf,win,scaled,walks", [
    (32, 8, 1024, 512, 300, None, 0, True, True),
    (32, 8, 1024, 512, 300, None, 0, False, True),
    (48, 8, 1024, 1024, 600, 1.1, 128, True, True),
    (64, 4, 2048, 768, 200, 1.1, 64, True, False),
    (256, 8, 6144, 2048, 512, None, 0, True, False),
    (256, 8, 6144, 2048, 2048, None, 0, True, True),
])
def test_l2_walk_matches_one_unit_kernel(E, K, H, I, T, zipf, win, scaled, walks):
    """The L2 walk (one workgroup per CU, the next unit's weights streamed during
    the current one) runs when the largest work item has 3..8 token tiles and
    I / 128 is a multiple of 4 (the host tries it above 16 routed rows per
    expert on average); otherwise the one-unit-per-workgroup kernel launched
    after it does.  y, the ffn bytes and the L2 rows are bit-identical with the
    walk disabled (l2_no_walk), including split experts (a 128-row window under
    skew) and the raw path; a graph of two launches replays to the same y."""
    _say(f"L2 walk E={E} T={T} zipf={zipf} win={win} scaled={scaled}")
    c = mc.normal_case(E, K, H, I, T, seed=T + 11, scaled=scaled, zipf=zipf, win=win)
    buf = mm.get_symm_buffer_for_mega_moe(None, E, T, K, H, I, expert_window=win)
    _load(buf, c)
    l1 = (c.w1, c.s1) if scaled else c.w1
    l2 = (c.w2, c.s2) if scaled else c.w2
    y = torch.empty((T, H), dtype=torch.bfloat16, device="cuda")
    buf.l2_walk = False
    mm.fp8_mega_moe(y, l1, l2, buf)
    torch.cuda.synchronize()
    want = _outputs(buf, c, y)
    st = buf.device_status()
    rows = st["max_item_rows"]
    assert st["error"] == 0 and rows > 0
    assert (32 < rows <= 128 and (I // 128) % 4 == 0) == walks, f"max item rows {rows}"
    buf.l2_walk = True
    for rep in range(2):
        y.zero_()
        buf.workspace[int(buf.layout.ffn):].zero_()
        mm.fp8_mega_moe(y, l1, l2, buf)
        torch.cuda.synchronize()
        got = _outputs(buf, c, y)
        for g, w, name in zip(got, want, ("y", "ffn", "l2")):
            assert np.array_equal(g, w), f"walk launch {rep}: {name} differs"
    assert buf.device_status()["error"] == 0
    # two launches (walk and one-unit kernel each) as one graph, replayed twice
    ys = [torch.empty((T, H), dtype=torch.bfloat16, device="cuda") for _ in range(2)]
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        g = torch.cuda.CUDAGraph()
        with torch.cuda.graph(g, stream=s):
            for yy in ys:
                mm.fp8_mega_moe(yy, l1, l2, buf)
    torch.cuda.current_stream().wait_stream(s)
    for rep in range(2):
        for yy in ys:
            yy.zero_()
        g.replay()
        torch.cuda.synchronize()
        for yy in ys:
            assert np.array_equal(yy.view(torch.int16).cpu().numpy(), want[0]), \
                f"walk graph replay {rep} differs"


def test_fused_l1l2_bounded_wait_reports_timeout():
    """The fused launch's give-up path, forced from the host: ready_bias = 1
    raises every L2 unit's ready target past the count its item's L1 blocks
    reach, and max_spins = 1 bounds each wait to one poll.  Every kernel still
    ends (every wait is bounded), every L2 unit gives up and sets
    kStatusWaitTimeout, and read_status reports it as a device error (7).  A
    launch whose counters all arrive (max_spins = 1, no bias) may or may not
    time out, and is exact when it does not.  The next launch with the
    default bound is exact again."""
    _say("fused L1->L2 give-up: ready_bias=1, max_spins=1")
    E, K, H, I, T = 256, 8, 6144, 2048, 2048
    c = mc.normal_case(E, K, H, I, T, seed=99, scaled=True)
    buf = mm.get_symm_buffer_for_mega_moe(None, E, T, K, H, I)
    _load(buf, c)
    y = torch.empty((T, H), dtype=torch.bfloat16, device="cuda")
    mm.fp8_mega_moe(y, (c.w1, c.s1), (c.w2, c.s2), buf)
    torch.cuda.synchronize()
    want = y.view(torch.int16).cpu().numpy()
    buf.fuse_l1l2 = True
    out = (ctypes.c_int * 5)()
    # forced: every wait gives up
    a = buf.make_args(T, (c.w1, c.s1), (c.w2, c.s2), y_bf16=y)
    a.max_spins, a.ready_bias = 1, 1
    assert mm.lib().mm_launch_full(ctypes.byref(a), _stream()) == 0
    torch.cuda.synchronize()
    st = buf.device_status()
    rc = mm.lib().mm_read_status(ctypes.byref(a), out, 5, _stream())
    _say(f"  forced: error bits {st['error']}, read_status {rc}")
    assert st["error"] == 2 and rc == 7
    # counters that all arrive, one poll each: exact unless a wait gave up
    a = buf.make_args(T, (c.w1, c.s1), (c.w2, c.s2), y_bf16=y)
    a.max_spins = 1
    assert mm.lib().mm_launch_full(ctypes.byref(a), _stream()) == 0
    torch.cuda.synchronize()
    st = buf.device_status()
    rc = mm.lib().mm_read_status(ctypes.byref(a), out, 5, _stream())
    timed_out = bool(st["error"] & 2)
    _say(f"  unforced: timeout bit set: {timed_out}")
    assert st["error"] & ~2 == 0
    assert rc == (7 if timed_out else 0)
    if not timed_out:
        assert np.array_equal(y.view(torch.int16).cpu().numpy(), want)
    mm.fp8_mega_moe(y, (c.w1, c.s1), (c.w2, c.s2), buf)
    torch.cuda.synchronize()
    assert buf.device_status()["error"] == 0
    assert np.array_equal(y.view(torch.int16).cpu().numpy(), want)
    buf.destroy()
