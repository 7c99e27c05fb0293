"""GPU parity tests: the HIP layer (through the C ABI) against the oracle.

Bars: routing / permutation / counts / byte work bit-exact; L1, L2, REDUCE at
check.cu's staged tolerances; the whole layer at max|d| <= 2e-2 rms(y) and
cos >= 0.9995 on the fp32 y, with the bf16 y its exact RNE cast and within
the same bar beyond its own half-ulp (moe_case.e2e_gate).
"""
import ctypes
import dataclasses
import sys

import numpy as np
import pytest
import torch

import mini_mega_amd as mm
from mini_mega_amd import inputs
from oracle import oracle as orc

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


# --------------------------------------------------------- device codecs --
def test_device_fp8_and_bf16_conversion_bit_exact():
    _say("convert selftest")
    t = orc.e4m3_decode_table()
    fin = np.sort(np.unique(t[np.isfinite(t)]))
    mids = (fin[1:] + fin[:-1]) / 2
    rng = np.random.default_rng(3)
    v = np.concatenate([fin, mids, np.nextafter(mids.astype(np.float32), np.float32(1e9)),
                        np.nextafter(mids.astype(np.float32), np.float32(-1e9)),
                        rng.standard_normal(20000) * 30, rng.standard_normal(5000) * 0.01,
                        [448.0, 464.0, 500.0, 1e6, -1e6, 0.0, -0.0]]).astype(np.float32)
    src = torch.from_numpy(v).cuda()
    o8 = torch.empty(v.size, dtype=torch.uint8, device="cuda")
    o16 = torch.empty(v.size, dtype=torch.int16, device="cuda")
    assert mm.lib().mm_selftest_convert(src.data_ptr(), v.size, o8.data_ptr(), o16.data_ptr(),
                                        _stream()) == 0
    torch.cuda.synchronize()
    assert np.array_equal(o8.cpu().numpy(), orc.e4m3_quantize(v))
    assert np.array_equal(o16.cpu().numpy().view(np.uint16), orc.f32_to_bf16(v))
    # bf16 rounding (the GEMM epilogue's v_cvt_pk_bf16_f32) on random fp32 bit
    # patterns, exact bf16 ties and their neighbours, denormals and the overflow
    # edge; NaN is excluded (the hardware quiets it, the reference keeps its bits)
    bits = rng.integers(0, 2**32, size=200000, dtype=np.uint64).astype(np.uint32)
    hb = rng.integers(0, 2**16, size=50000, dtype=np.uint64).astype(np.uint32) << 16
    ties = np.concatenate([hb | 0x8000, (hb | 0x8000) + 1, (hb | 0x8000) - 1, hb | 0x7FFF])
    edge = np.array([0x00000001, 0x00008000, 0x007FFFFF, 0x00800000, 0x7F7F7FFF, 0x7F7F8000,
                     0x7F7FFFFF, 0x7F800000, 0xFF800000, 0x80000001, 0xFF7FFFFF],
                    dtype=np.uint32)
    u = np.concatenate([bits, ties, edge])
    u = u[(u & 0x7FFFFFFF) <= 0x7F800000]
    vb = u.view(np.float32)
    srcb = torch.from_numpy(vb.copy()).cuda()
    o8b = torch.empty(vb.size, dtype=torch.uint8, device="cuda")
    o16b = torch.empty(vb.size, dtype=torch.int16, device="cuda")
    assert mm.lib().mm_selftest_convert(srcb.data_ptr(), vb.size, o8b.data_ptr(), o16b.data_ptr(),
                                        _stream()) == 0
    torch.cuda.synchronize()
    assert np.array_equal(o16b.cpu().numpy().view(np.uint16), orc.f32_to_bf16(vb))


def test_pack_weights_roundtrip():
    _say("pack roundtrip")
    rng = np.random.default_rng(4)
    w = rng.integers(0, 256, size=(3, 64, 384)).astype(np.uint8)
    packed = mm.pack_weights(torch.from_numpy(w).cuda().view(torch.float8_e4m3fn))
    torch.cuda.synchronize()
    p = packed.view(torch.uint8).cpu().numpy()
    for e in range(3):
        assert np.array_equal(inputs.unpack_tiles(p[e].ravel(), 64, 384), w[e])


@pytest.mark.parametrize("scaled", [False, True])
def test_transform_from_reference_layout(scaled):
    """Weights packed the reference's way (W1 gate/up paired every 256 rows,
    then its lane tiles, src/bench_check.cuh:268-272) convert to exactly the
    bytes transform_weights_for_mega_moe makes from the torch layout."""
    _say(f"transform from reference layout scaled={scaled}")
    E, H, I = 2, 384, 512
    rng = np.random.default_rng(11)
    w1 = rng.integers(0, 256, size=(E, 2 * I, H)).astype(np.uint8)
    w2 = rng.integers(0, 256, size=(E, H, I)).astype(np.uint8)
    # the reference's _interleave_weights(gran=256): [gate 0..255, up 0..255, gate 256..]
    g = w1[:, :I].reshape(E, I // 256, 256, H)
    u = w1[:, I:].reshape(E, I // 256, 256, H)
    w1_paired = np.stack([g, u], axis=2).reshape(E, 2 * I, H)
    r1 = torch.from_numpy(mc.ref_lane_pack(w1_paired)).cuda().view(torch.float8_e4m3fn)
    r2 = torch.from_numpy(mc.ref_lane_pack(w2)).cuda().view(torch.float8_e4m3fn)
    t1 = torch.from_numpy(w1).cuda().view(torch.float8_e4m3fn)
    t2 = torch.from_numpy(w2).cuda().view(torch.float8_e4m3fn)
    if scaled:
        s1 = torch.from_numpy(rng.integers(120, 135, size=(E, 2 * I // 128, H // 128))
                              .astype(np.uint8)).cuda()
        s2 = torch.from_numpy(rng.integers(120, 135, size=(E, H // 128, I // 128))
                              .astype(np.uint8)).cuda()
        (a1, as1), (a2, as2) = mm.transform_weights_from_reference((r1, s1), (r2, s2))
        (b1, bs1), (b2, bs2) = mm.transform_weights_for_mega_moe((t1, s1), (t2, s2))
        assert torch.equal(as1, bs1) and torch.equal(as2, bs2)
    else:
        a1, a2 = mm.transform_weights_from_reference(r1, r2)
        b1, b2 = mm.transform_weights_for_mega_moe(t1, t2)
    torch.cuda.synchronize()
    assert torch.equal(a1.view(torch.uint8), b1.view(torch.uint8))
    assert torch.equal(a2.view(torch.uint8), b2.view(torch.uint8))


def test_fill_weights_lane_matches_wprobe():
    _say("fill_weights_lane")
    n, k = 512, 768
    w = torch.empty(n * k, dtype=torch.uint8, device="cuda")
    assert mm.lib().mm_fill_weights_lane(w.data_ptr(), n, k, 17, _stream()) == 0
    torch.cuda.synchronize()
    got = inputs.unpack_tiles(w.cpu().numpy(), n, k)
    assert np.array_equal(got, orc.wprobe_matrix(17, 0, n, k))


@pytest.mark.parametrize("scaled", [True, False])
def test_quant_act_matches_oracle(scaled):
    _say(f"quant_act scaled={scaled}")
    xb, q, sf = inputs.make_x(64, 1024, seed=9, scaled=scaled)
    torch.cuda.synchronize()
    x32 = xb.float().cpu().numpy()
    if scaled:
        rq, rsf = orc.quant_rows_ue8m0(x32)
        assert np.array_equal(sf.cpu().numpy(), rsf)
    else:
        rq = orc.e4m3_quantize(x32).reshape(x32.shape)
    assert np.array_equal(q.cpu().numpy(), rq)


def test_weight_generator_scales_follow_recipe():
    _say("fill_weights_normal")
    (w1, s1), _ = inputs.make_weights_normal(2, 256, 128, seed=5)
    torch.cuda.synchronize()
    t = orc.e4m3_decode_table()
    wl = inputs.unpack_tiles(w1[1].view(torch.uint8).cpu().numpy().ravel(), 256, 256)
    s = s1[1].cpu().numpy().astype(np.int32)
    deq = t[wl].reshape(2, 128, 2, 128) * np.ldexp(1.0, s - 127)[:, None, :, None]
    amax_q = np.abs(t[wl]).reshape(2, 128, 2, 128).max(axis=(1, 3))
    assert np.all(amax_q <= 448) and np.all(amax_q >= 192)  # amax/sf in (224, 448] before RNE
    assert 0.015 < deq.std() < 0.025


# ----------------------------------------------------------------- routing --
def _route_only(E, K, H, I, idx, cap=0):
    T = idx.shape[0]
    buf = mm.get_symm_buffer_for_mega_moe(None, E, max(T, 1), K, H, I)
    if T:
        buf.topk_idx[:T].copy_(torch.from_numpy(idx))
    a = buf.make_args(T, buf.x, buf.x, slot_capacity=cap)  # weights unused by the prelude
    assert mm.lib().mm_launch_prelude(ctypes.byref(a), _stream()) == 0
    torch.cuda.synchronize()
    off = buf.offsets().cpu().numpy()
    slots = int(off[-1])
    return (buf.counts().cpu().numpy(), off,
            buf.perm(max(slots, 1)).cpu().numpy()[:slots].view(np.uint32),
            buf.pair_pos(max(T, 1)).cpu().numpy().ravel()[:T * K], buf.status().cpu().numpy())


def _check_route(E, K, idx, cap=0, H=256, I=128):
    counts, off, perm, pos, status = _route_only(E, K, H, I, idx, cap)
    rc, ro, rp, rpos = orc.route(idx, E, cap if cap else None)
    assert status[0] == 0
    assert np.array_equal(counts, rc)
    assert np.array_equal(off, ro)
    assert np.array_equal(perm, rp)
    assert np.array_equal(pos, rpos)


@pytest.mark.parametrize("T,K,E", [(32, 2, 8), (512, 8, 256), (2048, 8, 256), (8192, 8, 256),
                                   (1, 8, 256), (300, 6, 64), (1000, 8, 1024)])
def test_routing_bit_exact(T, K, E):
    _say(f"routing T={T} K={K} E={E}")
    idx, _ = inputs.route(T, E, K, seed=T + E)
    _check_route(E, K, idx)


def test_routing_invalid_ids_and_cap():
    _say("routing invalid ids + cap")
    rng = np.random.default_rng(7)
    idx = rng.integers(-3, 70, size=(700, 8)).astype(np.int64)  # E=64: ids 64..69 invalid
    _check_route(64, 8, idx)
    _check_route(64, 8, idx, cap=40)
    _check_route(64, 8, np.full((100, 8), 3, np.int64))  # one hot expert, duplicates


@pytest.mark.parametrize("launch", [804900, 809200, 853000])
def test_routing_tk_fixtures(launch):
    _say(f"routing TK launch {launch}")
    from test_oracle import _tk_launches
    per_expert = _tk_launches()[launch]
    idx = orc.routes_from_counts(per_expert, 32, 8, int(per_expert.sum()) // 256, 8)
    counts, *_ = _route_only(256, 8, 6144, 2048, idx)
    assert np.array_equal(counts, per_expert)
    _check_route(256, 8, idx, H=6144, I=2048)


def test_routing_skewed_zipf():
    _say("routing zipf")
    idx, _ = inputs.route(2048, 256, 8, seed=11, zipf_s=1.1)
    _check_route(256, 8, idx, H=6144, I=2048)


def test_dispatch_pool_is_gathered_rows():
    _say("dispatch pool")
    E, K, H, I, T = 16, 4, 512, 128, 100
    c = mc.normal_case(E, K, H, I, T, seed=21, scaled=False)
    r = mc.run_layer(c)
    slots = int(r.offsets[-1])
    pool = torch.empty((slots, H), dtype=torch.uint8, device="cuda")
    a = r.buf.make_args(T, c.w1, c.w2)
    assert mm.lib().mm_launch_dispatch(ctypes.byref(a), pool.data_ptr(), _stream()) == 0
    torch.cuda.synchronize()
    assert np.array_equal(pool.cpu().numpy(), c.x[r.perm // K])


# ------------------------------------------------------------- the layer --
SMALL = [
    # E, K, H, I, T, scaled, win
    (8, 2, 256, 128, 32, True, 0),      # the smoke workload
    (8, 2, 256, 128, 32, False, 0),
    (32, 8, 1024, 512, 200, True, 0),
    (32, 8, 1024, 512, 200, False, 16),
    (16, 4, 512, 256, 300, True, 64),
    (64, 8, 512, 256, 96, True, 32),
    # LDS-staged 8-wave kernels (work items of 64..256 rows, rows split evenly)
    (32, 8, 1024, 512, 160, False, 64),
    (16, 4, 512, 256, 600, True, 128),
    (8, 8, 256, 128, 300, True, 128),    # every token routed to every expert: 3 items each
    (8, 8, 256, 128, 250, True, 256),    # 250 rows per expert: one item of 16 token tiles
    (24, 6, 1024, 512, 700, True, 0),    # auto tile: 175 rows per expert -> one 256-row window
    (16, 4, 7168, 1280, 200, True, 0),   # H = 7168 (56 k-steps), I = 1280 (L2 k-loop remainder)
]


def test_every_token_tile_count():
    """Expert e gets 16(e+1) - 3 rows, so one 256-row window runs each of the
    big GEMMs' token-tile specialisations (1..16) on one item; every expert
    is checked staged."""
    E, K, H, I = 16, 8, 512, 256
    rows = [16 * (e + 1) - 3 for e in range(E)]
    ids = np.repeat(np.arange(E), rows)
    rng = np.random.default_rng(21)
    rng.shuffle(ids)
    T = ids.size // K
    idx = ids[:T * K].reshape(T, K).astype(np.int64)
    wts = rng.random((T, K)).astype(np.float32)
    wts /= wts.sum(axis=1, keepdims=True)
    _say(f"every token-tile count T={T}")
    c = mc.normal_case(E, K, H, I, T, seed=31, scaled=True, idx=idx, wts=wts)
    r = mc.run_layer(c)
    mc.check_routing(c, r)
    assert int(r.buf.layout.m_tile) == 256
    for e in range(E):
        mc.check_l1(c, r, e, max_rows=256)
        mc.check_l2(c, r, e, max_rows=256)
    mc.check_reduce(c, r)
    err, rms, cos = mc.check_e2e_tokens(c, r, [0, 1, T // 2, T - 1])
    _say(f"  subset e2e max_abs={err:.3e} rms={rms:.3e} cos={cos:.6f}")


@pytest.mark.parametrize("E,K,H,I,T,scaled,win", SMALL)
def test_layer_staged_and_e2e(E, K, H, I, T, scaled, win):
    _say(f"layer E={E} K={K} H={H} I={I} T={T} scaled={scaled} win={win}")
    c = mc.normal_case(E, K, H, I, T, seed=E + T, scaled=scaled, win=win)
    r = mc.run_layer(c)
    mc.check_routing(c, r)
    busiest = int(np.argmax(r.counts))
    for e in sorted({busiest, int(np.argmin(np.where(r.counts > 0, r.counts, 1 << 30)))}):
        mc.check_l1(c, r, e)
        mc.check_l2(c, r, e)
    mc.check_reduce(c, r)
    err, rms, cos = mc.check_e2e(c, r)
    _say(f"  e2e max_abs={err:.3e} rms={rms:.3e} cos={cos:.6f}")


def test_layer_bf16_input_fold():
    """bf16xfp8: x arrives as bf16 and is folded to fp8 inside the layer
    (reference x_fold_body, src/prologue.cuh:103-122)."""
    _say("bf16 input fold")
    E, K, H, I, T = 16, 4, 512, 256, 64
    xb, xq, xsf = inputs.make_x(T, H, seed=5, scaled=True)
    (w1, s1), (w2, s2) = inputs.make_weights_normal(E, H, I, seed=6)
    idx, wts = inputs.route(T, E, K, seed=7)
    buf = mm.get_symm_buffer_for_mega_moe(None, E, T, K, H, I, mma_type="bf16xfp8")
    buf.write_fp32_y = True
    buf.x[:T].copy_(xb)
    buf.topk_idx[:T].copy_(torch.from_numpy(idx))
    buf.topk_weights[:T].copy_(torch.from_numpy(wts))
    y = torch.empty((T, H), dtype=torch.bfloat16, device="cuda")
    mm.bf16_fp8_mega_moe(y, (w1, s1), (w2, s2), buf)
    torch.cuda.synchronize()
    c = mc.Case(E, K, H, I, T, xq.cpu().numpy(), xsf.cpu().numpy(), idx, wts, w1, s1, w2, s2)
    r = mc.Run(buf, y.float().cpu().numpy(), buf._y_fp32[:T].cpu().numpy(),
               buf.counts().cpu().numpy(), buf.offsets().cpu().numpy(), None, None, None)
    mc.check_e2e(c, r)


def test_single_token_then_empty_batch():
    """T=1 (K experts of one row each) at the staged and e2e tolerances; then
    T=0 on the same buffer: the launch succeeds, the expert counts are
    rewritten to zero (no stale counts from the previous call) and the
    cumulative per-expert stats gain nothing (reference
    mega/__init__.py:610-655 with num_tokens = 0)."""
    E, K, H, I = 32, 8, 1024, 512
    _say("single token T=1")
    c = mc.normal_case(E, K, H, I, 1, seed=43, scaled=True)
    r = mc.run_layer(c)
    mc.check_routing(c, r)
    for e in np.flatnonzero(r.counts):
        mc.check_l1(c, r, int(e))
        mc.check_l2(c, r, int(e))
    mc.check_reduce(c, r)
    mc.check_e2e(c, r)

    _say("empty batch T=0 after a T=1 call")
    buf = r.buf
    stats = torch.zeros(E, dtype=torch.int64, device="cuda")
    y1 = torch.empty((1, H), dtype=torch.bfloat16, device="cuda")
    mm.fp8_mega_moe(y1, (c.w1, c.s1), (c.w2, c.s2), buf,
                    cumulative_local_expert_recv_stats=stats)
    torch.cuda.synchronize()
    assert int(stats.sum()) == K and int(buf.counts().sum()) == K
    assert np.array_equal(y1.float().cpu().numpy(), r.y)
    y0 = torch.empty((0, H), dtype=torch.bfloat16, device="cuda")
    mm.fp8_mega_moe(y0, (c.w1, c.s1), (c.w2, c.s2), buf,
                    cumulative_local_expert_recv_stats=stats)
    torch.cuda.synchronize()
    assert int(buf.counts().abs().sum()) == 0
    assert int(buf.offsets().abs().sum()) == 0
    assert int(stats.sum()) == K


# -------------------------------------------------- check.cu-identical inputs --
@pytest.mark.parametrize("tpr", [1, 4, 16, 24, 32, 33, 64, 128, 256, 512])
def test_checkcu_inputs_full_size(tpr):
    """check.cu's own inputs at R=32 and every TPR of its balanced plans
    (kBalancedTprs, test/check.cu:49, and the smoke plan's 24, :922: T = 32
    .. 16384) remapped to one GPU:
    routing exact, every ffn byte saturated to 0x7E (closed form), L2 and
    REDUCE at check.cu tolerances."""
    _say(f"check.cu inputs TPR={tpr} (T={32 * tpr}) full size")
    c = mc.checkcu_case(32, tpr)
    r = mc.run_layer(c)
    mc.check_routing(c, r)
    slots = int(r.offsets[-1])
    assert slots == 32 * tpr * 8
    ffn = r.buf.ffn(slots).cpu().numpy()
    assert np.all(ffn == 0x7E)
    for e in (0, 7, 255):
        mc.check_l2(c, r, e)
    mc.check_reduce(c, r)


@pytest.mark.parametrize("launch", [804900, 809200])
def test_checkcu_tk_fixed_routes_full_layer(launch):
    """The reference smoke plan's recorded routes (TK_INFO launches 804900 and
    809200, its case0 / case2: test/check.cu:44-48,905-925) with check.cu's
    inputs at full size on one GPU: routing exact, every ffn byte saturated,
    L2 staged on the busiest and the lightest expert, REDUCE bit-exact, and a
    graph of three launches replayed bit-identical to the eager output (the
    plan's eager + graph x N pair)."""
    from test_oracle import _tk_launches
    per_expert = _tk_launches()[launch]
    tpr = int(per_expert.sum()) // (32 * 8)
    _say(f"check.cu inputs on TK launch {launch} (T={32 * tpr})")
    idx = orc.routes_from_counts(per_expert, 32, 8, tpr, 8)
    c = mc.checkcu_case(32, tpr, idx=idx)
    r = mc.run_layer(c)
    mc.check_routing(c, r)
    assert np.array_equal(r.counts, per_expert)
    slots = int(r.offsets[-1])
    assert np.all(r.buf.ffn(slots).cpu().numpy() == 0x7E)
    nz = np.nonzero(r.counts)[0]
    order = nz[np.argsort(r.counts[nz], kind="stable")]
    for e in {int(order[-1]), int(order[0])}:
        mc.check_l2(c, r, e)
    mc.check_reduce(c, r)
    ys = [torch.empty((c.T, c.H), dtype=torch.bfloat16, device="cuda") for _ in range(3)]
    torch.cuda.synchronize()
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        g = torch.cuda.CUDAGraph()
        with torch.cuda.graph(g, stream=s):
            for y in ys:
                mm.fp8_mega_moe(y, c.w1, c.w2, r.buf)
    torch.cuda.current_stream().wait_stream(s)
    for rep in range(2):
        for y in ys:
            y.zero_()
        torch.cuda.synchronize()
        g.replay()
        torch.cuda.synchronize()
        for y in ys:
            assert np.array_equal(y.float().cpu().numpy(), r.y), f"replay {rep} differs"


@pytest.mark.parametrize("launch", [45400, 84900, 151000])
def test_real_decode_routes_full_layer(launch):
    """Routes of the reference's real GLM-5.2 decode corpus (test/76.real_decode/
    dataset.tk_info: the most skewed launch, a median one and the smallest)
    through the full-size layer with the benchmark's scaled inputs: routing exact,
    staged L1/L2 on the busiest, a median and the lightest active expert,
    REDUCE bit-exact, and the whole chain on a token subset."""
    from test_oracle import _tk_launches
    per_expert = _tk_launches("tk_real_decode.log")[launch]
    tpr = int(per_expert.sum()) // (32 * 8)
    T = 32 * tpr
    _say(f"real decode launch {launch} (T={T}, busiest expert {int(per_expert.max())} rows)")
    idx = orc.routes_from_counts(per_expert, 32, 8, tpr, 8)
    _, wts = inputs.route(T, 256, 8, seed=launch)
    c = mc.normal_case(256, 8, 6144, 2048, T, seed=launch % 1000 + 5, scaled=True, idx=idx,
                       wts=wts)
    r = mc.run_layer(c)
    mc.check_routing(c, r)
    assert np.array_equal(r.counts, per_expert)
    nz = np.nonzero(r.counts)[0]
    order = nz[np.argsort(r.counts[nz], kind="stable")]
    for e in {int(order[-1]), int(order[len(order) // 2]), int(order[0])}:
        mc.check_l1(c, r, e, max_rows=48)
        mc.check_l2(c, r, e, max_rows=48)
    mc.check_reduce(c, r)
    err, rms, cos = mc.check_e2e_tokens(c, r, [0, T // 3, T - 1])
    _say(f"  subset e2e max_abs={err:.3e} rms={rms:.3e} cos={cos:.6f}")


# ------------------------------------------------------------ full sizes --
@pytest.mark.timeout(600)
@pytest.mark.parametrize("T,zipf", [(512, None), (2048, None), (2048, 1.1), (4096, None),
                                    (8192, None)])
def test_full_size_layer(T, zipf):
    """The benchmark workloads at full size: routing exact, staged L1/L2 on
    the busiest / a median / the lightest expert, REDUCE bit-exact, and the
    whole chain on a token subset.  T=4096 puts exactly 384 MiB of L2 rows in
    front of combine, the smallest size at which it streams them."""
    _say(f"full size T={T} zipf={zipf}")
    c = mc.normal_case(256, 8, 6144, 2048, T, seed=T + 1, scaled=True, zipf=zipf)
    r = mc.run_layer(c)
    mc.check_routing(c, r)
    nz = np.nonzero(r.counts)[0]
    order = nz[np.argsort(r.counts[nz], kind="stable")]
    # every row of the busiest expert (all its work items and token tiles),
    # 48 rows of a median and the lightest one
    busiest = int(order[-1])
    for e in {busiest, int(order[len(order) // 2]), int(order[0])}:
        rows = None if e == busiest else 48
        _say(f"  staged L1/L2 expert {e}: {int(r.counts[e])} rows, checking {rows or 'all'}")
        mc.check_l1(c, r, e, max_rows=rows)
        mc.check_l2(c, r, e, max_rows=rows)
    mc.check_reduce(c, r)
    err, rms, cos = mc.check_e2e_tokens(c, r, [0, 1, T // 2, T - 1])
    _say(f"  subset e2e max_abs={err:.3e} rms={rms:.3e} cos={cos:.6f}")


@pytest.mark.parametrize("win", [16, 32])
def test_full_size_decode_windows(win):
    """T=512 at full size through the decode-shaped kernels (windows of 16 /
    32 rows, the reference's small-window tasks): routing exact, staged L1/L2
    on the busiest and the lightest expert, REDUCE, the chain on a subset."""
    T = 512
    _say(f"full size T={T} win={win}")
    c = mc.normal_case(256, 8, 6144, 2048, T, seed=81, scaled=True, win=win)
    r = mc.run_layer(c)
    assert int(r.buf.layout.m_tile) == win
    mc.check_routing(c, r)
    nz = np.nonzero(r.counts)[0]
    order = nz[np.argsort(r.counts[nz], kind="stable")]
    for e in {int(order[-1]), int(order[0])}:
        mc.check_l1(c, r, e, max_rows=48)
        mc.check_l2(c, r, e, max_rows=48)
    mc.check_reduce(c, r)
    err, rms, cos = mc.check_e2e_tokens(c, r, [0, T // 3, T - 1])
    _say(f"  subset e2e max_abs={err:.3e} rms={rms:.3e} cos={cos:.6f}")


def test_layer_with_capacity_drops_and_invalid_ids():
    """Pairs over the slot capacity and pairs with an expert id outside [0, E)
    get no slot (src/prologue.cuh:150-175) and contribute nothing to y; the
    rest of the layer runs as usual."""
    E, K, H, I, T, cap = 32, 8, 1024, 512, 200, 30
    c = mc.normal_case(E, K, H, I, T, seed=51, scaled=True)
    idx = c.idx.copy()
    idx[3, 0], idx[7, 5], idx[100, 2] = -1, E + 3, E
    c = dataclasses.replace(c, idx=idx, cap=cap)
    _say(f"layer with cap={cap} and invalid ids")
    r = mc.run_layer(c)
    mc.check_routing(c, r)
    assert int((r.pair_pos < 0).sum()) > 3, "expected capacity drops"
    for e in range(0, E, 7):
        mc.check_l1(c, r, e)
        mc.check_l2(c, r, e)
    mc.check_reduce(c, r)
    mc.check_e2e(c, r)


def _sweep_case(seed):
    """A random small layer: shape, top-k, token count, scales, routing skew,
    expert window and slot capacity drawn from one seed."""
    rng = np.random.default_rng(1000 + seed)
    E = int(rng.choice([4, 8, 16, 32, 64, 128]))
    K = int(rng.integers(1, min(8, E) + 1))
    H = int(rng.choice([256, 512, 768, 1024]))
    I = int(rng.choice([128, 256, 512, 768]))
    T = int(rng.integers(1, 401))
    scaled = bool(rng.integers(0, 2))
    zipf = 1.1 if rng.random() < 0.4 else None
    win = int(rng.choice([0, 0, 16, 32, 64, 128, 256]))
    c = mc.normal_case(E, K, H, I, T, seed=300 + seed, scaled=scaled, zipf=zipf, win=win)
    if rng.random() < 0.3:
        # between one and two times the mean expert load: busy experts drop
        # pairs, but most tokens keep some (a cap that zeroes most rows makes
        # rms(y) small against the surviving rows, and the bf16 half-ulp of
        # those alone passes 2e-2 rms; test_layer_with_capacity_drops_and_
        # invalid_ids covers heavy drops)
        mean = -(-T * K // E)
        c = dataclasses.replace(c, cap=int(rng.integers(mean, 2 * mean + 1)))
    return c, zipf


@pytest.mark.parametrize("seed", range(24))
def test_random_shapes_sweep(seed):
    """Random small layers (seeded): routing bit-exact, L1 / L2 on the busiest
    and one other active expert at the staged tolerances, REDUCE, and the
    whole layer at the end-to-end bar (moe_case.e2e_gate); then the same layer with L1 and L2
    in one launch (fuse_l1l2) on the same buffer, bit-identical."""
    c, zipf = _sweep_case(seed)
    _say(f"sweep seed={seed}: E={c.E} K={c.K} H={c.H} I={c.I} T={c.T} scaled={c.scaled} "
         f"zipf={zipf} win={c.win} cap={c.cap}")
    r = mc.run_layer(c)
    mc.check_routing(c, r)
    active = np.flatnonzero(r.counts > 0)
    if active.size:
        busiest = int(np.argmax(r.counts))
        other = int(active[np.random.default_rng(seed).integers(0, active.size)])
        for e in sorted({busiest, other}):
            mc.check_l1(c, r, e)
            mc.check_l2(c, r, e)
    mc.check_reduce(c, r)
    err, rms, cos = mc.check_e2e(c, r)
    _say(f"  e2e max_abs={err:.3e} rms={rms:.3e} cos={cos:.6f}")
    r.buf.fuse_l1l2 = True
    r2 = mc.run_layer(c, buf=r.buf)
    assert np.array_equal(r2.y32.view(np.uint32), r.y32.view(np.uint32)), "fused launch differs"
    assert np.array_equal(r2.y, r.y)
    assert int(r2.status[0]) == 0


def test_full_size_extreme_skew():
    """T=1024 with every token routed among 16 experts (512 rows each: two
    256-row items, 16 token tiles) and 240 experts empty."""
    E, K, H, I, T = 256, 8, 6144, 2048, 1024
    rng = np.random.default_rng(61)
    hot = np.sort(rng.choice(E, size=16, replace=False))
    idx = np.stack([rng.permutation(hot)[:K] for _ in range(T)]).astype(np.int64)
    wts = rng.random((T, K)).astype(np.float32)
    wts /= wts.sum(axis=1, keepdims=True)
    _say("full size extreme skew T=1024 on 16 experts")
    c = mc.normal_case(E, K, H, I, T, seed=62, scaled=True, idx=idx, wts=wts)
    r = mc.run_layer(c)
    mc.check_routing(c, r)
    assert int((r.counts > 0).sum()) == 16
    for e in hot[:3]:
        mc.check_l1(c, r, int(e), max_rows=48)
        mc.check_l2(c, r, int(e), max_rows=48)
    mc.check_reduce(c, r)
    err, rms, cos = mc.check_e2e_tokens(c, r, [0, 1, T // 2, T - 1])
    _say(f"  subset e2e max_abs={err:.3e} rms={rms:.3e} cos={cos:.6f}")


def test_bf16_output_without_fp32_matches():
    """The torch mirror writes only the bf16 y unless write_fp32_y is set; the
    bf16 result is the same bits either way (combine computes one fp32 sum)."""
    _say("bf16 output with and without fp32 y")
    E, K, H, I, T = 16, 8, 512, 256, 96
    c = mc.normal_case(E, K, H, I, T, seed=41, scaled=True)
    r = mc.run_layer(c)                   # write_fp32_y = True
    buf = r.buf
    buf.write_fp32_y = False
    buf._y_fp32.fill_(12345.0)
    y = torch.empty((T, H), dtype=torch.bfloat16, device="cuda")
    mm.fp8_mega_moe(y, (c.w1, c.s1), (c.w2, c.s2), buf)
    torch.cuda.synchronize()
    assert np.array_equal(y.float().cpu().numpy(), r.y)
    assert bool((buf._y_fp32[:T] == 12345.0).all()), "fp32 y written although not requested"


def test_workspace_reuse_across_sizes():
    """One workspace, launches of 300, 37 and 300 tokens with different
    routings and weights: nothing of a larger earlier launch (work items, XCD
    unit ranges, chunk histograms) may leak into a smaller later one.  With
    1024 experts the routing alternates between the separate histogram launch
    (300 tokens: 10 chunks x 1024 counters) and the scan's own (37 tokens)."""
    E, K, H, I = 1024, 8, 256, 128
    buf = mm.get_symm_buffer_for_mega_moe(None, E, 300, K, H, I)
    for T, seed in ((300, 71), (37, 72), (300, 73)):
        _say(f"workspace reuse T={T} seed={seed}")
        c = mc.normal_case(E, K, H, I, T, seed=seed, scaled=True)
        r = mc.run_layer(c, buf=buf)
        mc.check_routing(c, r)
        mc.check_reduce(c, r)
        err, rms, cos = mc.check_e2e(c, r)
        _say(f"  e2e max_abs={err:.3e} rms={rms:.3e} cos={cos:.6f}")


def test_graph_replay_matches_eager():
    """N launches captured in one HIP graph, replayed three times with eager
    work in between; every replay must reproduce the eager output bit for bit
    (reference run_graph, test/check.cu:533-745)."""
    _say("graph replay")
    E, K, H, I, T = 32, 8, 1024, 512, 128
    c = mc.normal_case(E, K, H, I, T, seed=3, scaled=True)
    r = mc.run_layer(c)
    buf = r.buf
    ys = [torch.empty((T, H), dtype=torch.bfloat16, device="cuda") for _ in range(3)]
    torch.cuda.synchronize()
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        g = torch.cuda.CUDAGraph()
        with torch.cuda.graph(g, stream=s):
            for y in ys:
                mm.fp8_mega_moe(y, (c.w1, c.s1), (c.w2, c.s2), buf)
    torch.cuda.current_stream().wait_stream(s)
    for rep in range(3):
        for y in ys:
            y.zero_()
        torch.cuda.synchronize()
        g.replay()
        torch.cuda.synchronize()
        for y in ys:
            assert np.array_equal(y.float().cpu().numpy(), r.y), f"replay {rep} differs"
        # eager launch between replays must not disturb the graph's result
        y2 = torch.empty((T, H), dtype=torch.bfloat16, device="cuda")
        mm.fp8_mega_moe(y2, (c.w1, c.s1), (c.w2, c.s2), buf)
        torch.cuda.synchronize()
        assert np.array_equal(y2.float().cpu().numpy(), r.y)
