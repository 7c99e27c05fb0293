"""CPU tests of the weight-format helpers: the reference's on-device lane-tile
layout (as transform_weights_from_reference reads it) and the checkpoint
scale-folding recipe.  The GPU side of the converter is tested in
test_gpu_parity.py against the plain packer."""
import numpy as np
import pytest
import torch

import mini_mega_amd as mm
from moe_case import ref_lane_pack


def _swizzle_lane_numpy(w):
    """The reference's _swizzle_lane as a reshape/permute
    (torch/mxmegakernel/mega/__init__.py:527-530), for one matrix."""
    n, k = w.shape
    return (w.reshape(n // 32, 2, 16, k // 32, 4, 8)
            .transpose(0, 3, 4, 2, 1, 5).reshape(n, k))


def test_lane_closed_form_equals_reference_swizzle():
    """Two independent statements of the reference layout agree: the
    closed-form byte index (src/bench_check.cuh:268-272, which the HIP
    converter implements) and the torch-side permutation."""
    w = np.random.default_rng(1).integers(0, 256, size=(96, 256), dtype=np.uint8)
    assert np.array_equal(ref_lane_pack(w[None])[0], _swizzle_lane_numpy(w))


def test_lane_closed_form_is_a_permutation():
    n, k = 64, 128
    idx = np.arange(n * k, dtype=np.int64).reshape(n, k)
    # distinct values at distinct positions: pack the index pattern bytewise
    lo = ref_lane_pack((idx & 0xFF).astype(np.uint8)[None])[0]
    hi = ref_lane_pack((idx >> 8).astype(np.uint8)[None])[0]
    got = lo.astype(np.int64) | (hi.astype(np.int64) << 8)
    assert sorted(got.ravel().tolist()) == list(range(n * k))


def test_fold_checkpoint_block_scales_recipe():
    """patch_mega_scale.py:19-30: unit block scales leave W1 bit for bit;
    W2 is scaled by the power of two that brings its amax into (224, 448],
    exactly (a power-of-two product of an e4m3 value in range is exact)."""
    g = torch.Generator().manual_seed(0)
    w13 = (torch.randn(2, 256, 256, generator=g) * 2).to(torch.float8_e4m3fn)
    w2 = (torch.randn(2, 256, 128, generator=g) * 0.01).to(torch.float8_e4m3fn)
    s13 = torch.ones(2, 2, 2)
    s2 = torch.ones(2, 2, 1)
    w13_raw, w2_raw, w2_scale = mm.fold_checkpoint_block_scales(w13, s13, w2, s2)
    assert torch.equal(w13_raw.view(torch.uint8), w13.view(torch.uint8))
    amax = float(w2.float().abs().max())
    assert w2_scale == 2.0 ** np.floor(np.log2(448.0 / amax))
    assert 224.0 < amax * w2_scale <= 448.0
    assert torch.equal(w2_raw.float(), w2.float() * w2_scale)
    # a non-unit block scale is applied per 128x128 block before the cast
    s13b = s13.clone()
    s13b[0, 1, 0] = 0.5
    w13_b, _, _ = mm.fold_checkpoint_block_scales(w13, s13b, w2, s2)
    # (halving can round an e4m3 subnormal, hence the cast on the expected side)
    half = (w13[0, 128:, :128].float() * 0.5).to(torch.float8_e4m3fn)
    assert torch.equal(w13_b[0, 128:, :128].view(torch.uint8), half.view(torch.uint8))
    assert torch.equal(w13_b.view(torch.uint8)[0, 128:, 128:], w13.view(torch.uint8)[0, 128:, 128:])
    assert torch.equal(w13_b.view(torch.uint8)[0, :128], w13.view(torch.uint8)[0, :128])


def test_routes_with_counts_reproduce_logged_counts():
    """inputs.routes_with_counts (the bench's TK_INFO replay) gives exactly the
    logged per-expert counts with distinct experts per token, on every launch
    of both committed TK_INFO fixtures, and rejects counts that cannot form
    distinct top-k rows."""
    import os
    from mini_mega_amd import inputs
    for name in ("tk_info_anchors.log", "tk_real_decode.log"):
        launches = inputs.read_tk_info(os.path.join(os.path.dirname(__file__), "golden", name))
        assert launches
        for pe in launches.values():
            idx = inputs.routes_with_counts(pe, 8)
            assert np.array_equal(np.bincount(idx.ravel(), minlength=pe.size), pe)
            assert all(len(set(r.tolist())) == 8 for r in idx)
    with pytest.raises(ValueError):
        inputs.routes_with_counts(np.array([3, 1]), 2)    # 2 tokens, one expert with 3 rows
    with pytest.raises(ValueError):
        inputs.routes_with_counts(np.array([2, 1]), 2)    # 3 pairs: not whole top-2 tokens
