"""Python operator API of the fused FP8xFP8 MoE layer on one MI355X.

Mirrors the reference's torch layer (torch/mxmegakernel/mega/__init__.py):
same function names, argument meaning and error behaviour, single GPU.

* ``get_symm_buffer_for_mega_moe`` (reference :478-490) returns a
  :class:`SymmBuffer` (reference :144-475): input views ``x``, ``x_sf``,
  ``topk_idx``, ``topk_weights`` inside one device buffer, plus the
  caller-owned workspace of the HIP layer.  ``group`` must be None or a
  1-rank group: one GPU holds every expert.
* ``transform_weights_for_mega_moe`` (reference :553-573): torch-layout
  fp8 weights ``[E, 2I, H]`` ([gate; up]) and ``[E, H, I]`` -> gate/up paired
  (block G = min(256, I)) and packed into the MFMA tile layout.  Tuples
  ``(w, sf)`` carry 128x128 block scales (float powers of two or UE8M0 bytes).
* ``fp8_mega_moe`` (reference :610-655), ``fp8_mega_moe_compute`` /
  ``fp8_mega_moe_reduce`` (:658-712), ``bf16_fp8_mega_moe`` (:719-727).

Every call enqueues HIP kernels on torch's current stream through the C ABI
(mini_mega_amd/_lib.py); nothing here computes on the CPU.
"""
from __future__ import annotations

import ctypes
import math
from typing import Optional, Tuple, Union

import torch

from . import _lib
from ._lib import MegaLaunchArgs, check, lib

_SUPPORTED_MMA_TYPES = ("fp8xfp8", "bf16xfp8")
EXPERT_WINDOW_CHOICES = (0, 16, 32, 64, 128, 256)


def _align(x: int, a: int) -> int:
    return (x + a - 1) // a * a


def get_token_alignment_for_mega_moe() -> int:
    return 1


def pairing_block(intermediate_hidden: int) -> int:
    """Gate/up pairing block of the W1 row order (reference: 256,
    src/bench_check.cuh:444-445; min(256, I) here so that I = 128 works)."""
    return min(256, int(intermediate_hidden))


def get_symm_buffer_size_for_mega_moe(num_ranks: int, num_experts: int,
                                      num_max_tokens_per_rank: int, num_topk: int, hidden: int,
                                      intermediate_hidden: int, num_shared_experts: int = 0,
                                      mma_type: str = "fp8xfp8", num_tokens: int = 0,
                                      expert_window: int = 0) -> int:
    if num_ranks != 1:
        raise NotImplementedError("single-GPU build: num_ranks must be 1")
    L = _lib.layout(num_max_tokens_per_rank, num_topk, num_experts, hidden,
                    intermediate_hidden, expert_window)
    inputs = _inputs_bytes(num_max_tokens_per_rank, num_topk, hidden, mma_type)[-1]
    return int(L.total + inputs)


def _inputs_bytes(cap: int, topk: int, hidden: int, mma_type: str):
    xb = 2 if mma_type == "bf16xfp8" else 1
    x_off = 0
    sf_off = _align(x_off + cap * hidden * xb, 256)
    idx_off = _align(sf_off + cap * (hidden // 128), 256)
    w_off = _align(idx_off + cap * topk * 8, 256)
    total = _align(w_off + cap * topk * 4, 256)
    return x_off, sf_off, idx_off, w_off, total


def _view(buf: torch.Tensor, dtype: torch.dtype, shape, off: int) -> torch.Tensor:
    n = 1
    for s in shape:
        n *= s
    nbytes = n * torch.empty((), dtype=dtype).element_size()
    return buf[off:off + nbytes].view(dtype).view(*shape)


class SymmBuffer:
    """Inputs + workspace of one MoE layer on one GPU (reference SymmBuffer,
    torch/mxmegakernel/mega/__init__.py:144-475, minus the IPC / peer parts)."""

    def __init__(self, group, num_experts: int, num_max_tokens_per_rank: int, num_topk: int,
                 hidden: int, intermediate_hidden: int, num_shared_experts: int = 0,
                 mma_type: str = "fp8xfp8", activation: str = "swiglu",
                 grid_num_tokens: Optional[int] = None, expert_window: Optional[int] = None):
        if activation != "swiglu":
            raise ValueError(f"Only `swiglu` activation is supported, got `{activation}`")
        if mma_type not in _SUPPORTED_MMA_TYPES:
            raise NotImplementedError(f"only {_SUPPORTED_MMA_TYPES} are implemented, "
                                      f"got mma_type={mma_type!r}")
        if num_shared_experts != 0:
            raise NotImplementedError("shared experts are not supported")
        world = 1 if group is None else int(group.size())
        if world != 1:
            raise NotImplementedError("single-GPU build: the group must hold one rank")
        ew = 0 if expert_window is None else int(expert_window)
        if ew not in EXPERT_WINDOW_CHOICES:
            raise ValueError(f"expert_window must be one of {EXPERT_WINDOW_CHOICES}, got {ew}")
        lib()  # fail loudly if the HIP library is missing
        self.group = group
        self.world_size, self.rank = 1, 0
        self.num_experts = int(num_experts)
        self.num_max_tokens_per_rank = _align(int(num_max_tokens_per_rank),
                                              get_token_alignment_for_mega_moe())
        self.num_topk = int(num_topk)
        self.hidden = int(hidden)
        self.intermediate_hidden = int(intermediate_hidden)
        self.num_shared_experts = 0
        self.mma_type = mma_type
        self.activation = activation
        self.expert_window = ew
        self.device = torch.cuda.current_device()
        cap = self.num_max_tokens_per_rank
        self.layout = _lib.layout(cap, self.num_topk, self.num_experts, self.hidden,
                                  self.intermediate_hidden, ew)
        x_off, sf_off, idx_off, w_off, total = _inputs_bytes(cap, self.num_topk, self.hidden,
                                                             mma_type)
        self.buffer = torch.zeros(total, dtype=torch.uint8, device="cuda")
        xdtype = torch.bfloat16 if mma_type == "bf16xfp8" else torch.float8_e4m3fn
        self.x = _view(self.buffer, xdtype, (cap, self.hidden), x_off)
        self.x_sf = _view(self.buffer, torch.uint8, (cap, self.hidden // 128), sf_off)
        self.topk_idx = _view(self.buffer, torch.int64, (cap, self.num_topk), idx_off)
        self.topk_weights = _view(self.buffer, torch.float32, (cap, self.num_topk), w_off)
        self._x_off, self._w_off = x_off, w_off
        self.workspace = torch.zeros(int(self.layout.total), dtype=torch.uint8, device="cuda")
        self._y_fp32 = torch.empty((cap, self.hidden), dtype=torch.float32, device="cuda")
        # also write the fp32 y next to a bf16 output (staged checks read it)
        self.write_fp32_y = False
        # L1 and L2 in one launch, L2 units starting on an item once its L1
        # units are done (MegaLaunchArgs::fuse_l1l2)
        self.fuse_l1l2 = False
        # L2 as a walk of one workgroup per CU where the items allow it
        # (MegaLaunchArgs::l2_no_walk = 0)
        self.l2_walk = True
        # both GEMMs on the block-scaled fp8 MFMA (MegaLaunchArgs::mfma_fp8):
        # faster at large batches, outside the end-to-end bar of the default
        self.mfma_fp8 = False
        self.launch_count = 0

    # -- workspace views (staged parity checks read these, as check.cu dumps
    # -- the reference's pool / ffn / l2_out / combine buffers)
    def _ws(self, off: int, dtype, shape):
        return _view(self.workspace, dtype, shape, int(off))

    def counts(self):
        return self._ws(self.layout.counts, torch.int32, (self.num_experts,))

    def offsets(self):
        return self._ws(self.layout.offsets, torch.int32, (self.num_experts + 1,))

    def perm(self, slots: int):
        return self._ws(self.layout.perm, torch.int32, (slots,))

    def pair_pos(self, num_tokens: int):
        return self._ws(self.layout.pair_pos, torch.int32, (num_tokens, self.num_topk))

    def ffn(self, slots: int):
        return self._ws(self.layout.ffn, torch.uint8, (slots, self.intermediate_hidden))

    def ffn_sf(self, slots: int):
        return self._ws(self.layout.ffn_sf, torch.uint8,
                        (slots, self.intermediate_hidden // 128))

    def l2_out(self, slots: int):
        return self._ws(self.layout.l2, torch.int16, (slots, self.hidden))

    def status(self):
        return self._ws(self.layout.status, torch.int32, (64,))

    def tail_orders(self):
        """L1's tail-queue ticket order, uint8 [XCD][32]: ticket t of XCD x
        runs the tail's unit [x][t] (the status region's bytes after its 64
        words)."""
        return self._ws(int(self.layout.status) + 256, torch.uint8, (8, 32))

    def items(self, n: int):
        """Work items: (expert, first slot, end slot, j | n << 16 for item j of
        the expert's n)."""
        return self._ws(self.layout.items, torch.int32, (n, 4))

    def make_args(self, num_tokens: int, l1, l2, y_bf16: Optional[torch.Tensor] = None,
                  y_fp32: Optional[torch.Tensor] = None, skip_prologue: int = 0,
                  slot_capacity: int = 0) -> MegaLaunchArgs:
        """MegaLaunchArgs for one launch (reference mt::make_args,
        test/mega_common.cuh:344-376)."""
        w1, w1_sf = _split(l1)
        w2, w2_sf = _split(l2)
        a = MegaLaunchArgs()
        a.tokens = int(num_tokens)
        a.slot_capacity = int(slot_capacity)
        a.win_cap = self.expert_window
        a.rwk = self.workspace.data_ptr()
        a.self = self.buffer.data_ptr()
        a.x_off = self._x_off
        a.weights_off = self._w_off
        a.topk_idx = self.topk_idx.data_ptr()
        a.w1 = w1.data_ptr()
        a.w2 = w2.data_ptr()
        a.in_bf16 = 1 if self.mma_type == "bf16xfp8" else 0
        # fp32 y (the reference's MegaLaunchArgs::y) only when asked for, or
        # when there is no bf16 output: it is 4*T*H more bytes to write
        if y_fp32 is not None:
            a.y = y_fp32.data_ptr()
        elif self.write_fp32_y or y_bf16 is None:
            a.y = self._y_fp32.data_ptr()
        else:
            a.y = None
        a.y_bf16 = y_bf16.data_ptr() if y_bf16 is not None else None
        a.skip_prologue = int(skip_prologue)
        a.fuse_l1l2 = int(bool(self.fuse_l1l2))
        a.l2_no_walk = int(not self.l2_walk)
        a.mfma_fp8 = int(bool(self.mfma_fp8))
        a.num_experts, a.topk = self.num_experts, self.num_topk
        a.hidden, a.intermediate = self.hidden, self.intermediate_hidden
        a.max_tokens = self.num_max_tokens_per_rank
        a.workspace_bytes = int(self.layout.total)
        scaled = w1_sf is not None
        if scaled != (w2_sf is not None):
            raise ValueError("l1 and l2 weights must both carry scales or neither")
        if scaled:
            a.w1_sf, a.w2_sf = w1_sf.data_ptr(), w2_sf.data_ptr()
            if self.mma_type == "fp8xfp8":
                a.x_sf = self.x_sf.data_ptr()
            a.ffn_ue8m0 = 1
        return a

    def make_reduce_args(self, num_tokens: int, y_bf16: torch.Tensor) -> MegaLaunchArgs:
        """MegaLaunchArgs for launch_reduce alone: the reduce reads the
        workspace (L2 rows, slots) and the topk weights, no layer weights."""
        a = MegaLaunchArgs()
        a.tokens = int(num_tokens)
        a.win_cap = self.expert_window
        a.rwk = self.workspace.data_ptr()
        a.self = self.buffer.data_ptr()
        a.x_off = self._x_off
        a.weights_off = self._w_off
        a.topk_idx = self.topk_idx.data_ptr()
        a.in_bf16 = 1 if self.mma_type == "bf16xfp8" else 0
        a.y = self._y_fp32.data_ptr() if self.write_fp32_y else None
        a.y_bf16 = y_bf16.data_ptr()
        a.num_experts, a.topk = self.num_experts, self.num_topk
        a.hidden, a.intermediate = self.hidden, self.intermediate_hidden
        a.max_tokens = self.num_max_tokens_per_rank
        a.workspace_bytes = int(self.layout.total)
        return a

    def device_status(self) -> dict:
        """The device status words of the last launch on this buffer (through
        mm_read_status, which synchronises the current stream): error bits,
        work items, routed slots, pairs dropped by the slot capacity, pairs
        with an expert id outside [0, num_experts) and the rows of the largest
        work item."""
        import ctypes as _c
        a = self.make_reduce_args(0, self.workspace)
        out = (_c.c_int * 6)()
        rc = lib().mm_read_status(_c.byref(a), out, 6, _stream_ptr())
        if rc not in (0, _lib.ERR_DEVICE):
            check("mm_read_status", rc)
        return dict(error=int(out[0]), items=int(out[1]), slots=int(out[2]),
                    dropped_by_capacity=int(out[3]), invalid_ids=int(out[4]),
                    max_item_rows=int(out[5]))

    def destroy(self):
        self.buffer = self.workspace = self._y_fp32 = None


def get_symm_buffer_for_mega_moe(group, num_experts: int, num_max_tokens_per_rank: int,
                                 num_topk: int, hidden: int, intermediate_hidden: int,
                                 num_shared_experts: int = 0,
                                 use_fp8_dispatch: Optional[bool] = None,
                                 mma_type: str = "fp8xfp8", activation: str = "swiglu",
                                 num_tokens: Optional[int] = None,
                                 expert_window: Optional[int] = None) -> SymmBuffer:
    if use_fp8_dispatch is not None:
        assert use_fp8_dispatch == (mma_type.split("x")[0] == "fp8")
    return SymmBuffer(group, num_experts, num_max_tokens_per_rank, num_topk, hidden,
                      intermediate_hidden, num_shared_experts, mma_type=mma_type,
                      activation=activation, grid_num_tokens=num_tokens,
                      expert_window=expert_window)


def _split(w):
    if isinstance(w, tuple):
        return w[0], w[1]
    return w, None


def _stream_ptr() -> int:
    return torch.cuda.current_stream().cuda_stream


# ------------------------------------------------------------ weight packing
def _interleave_rows(t: torch.Tensor, gran: int) -> torch.Tensor:
    """[E, 2N, ...] with [gate | up] rows -> gate/up alternating every `gran`
    rows (reference _interleave_weights, mega/__init__.py:493-509)."""
    e, n = t.shape[0], t.shape[1]
    half = n // 2
    rest = t.shape[2:]
    gate = t[:, :half].reshape(e, half // gran, gran, *rest)
    up = t[:, half:].reshape(e, half // gran, gran, *rest)
    return torch.stack([gate, up], dim=2).reshape(e, n, *rest).contiguous()


def _sf_to_ue8m0(sf: torch.Tensor) -> torch.Tensor:
    if sf.dtype == torch.uint8:
        return sf.contiguous()
    if sf.dtype != torch.float32:
        raise TypeError("scales must be float32 powers of two or uint8 UE8M0 bytes")
    bits = sf.contiguous().view(torch.int32)
    if bool(((bits & 0x7FFFFF) != 0).any()) or bool((bits < 0).any()):
        raise ValueError("scales must be positive powers of two (UE8M0)")
    return ((bits >> 23) & 0xFF).to(torch.uint8)


def pack_weights(w: torch.Tensor) -> torch.Tensor:
    """Logical row-major fp8 [E, N, K] -> tile layout (device kernel)."""
    if w.dim() == 2:
        w = w.unsqueeze(0)
    e, n, k = w.shape
    src = w.contiguous().view(torch.uint8)
    dst = torch.empty_like(src)
    check("mm_pack_weights", lib().mm_pack_weights(dst.data_ptr(), src.data_ptr(), e, n, k,
                                                   _stream_ptr()))
    return dst.view(torch.float8_e4m3fn)


def transform_weights_for_mega_moe(
        l1_weights: Union[torch.Tensor, Tuple[torch.Tensor, torch.Tensor]],
        l2_weights: Union[torch.Tensor, Tuple[torch.Tensor, torch.Tensor]],
        activation: str = "swiglu"):
    """Offline weight packing (reference mega/__init__.py:553-573): W1 gate/up
    paired at block G = min(256, I) then tiled; W2 tiled.  Scale tensors (when
    given as tuples) are [E, 2I/128, H/128] and [E, H/128, I/128]."""
    assert activation == "swiglu", f"Only `swiglu` supported, got `{activation}`"
    w1, s1 = _split(l1_weights)
    w2, s2 = _split(l2_weights)
    for name, t in (("l1_weights", w1), ("l2_weights", w2)):
        if not isinstance(t, torch.Tensor) or t.dtype != torch.float8_e4m3fn:
            raise TypeError(f"{name} must be a float8_e4m3fn tensor")
    squeeze = w1.dim() == 2
    if squeeze:
        w1, w2 = w1.unsqueeze(0), w2.unsqueeze(0)
        s1 = None if s1 is None else s1.unsqueeze(0)
        s2 = None if s2 is None else s2.unsqueeze(0)
    I = w1.shape[1] // 2
    G = pairing_block(I)
    l1_t = pack_weights(_interleave_rows(w1.view(torch.uint8), G).view(torch.float8_e4m3fn))
    l2_t = pack_weights(w2)
    if (s1 is None) != (s2 is None):
        raise ValueError("give scales for both l1 and l2 or for neither")
    if s1 is None:
        return l1_t, l2_t
    s1p = _interleave_rows(_sf_to_ue8m0(s1), G // 128)
    return (l1_t, s1p), (l2_t, _sf_to_ue8m0(s2).contiguous())


def pack_weights_from_reference(w: torch.Tensor) -> torch.Tensor:
    """The reference's packed [E, N, K] fp8 (lane-tile layout of its
    _swizzle_lane, torch/mxmegakernel/mega/__init__.py:512-533) -> this
    library's tile layout, keeping the logical row order (device kernel)."""
    if w.dim() == 2:
        w = w.unsqueeze(0)
    e, n, k = w.shape
    src = w.contiguous().view(torch.uint8)
    dst = torch.empty_like(src)
    check("mm_pack_weights_from_reference",
          lib().mm_pack_weights_from_reference(dst.data_ptr(), src.data_ptr(), e, n, k,
                                               _stream_ptr()))
    return dst.view(torch.float8_e4m3fn)


def transform_weights_from_reference(
        l1_weights: Union[torch.Tensor, Tuple[torch.Tensor, torch.Tensor]],
        l2_weights: Union[torch.Tensor, Tuple[torch.Tensor, torch.Tensor]]):
    """Weights already packed for the reference (the output of its
    transform_weights_for_mega_moe, torch/mxmegakernel/mega/__init__.py:553-573:
    W1 gate/up paired every 256 rows, then lane-swizzled; W2 lane-swizzled)
    -> this library's packed weights, as transform_weights_for_mega_moe
    returns them.  The reference pairs W1 in blocks of 256, which equals
    this library's block min(256, I) since the reference needs I % 256 == 0.
    Optional UE8M0 scales, given as (w, sf) tuples, are in the torch layout
    ([E, 2I/128, H/128] with [gate | up] rows, [E, H/128, I/128])."""
    w1, s1 = _split(l1_weights)
    w2, s2 = _split(l2_weights)
    for name, t in (("l1_weights", w1), ("l2_weights", w2)):
        if not isinstance(t, torch.Tensor) or t.dtype != torch.float8_e4m3fn:
            raise TypeError(f"{name} must be a float8_e4m3fn tensor")
    I = w1.shape[-2] // 2
    if I % 256 != 0:
        raise ValueError(f"reference-packed W1 needs I % 256 == 0 (its pairing block); got I={I}")
    if (s1 is None) != (s2 is None):
        raise ValueError("give scales for both l1 and l2 or for neither")
    squeeze = w1.dim() == 2
    l1_t = pack_weights_from_reference(w1)
    l2_t = pack_weights_from_reference(w2)
    if squeeze:
        l1_t, l2_t = l1_t.squeeze(0), l2_t.squeeze(0)
    if s1 is None:
        return l1_t, l2_t
    s1 = s1.unsqueeze(0) if s1.dim() == 2 else s1
    s1p = _interleave_rows(_sf_to_ue8m0(s1), pairing_block(I) // 128)
    s2p = _sf_to_ue8m0(s2).contiguous()
    if squeeze:
        s1p = s1p.squeeze(0)
    return (l1_t, s1p), (l2_t, s2p)


def fold_checkpoint_block_scales(w13: torch.Tensor, w13_sf: torch.Tensor, w2: torch.Tensor,
                                 w2_sf: torch.Tensor):
    """The reference serving path's raw-E4M3 weight build from a block-scaled
    fp8 checkpoint (torch/sglang_patches/patch_mega_scale.py:19-30): dequantise
    with the 128x128 block scales, cast W1 directly (clamped to +-448; SwiGLU
    does not allow folding a scale back out), and scale W2 by the power of two
    w2_scale = 2^floor(log2(448 / amax(W2))) before its cast.  The caller
    divides the top-k weights by w2_scale so that REDUCE cancels it exactly.
    Returns (w13_raw, w2_raw, w2_scale).  (This library can instead keep the
    block scales: pass (w, sf) tuples to transform_weights_for_mega_moe.)"""
    def dequant(w, sf):
        e, n, k = w.shape
        f = sf.to(torch.float32).repeat_interleave(128, dim=1).repeat_interleave(128, dim=2)
        return w.to(torch.float32) * f[:, :n, :k]
    w13_f = dequant(w13, w13_sf)
    w2_f = dequant(w2, w2_sf)
    amax2 = float(w2_f.abs().max())
    w2_scale = 2.0 ** math.floor(math.log2(448.0 / amax2)) if amax2 > 0 else 1.0
    w13_raw = w13_f.clamp(-448.0, 448.0).to(torch.float8_e4m3fn)
    w2_raw = (w2_f * w2_scale).clamp(-448.0, 448.0).to(torch.float8_e4m3fn)
    return w13_raw, w2_raw, w2_scale


# ------------------------------------------------------------------ launches
def _check_common(fn: str, sym_buffer: SymmBuffer, activation: str):
    if sym_buffer.mma_type not in _SUPPORTED_MMA_TYPES:
        raise ValueError(f"{fn} requires fp8xfp8/bf16xfp8 SymmBuffer, got "
                         f"{sym_buffer.mma_type!r}")
    if activation != "swiglu":
        raise ValueError(f"fp8xfp8 requires activation='swiglu', got {activation!r}")


def _check_output(fn: str, y: torch.Tensor, sym_buffer: SymmBuffer, num_tokens: int) -> None:
    """y must be the contiguous bf16 [num_tokens, hidden] tensor on the buffer's
    device: the combine kernel writes num_tokens * hidden values through its
    pointer (the reference copies into y, which raises on a mismatch,
    mega/__init__.py:655)."""
    if not isinstance(y, torch.Tensor) or y.dtype != torch.bfloat16 or not y.is_contiguous():
        raise TypeError(f"{fn}: y must be a contiguous bfloat16 tensor")
    if y.dim() != 2 or int(y.shape[1]) != sym_buffer.hidden or int(y.shape[0]) < num_tokens:
        raise ValueError(f"{fn}: y has shape {tuple(y.shape)}, needs ({num_tokens}, "
                         f"{sym_buffer.hidden})")
    if num_tokens > 0 and (y.device.type != "cuda" or y.device.index != sym_buffer.device):
        raise ValueError(f"{fn}: y is on {y.device}, the buffer on cuda:{sym_buffer.device}")


def fp8_mega_moe(y: torch.Tensor, l1_weights, l2_weights, sym_buffer: SymmBuffer,
                 cumulative_local_expert_recv_stats=None, activation: str = "swiglu",
                 activation_clamp=None, expert_window: Optional[int] = None) -> None:
    """Full layer: y[:T] (bf16) = MoE(x, topk_idx, topk_weights) (reference
    mega/__init__.py:610-655).  activation_clamp is accepted and unused, as in
    the reference kernel."""
    _check_common("fp8_mega_moe", sym_buffer, activation)
    num_tokens = int(y.shape[0])
    if num_tokens > sym_buffer.num_max_tokens_per_rank:
        raise ValueError(f"num_tokens={num_tokens} exceeds capacity "
                         f"{sym_buffer.num_max_tokens_per_rank}")
    _check_output("fp8_mega_moe", y, sym_buffer, num_tokens)
    if expert_window is not None and int(expert_window) != sym_buffer.expert_window:
        raise ValueError("expert_window is fixed when the SymmBuffer is built")
    a = sym_buffer.make_args(num_tokens, l1_weights, l2_weights,
                             y_bf16=y if num_tokens > 0 else None)
    check("mm_launch_full", lib().mm_launch_full(ctypes.byref(a), _stream_ptr()))
    sym_buffer.launch_count += 1
    sym_buffer._last_compute_tokens = num_tokens
    if cumulative_local_expert_recv_stats is not None:
        cumulative_local_expert_recv_stats.add_(sym_buffer.counts()[
            :cumulative_local_expert_recv_stats.numel()].to(
                cumulative_local_expert_recv_stats.dtype))


def fp8_mega_moe_compute(l1_weights, l2_weights, sym_buffer: SymmBuffer, num_tokens: int,
                         activation: str = "swiglu", activation_clamp=None,
                         expert_window: Optional[int] = None, skip_prologue: int = 0) -> None:
    """Routing + L1 + L2 without the reduce (reference :658-693).  The L2 rows
    stay in the buffer's workspace until fp8_mega_moe_reduce; kernels that do
    not touch this buffer may run in between.  skip_prologue=1 reuses the
    routing of the buffer's previous launch (same topk_idx and num_tokens;
    the reference's graph-node option, src/megakernel.h:106): only x is
    folded again for a bf16xfp8 buffer."""
    _check_common("fp8_mega_moe_compute", sym_buffer, activation)
    num_tokens = int(num_tokens)
    if num_tokens < 0 or num_tokens > sym_buffer.num_max_tokens_per_rank:
        raise ValueError(f"num_tokens={num_tokens} exceeds capacity "
                         f"{sym_buffer.num_max_tokens_per_rank}")
    if expert_window is not None and int(expert_window) != sym_buffer.expert_window:
        raise ValueError("expert_window is fixed when the SymmBuffer is built")
    if skip_prologue and getattr(sym_buffer, "_last_compute_tokens", None) != num_tokens:
        raise ValueError("skip_prologue reuses the previous launch's routing: it needs a "
                         "previous launch with the same num_tokens")
    a = sym_buffer.make_args(num_tokens, l1_weights, l2_weights, skip_prologue=skip_prologue)
    check("mm_launch_compute", lib().mm_launch_compute(ctypes.byref(a), _stream_ptr()))
    sym_buffer.launch_count += 1
    sym_buffer._last_compute_tokens = num_tokens


def fp8_mega_moe_reduce(y: torch.Tensor, sym_buffer: SymmBuffer,
                        num_tokens: Optional[int] = None) -> None:
    """Top-k weighted reduce into y (bf16) of the buffer's last
    fp8_mega_moe_compute (reference :696-712).  The reduce reads only the
    workspace's L2 rows and slots and the buffer's topk_weights, so it needs no
    weights; num_tokens (default y.shape[0]) may not exceed the token count of
    that compute."""
    if sym_buffer.mma_type not in _SUPPORTED_MMA_TYPES:
        raise ValueError(f"fp8_mega_moe_reduce requires fp8xfp8/bf16xfp8 SymmBuffer, got "
                         f"{sym_buffer.mma_type!r}")
    nt = int(num_tokens) if num_tokens is not None else int(y.shape[0])
    if nt <= 0 or nt > sym_buffer.num_max_tokens_per_rank:
        raise ValueError(f"num_tokens={nt} out of range "
                         f"(capacity {sym_buffer.num_max_tokens_per_rank})")
    last = getattr(sym_buffer, "_last_compute_tokens", None)
    if last is None:
        raise RuntimeError("fp8_mega_moe_reduce needs a preceding fp8_mega_moe_compute")
    if nt > last:
        raise ValueError(f"num_tokens={nt} exceeds the {last} tokens of the last compute")
    _check_output("fp8_mega_moe_reduce", y, sym_buffer, nt)
    a = sym_buffer.make_reduce_args(nt, y)
    check("mm_launch_reduce", lib().mm_launch_reduce(ctypes.byref(a), _stream_ptr()))


def bf16_fp8_mega_moe(y: torch.Tensor, l1_weights, l2_weights, sym_buffer: SymmBuffer,
                      **kwargs) -> None:
    """bf16 x + fp8 weights: x is folded to fp8 inside the layer (reference
    :719-727)."""
    if sym_buffer.mma_type != "bf16xfp8":
        raise ValueError(f"bf16_fp8_mega_moe requires a bf16xfp8 SymmBuffer, got "
                         f"{sym_buffer.mma_type!r}")
    return fp8_mega_moe(y, l1_weights, l2_weights, sym_buffer, **kwargs)


def bf16_mega_moe(*args, **kwargs):
    raise NotImplementedError("only fp8xfp8 / bf16xfp8 are implemented")


def fp8_fp4_mega_moe(*args, **kwargs):
    raise NotImplementedError("only fp8xfp8 / bf16xfp8 are implemented")
