"""ctypes binding of libmegakernel.so (the C ABI declared in include/megakernel.h).

Loading fails loudly when the HIP library has not been built: there is no CPU
fallback anywhere in this package.
"""
from __future__ import annotations

import ctypes
import os

_HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(_HERE, "libmegakernel.so")

c_int, c_i64, c_vp, c_float = ctypes.c_int, ctypes.c_int64, ctypes.c_void_p, ctypes.c_float


class MegaLaunchArgs(ctypes.Structure):
    """Mirror of fp8mega::MegaLaunchArgs (include/megakernel.h; reference
    src/megakernel.h:54-114, appended fields after skip_prologue)."""
    _fields_ = [
        ("R", c_int), ("rank", c_int), ("tokens", c_int), ("slot_capacity", c_int),
        ("win_cap", c_int), ("grid", c_int), ("threads", c_int), ("smem", c_i64),
        ("rwk", c_vp), ("unk", c_vp), ("unk_peers", c_vp), ("self", c_vp),
        ("peer_bases", c_vp), ("topk_idx", c_vp), ("w1", c_vp), ("w2", c_vp),
        ("group_weights_ready", c_int), ("topk_idx_off", c_i64), ("x_off", c_i64),
        ("weights_off", c_i64), ("in_bf16", c_int), ("skip_combine", c_int),
        ("y", c_vp), ("max_spins", c_int), ("skip_prologue", c_int),
        ("num_experts", c_int), ("topk", c_int), ("hidden", c_int), ("intermediate", c_int),
        ("max_tokens", c_int), ("workspace_bytes", c_i64), ("x_sf", c_vp), ("w1_sf", c_vp),
        ("w2_sf", c_vp), ("ffn_ue8m0", c_int), ("y_bf16", c_vp), ("fuse_l1l2", c_int), ("l2_no_walk", c_int),
        ("ready_bias", c_int), ("mfma_fp8", c_int),
    ]

    def __init__(this, **kw):  # "self" is a field name (the reference's base pointer)
        super().__init__()
        this.R, this.rank = 1, 0
        this.num_experts, this.topk, this.hidden, this.intermediate = 256, 8, 6144, 2048
        for k, v in kw.items():
            setattr(this, k, v)


class MegaLayout(ctypes.Structure):
    """Mirror of fp8mega::MegaLayout (workspace byte offsets)."""
    _fields_ = [(n, c_i64) for n in (
        "status", "chunk_hist", "counts", "offsets", "items", "perm", "pair_pos", "xq",
        "xq_sf", "ffn", "ffn_sf", "l2", "total")] + [
        (n, c_int) for n in ("nchunks", "max_items", "max_pairs", "m_tile")]


STATUS_NAMES = {
    0: "ok", 1: "null pointer", 2: "unsupported dims", 3: "workspace too small",
    4: "tokens exceed max_tokens", 5: "kernel launch failed", 6: "unsupported option",
    7: "device status word reports an error",
    8: "layout larger than the no-alloc scratch",
}
ERR_DEVICE = 7


class MegaError(RuntimeError):
    def __init__(self, fn: str, code: int):
        super().__init__(f"{fn}: {STATUS_NAMES.get(code, 'error')} (status {code})")
        self.code = code


EXPORTS = (
    "mm_abi_version", "mm_args_size", "mm_args_offset", "mm_layout", "mm_launch_prelude",
    "mm_launch_compute", "mm_launch_l1", "mm_launch_l2", "mm_launch_reduce", "mm_launch_full",
    "mm_launch_full_noalloc", "mm_noalloc_scratch_bytes",
    "mm_launch_empty", "mm_launch_dispatch", "mm_read_status", "mm_fill_weights_lane", "mm_pack_weights",
    "mm_pack_weights_from_reference",
    "mm_fill_weights_normal", "mm_quant_act", "mm_selftest_convert", "mm_dump_kernel_resources",
    "mm_probe_mfma_dot", "mm_probe_l2_rows", "mm_probe_stream_read", "mm_probe_mfma_rate",
)

_lib = None


def lib():
    """Loads libmegakernel.so once; raises if it has not been built."""
    global _lib
    if _lib is not None:
        return _lib
    if not os.path.exists(LIB_PATH):
        raise ImportError(
            f"{LIB_PATH} is missing: build the HIP library first "
            "(python -m mini_mega_amd.build or __graft_entry__.build())")
    L = ctypes.CDLL(LIB_PATH)
    A = ctypes.POINTER(MegaLaunchArgs)
    L.mm_abi_version.restype = c_int
    L.mm_args_size.restype = ctypes.c_size_t
    L.mm_args_offset.restype = ctypes.c_longlong
    L.mm_args_offset.argtypes = [ctypes.c_char_p]
    L.mm_layout.restype = c_int
    L.mm_layout.argtypes = [c_int] * 6 + [ctypes.POINTER(MegaLayout)]
    for n in ("mm_launch_prelude", "mm_launch_compute", "mm_launch_l1", "mm_launch_l2",
              "mm_launch_reduce", "mm_launch_full", "mm_launch_full_noalloc"):
        getattr(L, n).restype = c_int
        getattr(L, n).argtypes = [A, c_vp]
    L.mm_launch_dispatch.restype = c_int
    L.mm_launch_dispatch.argtypes = [A, c_vp, c_vp]
    L.mm_noalloc_scratch_bytes.restype = ctypes.c_longlong
    L.mm_read_status.restype = c_int
    L.mm_read_status.argtypes = [A, c_vp, c_int, c_vp]
    L.mm_launch_empty.restype = c_int
    L.mm_launch_empty.argtypes = [c_int, c_int, ctypes.c_longlong, c_vp]
    L.mm_fill_weights_lane.restype = c_int
    L.mm_fill_weights_lane.argtypes = [c_vp, c_int, c_int, ctypes.c_uint, c_vp]
    L.mm_pack_weights.restype = c_int
    L.mm_pack_weights.argtypes = [c_vp, c_vp, c_int, c_int, c_int, c_vp]
    L.mm_pack_weights_from_reference.restype = c_int
    L.mm_pack_weights_from_reference.argtypes = [c_vp, c_vp, c_int, c_int, c_int, c_vp]
    L.mm_fill_weights_normal.restype = c_int
    L.mm_fill_weights_normal.argtypes = [c_vp, c_vp, c_int, c_int, c_int, ctypes.c_ulonglong,
                                         c_float, c_vp]
    L.mm_quant_act.restype = c_int
    L.mm_quant_act.argtypes = [c_vp, c_int, c_int, c_vp, c_vp, c_vp]
    L.mm_selftest_convert.restype = c_int
    L.mm_selftest_convert.argtypes = [c_vp, c_int, c_vp, c_vp, c_vp]
    L.mm_dump_kernel_resources.restype = None
    L.mm_probe_mfma_dot.restype = c_int
    L.mm_probe_mfma_dot.argtypes = [c_vp, c_vp, c_int, c_int, c_int, c_vp, c_vp]
    L.mm_probe_l2_rows.restype = c_int
    L.mm_probe_l2_rows.argtypes = [c_vp] * 5 + [c_int] * 4 + [c_vp, c_vp]
    L.mm_probe_stream_read.restype = c_int
    L.mm_probe_stream_read.argtypes = [c_vp, ctypes.c_ulonglong, c_vp, c_int, c_vp]
    L.mm_probe_mfma_rate.restype = c_int
    L.mm_probe_mfma_rate.argtypes = [c_int, c_int, c_int, c_vp, c_vp]
    if L.mm_args_size() != ctypes.sizeof(MegaLaunchArgs):
        raise ImportError("MegaLaunchArgs mirror does not match the library's struct size")
    for name, *_ in MegaLaunchArgs._fields_:
        off = L.mm_args_offset(name.encode())
        if off != getattr(MegaLaunchArgs, name).offset:
            raise ImportError(f"MegaLaunchArgs.{name}: offset {off} in the library, "
                              f"{getattr(MegaLaunchArgs, name).offset} in the mirror")
    _lib = L
    return _lib


def check(fn: str, code: int) -> None:
    if code != 0:
        raise MegaError(fn, code)


def layout(max_tokens: int, topk: int, num_experts: int, hidden: int, intermediate: int,
           win_cap: int = 0) -> MegaLayout:
    out = MegaLayout()
    check("mm_layout", lib().mm_layout(max_tokens, topk, num_experts, hidden, intermediate,
                                       win_cap, ctypes.byref(out)))
    return out
