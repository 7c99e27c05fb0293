"""ctypes wrapper around oracle/libmoe_oracle.so -- TEST INFRASTRUCTURE ONLY.

The oracle is the CPU restatement of the reference's host numeric path
(src/bench_check.cuh:326-625, src/prologue.cuh:126-226 routing semantics,
torch/mxmegakernel/utils/math.py:13-72 UE8M0 recipe).  Only tests/, the
smoke() entry point and bench.py's cpu_baseline leg import this module, and
only as the checker; the product package never touches it.

Every array argument is a contiguous numpy array; weights are LOGICAL
row-major ([E][2I][H] in paired gate/up order, [E][H][I]).
"""
from __future__ import annotations

import ctypes
import os
import subprocess

import numpy as np

_HERE = os.path.dirname(os.path.abspath(__file__))
_LIB_PATH = os.path.join(_HERE, "libmoe_oracle.so")
_lib = None


def build() -> str:
    """Compiles the oracle C restatement (gcc, see oracle/Makefile)."""
    subprocess.run(["make", "-s", "-C", _HERE], check=True)
    return _LIB_PATH


def lib():
    global _lib
    if _lib is None:
        if not os.path.exists(_LIB_PATH):
            build()
        L = ctypes.CDLL(_LIB_PATH)
        u8, f32, i32, u32, vp = (ctypes.c_uint8, ctypes.c_float, ctypes.c_int,
                                 ctypes.c_uint32, ctypes.c_void_p)
        L.orc_e4m3_decode.restype = f32
        L.orc_e4m3_decode.argtypes = [u8]
        L.orc_e4m3_quantize.restype = u8
        L.orc_e4m3_quantize.argtypes = [f32]
        L.orc_f32_to_bf16.restype = ctypes.c_uint16
        L.orc_f32_to_bf16.argtypes = [f32]
        L.orc_bf16_to_f32.restype = f32
        L.orc_bf16_to_f32.argtypes = [ctypes.c_uint16]
        L.orc_ceil_ue8m0.restype = u8
        L.orc_ceil_ue8m0.argtypes = [f32]
        L.orc_block_scale.restype = u8
        L.orc_block_scale.argtypes = [f32]
        L.orc_wprobe_val.restype = u8
        L.orc_wprobe_val.argtypes = [u32, u32, u32]
        L.orc_quant_rows_ue8m0.argtypes = [vp, i32, i32, i32, vp, vp]
        L.orc_quant_blocks_ue8m0.argtypes = [vp, i32, i32, i32, vp, vp]
        L.orc_checkcu_inputs.argtypes = [i32, i32, i32, i32, vp, vp]
        L.orc_balanced_routes.argtypes = [i32, i32, i32, i32, i32, vp]
        L.orc_routes_from_counts.restype = i32
        L.orc_routes_from_counts.argtypes = [vp, i32, i32, i32, i32, vp]
        L.orc_route.argtypes = [vp, i32, i32, i32, i32, vp, vp, vp, vp]
        L.orc_l1_rows.argtypes = [vp, vp, i32, vp, vp, i32, i32, i32, vp]
        L.orc_quant_ffn.argtypes = [vp, i32, i32, i32, vp, vp]
        L.orc_l2_rows.argtypes = [vp, vp, i32, vp, vp, i32, i32, vp]
        L.orc_reduce.argtypes = [vp, vp, vp, i32, i32, i32, vp, vp]
        L.orc_set_acc64.argtypes = [i32]
        L.orc_set_mutation.argtypes = [i32]
        L.orc_layer_slots.restype = i32
        L.orc_layer_slots.argtypes = [vp, vp, vp, vp, vp, vp, vp, vp, i32, i32, i32, i32,
                                      i32, i32, vp, vp, vp, vp, i32]
        _lib = L
    return _lib


def _p(a):
    if a is None:
        return None
    assert a.flags["C_CONTIGUOUS"], "oracle arrays must be C-contiguous"
    return a.ctypes.data


# ----------------------------------------------------------- scalar codecs --
def e4m3_decode_table() -> np.ndarray:
    L = lib()
    return np.array([L.orc_e4m3_decode(i) for i in range(256)], dtype=np.float32)


def e4m3_quantize(v: np.ndarray) -> np.ndarray:
    L = lib()
    v = np.ascontiguousarray(v, dtype=np.float32).ravel()
    return np.array([L.orc_e4m3_quantize(float(x)) for x in v], dtype=np.uint8)


def f32_to_bf16(v: np.ndarray) -> np.ndarray:
    L = lib()
    v = np.ascontiguousarray(v, dtype=np.float32).ravel()
    return np.array([L.orc_f32_to_bf16(float(x)) for x in v], dtype=np.uint16)


def ceil_ue8m0(v: float) -> int:
    return int(lib().orc_ceil_ue8m0(float(v)))


def block_scale(amax: float) -> int:
    return int(lib().orc_block_scale(float(amax)))


# ------------------------------------------------------------- casts --------
def quant_rows_ue8m0(x: np.ndarray, gran: int = 128):
    x = np.ascontiguousarray(x, dtype=np.float32)
    rows, cols = x.shape
    q = np.empty((rows, cols), np.uint8)
    sf = np.empty((rows, cols // gran), np.uint8)
    lib().orc_quant_rows_ue8m0(_p(x), rows, cols, gran, _p(q), _p(sf))
    return q, sf


def quant_blocks_ue8m0(w: np.ndarray, gran: int = 128):
    w = np.ascontiguousarray(w, dtype=np.float32)
    rows, cols = w.shape
    q = np.empty((rows, cols), np.uint8)
    sf = np.empty((rows // gran, cols // gran), np.uint8)
    lib().orc_quant_blocks_ue8m0(_p(w), rows, cols, gran, _p(q), _p(sf))
    return q, sf


# -------------------------------------------------------- generators --------
def wprobe_matrix(seed: int, row0: int, rows: int, cols: int) -> np.ndarray:
    """WPROBE_VAL(seed, row, k) over logical rows [row0, row0+rows)."""
    r = (np.arange(row0, row0 + rows, dtype=np.uint64)[:, None])
    k = np.arange(cols, dtype=np.uint64)[None, :]
    return ((seed + r * 131 + k * 7) & 0x3F).astype(np.uint8)


def checkcu_inputs(ranks: int, tpr: int, H: int, topk: int):
    x = np.empty((ranks * tpr, H), np.uint8)
    w = np.empty((ranks * tpr, topk), np.float32)
    lib().orc_checkcu_inputs(ranks, tpr, H, topk, _p(x), _p(w))
    return x, w


def balanced_routes(ranks: int, tokens: int, topk: int, epr: int, salt: int = 0):
    idx = np.empty((ranks * tokens, topk), np.int64)
    lib().orc_balanced_routes(ranks, tokens, topk, epr, salt, _p(idx))
    return idx


def routes_from_counts(per_expert, R: int, epr: int, tokens: int, topk: int):
    pe = np.ascontiguousarray(per_expert, dtype=np.int32)
    idx = np.empty((R * tokens, topk), np.int64)
    rc = lib().orc_routes_from_counts(_p(pe), R, epr, tokens, topk, _p(idx))
    if rc != 0:
        raise ValueError("routes_from_counts: duplicate expert within a token")
    return idx


# ------------------------------------------------------------- the path -----
def route(topk_idx: np.ndarray, E: int, cap: int | None = None):
    idx = np.ascontiguousarray(topk_idx, dtype=np.int64)
    T, K = idx.shape
    cap = T * K if cap is None else cap
    counts = np.empty(E, np.int32)
    offsets = np.empty(E + 1, np.int32)
    perm = np.zeros(max(T * K, 1), np.uint32)
    pair_pos = np.empty(T * K, np.int32)
    lib().orc_route(_p(idx), T, K, E, cap, _p(counts), _p(offsets), _p(perm), _p(pair_pos))
    return counts, offsets, perm[: offsets[E]], pair_pos


def set_mutation(m: int) -> None:
    """Plants a known mistake in the oracle (tests of the pins' sensitivity
    only; 0 restores the faithful restatement)."""
    lib().orc_set_mutation(int(m))


def l1_rows(x, xsf, w1e, w1sf, G: int):
    x = np.ascontiguousarray(x, np.uint8)
    rows, H = x.shape
    I = w1e.shape[0] // 2
    out = np.empty((rows, I), np.float32)
    lib().orc_l1_rows(_p(x), _p(xsf), rows, _p(np.ascontiguousarray(w1e)), _p(w1sf), H, I, G,
                      _p(out))
    return out


def quant_ffn(h: np.ndarray, scaled: bool):
    h = np.ascontiguousarray(h, np.float32)
    rows, I = h.shape
    q = np.empty((rows, I), np.uint8)
    sf = np.full((rows, I // 128), 127, np.uint8)
    lib().orc_quant_ffn(_p(h), rows, I, int(scaled), _p(q), _p(sf))
    return q, (sf if scaled else None)


def l2_rows(ffn, fsf, w2e, w2sf):
    ffn = np.ascontiguousarray(ffn, np.uint8)
    rows, I = ffn.shape
    H = w2e.shape[0]
    out = np.empty((rows, H), np.float32)
    lib().orc_l2_rows(_p(ffn), _p(fsf), rows, _p(np.ascontiguousarray(w2e)), _p(w2sf), H, I,
                      _p(out))
    return out


def reduce(l2_bits: np.ndarray, pair_pos: np.ndarray, w: np.ndarray, T: int, topk: int):
    l2_bits = np.ascontiguousarray(l2_bits, np.uint16)
    H = l2_bits.shape[1]
    y = np.empty((T, H), np.float32)
    yb = np.empty((T, H), np.uint16)
    lib().orc_reduce(_p(l2_bits), _p(np.ascontiguousarray(pair_pos, np.int32)),
                     _p(np.ascontiguousarray(w, np.float32)), T, topk, H, _p(y), _p(yb))
    return y, yb


def layer(x, xsf, w1, w1sf, w2, w2sf, topk_idx, topk_w, E: int, G: int, scaled: bool,
          nthreads: int = 8, expert_mask=None, cap: int | None = None, acc64: bool = False):
    """Full reference chain: route -> L1 -> quant -> L2 -> bf16 -> reduce.
    acc64=True sums the GEMMs in float64 (an exactly-summing device model).

    Returns dict with counts/offsets/perm/pair_pos/ffn/ffn_sf/l2/y/y_bf16."""
    T, K = topk_idx.shape
    H = x.shape[1]
    I = w2.shape[2]
    counts, offsets, perm, pair_pos = route(topk_idx, E, cap)
    slots = int(offsets[E])
    ffn = np.zeros((max(slots, 1), I), np.uint8)
    ffn_sf = np.full((max(slots, 1), I // 128), 127, np.uint8)
    l2 = np.zeros((max(slots, 1), H), np.uint16)
    perm_c = np.ascontiguousarray(np.concatenate([perm, np.zeros(1, np.uint32)]))
    mask = None if expert_mask is None else np.ascontiguousarray(expert_mask, np.uint8)
    lib().orc_set_acc64(int(acc64))
    lib().orc_layer_slots(_p(np.ascontiguousarray(x)), _p(xsf), _p(np.ascontiguousarray(w1)),
                          _p(w1sf), _p(np.ascontiguousarray(w2)), _p(w2sf), _p(offsets),
                          _p(perm_c), K, E, H, I, G, int(scaled), _p(mask), _p(ffn),
                          _p(ffn_sf), _p(l2), nthreads)
    lib().orc_set_acc64(0)
    y, yb = reduce(l2, pair_pos, topk_w, T, K)
    return dict(counts=counts, offsets=offsets, perm=perm, pair_pos=pair_pos,
                ffn=ffn[:slots], ffn_sf=ffn_sf[:slots] if scaled else None, l2=l2[:slots],
                y=y, y_bf16=yb)
