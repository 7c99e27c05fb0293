"""Seeded synthetic inputs for the MoE layer (the benchmark and test workloads).

* x: bf16 ~ N(0, 1) [T, H] cast to fp8 e4m3 with per-token per-128-column
  UE8M0 scales by the HIP quant_act kernel (or a direct RNE cast, unscaled).
* W1 [E, 2I, H], W2 [E, H, I]: ~ N(0, 0.02) generated on the device in tile
  layout with 128x128 UE8M0 block scales (fill_weights_normal), or the
  reference's deterministic WPROBE bytes (fill_weights_lane, check.cu inputs).
* Router: logits [T, E] ~ N(0, 1) (+ an optional Zipf(s) per-expert bias),
  softmax -> top-k (ties to the lower index) -> renormalised weights.

The router runs in float64 numpy on the host so that routing is identical on
every machine; it is input preparation, not part of the layer.
"""
from __future__ import annotations

import ctypes

import numpy as np
import torch

from ._lib import check, lib
from .mega import pairing_block


def _stream() -> int:
    return torch.cuda.current_stream().cuda_stream


ZIPF_STRENGTH = 0.4   # hottest 8 experts get ~8x the mean load at T=2048
ZIPF_DEAD = 16        # coldest-ranked experts that receive no tokens


def zipf_bias(E: int, s: float, seed: int, strength: float = ZIPF_STRENGTH,
              dead: int = ZIPF_DEAD) -> np.ndarray:
    """Per-expert logit bias strength*log(1/rank^s) over a seeded permutation
    of the experts (the hottest experts are spread over the id range); the
    `dead` coldest ranks get -inf (empty experts)."""
    rng = np.random.default_rng(seed ^ 0x5A5A)
    ranks = rng.permutation(E) + 1
    bias = strength * (-s) * np.log(ranks.astype(np.float64))
    if dead > 0 and dead < E:
        bias[ranks > E - dead] = -np.inf
    return bias


def route(T: int, E: int, topk: int, seed: int, zipf_s: float | None = None,
          zipf_strength: float = ZIPF_STRENGTH):
    """Softmax top-k router on N(0,1) logits; returns (topk_idx int64 [T,k],
    topk_weights float32 [T,k]) as numpy arrays."""
    rng = np.random.default_rng(seed)
    logits = rng.standard_normal((T, E))
    if zipf_s is not None:
        logits = logits + zipf_bias(E, zipf_s, seed, zipf_strength)[None, :]
    m = logits.max(axis=1, keepdims=True)
    p = np.exp(logits - m)
    p /= p.sum(axis=1, keepdims=True)
    # stable sort of -p: ties resolve to the lower expert index
    idx = np.argsort(-p, axis=1, kind="stable")[:, :topk]
    w = np.take_along_axis(p, idx, axis=1)
    w = w / w.sum(axis=1, keepdims=True)
    return idx.astype(np.int64), w.astype(np.float32)


def routes_with_counts(per_expert, topk: int) -> np.ndarray:
    """topk_idx int64 [T, topk] whose per-expert counts are exactly
    per_expert (T = sum / topk): every token takes the topk experts with the
    most rows left (ties to the lower index), so each token's experts are
    distinct as long as no expert holds more than T rows.  Used to replay a
    logged routing distribution (the reference bench's --tk-info inputs,
    test/mybench.cu), not to model any router."""
    left = np.asarray(per_expert, dtype=np.int64).copy()
    total = int(left.sum())
    if total % topk:
        raise ValueError(f"{total} routed pairs are not a multiple of top-{topk}")
    T = total // topk
    if left.max(initial=0) > T:
        raise ValueError("an expert holds more rows than there are tokens")
    idx = np.empty((T, topk), np.int64)
    for t in range(T):
        pick = np.argsort(-left, kind="stable")[:topk]
        idx[t] = pick
        left[pick] -= 1
    if left.min(initial=0) < 0:
        raise ValueError("counts cannot be split into distinct top-k rows")
    return idx


def read_tk_info(path: str) -> dict:
    """{launch: per-expert counts [ranks * experts per rank]} from a TK_INFO
    log ("[TK_INFO] rank=R launch=L n=N : c0 c1 ..."), the reference's
    routing-distribution format (test/mega_common.cuh:460-482)."""
    import re
    data: dict = {}
    for line in open(path, encoding="utf-8"):
        m = re.search(r"\[TK_INFO\] rank=(\d+) launch=(\d+) n=\d+ : (.*)", line)
        if m:
            data.setdefault(int(m.group(2)), {})[int(m.group(1))] = [int(v) for v in m.group(3).split()]
    return {l: np.array([c for r in sorted(rk) for c in rk[r]], np.int64) for l, rk in data.items()}


def make_x(T: int, H: int, seed: int, scaled: bool = True):
    """bf16 N(0,1) activations on the device -> (x_bf16, x_fp8 [T,H] uint8,
    x_sf [T,H/128] uint8 or None)."""
    g = torch.Generator(device="cuda")
    g.manual_seed(seed)
    xb = torch.randn((T, H), generator=g, device="cuda", dtype=torch.float32).to(torch.bfloat16)
    q = torch.empty((T, H), dtype=torch.uint8, device="cuda")
    sf = torch.empty((T, H // 128), dtype=torch.uint8, device="cuda") if scaled else None
    check("mm_quant_act", lib().mm_quant_act(xb.data_ptr(), T, H, q.data_ptr(),
                                             sf.data_ptr() if sf is not None else None,
                                             _stream()))
    return xb, q, sf


def make_weights_normal(E: int, H: int, I: int, seed: int, sigma: float = 0.02):
    """Packed W1 [E,2I,H] (+ scales [E,2I/128,H/128]) and W2 [E,H,I] (+ scales),
    N(0, sigma) with 128x128 UE8M0 block scales."""
    w1 = torch.empty((E, 2 * I, H), dtype=torch.uint8, device="cuda")
    s1 = torch.empty((E, 2 * I // 128, H // 128), dtype=torch.uint8, device="cuda")
    w2 = torch.empty((E, H, I), dtype=torch.uint8, device="cuda")
    s2 = torch.empty((E, H // 128, I // 128), dtype=torch.uint8, device="cuda")
    L = lib()
    check("mm_fill_weights_normal", L.mm_fill_weights_normal(
        w1.data_ptr(), s1.data_ptr(), E, 2 * I, H, seed, sigma, _stream()))
    check("mm_fill_weights_normal", L.mm_fill_weights_normal(
        w2.data_ptr(), s2.data_ptr(), E, H, I, seed + 1, sigma, _stream()))
    return (w1.view(torch.float8_e4m3fn), s1), (w2.view(torch.float8_e4m3fn), s2)


def make_weights_checkcu(E: int, H: int, I: int, epr: int = 8, seed1: int = 17, seed2: int = 91):
    """check.cu weights: every rank holds the same `epr` local experts filled
    with WPROBE_VAL(seed, row, k) over the whole [epr*2I, H] / [epr*H, I]
    tensors (test/mega_common.cuh:229-240); global expert e uses local e % epr."""
    epr = min(epr, E)
    L = lib()
    w1l = torch.empty((epr, 2 * I, H), dtype=torch.uint8, device="cuda")
    w2l = torch.empty((epr, H, I), dtype=torch.uint8, device="cuda")
    check("mm_fill_weights_lane",
          L.mm_fill_weights_lane(w1l.data_ptr(), epr * 2 * I, H, seed1, _stream()))
    check("mm_fill_weights_lane",
          L.mm_fill_weights_lane(w2l.data_ptr(), epr * H, I, seed2, _stream()))
    reps = (E + epr - 1) // epr
    w1 = w1l.repeat(reps, 1, 1)[:E].contiguous()
    w2 = w2l.repeat(reps, 1, 1)[:E].contiguous()
    return w1.view(torch.float8_e4m3fn), w2.view(torch.float8_e4m3fn)


# ------------------------------------------------------------- host views --
def unpack_tiles(packed: np.ndarray, n_rows: int, k_cols: int) -> np.ndarray:
    """Tile layout bytes of one [n_rows, k_cols] matrix -> logical row-major
    (numpy; the inverse of the device packing, used by checkers)."""
    KT = k_cols // 128
    t = packed.reshape(n_rows // 16, KT, 2, 4, 16, 16)  # nt, kt, h, kq, r, j
    # byte (r, k): k = 128*kt + 32*kq + 16*h + j
    out = t.transpose(0, 4, 1, 3, 2, 5).reshape(n_rows, k_cols)
    return np.ascontiguousarray(out)


def paired_to_torch_rows(I: int) -> np.ndarray:
    """Index map: paired-order row rho -> torch-order row ([gate(I); up(I)])."""
    G = pairing_block(I)
    rho = np.arange(2 * I)
    blk, r = rho // (2 * G), rho % (2 * G)
    is_up = r >= G
    h = blk * G + (r % G)
    return np.where(is_up, I + h, h)
