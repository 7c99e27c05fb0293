// gemm_big.hip -- the L1 / L2 grouped GEMMs for large per-expert row counts
// (work items of 64..128 token rows: T >= ~1024 and skewed routing), where
// the decode-shaped kernels of gemm.hip would re-stream each expert's weights
// once per 32 rows.
//
// Reference counterparts: r24_l1_big / r24_l2_big (src/compute_big.cuh:888-1161,
// 1375-1679), the reference's count-tiered big-window GEMMs.
//
// One 8-wave workgroup per (work item, block of 256 weight rows); each wave
// owns a 32-row weight slice across all of the item's token rows (every weight
// byte is loaded and converted exactly once):
//   * per 128-k step, all 512 threads gather the item's BM = 16*MT activation
//     rows (through perm[] for L1, slot order for L2), convert them once to
//     bf16 with the row's UE8M0 scale folded in (exact), and store them in a
//     double-buffered LDS tile: [token tile][k-group q][lane][8 bf16], so that
//     a wave's operand read for one MFMA is 1 KiB contiguous;
//   * each wave streams its two 16-row weight tiles (L1: gate and up rows of
//     16 hidden columns; L2: 32 output channels) from HBM through a 4-stage
//     register pipeline and converts them exactly to bf16;
//   * v_mfma_f32_16x16x32_bf16 (fp32-accurate sums; see gemm.hip) over the
//     item's NT active token tiles -- NT is a compile-time specialisation
//     picked per item, so there is no per-tile branch in the k loop and the
//     2*NT accumulators are independent chains;
//   * epilogues as in gemm.hip: L1 SwiGLU + fp8 (raw, or per-128 UE8M0 with
//     the 128-column amax reduced over the 8 waves in LDS), L2 bf16.
#include "mm_kernels.h"

namespace mm {

constexpr int kXTileBytes = 16 * kTileK * 2;   // one bf16 token tile: 16 rows x 128 k

template <int MT>
struct BigSmem {
    uint8_t x[2][MT * kXTileBytes];            // bf16 tiles, double buffered
    uint8_t sfx[MT * 16][kBigMaxKT];           // the item's row scales, all k-steps
    uint8_t sfw[16][kBigMaxKT];                // the block's 16 weight tiles' scales
};

// Loader: chunk i = tid + 512*u is row r = 16*(i/128) + i%16 of the item,
// fp8 bytes [16*cc, 16*cc+16) of the k-step with cc = (i/16)%8: k-group
// g = cc/2, MFMA groups q = 2*(cc%2) and q+1.  Rows vary fastest, so the 16
// lanes of an LDS write phase fill 16 consecutive 16-byte slots (no bank
// conflicts).  Two register stages: the rows of k-step kt+2 are in flight
// while kt+1 is written to LDS.  Row addresses are 32-bit offsets.
template <int MT>
struct XLoader {
    static constexpr int U = MT / 4;
    const uint8_t* base;
    uint32_t off[U];
    v4i reg[2][U];

    __device__ __forceinline__ static int row_of(int i) { return ((i >> 7) << 4) | (i & 15); }
    __device__ __forceinline__ static int cc_of(int i) { return (i >> 4) & 7; }

    __device__ __forceinline__ void issue(int kt, int rs) {
#pragma unroll
        for (int u = 0; u < U; ++u) reg[rs][u] = load16(base + off[u] + kt * kTileK);
    }
    __device__ __forceinline__ void commit(BigSmem<MT>& sm, int stage, int rs, int kt) {
#pragma unroll
        for (int u = 0; u < U; ++u) {
            const int i = threadIdx.x + kBigThreads * u;
            const int r = row_of(i), cc = cc_of(i);
            const int lane_slot = (r & 15) + 16 * (cc >> 1);
            const int q0 = 2 * (cc & 1);
            uint8_t* t = &sm.x[stage][(r >> 4) * kXTileBytes + q0 * 1024 + lane_slot * 16];
            const float s = ue8m0_to_f32(sm.sfx[r][kt]);
            *reinterpret_cast<v8bf*>(t) = fp8x8_to_bf16(reg[rs][u][0], reg[rs][u][1], s);
            *reinterpret_cast<v8bf*>(t + 1024) = fp8x8_to_bf16(reg[rs][u][2], reg[rs][u][3], s);
        }
    }
};

struct WStage {
    v4i a[2][2];   // two weight tiles, two 16-byte halves each
};

__device__ __forceinline__ void w_load(WStage& w, const uint8_t* const* wt, int kt) {
    const size_t o = (size_t)kt * kTileBytes;
#pragma unroll
    for (int t = 0; t < 2; ++t) {
        w.a[t][0] = load16_stream(wt[t] + o);
        w.a[t][1] = load16_stream(wt[t] + o + 1024);
    }
}

// acc[t][j] += weight tile t x token tile j, j < NT, one 128-k step.
template <int MT, int NT>
__device__ __forceinline__ void big_mma(v4f (&acc)[2][NT], const WStage& w,
                                        const BigSmem<MT>& sm, int stage, int kt) {
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const float s0 = ue8m0_to_f32(sm.sfw[2 * wave][kt]);
    const float s1 = ue8m0_to_f32(sm.sfw[2 * wave + 1][kt]);
#pragma unroll
    for (int q = 0; q < 4; ++q) {
        const v8bf a0 = fp8x8_to_bf16(w.a[0][q >> 1][2 * (q & 1)], w.a[0][q >> 1][2 * (q & 1) + 1], s0);
        const v8bf a1 = fp8x8_to_bf16(w.a[1][q >> 1][2 * (q & 1)], w.a[1][q >> 1][2 * (q & 1) + 1], s1);
#pragma unroll
        for (int j = 0; j < NT; ++j) {
            const v8bf b = *reinterpret_cast<const v8bf*>(
                &sm.x[stage][j * kXTileBytes + q * 1024 + lane * 16]);
            acc[0][j] = mfma_bf16(a0, b, acc[0][j]);
            acc[1][j] = mfma_bf16(a1, b, acc[1][j]);
        }
    }
}

constexpr int kBigStages = 4;   // weight register stages (even: x stages alternate)

// One k-step of the pipeline: prefetch activations for kt+2 and weights for
// kt+S-1 (indices clamped to the last step: a redundant in-bounds reload
// keeps the loop free of branches, so the compiler's wait counts stay
// partial), compute kt, write the activations of kt+1 to LDS, barrier.  All
// scale bytes come from LDS, so the only vector-memory loads in the loop are
// the prefetches themselves.
template <int MT, int NT, int S, int s>
__device__ __forceinline__ void big_step(v4f (&acc)[2][NT], BigSmem<MT>& sm, XLoader<MT>& xl,
                                         WStage (&w)[S], const uint8_t* const* wt, int kt,
                                         int KT) {
    xl.issue(min(kt + 2, KT - 1), s & 1);
    w_load(w[(s + S - 1) % S], wt, min(kt + S - 1, KT - 1));
    // keep the prefetch loads ahead of this step's MFMAs
    __builtin_amdgcn_sched_barrier(0);
    big_mma<MT, NT>(acc, w[s], sm, kt & 1, kt);
    __builtin_amdgcn_sched_barrier(0);
    xl.commit(sm, (kt + 1) & 1, (s + 1) & 1, min(kt + 1, KT - 1));
    __syncthreads();
}

template <int MT, int NT, int S, int s>
__device__ __forceinline__ void big_group(v4f (&acc)[2][NT], BigSmem<MT>& sm, XLoader<MT>& xl,
                                          WStage (&w)[S], const uint8_t* const* wt, int kb,
                                          int KT) {
    big_step<MT, NT, S, s>(acc, sm, xl, w, wt, kb + s, KT);
    if constexpr (s + 1 < S) big_group<MT, NT, S, s + 1>(acc, sm, xl, w, wt, kb, KT);
}

// Main loop: every wave runs the same KT + 1 barriers.  Activations: LDS
// double buffer fed from two register stages.  Weights: S register stages.
// Whole groups of S k-steps run without any branch; a remainder (only when
// KT is not a multiple of S: tiny shapes) runs through the guarded tail.
template <int MT, int NT>
__device__ __forceinline__ void big_mainloop(v4f (&acc)[2][NT], BigSmem<MT>& sm,
                                             XLoader<MT>& xl, const uint8_t* const* wt, int KT) {
    constexpr int S = kBigStages;
    WStage w[S];
    xl.issue(0, 0);
    xl.issue(min(1, KT - 1), 1);
#pragma unroll
    for (int s = 0; s < S - 1; ++s) w_load(w[s], wt, min(s, KT - 1));
    xl.commit(sm, 0, 0, 0);
    __syncthreads();
    const int KF = KT - KT % S;
#pragma unroll 1
    for (int kb = 0; kb < KF; kb += S) big_group<MT, NT, S, 0>(acc, sm, xl, w, wt, kb, KT);
    if (KF < KT) {
        big_step<MT, NT, S, 0>(acc, sm, xl, w, wt, KF, KT);
        if (KF + 1 < KT) big_step<MT, NT, S, 1>(acc, sm, xl, w, wt, KF + 1, KT);
        if (KF + 2 < KT) big_step<MT, NT, S, 2>(acc, sm, xl, w, wt, KF + 2, KT);
    }
}

// Loads the item's row scales and the block's weight-tile scales into LDS
// (2^0 where the operand has none).  row_scale_base(r) gives row r's scale
// row; tile_scale_base(t) tile t's (t = 2*wave + 0/1).
template <int MT, class RowF, class TileF>
__device__ __forceinline__ void big_load_scales(BigSmem<MT>& sm, int KT, bool has_x, bool has_w,
                                                RowF row_scale_base, TileF tile_scale_base) {
    for (int i = threadIdx.x; i < MT * 16 * KT; i += kBigThreads) {
        const int r = i / KT, k = i - r * KT;
        sm.sfx[r][k] = has_x ? row_scale_base(r)[k] : (uint8_t)127;
    }
    for (int i = threadIdx.x; i < 16 * KT; i += kBigThreads) {
        const int t = i / KT, k = i - t * KT;
        sm.sfw[t][k] = has_w ? tile_scale_base(t)[k] : (uint8_t)127;
    }
    __syncthreads();
}

// Per-item context shared by the two kernels.
struct BigItem {
    int e, m0, rows, off, ntiles;
};

__device__ __forceinline__ bool big_item(const GemmParams& p, BigItem& it) {
    const int item = blockIdx.y;
    if (item >= p.status[1]) return false;
    const int4 v = reinterpret_cast<const int4*>(p.items)[item];
    it.e = v.x;
    it.m0 = v.y;
    it.rows = v.z - v.y;
    it.off = p.offsets[it.e];
    it.ntiles = (it.rows + 15) >> 4;
    return true;
}

template <int NT>
__device__ __forceinline__ void zero2(v4f (&acc)[2][NT]) {
#pragma unroll
    for (int t = 0; t < 2; ++t)
#pragma unroll
        for (int j = 0; j < NT; ++j) acc[t][j] = v4f{0.f, 0.f, 0.f, 0.f};
}

// ---------------------------------------------------------------------- L1 --
template <int MT, int NT>
__device__ __forceinline__ void l1_big_body(const GemmParams& p, const BigItem& it,
                                            BigSmem<MT>& sm, XLoader<MT>& xl) {
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int H = p.H, I = p.I, G = p.G, KT = H >> 7;
    const int hw = blockIdx.x * kL1BlockH + wave * 16;   // this wave's hidden columns
    const int rho = (hw / G) * 2 * G + (hw % G);
    const int ntg = rho >> 4, ntu = ntg + (G >> 4);
    const uint8_t* we = p.w + (size_t)it.e * (size_t)(2 * I) * H;
    const size_t tstride = (size_t)KT * kTileBytes;
    const uint8_t* wt[2] = {we + (size_t)ntg * tstride + lane * 16,
                            we + (size_t)ntu * tstride + lane * 16};
    v4f acc[2][NT];
    zero2<NT>(acc);
    big_mainloop<MT, NT>(acc, sm, xl, wt, KT);

    // h = silu(g) * u: channels hw + 4*(L/16) + i, token 16*j + L%16
    float hv[NT][4];
#pragma unroll
    for (int j = 0; j < NT; ++j)
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const float g = acc[0][j][i], u = acc[1][j][i];
            hv[j][i] = (g / (1.0f + __expf(-g))) * u;
        }
    const int I128 = I >> 7;
    if (p.ffn_ue8m0) {
        // amax over the block's 128 hidden columns = the 8 waves; the LDS
        // tiles are free after the main loop's last barrier.
        float* red = reinterpret_cast<float*>(&sm.x[0][0]);   // [8][MT*16]
#pragma unroll
        for (int j = 0; j < NT; ++j) {
            float m = fmaxf(fmaxf(fabsf(hv[j][0]), fabsf(hv[j][1])),
                            fmaxf(fabsf(hv[j][2]), fabsf(hv[j][3])));
            m = fmaxf(m, __shfl_xor(m, 16, 64));
            m = fmaxf(m, __shfl_xor(m, 32, 64));
            if (lane < 16) red[wave * (MT * 16) + 16 * j + lane] = m;
        }
        __syncthreads();
#pragma unroll
        for (int j = 0; j < NT; ++j) {
            const int r = 16 * j + (lane & 15);
            float amax = red[r];
#pragma unroll
            for (int w = 1; w < 8; ++w) amax = fmaxf(amax, red[w * (MT * 16) + r]);
            const uint32_t sb = block_scale_byte(amax);
            const float inv = inv_scale(sb);
            if (r < it.rows) {
                const size_t slot = (size_t)(it.off + it.m0 + r);
                *reinterpret_cast<uint32_t*>(p.out8 + slot * I + hw + 4 * (lane >> 4)) =
                    pack4_fp8(hv[j][0] * inv, hv[j][1] * inv, hv[j][2] * inv, hv[j][3] * inv);
                if (wave == 0 && lane < 16) p.out_sf[slot * I128 + blockIdx.x] = (uint8_t)sb;
            }
        }
    } else {
#pragma unroll
        for (int j = 0; j < NT; ++j) {
            const int r = 16 * j + (lane & 15);
            if (r < it.rows) {
                const size_t slot = (size_t)(it.off + it.m0 + r);
                *reinterpret_cast<uint32_t*>(p.out8 + slot * I + hw + 4 * (lane >> 4)) =
                    pack4_fp8(hv[j][0], hv[j][1], hv[j][2], hv[j][3]);
            }
        }
    }
}

// NT (the item's token tiles) is uniform over the block, so every wave runs
// the same body and the same barriers.
template <int MT>
__global__ void __launch_bounds__(kBigThreads) l1_big_kernel(GemmParams p) {
    __shared__ BigSmem<MT> sm;
    BigItem it;
    if (!big_item(p, it)) return;
    XLoader<MT> xl;
    xl.base = p.x;
    const int KT = p.H >> 7;
#pragma unroll
    for (int u = 0; u < XLoader<MT>::U; ++u) {
        const int i = threadIdx.x + kBigThreads * u;
        const int r = XLoader<MT>::row_of(i), cc = XLoader<MT>::cc_of(i);
        const int slot = it.off + it.m0 + (r < it.rows ? r : 0);
        const uint32_t tok = p.perm[slot] / (uint32_t)p.topk;
        xl.off[u] = tok * (uint32_t)p.H + cc * 16;
    }
    {
        // scales: x rows through perm[]; W1 tiles 2*wave (gate), 2*wave+1 (up)
        const int I = p.I, G = p.G;
        big_load_scales<MT>(
            sm, KT, p.x_sf != nullptr, p.w_sf != nullptr,
            [&](int r) {
                const int slot = it.off + it.m0 + (r < it.rows ? r : 0);
                return p.x_sf + (size_t)(p.perm[slot] / (uint32_t)p.topk) * KT;
            },
            [&](int t) {
                const int hw = blockIdx.x * kL1BlockH + (t >> 1) * 16;
                const int rho = (hw / G) * 2 * G + (hw % G) + ((t & 1) ? G : 0);
                return p.w_sf + ((size_t)it.e * (2 * I / 128) + (rho >> 7)) * KT;
            });
    }
    switch (it.ntiles) {
        case 1: l1_big_body<MT, 1>(p, it, sm, xl); break;
        case 2: l1_big_body<MT, 2>(p, it, sm, xl); break;
        case 3: l1_big_body<MT, 3>(p, it, sm, xl); break;
        case 4: l1_big_body<MT, 4>(p, it, sm, xl); break;
        case 5: if constexpr (MT >= 5) l1_big_body<MT, 5>(p, it, sm, xl); break;
        case 6: if constexpr (MT >= 6) l1_big_body<MT, 6>(p, it, sm, xl); break;
        case 7: if constexpr (MT >= 7) l1_big_body<MT, 7>(p, it, sm, xl); break;
        default: if constexpr (MT >= 8) l1_big_body<MT, 8>(p, it, sm, xl); break;
    }
}

// ---------------------------------------------------------------------- L2 --
template <int MT, int NT>
__device__ __forceinline__ void l2_big_body(const GemmParams& p, const BigItem& it,
                                            BigSmem<MT>& sm, XLoader<MT>& xl) {
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int H = p.H, I = p.I, KT = I >> 7;
    const int n0 = blockIdx.x * kL2BlockN + wave * 32;
    const uint8_t* we = p.w + (size_t)it.e * (size_t)H * I;
    const size_t tstride = (size_t)KT * kTileBytes;
    const uint8_t* wt[2] = {we + (size_t)(n0 >> 4) * tstride + lane * 16,
                            we + (size_t)((n0 >> 4) + 1) * tstride + lane * 16};
    v4f acc[2][NT];
    zero2<NT>(acc);
    big_mainloop<MT, NT>(acc, sm, xl, wt, KT);
#pragma unroll
    for (int j = 0; j < NT; ++j) {
        const int r = 16 * j + (lane & 15);
        if (r < it.rows) {
            const size_t slot = (size_t)(it.off + it.m0 + r);
#pragma unroll
            for (int t = 0; t < 2; ++t) {
                uint2 v;
                v.x = bf16_rne(acc[t][j][0]) | (bf16_rne(acc[t][j][1]) << 16);
                v.y = bf16_rne(acc[t][j][2]) | (bf16_rne(acc[t][j][3]) << 16);
                *reinterpret_cast<uint2*>(p.out16 + slot * H + n0 + 16 * t + 4 * (lane >> 4)) = v;
            }
        }
    }
}

template <int MT>
__global__ void __launch_bounds__(kBigThreads) l2_big_kernel(GemmParams p) {
    __shared__ BigSmem<MT> sm;
    BigItem it;
    if (!big_item(p, it)) return;
    XLoader<MT> xl;
    xl.base = p.x;
    const int KT = p.I >> 7;
#pragma unroll
    for (int u = 0; u < XLoader<MT>::U; ++u) {
        const int i = threadIdx.x + kBigThreads * u;
        const int r = XLoader<MT>::row_of(i), cc = XLoader<MT>::cc_of(i);
        const uint32_t slot = (uint32_t)(it.off + it.m0 + (r < it.rows ? r : 0));
        xl.off[u] = slot * (uint32_t)p.I + cc * 16;
    }
    {
        // scales: ffn rows in slot order; W2 tiles of this block's 256 channels
        const int H = p.H;
        big_load_scales<MT>(
            sm, KT, p.x_sf != nullptr, p.w_sf != nullptr,
            [&](int r) {
                return p.x_sf + (size_t)(it.off + it.m0 + (r < it.rows ? r : 0)) * KT;
            },
            [&](int t) {
                const int n = blockIdx.x * kL2BlockN + t * 16;
                return p.w_sf + ((size_t)it.e * (H / 128) + (n >> 7)) * KT;
            });
    }
    switch (it.ntiles) {
        case 1: l2_big_body<MT, 1>(p, it, sm, xl); break;
        case 2: l2_big_body<MT, 2>(p, it, sm, xl); break;
        case 3: l2_big_body<MT, 3>(p, it, sm, xl); break;
        case 4: l2_big_body<MT, 4>(p, it, sm, xl); break;
        case 5: if constexpr (MT >= 5) l2_big_body<MT, 5>(p, it, sm, xl); break;
        case 6: if constexpr (MT >= 6) l2_big_body<MT, 6>(p, it, sm, xl); break;
        case 7: if constexpr (MT >= 7) l2_big_body<MT, 7>(p, it, sm, xl); break;
        default: if constexpr (MT >= 8) l2_big_body<MT, 8>(p, it, sm, xl); break;
    }
}

template __global__ void l1_big_kernel<4>(GemmParams);
template __global__ void l1_big_kernel<8>(GemmParams);
template __global__ void l2_big_kernel<4>(GemmParams);
template __global__ void l2_big_kernel<8>(GemmParams);

}  // namespace mm
