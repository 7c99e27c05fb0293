// gemm.hip -- the two grouped fp8 GEMMs of the MoE layer on CDNA4 MFMA.
//
// Both GEMMs read fp8 e4m3 operands from HBM and convert them in registers,
// exactly (UE8M0 scales folded in), to bf16 for v_mfma_f32_16x16x32_bf16.
// gfx950's fp8 MFMAs (v_mfma_scale_f32_16x16x128_f8f6f4 and
// v_mfma_f32_16x16x32_fp8_fp8 alike) return exact products but sum them with
// truncating alignment -- measured error up to ~2^-20 of sum|terms| against
// ~1e-8 for the bf16 MFMA and for sequential fp32 -- which flips the L1 fp8
// requantisation (and its 128-block scales) and the L2 bf16 rounding often
// enough, against the reference's fp32 host path, to break the layer's
// end-to-end tolerance.  The bf16 path keeps every sum fp32-accurate.
//
// L1 (reference: l1_gemm_swiglu_body_paired src/compute.cuh:280-484,
//     r19_l1_big / r24_l1_big src/compute_big.cuh:320-515, 888-1161):
//   for every work item (expert e, rows m0 .. m0+16*MT of e's slots) and every
//   block of 128 hidden columns, g/u = W1_e[gate/up rows] . x[token]^T, then
//   h = silu(g)*u and the fp8 cast of h
//   (raw RNE-saturating, or per-128 UE8M0 requant) into ffn[slot][I].
//   The activation rows are gathered straight from x through perm[] (the
//   fused DISPATCH gather: 16-byte loads of the routed tokens' rows).
// L2 (reference: l2_gemm_body src/compute.cuh:497-641, r24_l2_big
//     src/compute_big.cuh:1375-1679):
//   o = W2_e . ffn[slot]^T, bf16 RNE into l2[slot][H].
//
// Operand roles: the weight tile is the MFMA "A" operand (16 output channels
// x 128 k) and the 16 token rows are "B" (128 k x 16 tokens), so each lane's
// 4 accumulators are 4 consecutive output channels of one token, which packs
// into one 4-byte fp8 store (L1) or one 8-byte bf16 store (L2).
//
// Each wave owns 4 weight tiles (64 weight rows) for all MT token tiles of
// the item; weights stream from HBM once per item through an S-stage
// register pipeline (loads for k-step kt+S-1 are issued before the MFMAs of
// k-step kt).
#include "mm_kernels.h"

namespace mm {

template <int MT>
struct Stage {
    v4i a[4][2];   // 4 weight tiles, two 16-byte halves each
    v4i b[MT][2];  // MT token tiles
    int sa[2];     // weight scale bytes (two 128-row blocks at most)
    int sb[MT];    // token scale bytes
};

template <int MT>
__device__ __forceinline__ void load_stage(Stage<MT>& s, const WTiles<4>& wt,
                                           const uint8_t* const* xr, int kt,
                                           const uint8_t* wsf0, const uint8_t* wsf1,
                                           const uint8_t* const* xsf) {
#pragma unroll
    for (int t = 0; t < 4; ++t) {
        const uint8_t* a = wt.at(t, kt);
        s.a[t][0] = load16_stream(a);
        s.a[t][1] = load16_stream(a + 1024);
    }
#pragma unroll
    for (int j = 0; j < MT; ++j) {
        s.b[j][0] = load16(xr[j] + kt * kTileK);
        s.b[j][1] = load16(xr[j] + kt * kTileK + 16);
    }
    s.sa[0] = wsf0 ? (int)wsf0[kt] : 127;
    s.sa[1] = wsf1 ? (int)wsf1[kt] : 127;
#pragma unroll
    for (int j = 0; j < MT; ++j) s.sb[j] = xsf[j] ? (int)xsf[j][kt] : 127;
}

// bf16 MFMA step with fp32-accurate sums: each lane's 32 fp8 bytes per tile
// are converted (scale folded in, exact) to four groups of 8 bf16, group q
// feeding the q-th of four 16x16x32 MFMAs; A and B use the same grouping, so
// every k of the 128-step meets its partner exactly once.
struct MmaBf16 {
    template <int MT>
    __device__ __forceinline__ static void run(v4f (&acc)[4][MT], const Stage<MT>& s,
                                               int ntiles) {
        const float sa0 = ue8m0_to_f32(s.sa[0]), sa1 = ue8m0_to_f32(s.sa[1]);
#pragma unroll
        for (int q = 0; q < 4; ++q) {
            const int h = q >> 1, d = 2 * (q & 1);
            v8bf b[MT];
#pragma unroll
            for (int j = 0; j < MT; ++j)
                if (j < ntiles)
                    b[j] = fp8x8_to_bf16(s.b[j][h][d], s.b[j][h][d + 1], ue8m0_to_f32(s.sb[j]));
#pragma unroll
            for (int t = 0; t < 4; ++t) {
                const v8bf a = fp8x8_to_bf16(s.a[t][h][d], s.a[t][h][d + 1], t < 2 ? sa0 : sa1);
#pragma unroll
                for (int j = 0; j < MT; ++j)
                    if (j < ntiles) acc[t][j] = mfma_bf16(a, b[j], acc[t][j]);
            }
        }
    }
};

// K loop with an S-stage register pipeline over KT k-steps of 128.
template <class Mma, int MT, int S>
__device__ __forceinline__ void gemm_mainloop(v4f (&acc)[4][MT], const WTiles<4>& wt,
                                              const uint8_t* const* xr, int KT,
                                              const uint8_t* wsf0, const uint8_t* wsf1,
                                              const uint8_t* const* xsf, int ntiles) {
    Stage<MT> buf[S];
#pragma unroll
    for (int s = 0; s < S - 1; ++s)
        if (s < KT) load_stage<MT>(buf[s], wt, xr, s, wsf0, wsf1, xsf);
    for (int kb = 0; kb < KT; kb += S) {
#pragma unroll
        for (int s = 0; s < S; ++s) {
            const int kt = kb + s;
            const int kl = kt + S - 1;
            if (kl < KT) load_stage<MT>(buf[(s + S - 1) % S], wt, xr, kl, wsf0, wsf1, xsf);
            if (kt < KT) Mma::template run<MT>(acc, buf[s], ntiles);
        }
    }
}

template <int MT>
constexpr int stages_for() { return MT <= 2 ? 3 : 2; }

template <int MT>
__global__ void __launch_bounds__(kGemmThreads) l1_kernel(GemmParams p) {
    const int item = blockIdx.y;
    if (item >= p.status[1]) return;
    const int4 it = reinterpret_cast<const int4*>(p.items)[item];
    const int e = it.x, m0 = it.y;
    const int cnt = it.z;  // slots m0 .. cnt-1 (absolute) of expert e
    const int rows = cnt - m0;
    const int ntiles = (rows + 15) >> 4;
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int H = p.H, I = p.I, G = p.G, KT = H >> 7;

    // Four weight tiles: gate rows of hidden h0..h0+31 and the matching up rows
    // (paired order: gate row of h = (h/G)*2G + h%G, up row = gate row + G).
    const int h0 = blockIdx.x * kL1BlockH + wave * 32;
    const int rho = (h0 / G) * 2 * G + (h0 % G);
    const int ntg = rho >> 4, ntu = ntg + (G >> 4);
    const uint8_t* we = p.w + (size_t)e * (size_t)(2 * I) * H;
    WTiles<4> wt;
    wt.KT = KT;
    wt.set(0, we, ntg, lane);
    wt.set(1, we, ntg + 1, lane);
    wt.set(2, we, ntu, lane);
    wt.set(3, we, ntu + 1, lane);
    const uint8_t* wsf0 = nullptr;
    const uint8_t* wsf1 = nullptr;
    if (p.w_sf) {
        const uint8_t* se = p.w_sf + (size_t)e * (size_t)(2 * I / 128) * KT;
        wsf0 = se + (size_t)(ntg >> 3) * KT;
        wsf1 = se + (size_t)(ntu >> 3) * KT;
    }

    // Token rows (B operand): slot m0+16j+L%16 (absolute) of expert e.
    const uint8_t* xr[MT];
    const uint8_t* xsf[MT];
#pragma unroll
    for (int j = 0; j < MT; ++j) {
        const int r = m0 + 16 * j + (lane & 15);
        const int slot = r < cnt ? r : 0;
        const size_t tok = p.perm[slot] / (uint32_t)p.topk;
        xr[j] = p.x + tok * H + 32 * (lane >> 4);
        xsf[j] = p.x_sf ? p.x_sf + tok * KT : nullptr;
    }

    v4f acc[4][MT];
#pragma unroll
    for (int t = 0; t < 4; ++t)
#pragma unroll
        for (int j = 0; j < MT; ++j) acc[t][j] = v4f{0.f, 0.f, 0.f, 0.f};

    gemm_mainloop<MmaBf16, MT, stages_for<MT>()>(acc, wt, xr, KT, wsf0, wsf1, xsf, ntiles);

    // Epilogue: h = silu(g) * u for channels h0 + 16*pp + 4*(L/16) + i.
    float hv[MT][2][4];
#pragma unroll
    for (int j = 0; j < MT; ++j)
#pragma unroll
        for (int pp = 0; pp < 2; ++pp)
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                const float g = acc[pp][j][i], u = acc[2 + pp][j][i];
                hv[j][pp][i] = silu_mul(g, u);
            }

    const int I128 = I >> 7;
    if (p.ffn_ue8m0) {
        // Per token, per 128 hidden columns (this workgroup's block): amax over
        // the 4 waves x 32 columns -> UE8M0 scale -> quantise.
        __shared__ float red[4][MT][16];
#pragma unroll
        for (int j = 0; j < MT; ++j) {
            float m = 0.0f;
#pragma unroll
            for (int pp = 0; pp < 2; ++pp)
#pragma unroll
                for (int i = 0; i < 4; ++i) m = fmaxf(m, fabsf(hv[j][pp][i]));
            m = fmaxf(m, __shfl_xor(m, 16, 64));
            m = fmaxf(m, __shfl_xor(m, 32, 64));
            if (lane < 16) red[wave][j][lane] = m;
        }
        __syncthreads();
#pragma unroll
        for (int j = 0; j < MT; ++j) {
            const int r = m0 + 16 * j + (lane & 15);
            const float amax = fmaxf(fmaxf(red[0][j][lane & 15], red[1][j][lane & 15]),
                                     fmaxf(red[2][j][lane & 15], red[3][j][lane & 15]));
            const uint32_t sb = block_scale_byte(amax);
            const float inv = inv_scale(sb);
            if (j < ntiles && r < cnt) {
                const size_t slot = (size_t)r;
#pragma unroll
                for (int pp = 0; pp < 2; ++pp) {
                    const uint32_t q = pack4_fp8(hv[j][pp][0] * inv, hv[j][pp][1] * inv,
                                                 hv[j][pp][2] * inv, hv[j][pp][3] * inv);
                    *reinterpret_cast<uint32_t*>(p.out8 + slot * I + h0 + 16 * pp +
                                                 4 * (lane >> 4)) = q;
                }
                if (wave == 0 && lane < 16) p.out_sf[slot * I128 + blockIdx.x] = (uint8_t)sb;
            }
        }
    } else {
#pragma unroll
        for (int j = 0; j < MT; ++j) {
            const int r = m0 + 16 * j + (lane & 15);
            if (j < ntiles && r < cnt) {
                const size_t slot = (size_t)r;
#pragma unroll
                for (int pp = 0; pp < 2; ++pp) {
                    const uint32_t q =
                        pack4_fp8(hv[j][pp][0], hv[j][pp][1], hv[j][pp][2], hv[j][pp][3]);
                    *reinterpret_cast<uint32_t*>(p.out8 + slot * I + h0 + 16 * pp +
                                                 4 * (lane >> 4)) = q;
                }
            }
        }
    }
}

template <int MT>
__global__ void __launch_bounds__(kGemmThreads) l2_kernel(GemmParams p) {
    const int item = blockIdx.y;
    if (item >= p.status[1]) return;
    const int4 it = reinterpret_cast<const int4*>(p.items)[item];
    const int e = it.x, m0 = it.y;
    const int cnt = it.z;  // slots m0 .. cnt-1 (absolute) of expert e
    const int rows = cnt - m0;
    const int ntiles = (rows + 15) >> 4;
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int H = p.H, I = p.I, KT = I >> 7;

    const int n0 = blockIdx.x * kL2BlockN + wave * 64;
    const int nt0 = n0 >> 4;
    const uint8_t* we = p.w + (size_t)e * (size_t)H * I;
    WTiles<4> wt;
    wt.KT = KT;
#pragma unroll
    for (int t = 0; t < 4; ++t) wt.set(t, we, nt0 + t, lane);
    const uint8_t* wsf = p.w_sf ? p.w_sf + ((size_t)e * (H / 128) + (n0 >> 7)) * KT : nullptr;

    const uint8_t* xr[MT];
    const uint8_t* xsf[MT];
#pragma unroll
    for (int j = 0; j < MT; ++j) {
        const int r = m0 + 16 * j + (lane & 15);
        const size_t slot = (size_t)(r < cnt ? r : 0);
        xr[j] = p.x + slot * I + 32 * (lane >> 4);
        xsf[j] = p.x_sf ? p.x_sf + slot * KT : nullptr;
    }

    v4f acc[4][MT];
#pragma unroll
    for (int t = 0; t < 4; ++t)
#pragma unroll
        for (int j = 0; j < MT; ++j) acc[t][j] = v4f{0.f, 0.f, 0.f, 0.f};

    gemm_mainloop<MmaBf16, MT, stages_for<MT>()>(acc, wt, xr, KT, wsf, wsf, xsf, ntiles);

#pragma unroll
    for (int j = 0; j < MT; ++j) {
        const int r = m0 + 16 * j + (lane & 15);
        if (j < ntiles && r < cnt) {
            const size_t slot = (size_t)r;
#pragma unroll
            for (int t = 0; t < 4; ++t) {
                uint2 v;
                v.x = pack2_bf16(acc[t][j][0], acc[t][j][1]);
                v.y = pack2_bf16(acc[t][j][2], acc[t][j][3]);
                *reinterpret_cast<uint2*>(p.out16 + slot * H + n0 + 16 * t + 4 * (lane >> 4)) = v;
            }
        }
    }
}

template __global__ void l1_kernel<1>(GemmParams);
template __global__ void l1_kernel<2>(GemmParams);
template __global__ void l2_kernel<1>(GemmParams);
template __global__ void l2_kernel<2>(GemmParams);

}  // namespace mm
