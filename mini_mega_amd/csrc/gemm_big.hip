// gemm_big.hip -- the L1 / L2 grouped GEMMs for large per-expert row counts
// (work items of 33..256 token rows: T >= ~1024 and skewed routing), where
// the decode-shaped kernels of gemm.hip would re-stream each expert's weights
// once per 32 rows.
//
// Reference counterparts: r24_l1_big / r24_l2_big (src/compute_big.cuh:888-1161,
// 1375-1679), the reference's count-tiered big-window GEMMs.
//
// One 8-wave workgroup (two waves per SIMD) per work unit = (work item,
// block of 256 weight rows = 16 tiles); each wave owns a 32-row weight slice
// (two 16-row tiles).  The code is written for W waves of 16/W tiles each;
// W = 4 (one wave per SIMD, four tiles, accumulators in AGPRs: half the LDS
// operand traffic per MFMA) was measured slower at every T on MI355X (T =
// 8192 with items of <= 192 rows: L1 3423 vs 3254 us), so only W = 8 is
// instantiated.  Each wave covers all of the item's token rows (up to 256, so that at
// T = 8192 one item covers an expert and its weights stream from HBM once):
//   * per 128-k step, the workgroup gathers the item's active token rows
//     (through perm[] for L1, slot order for L2), converts them once to bf16
//     with the row's UE8M0 scale folded in (exact), and stores them in a
//     double-buffered LDS tile: [token tile][k-group q][lane][8 bf16], so that
//     a wave's operand read for one MFMA group is 1 KiB contiguous;
//   * each wave streams its weight tiles (L1: gate and up rows of its hidden
//     columns; L2: its output channels) from HBM through a 2- to 6-stage
//     register pipeline and converts them exactly to bf16;
//   * v_mfma_f32_16x16x32_bf16 (fp32-accurate sums; see gemm.hip) over the
//     item's NT active token tiles -- NT is a compile-time specialisation
//     picked per item (1..16), so the k loop has no branch
//     and the accumulator chains are independent;
//   * epilogues as in gemm.hip: L1 SwiGLU + fp8 (raw, or per-128 UE8M0 with
//     the 128-column amax reduced over the waves in LDS), L2 bf16.
// Work units are numbered so that each XCD runs a contiguous range of them:
// the N-blocks of one item share that XCD's L2 for the item's activations;
// in L1 the last units of each range go out through a per-XCD ticket queue
// that a few extra workgroups of the other XCDs also drain.  The two GEMMs
// run as two stream-ordered launches, or (gemm_fused_kernel, opt-in) as one
// launch whose L2 units wait on per-item ready counters (reference:
// src/compute_big.cuh:1948-1997).
#include <type_traits>

#include "mm_kernels.h"

// The kernels are written for gfx950 alone (MFMA shapes, buffer-resource
// words, cache-policy bits and the fused handoff's store semantics).
#if defined(__HIP_DEVICE_COMPILE__) && !defined(__gfx950__)
#error "gemm_big.hip is built for gfx950 only"
#endif

namespace mm {

constexpr int kXTileBytes = 16 * kTileK * 2;   // one bf16 token tile: 16 rows x 128 k
constexpr int kBlockTiles = 16;                 // weight tiles = 256 rows per workgroup
constexpr int kBigRows = kBigMaxTiles * 16;     // token rows per work item (max)
static_assert(kBlockTiles * 16 == kL2BlockN && kBlockTiles * 8 == kL1BlockH, "block shape");

// Workgroup shape: W waves, kWT = 16 / W weight tiles per wave.
template <int W>
struct Geo {
    static constexpr int kWaves = W;
    static constexpr int kThreads = 64 * W;
    static constexpr int kWT = kBlockTiles / W;
};

// Row pitch of the staged row scales: 16-byte aligned rows for the staging
// copies, and 20 dwords, so that the 16 rows one k-step reads per wave fall
// in 16 different LDS banks (a 64-byte pitch put them in 4).
constexpr int kSfxPitch = kBigMaxKT + 16;

struct alignas(16) BigSmem {
    uint8_t x[2][kBigMaxTiles * kXTileBytes];   // bf16 tiles, double buffered
    uint8_t sfx[kBigRows][kSfxPitch];           // the item's row scales [row][k-step]
    uint32_t tok[kBigRows];                      // L1: the token of each item row
    uint8_t sfw[kBigMaxKT][kBlockTiles];        // the block's weight-tile scales [k-step][tile]
};

// Loader for NT active token tiles: chunk i = (tid + T*u) mod (NT*128), T
// the workgroup's threads, is row r = 16*(i/128) + i%16 of the item, fp8
// bytes [16*cc, 16*cc+16) of the k-step with cc = (i/16)%8: k-group g = cc/2,
// MFMA groups q = 2*(cc%2) and q+1.  Rows vary fastest, so the 16 lanes of an
// LDS write phase fill 16 consecutive 16-byte slots (no bank conflicts).
// When NT*128 is not a multiple of T some threads redo another thread's
// chunk (same bytes to the same LDS slot), which keeps every thread's work
// uniform.  XS register stages: with two, the rows of k-step kt+2 are in
// flight while kt+1 is written to LDS; with one (above 12 token tiles, where
// registers go to accumulators, and a k-step's 4*NT MFMA groups alone cover
// an L2 hit; measured even with two at T = 8192), kt+1 is loaded during kt.
template <int W, int NT, int kAux = 0, bool kOpaqueTid = false, int kXS = (NT <= 12 ? 2 : 1)>
struct XLoader {
    static constexpr int kThreads = Geo<W>::kThreads;
    static constexpr int U = (NT * 128 + kThreads - 1) / kThreads;
    static constexpr int XS = kXS;
    const uint8_t* base;
    int tid_;   // kOpaqueTid: the thread index, read once per unit through an empty asm
    uint32_t off[U];
    v4i reg[XS][U];

    __device__ __forceinline__ int tid() const {
        if constexpr (kOpaqueTid) {
            __builtin_assume(tid_ >= 0 && tid_ < kThreads);
            return tid_;
        } else {
            return threadIdx.x;
        }
    }
    // the wave index, wave-uniform (in a scalar register)
    __device__ __forceinline__ int wave() const {
        return __builtin_amdgcn_readfirstlane(tid() >> 6);
    }
    __device__ __forceinline__ int chunk(int u) const { return (tid() + kThreads * u) % (NT * 128); }
    __device__ __forceinline__ static int row_of(int i) { return ((i >> 7) << 4) | (i & 15); }
    __device__ __forceinline__ static int cc_of(int i) { return (i >> 4) & 7; }
    __device__ __forceinline__ static int slot_of(int i) {
        const int r = row_of(i), cc = cc_of(i);
        return (r >> 4) * kXTileBytes + 2 * (cc & 1) * 1024 + ((r & 15) + 16 * (cc >> 1)) * 16;
    }

    __device__ __forceinline__ void issue(int kt, int rs) {
#pragma unroll
        for (int u = 0; u < U; ++u) reg[rs][u] = load16_rows<kAux>(base, off[u], kt * kTileK);
    }
    // Writes chunk u of register stage rs, scaled by 2^(e - 127), to LDS stage xw.
    __device__ __forceinline__ void commit_chunk(uint8_t* xw, int rs, int u, uint32_t e) {
        uint8_t* t = xw + slot_of(chunk(u));
        const float s = ue8m0_to_f32(e);
        *reinterpret_cast<v8bf*>(t) = fp8x8_to_bf16(reg[rs][u][0], reg[rs][u][1], s);
        *reinterpret_cast<v8bf*>(t + 1024) = fp8x8_to_bf16(reg[rs][u][2], reg[rs][u][3], s);
    }
    __device__ __forceinline__ void commit(BigSmem& sm, int stage, int rs, int kt) {
#pragma unroll
        for (int u = 0; u < U; ++u)
            commit_chunk(&sm.x[stage][0], rs, u, sm.sfx[row_of(chunk(u))][kt]);
    }
    // fp8 MFMA path: the chunk's 16 raw bytes go to the fp8 token tile in the
    // weight-tile layout ([half][lane][16 B], 2 KiB a tile), unconverted (the
    // MFMA applies the row scale).
    __device__ __forceinline__ static int slot_of_f8(int i) {
        const int r = row_of(i), cc = cc_of(i);
        return (r >> 4) * kTileBytes + (cc & 1) * 1024 + ((r & 15) + 16 * (cc >> 1)) * 16;
    }
    __device__ __forceinline__ void commit_chunk_f8(uint8_t* xw, int rs, int u) {
        *reinterpret_cast<v4i*>(xw + slot_of_f8(chunk(u))) = reg[rs][u];
    }
};

template <int WT>
struct WStage {
    v4i a[WT][2];   // the wave's weight tiles, two 16-byte halves each
};

template <int WT>
__device__ __forceinline__ void w_load(WStage<WT>& w, const WTiles<WT>& wt, int kt) {
#pragma unroll
    for (int t = 0; t < WT; ++t) {
        const int o = (int)wt.lane16, so = kt * kTileBytes;
        w.a[t][0] = load16_row_stream(wt.row[t], wt.KT * kTileBytes, o, so);
        w.a[t][1] = load16_row_stream(wt.row[t], wt.KT * kTileBytes, o + 1024, so);
    }
}

// Weight tile t's operand of k-group q (8 bf16 per lane) with scale s folded in.
template <int WT>
__device__ __forceinline__ v8bf w_group(const WStage<WT>& w, int t, int q, float s) {
    return fp8x8_to_bf16(w.a[t][q >> 1][2 * (q & 1)], w.a[t][q >> 1][2 * (q & 1) + 1], s);
}

// The wave's weight-tile scale bytes of k-step kt (byte t = tile t).
template <int WT>
__device__ __forceinline__ uint32_t w_scales(const BigSmem& sm, int kt, int wave) {
    if constexpr (WT == 2)
        return *reinterpret_cast<const uint16_t*>(&sm.sfw[kt][WT * wave]);
    else
        return *reinterpret_cast<const uint32_t*>(&sm.sfw[kt][WT * wave]);
}

__device__ __forceinline__ float scale_of(uint32_t bytes, int t) {
    return ue8m0_to_f32((bytes >> (8 * t)) & 0xffu);
}

// Weight register stages (even where the activations have two register
// stages, so that these alternate within a group of S k-steps).  Up to 8
// token tiles (8 waves): 4 for L1, 6 for L2, whose shorter units (K = I)
// gain from the deeper prefetch (measured on MI355X at T = 512: L2 543 vs
// 565 us; L1 prefers 4: 950 vs 961 us).  Above 12 tiles: 2, since the
// registers go to accumulators and one k-step of >= 4*NT MFMA groups covers
// the latency of the next step's weights.
template <int W, int NT, bool L2>
constexpr int big_stages() {
    return (W == 8 ? NT > 12 : NT > 8) ? 2 : (W == 8 && NT <= 8 && L2 ? 6 : 4);
}

// Activation operand reads in flight ahead of their MFMAs: 3, or 2 for W = 8
// above NT = 12 (registers).
template <int W, int NT>
constexpr int big_read_ahead() { return (W == 8 && NT > 12) ? 2 : 3; }

// Bodies of at most this many token tiles issue their first weight stages
// before the unit's scale staging, whose load round trip then overlaps the
// weights' HBM latency.  Measured on MI355X against issuing them after it:
// T = 512 layer 1515-1517 vs 1521 us (L2 537 vs 541-545 us); with the bound
// at 8 tiles, T = 2048 L1 took 1153-1155 vs 1146-1147 us, so larger bodies
// keep the later issue (at NT = 16 the early stages also made the body spill).
constexpr int kEarlyMaxTiles = 2;

// The next unit's weight tiles, for a workgroup that runs several units in a
// row (l2_walk): the last S - 1 k-steps of a unit issue the next unit's first
// weight stages where they would otherwise reload the unit's last k-step, so
// the weight stream runs on across the unit boundary.  NoNext: one unit.
struct NoNext {
    static constexpr bool kOn = false;
};
template <int WT>
struct NextW {
    static constexpr bool kOn = true;
    WTiles<WT> wt;
    bool has;
};

// One k-step, software-pipelined by hand.  The step's 4*NT chunks (k-group
// q, token tile j) each hold: the LDS read of the activation operand D
// chunks ahead, a share of the conversions of the next k-group's weight
// operands (in the last group: the next k-step's first), a share of the
// activation commit of k-step kt+1 (last group only), and the chunk's kWT
// MFMAs.  A scheduling fence closes every chunk, so the compiler keeps this
// order: operand reads stay ahead of their use, and conversions overlap the
// MFMAs instead of stalling them.  Before the chunks: the prefetches of
// weights (kt+S-1) and activations (kt+XS), with indices clamped to the last
// step (a redundant in-bounds reload keeps the loop free of branches, so the
// compiler's wait counts stay partial).  After: the barrier that publishes
// the committed activations.  a0 carries the converted k-group-0 operand from
// one step to the next.
template <int W, int NT, int S, int s, class XL, class NX = NoNext>
__device__ __forceinline__ void big_step(v4f (&acc)[Geo<W>::kWT][NT], BigSmem& sm,
                                         XL& xl, WStage<Geo<W>::kWT> (&w)[S],
                                         const WTiles<Geo<W>::kWT>& wt, v8bf (&a0)[Geo<W>::kWT],
                                         int kt, int KT, const NX& nx = NX{}) {
    constexpr int kWT = Geo<W>::kWT;
    constexpr int XS = XL::XS, U = XL::U;
    constexpr int G = 4 * NT, D = big_read_ahead<W, NT>() < G ? big_read_ahead<W, NT>() : G;
    constexpr int rs = XS == 2 ? ((s + 1) & 1) : 0;   // register stage holding k-step kt+1
    const int lane = xl.tid() & 63, wave = xl.wave();
    // weights first: vector loads complete in issue order, so the wait for
    // the next step's weights (end of this step) must not also wait for this
    // step's gathered activation rows, which can miss to HBM (measured:
    // T = 8192 L1 3136 vs 3252 us)
    // when walking (L2 units only): the activation rows first, so that the
    // commit's wait does not also wait for the weights issued ahead of them
    // (measured on MI355X with the walk at T = 2048: L2 610-611 vs 615-618 us)
    if constexpr (NX::kOn) xl.issue(min(kt + XS, KT - 1), XS == 2 ? (s & 1) : 0);
    if constexpr (NX::kOn) {
        const int kw = kt + S - 1;
        const bool cur = kw < KT, nxt = !cur && nx.has;
        WTiles<kWT> ws = wt;
#pragma unroll
        for (int t = 0; t < kWT; ++t) ws.row[t] = nxt ? nx.wt.row[t] : wt.row[t];
        w_load<kWT>(w[(s + S - 1) % S], ws, cur ? kw : nxt ? kw - KT : KT - 1);
    } else {
        w_load<kWT>(w[(s + S - 1) % S], wt, min(kt + S - 1, KT - 1));
    }
    if constexpr (!NX::kOn) xl.issue(min(kt + XS, KT - 1), XS == 2 ? (s & 1) : 0);
    // scale bytes, read here and decoded where used (no wait before the MFMAs)
    const int kn = min(kt + 1, KT - 1);
    const uint32_t sc = w_scales<kWT>(sm, kt, wave), sn = w_scales<kWT>(sm, kn, wave);
    uint32_t xs[U];
#pragma unroll
    for (int u = 0; u < U; ++u)
        xs[u] = sm.sfx[XL::row_of(xl.chunk(u))][kn];
    // LDS bases of this step's read and write buffers.  Opaque to the
    // optimiser: otherwise it hoists every operand address of the unrolled
    // group out of the loop into a register of its own (the buffer parity of
    // each step is known there) instead of using one base plus immediate
    // offsets.
    uint32_t xro = (kt & 1) * (uint32_t)sizeof(sm.x[0]) + lane * 16;
    uint32_t xwo = ((kt + 1) & 1) * (uint32_t)sizeof(sm.x[0]);
    asm volatile("" : "+v"(xro), "+v"(xwo));
    const uint8_t* xb = &sm.x[0][0] + xro;
    uint8_t* xw = &sm.x[0][0] + xwo;
    v8bf b[D + 1];
#pragma unroll
    for (int d = 0; d < D; ++d)
        b[d] = *reinterpret_cast<const v8bf*>(xb + (d % NT) * kXTileBytes + (d / NT) * 1024);
    __builtin_amdgcn_sched_barrier(0);
    v8bf ac[kWT], an[kWT];
#pragma unroll
    for (int t = 0; t < kWT; ++t) ac[t] = a0[t];
#pragma unroll
    for (int g = 0; g < G; ++g) {
        const int q = g / NT, j = g % NT;
        if (g + D < G) {
            const int gn = g + D;
            b[gn % (D + 1)] = *reinterpret_cast<const v8bf*>(xb + (gn % NT) * kXTileBytes +
                                                             (gn / NT) * 1024);
        }
#pragma unroll
        for (int t = 0; t < kWT; ++t)
            if (j == (t * NT) / kWT)
                an[t] = q < 3 ? w_group<kWT>(w[s], t, q + 1, scale_of(sc, t))
                              : w_group<kWT>(w[(s + 1) % S], t, 0, scale_of(sn, t));
        if (q == 3) {
#pragma unroll
            for (int u = 0; u < U; ++u)
                if (j == (u * NT) / U) xl.commit_chunk(xw, rs, u, xs[u]);
        }
#pragma unroll
        for (int t = 0; t < kWT; ++t) acc[t][j] = mfma_bf16(ac[t], b[g % (D + 1)], acc[t][j]);
        if (j == NT - 1) {
#pragma unroll
            for (int t = 0; t < kWT; ++t) ac[t] = an[t];
        }
        __builtin_amdgcn_sched_barrier(0);
    }
#pragma unroll
    for (int t = 0; t < kWT; ++t) a0[t] = ac[t];
    __syncthreads();
}

template <int W, int NT, int S, int s, class XL, class NX>
__device__ __forceinline__ void big_group(v4f (&acc)[Geo<W>::kWT][NT], BigSmem& sm,
                                          XL& xl, WStage<Geo<W>::kWT> (&w)[S],
                                          const WTiles<Geo<W>::kWT>& wt, v8bf (&a0)[Geo<W>::kWT],
                                          int kb, int KT, const NX& nx) {
    big_step<W, NT, S, s>(acc, sm, xl, w, wt, a0, kb + s, KT, nx);
    if constexpr (s + 1 < S) big_group<W, NT, S, s + 1>(acc, sm, xl, w, wt, a0, kb, KT, nx);
}

// The KT % S remaining k-steps, one guarded step each.
template <int W, int NT, int S, int r, class XL, class NX>
__device__ __forceinline__ void big_tail(v4f (&acc)[Geo<W>::kWT][NT], BigSmem& sm,
                                         XL& xl, WStage<Geo<W>::kWT> (&w)[S],
                                         const WTiles<Geo<W>::kWT>& wt, v8bf (&a0)[Geo<W>::kWT],
                                         int KF, int KT, const NX& nx) {
    if (KF + r < KT) {
        big_step<W, NT, S, r>(acc, sm, xl, w, wt, a0, KF + r, KT, nx);
        if constexpr (r + 2 < S) big_tail<W, NT, S, r + 1>(acc, sm, xl, w, wt, a0, KF, KT, nx);
    }
}

// Main loop: every wave runs the same KT + 1 barriers.  Activations: LDS
// double buffer fed from XS register stages.  Weights: S register stages.
// Whole groups of S k-steps run without any branch; a remainder (only when
// KT is not a multiple of S) runs through the guarded tail.
// The first S - 1 weight stages of a unit.
template <int WT, int S>
__device__ __forceinline__ void w_prologue(WStage<WT> (&w)[S], const WTiles<WT>& wt, int KT) {
#pragma unroll
    for (int s = 0; s < S - 1; ++s) w_load<WT>(w[s], wt, min(s, KT - 1));
}

// kEarly: the caller issued the first weight stages (w_prologue) before the
// unit's scale staging, so that their HBM latency overlaps it.
// NX::kOn (several units per workgroup): the previous unit issued the first
// `pref` weight stages already; the prologue issues the rest.
template <int W, int NT, int S, bool kEarly, class XL, class NX = NoNext>
__device__ __forceinline__ void big_mainloop(v4f (&acc)[Geo<W>::kWT][NT], BigSmem& sm,
                                             XL& xl, const WTiles<Geo<W>::kWT>& wt,
                                             int KT, WStage<Geo<W>::kWT> (&w)[S],
                                             const NX& nx = NX{}, int pref = 0) {
    constexpr int kWT = Geo<W>::kWT;
    constexpr int XS = XL::XS;
    static_assert(XS == 1 || S % 2 == 0, "two activation stages alternate within a group");
    static_assert(S >= 2 && S <= 8, "stages");
#pragma unroll
    for (int t = 0; t < kWT; ++t)
#pragma unroll
        for (int j = 0; j < NT; ++j) acc[t][j] = v4f{0.f, 0.f, 0.f, 0.f};
    xl.issue(0, 0);
    if constexpr (XS == 2) xl.issue(min(1, KT - 1), 1);
    if constexpr (NX::kOn) {
#pragma unroll
        for (int j = 0; j < S - 1; ++j)
            if (j >= pref) w_load<kWT>(w[j], wt, min(j, KT - 1));
    } else if constexpr (!kEarly) {
        w_prologue<kWT, S>(w, wt, KT);
    }
    xl.commit(sm, 0, 0, 0);
    __syncthreads();
    v8bf a0[kWT];
    {
        const uint32_t sc = w_scales<kWT>(sm, 0, xl.wave());
#pragma unroll
        for (int t = 0; t < kWT; ++t) a0[t] = w_group<kWT>(w[0], t, 0, scale_of(sc, t));
    }
    const int KF = KT - KT % S;
#pragma unroll 1
    for (int kb = 0; kb < KF; kb += S) big_group<W, NT, S, 0>(acc, sm, xl, w, wt, a0, kb, KT, nx);
    big_tail<W, NT, S, 0>(acc, sm, xl, w, wt, a0, KF, KT, nx);
}

// ---------------------------------------------------------- fp8 MFMA path --
// Opt-in (MegaLaunchArgs::mfma_fp8): both GEMMs on gfx950's block-scaled fp8
// MFMA, v_mfma_scale_f32_16x16x128_f8f6f4, one instruction per (weight tile,
// token tile, 128-k step), the UE8M0 bytes as its scale operands (the
// weight tile's byte from every lane, each token row's byte from its lane).
// Weights go from the register stages to the MFMA as they are loaded; token
// rows are committed to LDS unconverted (fp8 tiles of 2 KiB).  Its sums
// truncate (~2^-20 of sum|terms|; see the probes in tests), so it is outside
// the end-to-end bar the default bf16 path meets; it is the reference's
// arithmetic class (its own fp8 MMA, src/compute.cuh:414-417,593-596).
typedef int v8i __attribute__((ext_vector_type(8)));

__device__ __forceinline__ v4f mfma_f8(const v8i& a, const v8i& b, uint32_t sa, uint32_t sb,
                                       const v4f& c) {
    return __builtin_amdgcn_mfma_scale_f32_16x16x128_f8f6f4(a, b, c, 0, 0, 0, (int)sa, 0,
                                                            (int)sb);
}

// Weight register stages of the fp8 path: 2 above 8 token tiles, 4 up to 8.
// Measured on MI355X at T = 8192 (layer, fp8 path): three stages with one
// activation stage above 8 tiles 3722-3726 us, four 3814 us, against 3360-
// 3364 us; T = 2048 even or slower.
template <int NT>
constexpr int big_stages_f8() { return NT > 8 ? 2 : 4; }

// The fp8 path's weight stage: each tile's two 16-byte halves loaded straight
// into one 8-register operand.
template <int WT>
struct WStage8 {
    v8i a[WT];
};

template <int WT>
__device__ __forceinline__ void w_load8(WStage8<WT>& w, const WTiles<WT>& wt, int kt) {
#pragma unroll
    for (int t = 0; t < WT; ++t) {
        const int o = (int)wt.lane16, so = kt * kTileBytes;
        const v4i lo = load16_row_stream(wt.row[t], wt.KT * kTileBytes, o, so);
        const v4i hi = load16_row_stream(wt.row[t], wt.KT * kTileBytes, o + 1024, so);
        w.a[t] = __builtin_shufflevector(lo, hi, 0, 1, 2, 3, 4, 5, 6, 7);
    }
}

// One k-step: NT chunks, chunk j = token tile j: the LDS read of the operand
// D tiles ahead (two 16-byte halves and its row scale), a share of the
// commit of k-step kt+1 (spread over all chunks: the rows were loaded a step
// earlier; measured even with the second half or last quarter, and the only
// placement without spills in L1), and kWT MFMAs.
template <int W, int NT, int S, int s, class XL>
__device__ __forceinline__ void big_step_f8(v4f (&acc)[Geo<W>::kWT][NT], BigSmem& sm, XL& xl,
                                            WStage8<Geo<W>::kWT> (&w)[S],
                                            const WTiles<Geo<W>::kWT>& wt, int kt, int KT) {
    constexpr int kWT = Geo<W>::kWT;
    constexpr int XS = XL::XS, U = XL::U;
    constexpr int D = NT < 2 ? NT : 2;
    constexpr int rs = XS == 2 ? ((s + 1) & 1) : 0;
    const int lane = xl.tid() & 63, wave = xl.wave();
    w_load8<kWT>(w[(s + S - 1) % S], wt, min(kt + S - 1, KT - 1));   // s: step in the group
    xl.issue(min(kt + XS, KT - 1), XS == 2 ? (s & 1) : 0);
    const uint32_t sc = w_scales<kWT>(sm, kt, wave);
    uint32_t xro = (kt & 1) * (uint32_t)sizeof(sm.x[0]) + lane * 16;
    uint32_t xwo = ((kt + 1) & 1) * (uint32_t)sizeof(sm.x[0]);
    uint32_t sfo = (lane & 15) * kSfxPitch + kt;
    asm volatile("" : "+v"(xro), "+v"(xwo), "+v"(sfo));
    const uint8_t* xb = &sm.x[0][0] + xro;
    uint8_t* xw = &sm.x[0][0] + xwo;
    const uint8_t* sf = &sm.sfx[0][0] + sfo;
    v8i b[D + 1];
    uint32_t bs[D + 1];
    auto rd = [&](int d, int j) {
        const v4i lo = *reinterpret_cast<const v4i*>(xb + j * kTileBytes);
        const v4i hi = *reinterpret_cast<const v4i*>(xb + j * kTileBytes + 1024);
        b[d] = __builtin_shufflevector(lo, hi, 0, 1, 2, 3, 4, 5, 6, 7);
        bs[d] = sf[j * 16 * kSfxPitch];
    };
#pragma unroll
    for (int d = 0; d < D; ++d) rd(d, d);
    __builtin_amdgcn_sched_barrier(0);
#pragma unroll
    for (int j = 0; j < NT; ++j) {
        if (j + D < NT) rd((j + D) % (D + 1), j + D);
#pragma unroll
        for (int u = 0; u < U; ++u)
            if (j == (u * NT) / U) xl.commit_chunk_f8(xw, rs, u);
#pragma unroll
        for (int t = 0; t < kWT; ++t)
            acc[t][j] = mfma_f8(w[s % S].a[t], b[j % (D + 1)], (sc >> (8 * t)) & 0xffu,
                                bs[j % (D + 1)], acc[t][j]);
        __builtin_amdgcn_sched_barrier(0);
    }
    __syncthreads();
}

// A group of GS k-steps (a multiple of S, and even with two activation
// register stages), so that both stage indices are static within it.
template <int W, int NT, int S, int GS, int s, class XL>
__device__ __forceinline__ void big_group_f8(v4f (&acc)[Geo<W>::kWT][NT], BigSmem& sm, XL& xl,
                                             WStage8<Geo<W>::kWT> (&w)[S],
                                             const WTiles<Geo<W>::kWT>& wt, int kb, int KT) {
    big_step_f8<W, NT, S, s>(acc, sm, xl, w, wt, kb + s, KT);
    if constexpr (s + 1 < GS) big_group_f8<W, NT, S, GS, s + 1>(acc, sm, xl, w, wt, kb, KT);
}

template <int W, int NT, int S, int GS, int r, class XL>
__device__ __forceinline__ void big_tail_f8(v4f (&acc)[Geo<W>::kWT][NT], BigSmem& sm, XL& xl,
                                            WStage8<Geo<W>::kWT> (&w)[S],
                                            const WTiles<Geo<W>::kWT>& wt, int KF, int KT) {
    if (KF + r < KT) {
        big_step_f8<W, NT, S, r>(acc, sm, xl, w, wt, KF + r, KT);
        if constexpr (r + 2 < GS) big_tail_f8<W, NT, S, GS, r + 1>(acc, sm, xl, w, wt, KF, KT);
    }
}

// The fp8 path's main loop (big_mainloop's structure, no operand conversion).
template <int W, int NT, int S, bool kEarly, class XL>
__device__ __forceinline__ void big_mainloop_f8(v4f (&acc)[Geo<W>::kWT][NT], BigSmem& sm,
                                                XL& xl, const WTiles<Geo<W>::kWT>& wt, int KT,
                                                WStage8<Geo<W>::kWT> (&w)[S]) {
    constexpr int kWT = Geo<W>::kWT;
    constexpr int XS = XL::XS, U = XL::U;
    constexpr int GS = (XS == 2 && S % 2) ? 2 * S : S;
#pragma unroll
    for (int t = 0; t < kWT; ++t)
#pragma unroll
        for (int j = 0; j < NT; ++j) acc[t][j] = v4f{0.f, 0.f, 0.f, 0.f};
    xl.issue(0, 0);
    if constexpr (XS == 2) xl.issue(min(1, KT - 1), 1);
    if constexpr (!kEarly) {
#pragma unroll
        for (int st = 0; st < S - 1; ++st) w_load8<kWT>(w[st], wt, min(st, KT - 1));
    }
#pragma unroll
    for (int u = 0; u < U; ++u) xl.commit_chunk_f8(&sm.x[0][0], 0, u);
    __syncthreads();
    const int KF = KT - KT % GS;
#pragma unroll 1
    for (int kb = 0; kb < KF; kb += GS) big_group_f8<W, NT, S, GS, 0>(acc, sm, xl, w, wt, kb, KT);
    big_tail_f8<W, NT, S, GS, 0>(acc, sm, xl, w, wt, KF, KT);
}

// Per-unit context shared by the two kernels.
struct BigItem {
    int e, m0, rows, bx, item;   // m0: first slot (absolute)
};

// Work units: an expert with n items has n * nb units, numbered from
// nb * (its first item) on, block-major: unit nb*i0 + bx*n + j is block bx of
// item i0 + j.  The n items of an expert read the same weight blocks, and
// this order runs the n readers of each block on neighbouring CUs of one XCD
// at the same time, so all but one take the block from that XCD's L2.  (The
// expert of unit u is the one of item u / nb: its items are consecutive.)
// The routing scan cuts the unit list into one contiguous range per XCD at
// equal modelled cost, and the XCDs take workgroups round-robin: workgroup L
// is the k-th of XCD x = L%8, k = L/8 (measured on MI355X with the XCC_ID
// register: every workgroup ran on XCD L%8).
// Static bulk, dynamic tail.  While k < (range of x) - kQueueTail, workgroup
// L runs unit cuts[x] + k, with no atomic on its way to its first load.  The
// last kQueueTail units of each range go out by ticket from that XCD's
// counter, to its workgroups k < range; the next kStealers workgroups of the
// XCD take tickets from the other XCDs' tails, so that an XCD that runs
// ahead of its modelled cost finishes the others' last units instead of
// idling.  Every later workgroup exits at once: the grid (nb * max_items +
// 8) is sized for the largest item count, and a surplus workgroup that paid
// atomics while holding a CU's LDS delayed the real tail (L2 650 -> 900 us
// at T = 2048).  The last ticket taker of a launch zeroes the counters for
// the next one.  Measured on MI355X (time-stamped workgroups): without the
// queue the XCDs' last L1 units ended up to 55 us apart at T = 512, 175 us
// at T = 8192 and 120 us with Zipf(1.1) skew; with it 22, 55 and 91 us.  A
// stolen unit runs without the victim XCD's L2 contents, so the kernel span
// shrinks less than the spread: L1 with Zipf(1.1) T = 2048 1260 -> 1216 us,
// T = 8192 -9 us, T = 512 and 2048 even.  L2's units are a third as long:
// there the queue cost 6-10 us at T = 512 and 2048 (items of 1-4 token
// tiles), and saved 2-4% of L2 at T = 8192 (1571-1586 vs 1603-1612 us) and
// with Zipf(1.1) skew at T = 2048 (651-663 vs 678-679 us), so L2 takes
// tickets only when its largest item has more than 32 rows (at T = 2048 the
// walk runs those launches).  L1's tickets go out costliest unit first (by
// the token tiles of the unit's item; the order is the routing scan's
// tail_ord), so that no heavy unit starts after the light ones of its tail:
// Zipf(1.1) T = 2048 L1 1193-1195 vs 1223-1231 us, T = 512 / 2048 / 8192
// even (measured on MI355X).  L2's tickets gained nothing from the order
// and go out in unit order.
__device__ __forceinline__ int claim_tail_unit(const GemmParams& p, int x, bool own, int grid) {
    int u = -1;
    for (int d = own ? 0 : 1; d < 8 && u < 0; ++d) {
        const int xx = (x + d) & 7;
        const int lo = p.xcd_cuts[xx], hi = p.xcd_cuts[xx + 1];
        const int tail = min(hi - lo, kQueueTail);
        if (tail <= 0) continue;
        const int t = atomicAdd(&p.queue[xx], 1);
        if (t < tail) u = hi - tail + (p.tail_ord ? p.tail_ord[kQueueTail * xx + t] : t);
    }
    // ticket takers of this launch: per XCD, its workgroups from the tail
    // through its stealers (as many as the grid holds)
    int takers = 0;
    for (int xx = 0; xx < 8; ++xx) {
        const int range = p.xcd_cuts[xx + 1] - p.xcd_cuts[xx];
        const int wgs = (grid - xx + 7) >> 3;
        takers += min(wgs, range + kStealers) - (range - min(range, kQueueTail));
    }
    if (atomicAdd(&p.queue[8], 1) == takers - 1) {
#pragma unroll
        for (int i = 0; i < kQueueInts; ++i) p.queue[i] = 0;
    }
    return u;
}

// Workgroup L of a grid of `grid` (the big GEMM's own share of the launch).
template <bool kTailQueue>
__device__ __forceinline__ bool big_unit(const GemmParams& p, int nb, BigItem& it, int* s_unit,
                                         int L, int grid) {
    const int x = L & 7, k = L >> 3;
    const int lo = p.xcd_cuts[x], hi = p.xcd_cuts[x + 1], range = hi - lo;
    int u = lo + k;
    if (!kTailQueue) {
        if (k >= range) return false;
    } else if (k >= range + kStealers) {
        return false;
    }
    if (kTailQueue && k >= range - min(range, kQueueTail)) {
        if (threadIdx.x == 0) *s_unit = claim_tail_unit(p, x, k < range, grid);
        __syncthreads();
        u = *s_unit;
        if (u < 0) return false;
    }
    // One dependent load for an expert of one item (every expert up to
    // 256 rows), a second one otherwise; the items hold absolute slots.
    const int4* items = reinterpret_cast<const int4*>(p.items);
    const int im = u / nb;                 // item-major item: same expert
    int4 v = items[im];
    const int i0 = im - (v.w & 0xffff), n = v.w >> 16;
    const int local = u - nb * i0;
    it.bx = local / n;
    it.item = i0 + local % n;
    if (n != 1) v = items[it.item];
    it.e = v.x;
    it.m0 = v.y;
    it.rows = v.z - v.y;
    return true;
}

// Stages the item's row scales ([k-step][row], 2^0 without x_sf) and the
// block's 16 weight-tile scales ([k-step][tile], 2^0 without w_sf) in LDS.
// row_scale(r) points at row r's KT scale bytes (null: 2^0), called once
// for every row r < nrows; tile_scale(t) points at tile t's.  A row's bytes
// go to LDS as 16-byte copies where KT and the source allow (one load and one
// LDS write per 16 k-steps instead of one per byte); L1 also keeps each row's
// token here, so its activation loader reads LDS instead of perm[] a second
// time.  Measured on MI355X against byte-wise staging into [k-step][row]:
// L1 T = 512 944-945 vs 948 us, T = 2048 1133-1135 vs 1144-1151, T = 8192
// 2910-2928 vs 2936-2961; layer -0.3 to -0.8%.
// kCoherent: the row scales were written by another XCD during this launch
// (the fused L1 -> L2 handoff) and are read at device scope.
template <int W, bool kCoherent = false, class RowF, class TileF>
__device__ __forceinline__ void big_load_scales(BigSmem& sm, int KT, int nrows, bool has_w,
                                                RowF row_scale, TileF tile_scale,
                                                int tid = threadIdx.x) {
    constexpr int T = Geo<W>::kThreads;
    for (int r = tid; r < nrows; r += T) {
        const uint8_t* src = row_scale(r);
        uint8_t* dst = &sm.sfx[r][0];
        if (src && (KT & 15) == 0 && (reinterpret_cast<uintptr_t>(src) & 15) == 0) {
            for (int k = 0; k < KT; k += 16)
                *reinterpret_cast<v4i*>(dst + k) =
                    kCoherent ? load16_rows<kBufferSc1>(src, 0, k) : load16(src + k);
        } else if (src) {
            for (int k = 0; k < KT; ++k)
                dst[k] = kCoherent ? __hip_atomic_load(src + k, __ATOMIC_RELAXED,
                                                       __HIP_MEMORY_SCOPE_AGENT)
                                   : src[k];
        } else {
            for (int k = 0; k < KT; k += 4) *reinterpret_cast<uint32_t*>(dst + k) = 0x7f7f7f7fu;
        }
    }
    for (int i = tid; i < kBlockTiles * KT; i += T) {
        const int t = i % kBlockTiles, k = i / kBlockTiles;
        sm.sfw[k][t] = has_w ? tile_scale(t)[k] : (uint8_t)127;
    }
    __syncthreads();
}

// NT as run for an item of `tiles` (<= kBigMaxTiles) token tiles: exact, so
// that the MFMAs cover no more than the item's partial last tile (at T =
// 8192 rounding to even counts above 8 tiles ran 6% more MFMA work: padding
// 11.7% vs 5.2% of the routed rows; layer 5122 -> 4782 us on MI355X).
#define MM_BIG_DISPATCH(BODY)    \
    switch (tiles) {             \
        case 1: BODY(1); break;  \
        case 2: BODY(2); break;  \
        case 3: BODY(3); break;  \
        case 4: BODY(4); break;  \
        case 5: BODY(5); break;  \
        case 6: BODY(6); break;  \
        case 7: BODY(7); break;  \
        case 8: BODY(8); break;  \
        case 9: BODY(9); break;  \
        case 10: BODY(10); break; \
        case 11: BODY(11); break; \
        case 12: BODY(12); break; \
        case 13: BODY(13); break; \
        case 14: BODY(14); break; \
        case 15: BODY(15); break; \
        default: BODY(16); break; \
    }

// Sets the loader's row offsets: row r of the item (r >= rows: row 0,
// whose bytes are loaded but whose results are never stored).
template <class XL, class RowOff>
__device__ __forceinline__ void big_loader_init(XL& xl, RowOff row_off) {
#pragma unroll
    for (int u = 0; u < XL::U; ++u) {
        const int i = xl.chunk(u);
        xl.off[u] = row_off(XL::row_of(i)) + XL::cc_of(i) * 16;
    }
}

// ---------------------------------------------------------------------- L1 --
// Block tile bt = kWT*wave + t of an L1 block: the wave's hidden columns are
// hw0 = bx*128 + wave*(128/W) .. +128/W; tiles t < kWT/2 are the gate rows of
// columns hw0 + 16t .. +16, tiles t >= kWT/2 the up rows of the same columns
// (t - kWT/2).  Returns the W1 row of the tile's first row (paired order:
// gate and up alternate in blocks of G rows).
template <int W>
__device__ __forceinline__ int l1_tile_row(int bx, int bt, int G) {
    constexpr int kWT = Geo<W>::kWT;
    const int wave = bt / kWT, t = bt % kWT;
    const int c = t % (kWT / 2), up = t >= kWT / 2;
    const int hw = bx * kL1BlockH + wave * (kL1BlockH / W) + 16 * c;
    return (hw / G) * 2 * G + (hw % G) + (up ? G : 0);
}

// kFused: the L2 units of the same launch read this item's ffn rows (the
// fused L1 -> L2 handoff).  The rows and scales are then written with
// agent-scope relaxed atomic stores (on gfx950 write-through stores, so the
// release below has few dirty L2 lines to write back), every wave waits for
// its stores, and after the workgroup barrier one thread bumps the item's
// ready counter with an agent-scope release; the L2 side acquires it.
template <int W, int NT, bool kFused, bool kF8, class ScalesF>
__device__ __forceinline__ void l1_big_body(const GemmParams& p, const BigItem& it, BigSmem& sm,
                                            ScalesF stage_scales) {
    constexpr int kWT = Geo<W>::kWT, kH = kWT / 2;
    auto put4 = [](uint8_t* dst, uint32_t v) {
        if constexpr (kFused)
            __hip_atomic_store(reinterpret_cast<uint32_t*>(dst), v, __ATOMIC_RELAXED,
                               __HIP_MEMORY_SCOPE_AGENT);
        else
            *reinterpret_cast<uint32_t*>(dst) = v;
    };
    constexpr int S = kF8 ? big_stages_f8<NT>() : big_stages<W, NT, false>();
    constexpr bool kEarly = NT <= kEarlyMaxTiles;
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int H = p.H, I = p.I, G = p.G, KT = H >> 7;
    const uint8_t* we = p.w + (size_t)it.e * (size_t)(2 * I) * H;
    WTiles<kWT> wt;
    wt.KT = KT;
#pragma unroll
    for (int t = 0; t < kWT; ++t) wt.set(t, we, l1_tile_row<W>(it.bx, kWT * wave + t, G) >> 4, lane);
    std::conditional_t<kF8, WStage8<kWT>, WStage<kWT>> w[S];
    if constexpr (kEarly) {
        if constexpr (kF8) {
#pragma unroll
            for (int st = 0; st < S - 1; ++st) w_load8<kWT>(w[st], wt, min(st, KT - 1));
        } else {
            w_prologue<kWT, S>(w, wt, KT);
        }
    }
    stage_scales();
    // the fp8 path keeps two activation register stages at every tile count
    // (measured on MI355X at T = 8192: layer 3267-3269 vs 3399-3417 us with
    // one stage above 10 tiles)
    XLoader<W, NT, 0, false, (kF8 || NT <= 12 ? 2 : 1)> xl;
    xl.base = p.x;
    big_loader_init(xl, [&](int r) { return sm.tok[r] * (uint32_t)H; });
    v4f acc[kWT][NT];
    if constexpr (kF8)
        big_mainloop_f8<W, NT, S, kEarly>(acc, sm, xl, wt, KT, w);
    else
        big_mainloop<W, NT, S, kEarly>(acc, sm, xl, wt, KT, w);

    // h = silu(g) * u: hidden column hw + 16c + 4*(L/16) + i, token 16*j + L%16
    const int hw = it.bx * kL1BlockH + wave * (kL1BlockH / W);
    float hv[kH][NT][4];
#pragma unroll
    for (int c = 0; c < kH; ++c)
#pragma unroll
        for (int j = 0; j < NT; ++j)
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                const float g = acc[c][j][i], u = acc[c + kH][j][i];
                hv[c][j][i] = silu_mul(g, u);
            }
    const int I128 = I >> 7;
    if (p.ffn_ue8m0) {
        // amax over the block's 128 hidden columns = the W waves; the LDS
        // tiles are free after the main loop's last barrier.
        float* red = reinterpret_cast<float*>(&sm.x[0][0]);   // [W][kBigRows]
#pragma unroll
        for (int j = 0; j < NT; ++j) {
            float m = 0.0f;
#pragma unroll
            for (int c = 0; c < kH; ++c)
                m = fmaxf(m, fmaxf(fmaxf(fabsf(hv[c][j][0]), fabsf(hv[c][j][1])),
                                   fmaxf(fabsf(hv[c][j][2]), fabsf(hv[c][j][3]))));
            m = fmaxf(m, __shfl_xor(m, 16, 64));
            m = fmaxf(m, __shfl_xor(m, 32, 64));
            if (lane < 16) red[wave * kBigRows + 16 * j + lane] = m;
        }
        __syncthreads();
#pragma unroll
        for (int j = 0; j < NT; ++j) {
            const int r = 16 * j + (lane & 15);
            float amax = red[r];
#pragma unroll
            for (int w = 1; w < W; ++w) amax = fmaxf(amax, red[w * kBigRows + r]);
            const uint32_t sb = block_scale_byte(amax);
            const float inv = inv_scale(sb);
            if (r < it.rows) {
                const size_t slot = (size_t)(it.m0 + r);
#pragma unroll
                for (int c = 0; c < kH; ++c)
                    put4(p.out8 + slot * I + hw + 16 * c + 4 * (lane >> 4),
                         pack4_fp8(hv[c][j][0] * inv, hv[c][j][1] * inv, hv[c][j][2] * inv,
                                   hv[c][j][3] * inv));
                if (wave == 0 && lane < 16) {
                    if constexpr (kFused)
                        __hip_atomic_store(p.out_sf + slot * I128 + it.bx, (uint8_t)sb,
                                           __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
                    else
                        p.out_sf[slot * I128 + it.bx] = (uint8_t)sb;
                }
            }
        }
    } else {
#pragma unroll
        for (int j = 0; j < NT; ++j) {
            const int r = 16 * j + (lane & 15);
            if (r < it.rows) {
                const size_t slot = (size_t)(it.m0 + r);
#pragma unroll
                for (int c = 0; c < kH; ++c)
                    put4(p.out8 + slot * I + hw + 16 * c + 4 * (lane >> 4),
                         pack4_fp8(hv[c][j][0], hv[c][j][1], hv[c][j][2], hv[c][j][3]));
            }
        }
    }
    if constexpr (kFused) {
        __builtin_amdgcn_s_waitcnt(0);   // this wave's stores are complete at device scope
        __syncthreads();
        if (threadIdx.x == 0)
            __hip_atomic_fetch_add(p.ready + it.item, 1, __ATOMIC_RELEASE,
                                   __HIP_MEMORY_SCOPE_AGENT);
    }
}

// NT (the item's token tiles) is uniform over the block, so every wave runs
// the same body and the same barriers.
// Workgroup L of the `grid` L1 workgroups.
template <int W, bool kFused, bool kF8 = false>
__device__ __forceinline__ void l1_big(const GemmParams& p, BigSmem& sm, int* s_unit, int L,
                                       int grid) {
    BigItem it;
    if (!big_unit<true>(p, p.I / kL1BlockH, it, s_unit, L, grid)) return;
    const int KT = p.H >> 7, I = p.I, G = p.G;
    const int tiles = (it.rows + 15) >> 4;
    // scales: x rows through perm[] (each row's token kept in LDS for the
    // activation loader); W1 tiles as l1_tile_row places them
    auto stage_scales = [&]() {
        big_load_scales<W>(
            sm, KT, min(tiles * 16, kBigRows), p.w_sf != nullptr,
            [&](int r) -> const uint8_t* {
                const int slot = it.m0 + (r < it.rows ? r : 0);
                const uint32_t tok = p.perm[slot] / (uint32_t)p.topk;
                sm.tok[r] = tok;
                return p.x_sf ? p.x_sf + (size_t)tok * KT : nullptr;
            },
            [&](int t) {
                const int rho = l1_tile_row<W>(it.bx, t, G);
                return p.w_sf + ((size_t)it.e * (2 * I / 128) + (rho >> 7)) * KT;
            });
    };
#define MM_L1_BODY(n) l1_big_body<W, n, kFused, kF8>(p, it, sm, stage_scales)
    MM_BIG_DISPATCH(MM_L1_BODY)
#undef MM_L1_BODY
}

__global__ void __launch_bounds__(512) l1_big_kernel(GemmParams p) {
    __shared__ BigSmem sm;
    __shared__ int s_unit;
    l1_big<8, false>(p, sm, &s_unit, blockIdx.x, gridDim.x);
}

__global__ void __launch_bounds__(512) l1_big_f8_kernel(GemmParams p) {
    __shared__ BigSmem sm;
    __shared__ int s_unit;
    l1_big<8, false, true>(p, sm, &s_unit, blockIdx.x, gridDim.x);
}

// ---------------------------------------------------------------------- L2 --
// L2 epilogue: the unit's bf16 tile (rows x 256 channels) goes through LDS so
// that every global store writes whole rows (a wave: two 512-byte rows per
// instruction) instead of 32-byte pieces of 16 rows from the MFMA layout.
// The caller's main loop ended on a barrier; the tile (<= 256 rows at a
// 528-byte pitch, 132 KiB) overlays the LDS operand tiles and the scales.
// The pitch is 132 dwords, 4 banks past a multiple of 64: the 16 rows of a
// quarter-wave's 8-byte writes fall in distinct banks (measured on MI355X at
// T = 8192 / 2048: L2's LDS bank conflicts halved against a 544-byte pitch,
// bf16 L2 1561 vs 1569-1570 us, fp8 L2 1071-1075 vs 1078-1089 us).
constexpr int kL2TilePitch = kL2BlockN * 2 + 16;
static_assert(kBigRows * kL2TilePitch <= (int)sizeof(BigSmem), "L2 store tile");
template <int W, int NT>
__device__ __forceinline__ void l2_store_tile(const GemmParams& p, const BigItem& it, BigSmem& sm,
                                              v4f (&acc)[Geo<W>::kWT][NT], int c0, int lane,
                                              int wave) {
    constexpr int kWT = Geo<W>::kWT;
    uint8_t* tile = reinterpret_cast<uint8_t*>(&sm);
    // channel 32w + 16t + 4(L/16) + i, row 16j + L%16 (the MFMA output layout)
#pragma unroll
    for (int j = 0; j < NT; ++j)
#pragma unroll
        for (int t = 0; t < kWT; ++t) {
            uint2 v;
            v.x = pack2_bf16(acc[t][j][0], acc[t][j][1]);
            v.y = pack2_bf16(acc[t][j][2], acc[t][j][3]);
            const int r = 16 * j + (lane & 15);
            const int c = wave * (kL2BlockN / W) + 16 * t + 4 * (lane >> 4);
            *reinterpret_cast<uint2*>(tile + r * kL2TilePitch + c * 2) = v;
        }
    __syncthreads();
    // 16 rows per pass: thread T copies 16 bytes (8 channels) of row T / 32
    constexpr int kThreads = Geo<W>::kThreads;
    const int tid = wave * 64 + lane;
#pragma unroll
    for (int pass = 0; pass < NT * 16 * 32 / kThreads; ++pass) {
        const int i = pass * kThreads + tid, r = i >> 5, ch = (i & 31) * 8;
        if (r < it.rows)
            *reinterpret_cast<v4i*>(p.out16 + (size_t)(it.m0 + r) * p.H + c0 + ch) =
                *reinterpret_cast<const v4i*>(tile + r * kL2TilePitch + ch * 2);
    }
}

// kFused: the item's ffn rows come from L1 units of the same launch, read at
// device scope (the caller's stage_scales waits for them first).
template <int W, int NT, bool kFused, bool kF8, class ScalesF>
__device__ __forceinline__ void l2_big_body(const GemmParams& p, const BigItem& it, BigSmem& sm,
                                            ScalesF stage_scales) {
    constexpr int kWT = Geo<W>::kWT;
    constexpr int S = kF8 ? big_stages_f8<NT>() : big_stages<W, NT, true>();
    constexpr bool kEarly = NT <= kEarlyMaxTiles;
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int H = p.H, I = p.I, KT = I >> 7;
    const int n0 = it.bx * kL2BlockN + wave * (kL2BlockN / W);   // the wave's output channels
    const uint8_t* we = p.w + (size_t)it.e * (size_t)H * I;
    WTiles<kWT> wt;
    wt.KT = KT;
#pragma unroll
    for (int t = 0; t < kWT; ++t) wt.set(t, we, (n0 >> 4) + t, lane);
    v4f acc[kWT][NT];
    std::conditional_t<kF8, WStage8<kWT>, WStage<kWT>> w[S];
    if constexpr (kEarly) {
        if constexpr (kF8) {
#pragma unroll
            for (int st = 0; st < S - 1; ++st) w_load8<kWT>(w[st], wt, min(st, KT - 1));
        } else {
            w_prologue<kWT, S>(w, wt, KT);
        }
    }
    stage_scales();
    XLoader<W, NT, kFused ? kBufferSc1 : 0, false, (kF8 || NT <= 12 ? 2 : 1)> xl;
    xl.base = p.x;
    big_loader_init(xl, [&](int r) {
        return (uint32_t)(it.m0 + (r < it.rows ? r : 0)) * (uint32_t)I;
    });
    if constexpr (kF8)
        big_mainloop_f8<W, NT, S, kEarly>(acc, sm, xl, wt, KT, w);
    else
        big_mainloop<W, NT, S, kEarly>(acc, sm, xl, wt, KT, w);
    l2_store_tile<W, NT>(p, it, sm, acc, it.bx * kL2BlockN, lane, wave);
}

// Workgroup L of the `grid` L2 workgroups.  kFused: before reading the
// item's ffn rows, wait until its ready counter reaches p.ready_target (the
// L1 blocks of an item), polling with a sleep; after p.spin_limit polls the
// workgroup gives up, sets kStatusWaitTimeout in the status word and goes on
// (the output is then wrong and the status says so; the kernel never hangs).
// After the poll, an agent-scope acquire fence pairs with the L1 units'
// release increments, and the workgroup barrier carries it to every wave;
// the rows are then read with sc1 (device-coherent) loads.
template <int W, bool kFused, bool kF8 = false>
__device__ __forceinline__ void l2_big(const GemmParams& p, BigSmem& sm, int* s_unit, int L,
                                       int grid) {
    BigItem it;
    // the tail queue for items of more than 32 rows (at 1-2 token tiles the
    // units are short and the tickets cost more than they balance)
    const bool tail = !kFused && p.status[kStatusMaxRows] > 32;
    if (tail ? !big_unit<true>(p, p.H / kL2BlockN, it, s_unit, L, grid)
             : !big_unit<false>(p, p.H / kL2BlockN, it, s_unit, L, grid))
        return;
    const int KT = p.I >> 7, H = p.H;
    const int tiles = (it.rows + 15) >> 4;
    // scales: ffn rows in slot order; W2 tiles of this block's 256 channels
    auto stage_scales = [&]() {
        if constexpr (kFused) {
            if (threadIdx.x == 0) {
                for (int n = 0; __hip_atomic_load(p.ready + it.item, __ATOMIC_RELAXED,
                                                  __HIP_MEMORY_SCOPE_AGENT) < p.ready_target;) {
                    if (++n >= p.spin_limit) {
                        atomicOr(p.err, kStatusWaitTimeout);
                        break;
                    }
                    __builtin_amdgcn_s_sleep(8);
                }
                __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "agent");
            }
            __syncthreads();
        }
        big_load_scales<W, kFused>(
            sm, KT, min(tiles * 16, kBigRows), p.w_sf != nullptr,
            [&](int r) -> const uint8_t* {
                return p.x_sf ? p.x_sf + (size_t)(it.m0 + (r < it.rows ? r : 0)) * KT
                              : nullptr;
            },
            [&](int t) {
                const int n = it.bx * kL2BlockN + t * 16;
                return p.w_sf + ((size_t)it.e * (H / 128) + (n >> 7)) * KT;
            });
    };
#define MM_L2_BODY(n) l2_big_body<W, n, kFused, kF8>(p, it, sm, stage_scales)
    MM_BIG_DISPATCH(MM_L2_BODY)
#undef MM_L2_BODY
}

__global__ void __launch_bounds__(512) l2_big_kernel(GemmParams p) {
    __shared__ BigSmem sm;
    __shared__ int s_unit;
    if (walk_taken(p)) return;   // the walk (launched just before) ran the units
    l2_big<8, false>(p, sm, &s_unit, blockIdx.x, gridDim.x);
}

__global__ void __launch_bounds__(512) l2_big_f8_kernel(GemmParams p) {
    __shared__ BigSmem sm;
    __shared__ int s_unit;
    l2_big<8, false, true>(p, sm, &s_unit, blockIdx.x, gridDim.x);
}

// ------------------------------------------------------------- L2 walker --
// One workgroup per CU walks its XCD's unit range at a stride of the XCD's
// workgroup count (the same units in flight as with one unit per workgroup).
// A unit's last k-steps issue the next unit's first weight stages (NextW), so
// the CU's weight stream does not drain at the unit boundary: the next unit's
// scale staging and first activation commit wait for loads that were issued
// during the previous unit, its epilogue overlaps them, and no workgroup is
// dispatched in between.  kWalkStages (4) weight stages divide K / 128 = 16,
// so the ring's slots line up across units; the ring stays live across the
// walk, which therefore holds bodies of at most kWalkMaxTiles token tiles
// (with the larger ones the compiler spilled 250-600 VGPRs).

// (item, block) of unit u, as big_unit decodes it.
__device__ __forceinline__ BigItem walk_unit(const GemmParams& p, int nb, int u) {
    BigItem it;
    const int4* items = reinterpret_cast<const int4*>(p.items);
    const int im = u / nb;
    int4 v = items[im];
    const int i0 = im - (v.w & 0xffff), n = v.w >> 16;
    const int local = u - nb * i0;
    it.bx = local / n;
    it.item = i0 + local % n;
    if (n != 1) v = items[it.item];
    it.e = v.x;
    it.m0 = v.y;
    it.rows = v.z - v.y;
    return it;
}

template <int W>
__device__ __forceinline__ WTiles<Geo<W>::kWT> l2_tiles(const GemmParams& p, const BigItem& it,
                                                          int wave, int lane) {
    constexpr int kWT = Geo<W>::kWT;
    const int n0 = it.bx * kL2BlockN + wave * (kL2BlockN / W);
    const uint8_t* we = p.w + (size_t)it.e * (size_t)p.H * p.I;
    WTiles<kWT> wt;
    wt.KT = p.I >> 7;
#pragma unroll
    for (int t = 0; t < kWT; ++t) wt.set(t, we, (n0 >> 4) + t, lane);
    return wt;
}


// One unit of the walk.  ring: the kWalkStages weight stages; pref: stages of
// this unit the previous one issued; nx: the next unit.  The thread index
// goes through an empty asm once per unit, so that the optimiser does not
// hoist every body's thread-index arithmetic out of the walk (where it stays
// live across all the bodies and spills).
template <int W, int NT>
__device__ __forceinline__ void l2_walk_body(const GemmParams& p, const BigItem& it, BigSmem& sm,
                                             WStage<Geo<W>::kWT> (&ring)[4],
                                             const NextW<Geo<W>::kWT>& nx, int pref) {
    constexpr int kWT = Geo<W>::kWT;
    constexpr int S = kWalkStages;
    int tid = threadIdx.x;
    asm volatile("" : "+v"(tid));
    __builtin_assume(tid >= 0 && tid < Geo<W>::kThreads);
    const int lane = tid & 63, wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int H = p.H, I = p.I, KT = I >> 7;
    const WTiles<kWT> wt = l2_tiles<W>(p, it, wave, lane);
    const int tiles = (it.rows + 15) >> 4;
    big_load_scales<W>(
        sm, KT, min(tiles * 16, kBigRows), p.w_sf != nullptr,
        [&](int r) -> const uint8_t* {
            return p.x_sf ? p.x_sf + (size_t)(it.m0 + (r < it.rows ? r : 0)) * KT : nullptr;
        },
        [&](int t) {
            const int n = it.bx * kL2BlockN + t * 16;
            return p.w_sf + ((size_t)it.e * (H / 128) + (n >> 7)) * KT;
        },
        tid);
    XLoader<W, NT, 0, true> xl;
    xl.base = p.x;
    xl.tid_ = tid;
    big_loader_init(xl, [&](int r) {
        return (uint32_t)(it.m0 + (r < it.rows ? r : 0)) * (uint32_t)I;
    });
    v4f acc[kWT][NT];
    big_mainloop<W, NT, S, false>(acc, sm, xl, wt, KT, ring, nx, pref);
    l2_store_tile<W, NT>(p, it, sm, acc, it.bx * kL2BlockN, lane, wave);
}

template <int W>
__device__ __forceinline__ void l2_walk(const GemmParams& p, BigSmem& sm, int L, int grid) {
    constexpr int kWT = Geo<W>::kWT;
    const int x = L & 7, k = L >> 3, stride = (grid - x + 7) >> 3;
    const int lo = p.xcd_cuts[x], hi = p.xcd_cuts[x + 1];
    int u = lo + k;
    if (u >= hi) return;
    const int nb = p.H / kL2BlockN;
    BigItem it = walk_unit(p, nb, u);
    WStage<kWT> ring[4];
    int pref = 0;
#pragma unroll 1
    for (;;) {
        const int un = u + stride;
        NextW<kWT> nx;
        nx.has = un < hi;
        const BigItem itn = nx.has ? walk_unit(p, nb, un) : it;
        {
            int tid = threadIdx.x;
            asm volatile("" : "+v"(tid));
            nx.wt = l2_tiles<W>(p, itn, __builtin_amdgcn_readfirstlane(tid >> 6), tid & 63);
        }
        // items of at most 16 * kWalkMaxTiles rows (walk_taken)
        const int tiles = (it.rows + 15) >> 4;
        switch (tiles) {
#define MM_WALK_BODY(n) \
    case n: l2_walk_body<W, n>(p, it, sm, ring, nx, pref); break;
            MM_WALK_BODY(1) MM_WALK_BODY(2) MM_WALK_BODY(3) MM_WALK_BODY(4)
            MM_WALK_BODY(5) MM_WALK_BODY(6) MM_WALK_BODY(7) default: MM_WALK_BODY(8)
#undef MM_WALK_BODY
        }
        pref = nx.has ? kWalkStages - 1 : 0;
        if (un >= hi) break;
        __syncthreads();   // the next unit's staging reuses the LDS
        u = un;
        it = itn;
    }
}

__global__ void __launch_bounds__(512) l2_walk_kernel(GemmParams p) {
    __shared__ BigSmem sm;
    if (!walk_taken(p)) return;   // l2_big_kernel, launched next, runs the units
    l2_walk<8>(p, sm, blockIdx.x, gridDim.x);
}

// L1 and L2 in one launch: workgroups [0, g1) run L1 units, the rest L2
// units, which start on an item as soon as its L1 units are done (g1 is a
// multiple of 8, so both keep the workgroup -> XCD mapping L % 8).  Each
// XCD's dispatcher starts all its L1 workgroups before any of its L2
// workgroups, and no L1 unit waits for anything, so every wait ends.
__global__ void __launch_bounds__(512) gemm_fused_kernel(GemmParams p1, GemmParams p2, int g1) {
    __shared__ BigSmem sm;
    __shared__ int s_unit;
    if ((int)blockIdx.x < g1)
        l1_big<8, true>(p1, sm, &s_unit, blockIdx.x, g1);
    else
        l2_big<8, true>(p2, sm, &s_unit, (int)blockIdx.x - g1, (int)gridDim.x - g1);
}

#undef MM_BIG_DISPATCH

}  // namespace mm
