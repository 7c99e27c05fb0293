// route.hip -- token-to-expert permutation on one GPU (the intra-GPU form of
// the reference's EP dispatch metadata: route_build_body, src/prologue.cuh:
// 126-226; publish_counts_body :230-256; task_setup_body :269-498).
//
// Three stream-ordered kernels over P = tokens * topk (token, k) pairs (two
// for small P, where route_scan builds the histograms itself):
//   1. route_hist:    per chunk of pairs, an LDS histogram over experts.
//   2. route_scan:    one workgroup; per expert the exclusive prefix over chunks,
//                     the capped count, the exclusive prefix over experts
//                     (slot offsets), the work-item list (expert, first row),
//                     the big GEMMs' XCD unit ranges and the ticket order
//                     of L1's tail queues.
//   3. route_scatter: per chunk, a stable rank of every pair among the pairs of
//                     the same expert (wave ballots over the expert-id bits +
//                     an LDS prefix across waves), giving the canonical slot
//                     order = ascending pair index.  Writes perm[slot] and
//                     pair_pos[pair].
// Pairs whose id is outside [0, E) or whose rank is >= slot_capacity get
// pair_pos = -1 (reference: dropped at route_build_body, prologue.cuh:150-175).
#include "mm_kernels.h"

namespace mm {

__global__ void __launch_bounds__(kRouteThreads)
route_hist_kernel(const int64_t* __restrict__ topk_idx, int P, int E, int chunk,
                  int* __restrict__ chunk_hist) {
    __shared__ int hist[kMaxExperts];
    for (int i = threadIdx.x; i < E; i += blockDim.x) hist[i] = 0;
    __syncthreads();
    const int base = blockIdx.x * chunk;
    const int end = min(base + chunk, P);
    for (int p = base + threadIdx.x; p < end; p += blockDim.x) {
        const int64_t e = topk_idx[p];
        if (e >= 0 && e < E) atomicAdd(&hist[(int)e], 1);
    }
    __syncthreads();
    for (int i = threadIdx.x; i < E; i += blockDim.x)
        chunk_hist[(size_t)blockIdx.x * E + i] = hist[i];
}

// Block-wide exclusive scan of one int per thread (blockDim = kScanThreads).
__device__ int block_exclusive_scan(int v, int* smem, int* total) {
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    int x = v;
#pragma unroll
    for (int d = 1; d < 64; d <<= 1) {
        const int y = __shfl_up(x, d, 64);
        if (lane >= d) x += y;
    }
    if (lane == 63) smem[wave] = x;
    __syncthreads();
    if (threadIdx.x == 0) {
        int run = 0;
        for (int w = 0; w < kScanThreads / 64; ++w) {
            const int t = smem[w];
            smem[w] = run;
            run += t;
        }
        smem[kScanThreads / 64] = run;
    }
    __syncthreads();
    const int r = smem[wave] + x - v;
    *total = smem[kScanThreads / 64];
    __syncthreads();
    return r;
}

__global__ void __launch_bounds__(kScanThreads)
route_scan_kernel(const int64_t* __restrict__ topk_idx, int P, int chunk,
                  int* __restrict__ chunk_hist, int nchunks, int E, int cap, int m_tile,
                  int max_items, int nb1, int nb2, int* __restrict__ counts,
                  int* __restrict__ offsets, int* __restrict__ items, int* __restrict__ status) {
    __shared__ int smem[kScanThreads / 64 + 1];
    __shared__ int cut_s[2][8];
    __shared__ int lh[kFusedHist];   // [chunk][expert] when topk_idx is given
    __shared__ int s_rows;           // rows of the largest work item
    __shared__ int cuts_sh[9];       // the L1 XCD unit ranges
    __shared__ int s_ioff[kMaxExperts + 1];     // first item of each expert (+ the item count)
    __shared__ int s_cnt[kMaxExperts];          // routed rows of each expert
    __shared__ uint8_t tnt[8][kQueueTail];      // token tiles of L1's tail units
    // the status word of this launch (only this kernel sets its error bits;
    // thread 0 clears it before its own atomicOr below)
    if (threadIdx.x == 0) {
        status[0] = 0;
        s_rows = 0;
    }
    // Small launches (topk_idx given, nchunks * E <= kFusedHist): the chunk
    // histograms of route_hist_kernel, built here in LDS, 8 pairs' loads in
    // flight per thread.
    const bool fused = topk_idx != nullptr;
    if (fused) {
        for (int i = threadIdx.x; i < nchunks * E; i += kScanThreads) lh[i] = 0;
        __syncthreads();
        for (int p0 = threadIdx.x; p0 < P; p0 += 8 * kScanThreads) {
            int64_t ev[8];
#pragma unroll
            for (int u = 0; u < 8; ++u) {
                const int p = p0 + u * kScanThreads;
                ev[u] = p < P ? topk_idx[p] : -1;
            }
#pragma unroll
            for (int u = 0; u < 8; ++u) {
                const int p = p0 + u * kScanThreads;
                if (ev[u] >= 0 && ev[u] < E) atomicAdd(&lh[(p / chunk) * E + (int)ev[u]], 1);
            }
        }
        __syncthreads();
    }
    // E <= kMaxExperts = kScanThreads: one expert per thread.
    const int e = threadIdx.x;
    int cnt = 0, run = 0;
    if (e < E) {
        // exclusive prefix over chunks (uncapped rank base), 8 chunks' loads
        // in flight at a time
        for (int c0 = 0; c0 < nchunks; c0 += 8) {
            int h[8];
#pragma unroll
            for (int u = 0; u < 8; ++u)
                h[u] = c0 + u >= nchunks ? 0
                       : fused           ? lh[(c0 + u) * E + e]
                                         : chunk_hist[(size_t)(c0 + u) * E + e];
#pragma unroll
            for (int u = 0; u < 8; ++u)
                if (c0 + u < nchunks) {
                    chunk_hist[(size_t)(c0 + u) * E + e] = run;
                    run += h[u];
                }
        }
        cnt = min(run, cap);
        counts[e] = cnt;
    }
    // pairs with an id in [0, E) before the slot cap (the rest of P had ids
    // outside [0, E))
    int valid = 0;
    (void)block_exclusive_scan(run, smem, &valid);
    int slots = 0;
    const int off = block_exclusive_scan(cnt, smem, &slots);
    if (e < E) offsets[e] = off;
    if (threadIdx.x == 0) offsets[E] = slots;
    // Work items: the expert's rows split evenly into ceil(cnt / m_tile)
    // items of at most m_tile rows (no item re-streams the expert's weights
    // for a small remainder).  The items of one expert then have equal token
    // tile counts, so the units that read one weight block run in lockstep
    // and all but the first take it from L2.  (Measured on MI355X at T =
    // 8192: splitting at 16-row multiples instead ran 2% less MFMA work but
    // its unequal items drifted apart; L1 fetched 9.30 vs 7.33 GB and the
    // layer took 4908-4943 vs 4841-4854 us.)  Record: (expert, first slot,
    // end slot, index within the expert | item count of the expert << 16),
    // the slots absolute (the expert's offset included), so that a GEMM unit
    // needs no offsets[] load after its item.
    const int nm = (cnt + m_tile - 1) / m_tile;
    const int sz = nm > 0 ? (cnt + nm - 1) / nm : 0;
    if (sz > 0) atomicMax(&s_rows, sz);   // ordered before the read by the scan's barriers
    int nitems = 0;
    const int ioff = block_exclusive_scan(nm, smem, &nitems);
    for (int j = 0; j < nm; ++j) {
        const int it = ioff + j;
        if (it < max_items) {
            const int m0 = j * sz;
            reinterpret_cast<int4*>(items)[it] =
                make_int4(e, off + m0, off + min(cnt, m0 + sz), j | (nm << 16));
        }
    }
    if (threadIdx.x < 2 * kQueueInts) status[kQueueL1 + threadIdx.x] = 0;   // tail queues
    // per-item L1 ready counters of the fused L1 -> L2 launch (after the table)
    for (int i = threadIdx.x; i < max_items; i += kScanThreads) items[4 * max_items + i] = 0;
    if (threadIdx.x == 0) {
        status[1] = min(nitems, max_items);
        status[2] = slots;
        status[3] = valid - slots;   // pairs dropped by the slot capacity
        status[4] = P - valid;       // pairs whose expert id is outside [0, E)
        status[kStatusMaxRows] = s_rows;
        if (nitems > max_items) atomicOr(&status[0], kStatusItemOverflow);
    }
    // XCD ranges of the big GEMMs' units (nb blocks per item; an expert's
    // nb * nm units are contiguous in the kernels' numbering).  Modelled cost
    // of one of the expert's units per k-step, in token-tile MFMA times:
    // max(9, 2 + token tiles of its largest item) -- the fixed per-step work
    // (barrier, conversions, operand reads) is worth ~2 token tiles and the
    // weight stream at the full-chip HBM rate ~9 (measured on MI355X: a
    // k-step costs ~0.33 us + 0.137 us per token tile without weight loads,
    // and a weight block's k-step streams in ~1.23 us).  XCD x starts where
    // the running cost crosses x/8 of the total (the same expert for L1 and
    // L2, whose costs differ by the factor nb); each range is then clamped to
    // its share of the grid, nb * max_items + 8 workgroups.
    const int uc = max(9, 2 + min((sz + 15) >> 4, kBigMaxTiles));
    const int w = nm * uc;
    int wtot = 0;
    const int wpre = block_exclusive_scan(w, smem, &wtot);
    if (nm > 0 && ioff + nm <= max_items) {
        for (int x = 1; x < 8; ++x) {
            const int64_t t1 = (int64_t)wtot * nb1 * x / 8, t2 = (int64_t)wtot * nb2 * x / 8;
            const int64_t lo1 = (int64_t)wpre * nb1, lo2 = (int64_t)wpre * nb2;
            if (t1 >= lo1 && t1 < lo1 + (int64_t)w * nb1)
                cut_s[0][x] = nb1 * ioff + (int)((t1 - lo1) / uc);
            if (t2 >= lo2 && t2 < lo2 + (int64_t)w * nb2)
                cut_s[1][x] = nb2 * ioff + (int)((t2 - lo2) / uc);
        }
    }
    __syncthreads();
    if (threadIdx.x < 2) {
        const int nb = threadIdx.x == 0 ? nb1 : nb2;
        const int n = min(nitems, max_items), units = nb * n, cap = (nb * max_items + 8) / 8;
        int* cuts = status + (threadIdx.x == 0 ? kCutsL1 : kCutsL2);
        int prev = 0;
        cuts[0] = 0;
        for (int x = 1; x < 8; ++x) {
            // a target past the last complete expert (item overflow) cuts at the end
            int v = nitems <= max_items && n > 0 ? cut_s[threadIdx.x][x] : units;
            v = min(max(v, prev), prev + cap);
            v = max(v, units - (8 - x) * cap);
            cuts[x] = v;
            if (threadIdx.x == 0) cuts_sh[x] = v;
            prev = v;
        }
        cuts[8] = units;
        if (threadIdx.x == 0) {
            cuts_sh[0] = 0;
            cuts_sh[8] = units;
        }
    }
    // Ticket order of L1's tail queues (the last t = min(range, kQueueTail)
    // units of each XCD range): costliest unit first, i.e. by the token tiles
    // of its item, descending, ties in unit order, so that heavy units do not
    // start after light ones at the end of the kernel.  Tail unit i of XCD x
    // is unit cuts[x + 1] - t + i; L1 runs ticket k as tail unit order[k]
    // (gemm_big.hip: claim_tail_unit).  One thread per tail slot finds its
    // unit's expert by binary search over the item offsets.  Only when some
    // item holds more than kTailOrderRows rows (skewed routing, T = 8192):
    // below, the units differ by a few token tiles at most, and the order is
    // the identity.  (Measured on MI355X: a loop over the 8 tails in every
    // expert thread added 10.6 us to this one-workgroup kernel; L2's tails
    // gained nothing from the order and keep ticket order.)
    uint8_t* order = reinterpret_cast<uint8_t*>(status + kTailOrdL1);
    __syncthreads();   // cuts_sh, and s_rows of every expert
    if (s_rows > kTailOrderRows) {   // uniform over the workgroup
        if (e < E) {
            s_ioff[e] = ioff;
            s_cnt[e] = cnt;
        }
        if (threadIdx.x == 0) s_ioff[E] = nitems;
        __syncthreads();
        if (threadIdx.x < 8 * kQueueTail) {
            const int x = threadIdx.x / kQueueTail, i = threadIdx.x % kQueueTail;
            const int lo = cuts_sh[x], hi = cuts_sh[x + 1], t = min(hi - lo, kQueueTail);
            if (i < t) {
                const int u = hi - t + i, im = u / nb1;
                int a = 0, b = E - 1;   // the last expert whose first item is <= im
                while (a < b) {
                    const int m = (a + b + 1) >> 1;
                    if (s_ioff[m] <= im) a = m; else b = m - 1;
                }
                const int n = max(s_ioff[a + 1] - s_ioff[a], 1), c = s_cnt[a];
                const int z = (c + n - 1) / n, j = (u - nb1 * s_ioff[a]) % n;
                tnt[x][i] = (uint8_t)min((min(c, (j + 1) * z) - j * z + 15) >> 4, kBigMaxTiles);
            }
        }
        __syncthreads();
        if (threadIdx.x < 8 * kQueueTail) {
            const int x = threadIdx.x / kQueueTail, i = threadIdx.x % kQueueTail;
            const int t = min(cuts_sh[x + 1] - cuts_sh[x], kQueueTail);
            if (i < t) {
                const int v = tnt[x][i];
                int r = 0;
                for (int k = 0; k < t; ++k) {
                    const int w = tnt[x][k];
                    r += (w > v) || (w == v && k < i);
                }
                order[kQueueTail * x + r] = (uint8_t)i;
            }
        }
    } else if (threadIdx.x < 8 * kQueueTail) {
        order[threadIdx.x] = (uint8_t)(threadIdx.x % kQueueTail);
    }
}

__global__ void __launch_bounds__(kRouteThreads)
route_scatter_kernel(const int64_t* __restrict__ topk_idx, int P, int E, int nbits, int chunk,
                     const int* __restrict__ chunk_hist, const int* __restrict__ counts,
                     const int* __restrict__ offsets, uint32_t* __restrict__ perm,
                     int* __restrict__ pair_pos) {
    constexpr int kWaves = kRouteThreads / 64;
    __shared__ int run[kMaxExperts];
    __shared__ int cntw[kWaves][kMaxExperts];
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    for (int i = threadIdx.x; i < E; i += blockDim.x) {
        run[i] = chunk_hist[(size_t)blockIdx.x * E + i];
#pragma unroll
        for (int w = 0; w < kWaves; ++w) cntw[w][i] = 0;
    }
    __syncthreads();
    const int base = blockIdx.x * chunk;
    const uint64_t lt_mask = (lane == 0) ? 0ull : (~0ull >> (64 - lane));
    for (int r0 = base; r0 < min(base + chunk, P); r0 += kRouteThreads) {
        const int p = r0 + threadIdx.x;
        const bool in = p < P;
        const int64_t e64 = in ? topk_idx[p] : -1;
        const bool ok = e64 >= 0 && e64 < E;
        const int e = ok ? (int)e64 : 0;
        // lanes holding the same expert id: AND of per-bit ballots
        uint64_t m = __ballot(ok);
        for (int b = 0; b < nbits; ++b) {
            const uint64_t bb = __ballot(ok && ((e >> b) & 1));
            m &= ((e >> b) & 1) ? bb : ~bb;
        }
        const int rank = __popcll(m & lt_mask);
        const int wcnt = __popcll(m);
        if (ok && rank == 0) cntw[wave][e] = wcnt;
        __syncthreads();
        if (ok) {
            int pre = run[e];
            for (int w = 0; w < wave; ++w) pre += cntw[w][e];
            const int r = pre + rank;
            if (r < counts[e]) {
                const int pos = offsets[e] + r;
                perm[pos] = (uint32_t)p;
                pair_pos[p] = pos;
            } else {
                pair_pos[p] = -1;
            }
        } else if (in) {
            pair_pos[p] = -1;
        }
        __syncthreads();
        if (ok && rank == 0) {
            atomicAdd(&run[e], wcnt);
            cntw[wave][e] = 0;
        }
        __syncthreads();
    }
}

// DISPATCH pool (diagnostic / parity): pool[slot][:] = x[perm[slot] / topk][:],
// 16 bytes per thread.
__global__ void __launch_bounds__(256)
dispatch_gather_kernel(const uint8_t* __restrict__ x, int H, int topk,
                       const uint32_t* __restrict__ perm, const int* __restrict__ status,
                       uint8_t* __restrict__ pool) {
    const int slot = blockIdx.x;
    if (slot >= status[2]) return;
    const size_t tok = perm[slot] / (uint32_t)topk;
    const v4i* src = reinterpret_cast<const v4i*>(x + tok * H);
    v4i* dst = reinterpret_cast<v4i*>(pool + (size_t)slot * H);
    for (int c = threadIdx.x; c < H / 16; c += blockDim.x) dst[c] = src[c];
}

}  // namespace mm
