// mm_kernels.h -- kernel declarations and launch constants shared by the
// host launcher (megakernel.hip) and the kernel translation units.
#pragma once

#include "mm_device.h"
#include "megakernel.h"

namespace mm {

constexpr int kMaxExperts = 1024;   // E upper bound (one scan thread per expert)
constexpr int kScanThreads = 1024;
constexpr int kRouteThreads = 256;
// Pairs per routing chunk: 256 (one scatter round of kRouteThreads) up to
// kRouteSmallP pairs, 1024 above, where the scan's serial walk over chunks
// would grow (measured on MI355X, route_* total: T=512 13.5 vs 15.9 us,
// T=8192 37.2 vs 22.7 us).
constexpr int kRouteChunkSmall = 256;
constexpr int kRouteChunkLarge = 1024;
constexpr int kRouteSmallP = 8192;
inline int route_chunk(int P) { return P <= kRouteSmallP ? kRouteChunkSmall : kRouteChunkLarge; }
// The scan builds the chunk histograms itself (in LDS, no histogram launch)
// when they fit: nchunks * E <= kFusedHist counters.
constexpr int kFusedHist = 8192;

constexpr int kGemmThreads = 256;   // 4 waves per workgroup (decode-shaped GEMMs)
constexpr int kBigThreads = 512;    // 8 waves per workgroup, two per SIMD (large-M GEMMs)
constexpr int kBigMaxTiles = 16;    // large-M GEMMs: up to 16 token tiles (256 rows) per item
constexpr int kBigMaxKT = 64;       // large-M GEMMs: K / 128 <= 64 (H, I <= 8192)
constexpr int kL1BlockH = 128;      // hidden columns (gate+up pairs) per L1 workgroup
constexpr int kL2BlockN = 256;      // output channels per L2 workgroup
constexpr int kStatusWords = 64;    // status words (readable with read_status)
constexpr int kTailOrdL1 = 64;      // status[64..127] as bytes [8][kQueueTail]: L1 tail ticket order
constexpr int kStatusInts = 128;    // the workspace's status region
constexpr int kStatusItemOverflow = fp8mega::kStatusItemOverflow;
constexpr int kStatusWaitTimeout = fp8mega::kStatusWaitTimeout;
constexpr int kReadySpinLimit = 1 << 20;   // default polls (~1 s with the sleep between)
constexpr int kStatusMaxRows = 5;   // status[5]: rows of the largest work item
constexpr int kCutsL1 = 16;         // status[16..24]: XCD unit ranges of the L1 big GEMM
constexpr int kCutsL2 = 32;         // status[32..40]: the same for L2
// Tail queues of the big GEMMs: per XCD a ticket counter over the last
// kQueueTail units of its range, plus a count of the workgroups that took
// tickets (status[44..52] for L1, [53..61] for L2; zeroed by the routing
// scan and again by the last ticket taker of each launch).  L1 always takes
// tickets, L2 when its largest item has more than 32 rows (gemm_big.hip:
// big_unit<true>).  L1's tickets go out costliest unit first: the routing
// scan writes each tail's order (kTailOrdL1); L2's go out in unit order.
constexpr int kQueueInts = 9;
constexpr int kQueueL1 = 44;
constexpr int kQueueL2 = kQueueL1 + kQueueInts;
constexpr int kQueueTail = 32;      // units per XCD handed out by ticket (one per CU)
constexpr int kStealers = 8;        // workgroups per XCD past its range that take others' tickets
static_assert(kQueueTail * 8 <= (kStatusInts - kTailOrdL1) * 4, "the tail order fits");
constexpr int kTailOrderRows = 128;   // L1's tail order is costliest-first above this item size

// Parameters of the two grouped GEMMs (one struct so that the launcher and
// the kernels agree on one argument list).
struct GemmParams {
    const uint8_t* x;         // L1: activations fp8 [tokens][H]; L2: ffn [P][I]
    const uint8_t* x_sf;      // matching UE8M0 scales or null
    const uint8_t* w;         // packed weights of all experts
    const uint8_t* w_sf;      // UE8M0 block scales [E][N/128][K/128] or null
    const int* counts;        // [E]
    const int* offsets;       // [E+1]
    const int* items;         // [max_items][4]: expert, first slot, end slot (absolute), j | n << 16
                              // (item j of the expert's n)
    const int* status;        // [1] = number of items
    const int* xcd_cuts;      // [9]: XCD x runs big-GEMM units [cuts[x], cuts[x+1])
    int* queue;               // [kQueueInts]: the tail queue of these units
    const uint8_t* tail_ord;  // [8][kQueueTail]: ticket t of XCD x runs tail unit tail_ord[32x + t]
                              // (null: tail unit t)
    const uint32_t* perm;     // slot -> pair (L1 gathers x rows through it)
    uint8_t* out8;            // L1: ffn fp8 [P][I]
    uint8_t* out_sf;          // L1: ffn scales [P][I/128] (ffn_ue8m0)
    uint16_t* out16;          // L2: bf16 [P][H]
    int H, I, G, topk;
    int ffn_ue8m0;
    // fused L1 -> L2 launch only (gemm_fused_kernel)
    int* ready;               // [max_items]: L1 blocks done per work item
    int ready_target;         // L1 blocks per item (L2 waits for this count)
    int spin_limit;           // L2: polls of a ready counter before giving up
    int* err;                 // status word [0]: kStatusWaitTimeout on give-up
    // L2 launched as the walk plus the one-unit-per-workgroup kernel: exactly
    // one of the two runs the units (walk_taken decides from the item size)
    int walk;
};

// The L2 walk takes the launch when its largest work item has 3..8 token tiles
// and K / 128 is a multiple of its weight stages: its bodies hold at most 8
// tiles (the weight ring stays live across units), and at 1-2 tiles the
// one-unit kernel's six weight stages stream faster.
constexpr int kWalkMaxTiles = 8;
constexpr int kWalkStages = 4;     // weight stages of the walk; must divide K / 128
__device__ __forceinline__ bool walk_taken(const GemmParams& p) {
    if (!p.walk) return false;
    const int rows = p.status[kStatusMaxRows];
    return rows > 32 && rows <= 16 * kWalkMaxTiles && (p.I >> 7) % kWalkStages == 0;
}

template <int MT> __global__ void l1_kernel(GemmParams p);
template <int MT> __global__ void l2_kernel(GemmParams p);
__global__ void l1_big_kernel(GemmParams p);
__global__ void l2_big_kernel(GemmParams p);
__global__ void l1_big_f8_kernel(GemmParams p);   // MegaLaunchArgs::mfma_fp8
__global__ void l2_big_f8_kernel(GemmParams p);
__global__ void l2_walk_kernel(GemmParams p);
__global__ void gemm_fused_kernel(GemmParams p1, GemmParams p2, int g1);

__global__ void route_hist_kernel(const int64_t*, int, int, int, int*);
__global__ void route_scan_kernel(const int64_t*, int, int, int*, int, int, int, int, int, int, int,
                                  int*, int*, int*, int*);
__global__ void route_scatter_kernel(const int64_t*, int, int, int, int, const int*, const int*,
                                     const int*, uint32_t*, int*);
__global__ void dispatch_gather_kernel(const uint8_t*, int, int, const uint32_t*, const int*,
                                       uint8_t*);
template <bool kStreamRows>
__global__ void combine_kernel(const uint16_t*, const int*, const float*, int, int, float*,
                               uint16_t*);
__global__ void fill_w_lane_kernel(uint8_t*, int, int, uint32_t);
__global__ void pack_weights_kernel(uint8_t*, const uint8_t*, int, int, int);
__global__ void pack_weights_ref_kernel(uint8_t*, const uint8_t*, int, int, int);
__global__ void fill_weights_normal_kernel(uint8_t*, uint8_t*, int, int, uint64_t, float);
__global__ void quant_act_kernel(const uint16_t*, int, int, uint8_t*, uint8_t*);
__global__ void convert_selftest_kernel(const float*, int, uint8_t*, uint16_t*);
__global__ void empty_kernel();
__global__ void fill_int_kernel(int*, int, int);

}  // namespace mm
