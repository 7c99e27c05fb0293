// megakernel.hip -- host side of the public API (include/megakernel.h): shape
// validation, workspace layout, stream-ordered kernel launches, and the thin
// extern "C" layer.  Reference counterpart: src/megakernel.cu:1-284 (launch
// entry points) and test/mega_common.cuh:69-88,344-376 (geometry / args).
//
// Nothing here allocates or reads the environment, and only read_status
// synchronises: every launch entry point only validates its arguments and
// enqueues kernels on `stream`, so the layer is capture-safe.  The workspace
// is caller-owned, or (mm_launch_full_noalloc) the file-scope `scratch`.
#include <cstddef>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <mutex>

#include "mm_kernels.h"

namespace fp8mega {
namespace {

thread_local int g_last_error = kOk;

inline int64_t align256(int64_t v) { return (v + 255) & ~(int64_t)255; }

int auto_m_tile(int tokens, int topk, int E) {
    // Rows per work item: the largest window of the LDS-staged kernels (256),
    // so that an expert's weights stream from HBM once whenever its load fits
    // and a hot expert splits into as few items as possible.  Measured on
    // MI355X (L1 / L2 us): balanced routing gives the same items for every
    // window up to T = 2048; T = 4096: 1783 / 986 vs 1960 / 1079 with 128;
    // T = 8192: 3363 / 1813 vs 3406 / 1845 with 128; Zipf(1.1) T = 1024: 960 /
    // 554 vs 1000 / 585 with 64, T = 2048: 1240 / 682 vs 1277 / 701 with 128.
    // The decode-shaped kernels (win_cap 16/32) are slower from T = 512 on.
    (void)tokens;
    (void)topk;
    (void)E;
    return 16 * mm::kBigMaxTiles;
}

int pairing_block(int I) { return I < 256 ? I : 256; }

int check_dims(int topk, int E, int H, int I, int win_cap) {
    if (topk < 1 || topk > 64 || E < 1 || E > mm::kMaxExperts) return kErrBadDims;
    if (H < 256 || H % 256 != 0 || I < 128 || I % 128 != 0) return kErrBadDims;
    if (H > 128 * mm::kBigMaxKT || I > 128 * mm::kBigMaxKT) return kErrBadDims;
    if (I % pairing_block(I) != 0) return kErrBadDims;
    if (win_cap != 0 && win_cap != 16 && win_cap != 32 && win_cap != 64 && win_cap != 128 &&
        win_cap != 16 * mm::kBigMaxTiles)
        return kErrBadDims;
    return kOk;
}

// The GEMMs' activation loaders address a row as a 32-bit byte offset
// (token * H into x for L1, slot * I into the intermediate for L2), and slots
// are int: capacities past those ranges are rejected rather than wrapped.
// A work item records (index within its expert) | (items of the expert << 16)
// and the big GEMMs decode it with & 0xffff and an arithmetic >> 16, so one
// expert may hold at most 32767 items: ceil(max_tokens * topk / m_tile).
int check_capacity(int64_t max_tokens, int topk, int H, int I, int win_cap) {
    if (max_tokens <= 0) return kErrBadDims;
    const int64_t pairs = max_tokens * topk;
    if (pairs > INT32_MAX || max_tokens * H > (int64_t(1) << 32) ||
        pairs * I > (int64_t(1) << 32))
        return kErrBadDims;
    const int64_t m_tile = win_cap > 0 ? win_cap : auto_m_tile((int)max_tokens, topk, 0);
    if ((pairs + m_tile - 1) / m_tile > 32767) return kErrBadDims;
    return kOk;
}

struct Bound {
    const uint8_t* x = nullptr;
    const uint8_t* x_sf = nullptr;
    const float* w = nullptr;
    MegaLayout L{};
    uint8_t* ws = nullptr;
    int m_tile = 32;
};

int bind(const MegaLaunchArgs& a, Bound& b, bool need_weights) {
    int st = check_dims(a.topk, a.num_experts, a.hidden, a.intermediate, a.win_cap);
    if (st != kOk) return st;
    if (a.rwk == nullptr || a.topk_idx == nullptr || a.self == nullptr) return kErrNullPointer;
    if (need_weights && (a.w1 == nullptr || a.w2 == nullptr)) return kErrNullPointer;
    if (a.tokens < 0) return kErrBadDims;
    st = check_capacity(a.max_tokens, a.topk, a.hidden, a.intermediate, a.win_cap);
    if (st != kOk) return st;
    if (a.tokens > a.max_tokens) return kErrTooManyTokens;
    if (a.R != 1 || a.rank != 0) return kErrUnsupported;
    const bool any_sf = a.x_sf || a.w1_sf || a.w2_sf;
    if (any_sf && !(a.w1_sf && a.w2_sf)) return kErrNullPointer;
    if (any_sf && !a.in_bf16 && !a.x_sf) return kErrNullPointer;
    // the L1 output's quantisation follows the scale mode, as in the reference
    // (per-128 UE8M0 with block-scaled operands, torch/mxmegakernel/utils/
    // math.py:13-72; the saturating e4m3 cast without, src/bench_check.cuh:
    // 362-380); a mixed mode is no reference path
    if ((a.ffn_ue8m0 != 0) != any_sf) return kErrUnsupported;
    b.L = layout(a.max_tokens, a.topk, a.num_experts, a.hidden, a.intermediate, a.win_cap);
    if (a.workspace_bytes < b.L.total) return kErrWorkspace;
    // the fp8 MFMA path exists for the LDS-staged kernels and two launches
    if (a.mfma_fp8 && (a.fuse_l1l2 || b.L.m_tile <= 32)) return kErrUnsupported;
    b.ws = reinterpret_cast<uint8_t*>(a.rwk);
    b.x = a.self + a.x_off;
    b.x_sf = a.x_sf;
    b.w = reinterpret_cast<const float*>(a.self + a.weights_off);
    b.m_tile = b.L.m_tile;
    if (a.in_bf16) {
        b.x = b.ws + b.L.xq;
        b.x_sf = a.w1_sf ? b.ws + b.L.xq_sf : nullptr;
    }
    return kOk;
}

template <class T>
T* at(const Bound& b, int64_t off) { return reinterpret_cast<T*>(b.ws + off); }

int launched(int st) {
    if (st != kOk) return st;
    return hipPeekAtLastError() == hipSuccess ? kOk : kErrLaunch;
}

// bf16 x -> fp8 (+ per-128 UE8M0 scales) in the workspace (reference
// x_fold_body, src/prologue.cuh:103-122).  Runs on every launch with bf16
// input, also when skip_prologue reuses the routing: the tokens' routes may
// repeat while x changes (the reference's kernel.cuh:69-101 folds x before
// its skip_prologue test).
void fold_x(const MegaLaunchArgs& a, const Bound& b, hipStream_t s) {
    if (!a.in_bf16) return;
    const size_t n8 = (size_t)a.tokens * a.hidden / 8;
    if (n8 > 0)
        hipLaunchKernelGGL(mm::quant_act_kernel, dim3((unsigned)((n8 + 255) / 256)), dim3(256), 0,
                           s, reinterpret_cast<const uint16_t*>(a.self + a.x_off), a.tokens,
                           a.hidden, b.ws + b.L.xq, a.w1_sf ? b.ws + b.L.xq_sf : nullptr);
}

int do_prelude(const MegaLaunchArgs& a, hipStream_t s) {
    Bound b;
    int st = bind(a, b, false);
    if (st != kOk) return st;
    const int E = a.num_experts, P = a.tokens * a.topk;
    int* status = at<int>(b, b.L.status);   // reset and written by route_scan_kernel
    fold_x(a, b, s);
    const int chunk = mm::route_chunk(P);
    const int nchunks = P > 0 ? (P + chunk - 1) / chunk : 0;
    int* hist = at<int>(b, b.L.chunk_hist);
    // small launches: the scan builds the chunk histograms itself (one launch
    // fewer; measured on MI355X: routing 10.6 vs 11.8 us at T = 512, 12.3 vs 13.6 at T = 1024)
    const bool fused = (int64_t)nchunks * E <= mm::kFusedHist;
    if (nchunks > 0 && !fused)
        hipLaunchKernelGGL(mm::route_hist_kernel, dim3(nchunks), dim3(mm::kRouteThreads), 0, s,
                           a.topk_idx, P, E, chunk, hist);
    const int cap = a.slot_capacity > 0 ? a.slot_capacity : (P > 0 ? P : 1);
    hipLaunchKernelGGL(mm::route_scan_kernel, dim3(1), dim3(mm::kScanThreads), 0, s,
                       fused ? a.topk_idx : nullptr, P, chunk, hist,
                       nchunks, E, cap, b.m_tile, b.L.max_items, a.intermediate / mm::kL1BlockH,
                       a.hidden / mm::kL2BlockN, at<int>(b, b.L.counts),
                       at<int>(b, b.L.offsets), at<int>(b, b.L.items), status);
    int nbits = 0;
    while ((1 << nbits) < E) ++nbits;
    if (nchunks > 0)
        hipLaunchKernelGGL(mm::route_scatter_kernel, dim3(nchunks), dim3(mm::kRouteThreads), 0,
                           s, a.topk_idx, P, E, nbits, chunk, hist, at<int>(b, b.L.counts),
                           at<int>(b, b.L.offsets), at<uint32_t>(b, b.L.perm),
                           at<int>(b, b.L.pair_pos));
    return launched(kOk);
}

mm::GemmParams gemm_params(const MegaLaunchArgs& a, const Bound& b) {
    mm::GemmParams p{};
    p.counts = at<int>(b, b.L.counts);
    p.offsets = at<int>(b, b.L.offsets);
    p.items = at<int>(b, b.L.items);
    p.status = at<int>(b, b.L.status);
    p.perm = at<uint32_t>(b, b.L.perm);
    p.H = a.hidden;
    p.I = a.intermediate;
    p.G = pairing_block(a.intermediate);
    p.topk = a.topk;
    p.ffn_ue8m0 = a.ffn_ue8m0;
    return p;
}

using GemmKernel = void (*)(mm::GemmParams);

// Compute units of the current device (the L2 walk runs one workgroup on each).
int cu_count() {
    static int cached[64] = {};
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return 256;
    if (!cached[dev]) {
        int n = 0;
        if (hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess ||
            n <= 0)
            n = 256;
        cached[dev] = n;
    }
    return cached[dev];
}

// Decode-shaped kernels (MT = 1, 2) for m_tile <= 32; above, the LDS-staged
// kernels on a 1-D grid of nb * max_items + 8 workgroups (the kernel maps
// workgroups to (item, block) units XCD by XCD and drops the surplus).
void launch_gemm(const GemmKernel (&small)[2], GemmKernel big, int m_tile, int nb,
                 int max_items, hipStream_t s, const mm::GemmParams& p) {
    if (m_tile <= 32) {
        hipLaunchKernelGGL(small[m_tile <= 16 ? 0 : 1], dim3(nb, max_items),
                           dim3(mm::kGemmThreads), 0, s, p);
    } else {
        hipLaunchKernelGGL(big, dim3(nb * max_items + 8), dim3(mm::kBigThreads), 0, s, p);
    }
}

const GemmKernel kL1Small[2] = {mm::l1_kernel<1>, mm::l1_kernel<2>};
const GemmKernel kL2Small[2] = {mm::l2_kernel<1>, mm::l2_kernel<2>};

int do_l1(const MegaLaunchArgs& a, hipStream_t s) {
    Bound b;
    int st = bind(a, b, true);
    if (st != kOk) return st;
    if (a.tokens == 0) return kOk;
    mm::GemmParams p = gemm_params(a, b);
    p.x = b.x;
    p.x_sf = b.x_sf;
    p.w = a.w1;
    p.w_sf = a.w1_sf;
    p.out8 = b.ws + b.L.ffn;
    p.out_sf = b.ws + b.L.ffn_sf;
    p.xcd_cuts = p.status + mm::kCutsL1;
    p.queue = at<int>(b, b.L.status) + mm::kQueueL1;
    p.tail_ord = reinterpret_cast<const uint8_t*>(p.status + mm::kTailOrdL1);
    const int nb = a.intermediate / mm::kL1BlockH;
    launch_gemm(kL1Small, a.mfma_fp8 ? mm::l1_big_f8_kernel : mm::l1_big_kernel, b.m_tile, nb,
                b.L.max_items, s, p);
    return launched(kOk);
}

int do_l2(const MegaLaunchArgs& a, hipStream_t s) {
    Bound b;
    int st = bind(a, b, true);
    if (st != kOk) return st;
    if (a.tokens == 0) return kOk;
    mm::GemmParams p = gemm_params(a, b);
    p.x = b.ws + b.L.ffn;
    p.x_sf = a.ffn_ue8m0 ? b.ws + b.L.ffn_sf : nullptr;
    p.w = a.w2;
    p.w_sf = a.w2_sf;
    p.out16 = at<uint16_t>(b, b.L.l2);
    p.xcd_cuts = p.status + mm::kCutsL2;
    p.queue = at<int>(b, b.L.status) + mm::kQueueL2;
    const int nb = a.hidden / mm::kL2BlockN;
    // The walk and the one-unit kernel back to back: the device picks one of
    // them from the routing of this launch (mm::walk_taken).  Tried for 17 to
    // 128 routed rows per expert on average: below, items of more than 32
    // rows are rare; above, items of at most 128 rows are (T = 8192); there
    // the empty launch would only cost time (~5 us for the walk's, ~7 us for
    // the one-unit kernel's, measured).
    // Measured on MI355X, walk on vs off: T = 2048 layer 1819-1820 vs
    // 1846-1847 us (L2 613 vs 645-646); Zipf(1.1) T = 2048 and T = 8192 even
    // (the one-unit kernel runs them).
    const int64_t pairs = (int64_t)a.tokens * a.topk;
    if (b.m_tile > 32 && !a.l2_no_walk && !a.mfma_fp8 && pairs > 16LL * a.num_experts &&
        pairs <= 128LL * a.num_experts) {
        p.walk = 1;
        // at least one workgroup per XCD range (workgroup L walks range L % 8)
        const int walkers = cu_count() < 8 ? 8 : cu_count();
        hipLaunchKernelGGL(mm::l2_walk_kernel, dim3(walkers), dim3(mm::kBigThreads), 0, s, p);
    }
    launch_gemm(kL2Small, a.mfma_fp8 ? mm::l2_big_f8_kernel : mm::l2_big_kernel, b.m_tile, nb,
                b.L.max_items, s, p);
    return launched(kOk);
}

// The reference's diagnostic switches, read at every launch as it reads them
// (src/megakernel.cu:137-139,255-258): MX_SKIP_COMBINE != 0 acts as
// skip_combine (launch_reduce does nothing), MX_SKIP_REDUCE != 0 makes
// launch_full skip its reduce (compute only).
bool env_on(const char* name) {
    const char* v = std::getenv(name);
    return v != nullptr && std::atoi(v) != 0;
}

int do_reduce(const MegaLaunchArgs& a, hipStream_t s) {
    Bound b;
    int st = bind(a, b, false);
    if (st != kOk) return st;
    // an empty batch writes nothing, so it needs no output (a (0, H) tensor
    // has a null data pointer)
    if (a.skip_combine || a.tokens == 0 || env_on("MX_SKIP_COMBINE")) return kOk;
    if (a.y == nullptr && a.y_bf16 == nullptr) return kErrNullPointer;
    // a token per workgroup (H / 8 threads, whole waves) up to 1024 threads
    const int threads = a.hidden / 8 <= 1024 ? (a.hidden / 8 + 63) / 64 * 64 : 256;
    const int per_block = threads * 8;
    const dim3 grid(a.tokens, (a.hidden + per_block - 1) / per_block);
    // The L2 rows stream past the caches once they are well over the 256 MiB
    // Infinity Cache; smaller ones are still cached from L2's stores.  Measured
    // on MI355X (combine us, cached vs streamed loads, streamed stores both):
    // T = 2048 (192 MiB of rows) 34.4 vs 37.0, T = 3072 52.2 vs 57.9,
    // T = 4096 86.6 vs 77.3, T = 8192 171.6 vs 155.5 (before: 34.8, 61.8,
    // 93, 183 with 256-thread blocks and cached stores).
    const bool stream_rows = 2LL * a.tokens * a.topk * a.hidden >= (384LL << 20);
    hipLaunchKernelGGL(stream_rows ? mm::combine_kernel<true> : mm::combine_kernel<false>, grid,
                       dim3(threads), 0, s, at<uint16_t>(b, b.L.l2), at<int>(b, b.L.pair_pos), b.w,
                       a.topk, a.hidden, a.y, a.y_bf16);
    return launched(kOk);
}

// L1 and L2 as one launch (fuse_l1l2): gemm_fused_kernel's first g1
// workgroups run the L1 units, the rest the L2 units, each L2 unit waiting on
// its item's ready counter (zeroed by the routing scan, or here when the
// routing is reused).
int do_l1_l2_fused(const MegaLaunchArgs& a, hipStream_t s) {
    Bound b;
    int st = bind(a, b, true);
    if (st != kOk) return st;
    if (a.tokens == 0) return kOk;
    int* ready = at<int>(b, b.L.items) + 4 * b.L.max_items;
    if (a.skip_prologue) {
        const int n = b.L.max_items;
        hipLaunchKernelGGL(mm::fill_int_kernel, dim3((n + 255) / 256), dim3(256), 0, s, ready, n,
                           0);
    }
    const int nb1 = a.intermediate / mm::kL1BlockH, nb2 = a.hidden / mm::kL2BlockN;
    mm::GemmParams p1 = gemm_params(a, b), p2 = gemm_params(a, b);
    p1.x = b.x;
    p1.x_sf = b.x_sf;
    p1.w = a.w1;
    p1.w_sf = a.w1_sf;
    p1.out8 = b.ws + b.L.ffn;
    p1.out_sf = b.ws + b.L.ffn_sf;
    p1.xcd_cuts = p1.status + mm::kCutsL1;
    p1.queue = at<int>(b, b.L.status) + mm::kQueueL1;
    p1.tail_ord = reinterpret_cast<const uint8_t*>(p1.status + mm::kTailOrdL1);
    p2.x = b.ws + b.L.ffn;
    p2.x_sf = a.ffn_ue8m0 ? b.ws + b.L.ffn_sf : nullptr;
    p2.w = a.w2;
    p2.w_sf = a.w2_sf;
    p2.out16 = at<uint16_t>(b, b.L.l2);
    p2.xcd_cuts = p2.status + mm::kCutsL2;
    p2.queue = at<int>(b, b.L.status) + mm::kQueueL2;
    for (mm::GemmParams* q : {&p1, &p2}) {
        q->ready = ready;
        q->ready_target = nb1 + (a.ready_bias > 0 ? a.ready_bias : 0);
        q->spin_limit = a.max_spins > 0 ? a.max_spins : mm::kReadySpinLimit;
        q->err = at<int>(b, b.L.status);
    }
    const int g1 = (nb1 * b.L.max_items + 8 + 7) & ~7, g2 = nb2 * b.L.max_items + 8;
    hipLaunchKernelGGL(mm::gemm_fused_kernel, dim3(g1 + g2), dim3(mm::kBigThreads), 0, s, p1, p2,
                       g1);
    return launched(kOk);
}

int do_compute(const MegaLaunchArgs& a, hipStream_t s) {
    int st = kOk;
    if (!a.skip_prologue) {
        st = do_prelude(a, s);
    } else {
        // routing reused from the previous launch; x is still folded
        Bound b;
        st = bind(a, b, false);
        if (st == kOk) fold_x(a, b, s);
    }
    if (a.fuse_l1l2 && st == kOk) {
        Bound b;
        st = bind(a, b, true);
        if (st == kOk && b.m_tile > 32) return do_l1_l2_fused(a, s);
    }
    if (st == kOk) st = do_l1(a, s);
    if (st == kOk) st = do_l2(a, s);
    return st;
}

int do_full(const MegaLaunchArgs& a, hipStream_t s) {
    int st = do_compute(a, s);
    if (st == kOk && !env_on("MX_SKIP_REDUCE")) st = do_reduce(a, s);
    return st;
}

int do_dispatch(const MegaLaunchArgs& a, uint8_t* pool, hipStream_t s) {
    Bound b;
    int st = bind(a, b, false);
    if (st != kOk) return st;
    if (pool == nullptr) return kErrNullPointer;
    const int P = a.tokens * a.topk;
    if (P == 0) return kOk;
    hipLaunchKernelGGL(mm::dispatch_gather_kernel, dim3(P), dim3(256), 0, s, b.x, a.hidden,
                       a.topk, at<uint32_t>(b, b.L.perm), at<int>(b, b.L.status), pool);
    return launched(kOk);
}

// ---- the allocation-free entry point's workspace --------------------------
// One fixed device array per GPU the library runs on, held until the process
// ends.  Host code never uses its name as an address (on the host it is a
// stand-in symbol): scratch_on_device() resolves the device address once per
// device with hipGetSymbolAddress, with that device current.
constexpr int64_t kScratchBytes = int64_t(64) << 20;
constexpr int kMaxDevices = 64;
static __device__ __align__(256) uint8_t scratch[kScratchBytes];

std::mutex g_scratch_mu;
uint8_t* g_scratch_ptr[kMaxDevices] = {};

// What the routing held in a device's scratch was built for: a skip_prologue
// call reuses it only with the same shape, since the workspace regions it
// reads (items, slots, XCD cuts) sit at offsets that move with these.
struct RouteKey {
    int valid, E, topk, H, I, max_tokens, win_cap, tokens;
    bool operator==(const RouteKey& o) const {
        return valid == o.valid && E == o.E && topk == o.topk && H == o.H && I == o.I &&
               max_tokens == o.max_tokens && win_cap == o.win_cap && tokens == o.tokens;
    }
};
RouteKey g_scratch_route[kMaxDevices] = {};

// Device address of `scratch` on the current device, or null (status in *st);
// *dev_out: the device.
uint8_t* scratch_on_device(int* st, int* dev_out) {
    int dev = -1;
    if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= kMaxDevices) {
        *st = kErrLaunch;
        return nullptr;
    }
    *dev_out = dev;
    std::lock_guard<std::mutex> lock(g_scratch_mu);
    if (g_scratch_ptr[dev] == nullptr) {
        void* ptr = nullptr;
        if (hipGetSymbolAddress(&ptr, HIP_SYMBOL(scratch)) != hipSuccess || ptr == nullptr) {
            *st = kErrLaunch;
            return nullptr;
        }
        g_scratch_ptr[dev] = static_cast<uint8_t*>(ptr);
    }
    *st = kOk;
    return g_scratch_ptr[dev];
}

// launch_full with the workspace taken from `scratch` instead of a.rwk (which
// is ignored, as is a.workspace_bytes).  The layout of a.max_tokens must fit
// kScratchBytes (kErrScratch otherwise).  Every region the kernels read is
// written earlier in the same launch (status, histograms, items, slots, the
// intermediate rows), so nothing needs clearing between calls.  With
// skip_prologue the routing of the previous routed call on this device is
// reused; the call is rejected (kErrUnsupported, before any launch) unless
// that call had the same E, topk, H, I, max_tokens, win_cap and tokens.
int do_full_noalloc(const MegaLaunchArgs& a, hipStream_t s) {
    const int st0 = check_dims(a.topk, a.num_experts, a.hidden, a.intermediate, a.win_cap);
    if (st0 != kOk) return st0;
    const int st1 = check_capacity(a.max_tokens, a.topk, a.hidden, a.intermediate, a.win_cap);
    if (st1 != kOk) return st1;
    const MegaLayout L =
        layout(a.max_tokens, a.topk, a.num_experts, a.hidden, a.intermediate, a.win_cap);
    if (L.total > kScratchBytes) return kErrScratch;
    int st = kOk, dev = 0;
    uint8_t* ws = scratch_on_device(&st, &dev);
    if (st != kOk) return st;
    const RouteKey key{1, a.num_experts, a.topk, a.hidden, a.intermediate, a.max_tokens,
                       a.win_cap, a.tokens};
    {
        std::lock_guard<std::mutex> lock(g_scratch_mu);
        if (a.skip_prologue) {
            if (!(g_scratch_route[dev] == key)) return kErrUnsupported;
        } else {
            g_scratch_route[dev] = RouteKey{};   // no usable routing until this call launched
        }
    }
    MegaLaunchArgs b = a;
    b.rwk = reinterpret_cast<rwk_data*>(ws);
    b.workspace_bytes = kScratchBytes;
    st = do_full(b, s);
    if (st == kOk && !a.skip_prologue) {
        std::lock_guard<std::mutex> lock(g_scratch_mu);
        g_scratch_route[dev] = key;
    }
    return st;
}

int record(int st) {
    g_last_error = st;
    if (st != kOk) std::fprintf(stderr, "[fp8mega] error %d\n", st);
    return st;
}

unsigned grid_for(size_t n, unsigned cap = 1u << 16) {
    size_t g = (n + 255) / 256;
    if (g < 1) g = 1;
    return (unsigned)(g > cap ? cap : g);
}

}  // namespace

MegaLayout layout(int max_tokens, int topk, int num_experts, int hidden, int intermediate,
                  int win_cap) {
    MegaLayout L{};
    const int64_t P = (int64_t)(max_tokens > 0 ? max_tokens : 1) * topk;
    const int64_t E = num_experts;
    L.max_pairs = (int)P;
    // room for the per-chunk histograms of any launch up to P pairs
    const int64_t ps = P < mm::kRouteSmallP ? P : mm::kRouteSmallP;
    const int64_t n_small = (ps + mm::kRouteChunkSmall - 1) / mm::kRouteChunkSmall;
    const int64_t n_large = (P + mm::kRouteChunkLarge - 1) / mm::kRouteChunkLarge;
    L.nchunks = (int)(n_small > n_large ? n_small : n_large);
    L.m_tile = win_cap > 0 ? win_cap : auto_m_tile(max_tokens, topk, num_experts);
    L.max_items = (int)((P + L.m_tile - 1) / L.m_tile + E);
    int64_t o = 0;
    L.status = o;      o = align256(o + mm::kStatusInts * 4);
    L.chunk_hist = o;  o = align256(o + (int64_t)L.nchunks * E * 4);
    L.counts = o;      o = align256(o + E * 4);
    L.offsets = o;     o = align256(o + (E + 1) * 4);
    L.items = o;       o = align256(o + (int64_t)L.max_items * 20);   // + ready counters
    L.perm = o;        o = align256(o + P * 4);
    L.pair_pos = o;    o = align256(o + P * 4);
    L.xq = o;          o = align256(o + (int64_t)max_tokens * hidden);
    L.xq_sf = o;       o = align256(o + (int64_t)max_tokens * (hidden / 128));
    L.ffn = o;         o = align256(o + P * intermediate);
    L.ffn_sf = o;      o = align256(o + P * (intermediate / 128));
    L.l2 = o;          o = align256(o + P * hidden * 2);
    L.total = o;
    return L;
}

void launch_prelude(const MegaLaunchArgs& a, hipStream_t s) { record(do_prelude(a, s)); }
void launch_compute(const MegaLaunchArgs& a, hipStream_t s) { record(do_compute(a, s)); }
void launch_l1(const MegaLaunchArgs& a, hipStream_t s) { record(do_l1(a, s)); }
void launch_l2(const MegaLaunchArgs& a, hipStream_t s) { record(do_l2(a, s)); }
void launch_reduce(const MegaLaunchArgs& a, hipStream_t s) { record(do_reduce(a, s)); }
void launch_full(const MegaLaunchArgs& a, hipStream_t s) { record(do_full(a, s)); }
void launch_dispatch(const MegaLaunchArgs& a, uint8_t* pool, hipStream_t s) {
    record(do_dispatch(a, pool, s));
}

void launch_empty(int grid, int threads, int64_t smem, hipStream_t s) {
    hipLaunchKernelGGL(mm::empty_kernel, dim3(grid > 0 ? grid : 1),
                       dim3(threads > 0 ? threads : 64), (unsigned)smem, s);
    record(launched(kOk));
}

void fill_weights_lane(uint8_t* w, int n_rows, int k_cols, uint32_t seed, hipStream_t s) {
    if (w == nullptr) { record(kErrNullPointer); return; }
    if (n_rows <= 0 || n_rows % 16 || k_cols <= 0 || k_cols % 128) { record(kErrBadDims); return; }
    const size_t slots = (size_t)(n_rows / 16) * (k_cols / 128) * 128;
    hipLaunchKernelGGL(mm::fill_w_lane_kernel, dim3(grid_for(slots)), dim3(256), 0, s, w, n_rows,
                       k_cols, seed);
    record(launched(kOk));
}

void pack_weights(uint8_t* dst, const uint8_t* src, int n_mats, int n_rows, int k_cols,
                  hipStream_t s) {
    if (!dst || !src) { record(kErrNullPointer); return; }
    if (n_mats <= 0 || n_rows <= 0 || n_rows % 16 || k_cols <= 0 || k_cols % 128) {
        record(kErrBadDims);
        return;
    }
    const size_t slots = (size_t)n_mats * (n_rows / 16) * (k_cols / 128) * 128;
    hipLaunchKernelGGL(mm::pack_weights_kernel, dim3(grid_for(slots)), dim3(256), 0, s, dst, src,
                       n_mats, n_rows, k_cols);
    record(launched(kOk));
}

void pack_weights_from_reference(uint8_t* dst, const uint8_t* src, int n_mats, int n_rows,
                                 int k_cols, hipStream_t s) {
    if (!dst || !src) { record(kErrNullPointer); return; }
    if (n_mats <= 0 || n_rows <= 0 || n_rows % 32 || k_cols <= 0 || k_cols % 128) {
        record(kErrBadDims);
        return;
    }
    const size_t slots = (size_t)n_mats * (n_rows / 16) * (k_cols / 128) * 128;
    hipLaunchKernelGGL(mm::pack_weights_ref_kernel, dim3(grid_for(slots)), dim3(256), 0, s, dst,
                       src, n_mats, n_rows, k_cols);
    record(launched(kOk));
}

void fill_weights_normal(uint8_t* w, uint8_t* w_sf, int n_mats, int n_rows, int k_cols,
                         uint64_t seed, float sigma, hipStream_t s) {
    if (!w || !w_sf) { record(kErrNullPointer); return; }
    if (n_mats <= 0 || n_rows <= 0 || n_rows % 128 || k_cols <= 0 || k_cols % 128 ||
        n_mats > 65535 || n_rows / 128 > 65535) {
        record(kErrBadDims);
        return;
    }
    hipLaunchKernelGGL(mm::fill_weights_normal_kernel, dim3(k_cols / 128, n_rows / 128, n_mats),
                       dim3(256), 0, s, w, w_sf, n_rows, k_cols, seed, sigma);
    record(launched(kOk));
}

void quant_act(const uint16_t* x, int rows, int cols, uint8_t* q, uint8_t* sf, hipStream_t s) {
    if (!x || !q) { record(kErrNullPointer); return; }
    if (rows < 0 || cols <= 0 || cols % 128) { record(kErrBadDims); return; }
    const size_t n8 = (size_t)rows * cols / 8;
    if (n8 > 0)
        hipLaunchKernelGGL(mm::quant_act_kernel, dim3((unsigned)((n8 + 255) / 256)), dim3(256), 0,
                           s, x, rows, cols, q, sf);
    record(launched(kOk));
}

static void print_attr(const char* name, const void* fn) {
    hipFuncAttributes at{};
    if (hipFuncGetAttributes(&at, fn) != hipSuccess) {
        std::printf("[resources] %-26s (unavailable)\n", name);
        return;
    }
    std::printf("[resources] %-26s regs=%3d lds=%6zu B scratch=%5zu B max_threads=%d\n", name,
                at.numRegs, at.sharedSizeBytes, at.localSizeBytes, at.maxThreadsPerBlock);
}

void dump_kernel_resources() {
    print_attr("route_hist", (const void*)mm::route_hist_kernel);
    print_attr("route_scan", (const void*)mm::route_scan_kernel);
    print_attr("route_scatter", (const void*)mm::route_scatter_kernel);
    print_attr("l1_kernel<1>", (const void*)mm::l1_kernel<1>);
    print_attr("l1_kernel<2>", (const void*)mm::l1_kernel<2>);
    print_attr("l1_big_kernel", (const void*)mm::l1_big_kernel);
    print_attr("l2_kernel<1>", (const void*)mm::l2_kernel<1>);
    print_attr("l2_kernel<2>", (const void*)mm::l2_kernel<2>);
    print_attr("l2_big_kernel", (const void*)mm::l2_big_kernel);
    print_attr("l1_big_f8_kernel", (const void*)mm::l1_big_f8_kernel);
    print_attr("l2_big_f8_kernel", (const void*)mm::l2_big_f8_kernel);
    print_attr("l2_walk_kernel", (const void*)mm::l2_walk_kernel);
    print_attr("gemm_fused_kernel", (const void*)mm::gemm_fused_kernel);
    print_attr("combine<cached rows>", (const void*)mm::combine_kernel<false>);
    print_attr("combine<streamed rows>", (const void*)mm::combine_kernel<true>);
    std::fflush(stdout);
}

int last_error() { return g_last_error; }

int read_status(const MegaLaunchArgs& a, int32_t* out, int n, hipStream_t s) {
    if (out == nullptr) return record(kErrNullPointer);
    if (n < 1 || n > mm::kStatusWords) return record(kErrBadDims);
    Bound b;
    int st = bind(a, b, false);
    if (st != kOk) return record(st);
    if (hipMemcpyAsync(out, b.ws + b.L.status, sizeof(int32_t) * (size_t)n, hipMemcpyDeviceToHost,
                       s) != hipSuccess ||
        hipStreamSynchronize(s) != hipSuccess)
        return record(kErrLaunch);
    return record(out[0] != 0 ? kErrDevice : kOk);
}

}  // namespace fp8mega

// ------------------------------------------------------------------ C ABI --
using fp8mega::MegaLaunchArgs;

extern "C" {

int mm_abi_version(void) { return 4; }

long long mm_noalloc_scratch_bytes(void) { return (long long)fp8mega::kScratchBytes; }

size_t mm_args_size(void) { return sizeof(MegaLaunchArgs); }

long long mm_args_offset(const char* f) {
#define MM_FIELD(n) if (std::strcmp(f, #n) == 0) return (long long)offsetof(MegaLaunchArgs, n);
    MM_FIELD(R) MM_FIELD(rank) MM_FIELD(tokens) MM_FIELD(slot_capacity) MM_FIELD(win_cap)
    MM_FIELD(grid) MM_FIELD(threads) MM_FIELD(smem) MM_FIELD(rwk) MM_FIELD(unk)
    MM_FIELD(unk_peers) MM_FIELD(self) MM_FIELD(peer_bases) MM_FIELD(topk_idx) MM_FIELD(w1)
    MM_FIELD(w2) MM_FIELD(group_weights_ready) MM_FIELD(topk_idx_off) MM_FIELD(x_off)
    MM_FIELD(weights_off) MM_FIELD(in_bf16) MM_FIELD(skip_combine) MM_FIELD(y)
    MM_FIELD(max_spins) MM_FIELD(skip_prologue) MM_FIELD(num_experts) MM_FIELD(topk)
    MM_FIELD(hidden) MM_FIELD(intermediate) MM_FIELD(max_tokens) MM_FIELD(workspace_bytes)
    MM_FIELD(x_sf) MM_FIELD(w1_sf) MM_FIELD(w2_sf) MM_FIELD(ffn_ue8m0) MM_FIELD(y_bf16)
    MM_FIELD(fuse_l1l2)
    MM_FIELD(l2_no_walk) MM_FIELD(ready_bias) MM_FIELD(mfma_fp8)
#undef MM_FIELD
    return -1;
}

int mm_layout(int max_tokens, int topk, int num_experts, int hidden, int intermediate,
              int win_cap, fp8mega::MegaLayout* out) {
    if (!out) return fp8mega::kErrNullPointer;
    const int st = fp8mega::check_dims(topk, num_experts, hidden, intermediate, win_cap);
    if (st != fp8mega::kOk) return st;
    const int cst = fp8mega::check_capacity(max_tokens, topk, hidden, intermediate, win_cap);
    if (cst != fp8mega::kOk) return cst;
    *out = fp8mega::layout(max_tokens, topk, num_experts, hidden, intermediate, win_cap);
    return fp8mega::kOk;
}

#define MM_WRAP(name, call)                                           \
    int name(const MegaLaunchArgs* a, void* stream) {                 \
        if (!a) return fp8mega::kErrNullPointer;                       \
        return fp8mega::record(call(*a, (hipStream_t)stream));         \
    }
MM_WRAP(mm_launch_prelude, fp8mega::do_prelude)
MM_WRAP(mm_launch_compute, fp8mega::do_compute)
MM_WRAP(mm_launch_l1, fp8mega::do_l1)
MM_WRAP(mm_launch_l2, fp8mega::do_l2)
MM_WRAP(mm_launch_reduce, fp8mega::do_reduce)
MM_WRAP(mm_launch_full, fp8mega::do_full)
MM_WRAP(mm_launch_full_noalloc, fp8mega::do_full_noalloc)
#undef MM_WRAP

int mm_launch_dispatch(const MegaLaunchArgs* a, uint8_t* pool, void* stream) {
    if (!a) return fp8mega::kErrNullPointer;
    return fp8mega::record(fp8mega::do_dispatch(*a, pool, (hipStream_t)stream));
}

int mm_read_status(const MegaLaunchArgs* a, int* out, int n, void* stream) {
    if (!a) return fp8mega::kErrNullPointer;
    return fp8mega::read_status(*a, out, n, (hipStream_t)stream);
}

int mm_launch_empty(int grid, int threads, long long smem, void* stream) {
    fp8mega::launch_empty(grid, threads, smem, (hipStream_t)stream);
    return fp8mega::last_error();
}

int mm_fill_weights_lane(uint8_t* w, int n_rows, int k_cols, unsigned seed, void* stream) {
    fp8mega::fill_weights_lane(w, n_rows, k_cols, seed, (hipStream_t)stream);
    return fp8mega::last_error();
}

int mm_pack_weights(uint8_t* dst, const uint8_t* src, int n_mats, int n_rows, int k_cols,
                    void* stream) {
    fp8mega::pack_weights(dst, src, n_mats, n_rows, k_cols, (hipStream_t)stream);
    return fp8mega::last_error();
}

int mm_pack_weights_from_reference(uint8_t* dst, const uint8_t* src, int n_mats, int n_rows,
                                   int k_cols, void* stream) {
    fp8mega::pack_weights_from_reference(dst, src, n_mats, n_rows, k_cols, (hipStream_t)stream);
    return fp8mega::last_error();
}

int mm_fill_weights_normal(uint8_t* w, uint8_t* w_sf, int n_mats, int n_rows, int k_cols,
                           unsigned long long seed, float sigma, void* stream) {
    fp8mega::fill_weights_normal(w, w_sf, n_mats, n_rows, k_cols, seed, sigma,
                                 (hipStream_t)stream);
    return fp8mega::last_error();
}

int mm_quant_act(const uint16_t* x, int rows, int cols, uint8_t* q, uint8_t* sf, void* stream) {
    fp8mega::quant_act(x, rows, cols, q, sf, (hipStream_t)stream);
    return fp8mega::last_error();
}

int mm_selftest_convert(const float* in, int n, uint8_t* out8, uint16_t* out16, void* stream) {
    if (!in) return fp8mega::kErrNullPointer;
    if (n <= 0) return fp8mega::kOk;
    hipLaunchKernelGGL(mm::convert_selftest_kernel, dim3((n + 255) / 256), dim3(256), 0,
                       (hipStream_t)stream, in, n, out8, out16);
    return fp8mega::record(fp8mega::launched(fp8mega::kOk));
}

void mm_dump_kernel_resources(void) { fp8mega::dump_kernel_resources(); }

}  // extern "C"
