// ============================================================================
// megakernel.h -- host C++ API of the MI355X (gfx950) fused FP8xFP8 MoE layer.
//
// Drop-in for the reference's public header src/megakernel.h:18-139
// (namespace fp8mega, POD MegaLaunchArgs, launch_prelude / launch_compute /
// launch_reduce / launch_full / launch_empty / fill_weights_lane /
// dump_kernel_resources).  Differences a caller sees:
//   * streams are hipStream_t (reference: mcStream_t);
//   * one GPU holds all experts: R = 1, rank = 0, the peer/IPC fields are
//     accepted and ignored;
//   * MegaLaunchArgs is extended append-only with the layer dimensions, the
//     optional UE8M0 scale tensors, a bf16 output and the workspace size;
//   * weights are in this library's MFMA tile layout (fp8mega::pack_weights
//     converts from logical row-major, fill_weights_lane generates directly);
//   * errors: the C++ entry points keep the reference's void signatures and
//     record a status readable through fp8mega::last_error(); the extern "C"
//     mm_* layer below returns that status directly.
//
// All launch entry points are asynchronous and stream-ordered, never allocate,
// never synchronise and are safe under hipGraph capture.  The caller owns all
// memory: inputs, weights, outputs and the workspace (size: workspace_bytes).
// ============================================================================
#pragma once

#include <cstddef>
#include <cstdint>

#include <hip/hip_runtime_api.h>

// Opaque device workspace types (reference: src/megakernel.h:27-32 forward
// declares local_flags/ranks_flags/local_data/ranks_data/rwk_data/unk_data).
// Here rwk_data is the single caller-owned workspace laid out by
// fp8mega::layout(); unk_data is kept only so the field types match.
struct rwk_data;
struct unk_data;

// Deterministic weight byte used by fill_weights_lane (reference:
// src/megakernel.h:46-47, WPROBE = 0 form), on the logical row order.
#define WPROBE_VAL(seed, row, k) \
    ((uint8_t)(((seed) + (row) * 131 + (k) * 7) & 0x3f))

namespace fp8mega {

// Error codes (also returned by the extern "C" layer).
enum MegaStatus : int {
    kOk = 0,
    kErrNullPointer = 1,    // a required pointer is null
    kErrBadDims = 2,        // dims not supported (H, I multiples of 128, ...)
    kErrWorkspace = 3,      // workspace missing or smaller than layout().total
    kErrTooManyTokens = 4,  // tokens > max_tokens the workspace was laid out for
    kErrLaunch = 5,         // hipLaunchKernel failed
    kErrUnsupported = 6,    // option not supported by this build
    kErrDevice = 7,         // read_status: the device status word reports an error
    kErrScratch = 8,        // mm_launch_full_noalloc: layout larger than its scratch
};

// Device status words: the workspace region MegaLayout::status, rewritten by
// the routing of every launch (launch_prelude / launch_compute / launch_full
// without skip_prologue) and readable after it with read_status():
//   [0]  error bits (kStatusItemOverflow: the work-item table overflowed; the
//        GEMMs then skip the experts past it -- the layout's bound makes this
//        unreachable, the bit guards the kernels' assumption; kStatusWaitTimeout:
//        with fuse_l1l2, an L2 unit stopped waiting after max_spins polls)
//   [1]  work items, [2] routed slots,
//   [3]  pairs dropped by slot_capacity,
//   [4]  pairs whose expert id is outside [0, num_experts) (dropped)
//   [5]  rows of the largest work item (the L2 walk runs when 33..128)
//   [16..24], [32..40] the big GEMMs' XCD unit ranges (L1, L2)
// (read_status returns these 64 words; the region's next 256 bytes hold the
// L1 tail queues' ticket order, also written by the routing)
// The reference returns no status (src/megakernel.h:117-130): its launches
// are void and its host CHECKs exit (src/host_layout.cuh:18-26).
enum MegaDeviceStatus : int {
    kStatusItemOverflow = 1,
    kStatusWaitTimeout = 2,   // fuse_l1l2: an L2 unit gave up waiting for its item's L1 units
};

// One launch's host arguments (reference: src/megakernel.h:54-114; fields
// [1]..[5] keep the reference's names and order, [6] is appended).
struct MegaLaunchArgs {
    // [1] grid planning
    int R = 1, rank = 0;         // single GPU: R = 1, rank = 0
    int tokens = 0;              // tokens in this launch
    int slot_capacity = 0;       // per-expert slot cap; 0 = no cap (tokens*topk)
    int win_cap = 0;             // max rows per work item: 0 (auto), 16, 32, 64, 128, 256
    int grid = 0, threads = 0;   // informational (filled by make_args)
    int64_t smem = 0;

    // [2] pointers, offsets
    rwk_data* rwk = nullptr;               // caller-owned workspace (layout())
    unk_data* unk = nullptr;               // unused (multi-rank only)
    unk_data* const* unk_peers = nullptr;  // unused (multi-rank only)
    const uint8_t* self = nullptr;         // base of x / topk_weights views
    uint8_t* const* peer_bases = nullptr;  // unused (multi-rank only)
    const int64_t* topk_idx = nullptr;     // [tokens][topk] int64
    const uint8_t* w1 = nullptr;           // [E][2I][H] fp8 e4m3, tile layout
    const uint8_t* w2 = nullptr;           // [E][H][I]  fp8 e4m3, tile layout
    int group_weights_ready = 0;           // unused (multi-rank only)
    int64_t topk_idx_off = 0;              // unused (topk_idx is a pointer)
    int64_t x_off = 0, weights_off = 0;    // x = self + x_off, w = self + weights_off
    int in_bf16 = 0;                       // x is bf16 [tokens][H] (folded to fp8)
    int skip_combine = 0;                  // diagnostic: launch_reduce does nothing
                                           // (also while MX_SKIP_COMBINE != 0)

    // [3] output
    float* y = nullptr;                    // [tokens][H] fp32 (may be null if y_bf16)

    // [4] tuning
    int max_spins = 0;                     // fuse_l1l2: polls per L1 -> L2 wait (0: ~1 s);
                                           // no cross-rank waits on one GPU
    int skip_prologue = 0;                 // >0: reuse routing of the previous launch

    // [5] debug: none

    // [6] appended: layer dims, block scales, bf16 output, workspace size
    int num_experts = 256;
    int topk = 8;
    int hidden = 6144;                     // H
    int intermediate = 2048;               // I
    int max_tokens = 0;                    // tokens the workspace was laid out for; with
                                           // topk, H, I: max_tokens*H <= 2^32 and
                                           // max_tokens*topk*I <= 2^32 (kErrBadDims)
    int64_t workspace_bytes = 0;           // size of *rwk
    const uint8_t* x_sf = nullptr;         // [tokens][H/128] UE8M0 bytes, null = 2^0
    const uint8_t* w1_sf = nullptr;        // [E][2I/128][H/128] UE8M0, null = 2^0
    const uint8_t* w2_sf = nullptr;        // [E][H/128][I/128]  UE8M0, null = 2^0
    int ffn_ue8m0 = 0;                     // L1 output requant: per-128 UE8M0 (1) or raw (0);
                                           // must be 1 exactly when scales are given
    uint16_t* y_bf16 = nullptr;            // [tokens][H] bf16 (may be null if y)
    int fuse_l1l2 = 0;                     // 1: L1 and L2 in one launch, L2 units starting on
                                           // an item once its L1 units are done (per-item
                                           // ready counters; reference src/compute_big.cuh:
                                           // 1948-1997).  Windows > 32 rows; max_spins > 0
                                           // bounds each wait (else ~1 s).
    int l2_no_walk = 0;                    // 1: L2 always one unit per workgroup; 0: when the
                                           // largest work item has 3-8 token tiles (tried
                                           // for 17-128 routed rows per expert on average),
                                           // one workgroup per CU walks the units, streaming
                                           // the next unit's weights during the current one
    int ready_bias = 0;                    // test hook (fuse_l1l2): added to the count of L1
                                           // blocks an L2 unit waits for; > 0 makes every
                                           // wait give up after max_spins polls, so a test
                                           // drives the bounded wait's timeout report
    int mfma_fp8 = 0;                      // 1: both GEMMs on gfx950's block-scaled fp8 MFMA
                                           // (v_mfma_scale_f32_16x16x128_f8f6f4, the
                                           // reference's fp8 MMA class) instead of the bf16
                                           // MFMA after an exact conversion.  Faster at large
                                           // T; its truncating sums put the layer outside
                                           // the end-to-end bar the default meets (within
                                           // check.cu's staged tolerances).  Windows > 32
                                           // rows, two launches (not with fuse_l1l2):
                                           // kErrUnsupported otherwise.
};

// Byte offsets of every region inside the workspace (the single-GPU
// counterpart of mt::make_geo / compute_layout, test/mega_common.cuh:69-88,
// src/host_layout.cuh:59-100).  All offsets are 256-byte aligned.
struct MegaLayout {
    int64_t status;        // int32[128]: [0] status word, [1] items, [2] slots,
                           // [16..24] / [32..40] XCD unit ranges of the L1 / L2 GEMMs;
                           // bytes [256..512): L1's tail-queue ticket order [8][32]
    int64_t chunk_hist;    // int32[nchunks][E] per-chunk histograms -> prefixes
    int64_t counts;        // int32[E]   per-expert routed rows (after cap)
    int64_t offsets;       // int32[E+1] exclusive prefix of counts
    int64_t items;         // int32[max_items][4] (expert, first slot, end slot, j | n << 16) work
                           // items, then int32[max_items] per-item L1 ready counters (fuse_l1l2)
    int64_t perm;          // uint32[P]  pair index per slot (canonical order)
    int64_t pair_pos;      // int32[P]   slot per pair or -1
    int64_t xq;            // uint8[max_tokens][H]     folded fp8 x (in_bf16)
    int64_t xq_sf;         // uint8[max_tokens][H/128] folded x scales
    int64_t ffn;           // uint8[P][I]   L1 output (fp8, slot order)
    int64_t ffn_sf;        // uint8[P][I/128] L1 output scales
    int64_t l2;            // uint16[P][H]  L2 output (bf16, slot order)
    int64_t total;         // bytes
    int nchunks;           // routing chunk histograms held (256 pairs each up to 8192 pairs, 1024 above)
    int max_items;         // upper bound on work items for the chosen M tile
    int max_pairs;         // P = max_tokens * topk
    int m_tile;            // rows per work item
};

// Workspace layout for a launch shape (max_tokens bounds every launch that
// uses this workspace).  win_cap = rows per work item (0 = auto).
MegaLayout layout(int max_tokens, int topk, int num_experts, int hidden,
                  int intermediate, int win_cap);

// Routing only: per-expert counts, offsets, canonical permutation, pair slots,
// work items (reference: launch_prelude, src/megakernel.h:117).
void launch_prelude(const MegaLaunchArgs& a, hipStream_t stream);
// Routing (unless skip_prologue) + L1 GEMM/SwiGLU + L2 GEMM, no reduce
// (reference: launch_compute, src/megakernel.h:119).
void launch_compute(const MegaLaunchArgs& a, hipStream_t stream);
// Stage entry points (reference: launch_l1 / launch_l2, src/megakernel.h:123-126,
// compiled there under CM_L1L2_SPLIT).  Both need launch_prelude first.
void launch_l1(const MegaLaunchArgs& a, hipStream_t stream);
void launch_l2(const MegaLaunchArgs& a, hipStream_t stream);
// Top-k weighted reduce into y / y_bf16 (reference: launch_reduce, :128).
// Does nothing while the environment has MX_SKIP_COMBINE != 0 (read at each
// launch, as the reference reads it: src/megakernel.cu:137-139).
void launch_reduce(const MegaLaunchArgs& a, hipStream_t stream);
// launch_compute + launch_reduce on one stream (reference: launch_full, :130).
// While MX_SKIP_REDUCE != 0, launch_compute only (src/megakernel.cu:255-258).
void launch_full(const MegaLaunchArgs& a, hipStream_t stream);
// Empty kernel (launch floor; reference: launch_empty, :132).
void launch_empty(int grid, int threads, int64_t smem, hipStream_t stream);
// Device-side deterministic weights WPROBE_VAL(seed, row, k) over a logical
// n_rows x k_cols matrix, written in this library's tile layout (reference:
// fill_weights_lane, src/megakernel.h:134; its own lane layout differs).
void fill_weights_lane(uint8_t* w, int n_rows, int k_cols, uint32_t seed,
                       hipStream_t stream);
// Print register / LDS / scratch use of every kernel (reference:
// dump_kernel_resources, src/megakernel.h:137).
void dump_kernel_resources();
// Status of the last call made by this host thread (kOk when it succeeded).
int last_error();
// Copies the first n (1..64) device status words of the workspace a.rwk into
// host memory `out` once the work queued on `stream` has finished: it
// synchronises `stream`, so it is not for use under graph capture.  Returns
// kOk, kErrDevice when out[0] (the error bits) is non-zero, or an argument
// error (no reference counterpart; the single-GPU form of the device error
// word a caller reads after sync).
int read_status(const MegaLaunchArgs& a, int32_t* out, int n, hipStream_t stream);

// ---- layout / data-preparation helpers (no reference counterpart in the
// ---- C++ header; the reference does these in torch/mxmegakernel/mega/__init__.py)
// Logical row-major [n_mats][n_rows][k_cols] fp8 -> tile layout.
void pack_weights(uint8_t* dst, const uint8_t* src, int n_mats, int n_rows,
                  int k_cols, hipStream_t stream);
// The reference's packed on-device weights (lane-tile layout: fill_w_lane
// bytes, src/megakernel.cu:66-105, closed form src/bench_check.cuh:268-272;
// the output of its transform_weights_for_mega_moe,
// torch/mxmegakernel/mega/__init__.py:553-573) -> tile layout.  The logical
// row order is kept (W1 rows stay gate/up paired).  n_rows % 32 == 0,
// k_cols % 128 == 0.
void pack_weights_from_reference(uint8_t* dst, const uint8_t* src, int n_mats,
                                 int n_rows, int k_cols, hipStream_t stream);
// Synthetic N(0, sigma) weights quantised with 128x128 UE8M0 block scales,
// written in tile layout + scales [n_mats][n_rows/128][k_cols/128].
void fill_weights_normal(uint8_t* w, uint8_t* w_sf, int n_mats, int n_rows,
                         int k_cols, uint64_t seed, float sigma,
                         hipStream_t stream);
// bf16 [rows][cols] -> fp8 e4m3 [rows][cols] (+ per-128 UE8M0 scales when
// sf != null, else a direct RNE saturating cast).
void quant_act(const uint16_t* x_bf16, int rows, int cols, uint8_t* q,
               uint8_t* sf, hipStream_t stream);
// Copies routed fp8 x rows into slot order: pool[slot][H] = x[perm[slot]/topk]
// (the reference DISPATCH pool, src/compute_big.cuh:1691-1946; the hot path
// gathers these rows directly inside L1 instead).
void launch_dispatch(const MegaLaunchArgs& a, uint8_t* pool, hipStream_t stream);

}  // namespace fp8mega

// ============================================================================
// Thin C ABI (for ctypes / FFI).  Every function returns a MegaStatus code.
// `stream` is a hipStream_t passed as void*.  The MegaLaunchArgs pointer is
// the POD above; mm_args_size()/mm_args_offset() let a binding check its own
// mirror of the struct.
// ============================================================================
extern "C" {
int mm_abi_version(void);
size_t mm_args_size(void);
// Offset of a MegaLaunchArgs field by name, or -1 if unknown.
long long mm_args_offset(const char* field);
// Writes layout(...) into *out; returns status (kErrBadDims for unsupported
// dims or a capacity past the 32-bit activation row offsets, see max_tokens).
int mm_layout(int max_tokens, int topk, int num_experts, int hidden,
              int intermediate, int win_cap, fp8mega::MegaLayout* out);
int mm_launch_prelude(const fp8mega::MegaLaunchArgs* a, void* stream);
int mm_launch_compute(const fp8mega::MegaLaunchArgs* a, void* stream);
int mm_launch_l1(const fp8mega::MegaLaunchArgs* a, void* stream);
int mm_launch_l2(const fp8mega::MegaLaunchArgs* a, void* stream);
int mm_launch_reduce(const fp8mega::MegaLaunchArgs* a, void* stream);
int mm_launch_full(const fp8mega::MegaLaunchArgs* a, void* stream);
// launch_full for callers that cannot allocate (code under graph capture,
// tight serving loops, harnesses that forbid hipMalloc).  No reference
// counterpart.  The workspace is a fixed device array inside the library
// (mm_noalloc_scratch_bytes() bytes, 64 MiB, one per GPU, held until the
// process ends) instead of a->rwk, which is ignored with workspace_bytes:
// the layout of a->max_tokens must fit it (kErrScratch otherwise; e.g. up to
// ~550 tokens at E=256, top-8, H=6144, I=2048).  The caller still passes the
// inputs and outputs.  The call allocates nothing.  Every call on one GPU
// shares that array: calls that overlap on one GPU (other streams, other
// threads) race.  skip_prologue reuses the routing of the previous routed
// call on this GPU, and is rejected with kErrUnsupported (before any launch)
// unless that call had the same num_experts, topk, hidden, intermediate,
// max_tokens, win_cap and tokens.
int mm_launch_full_noalloc(const fp8mega::MegaLaunchArgs* a, void* stream);
long long mm_noalloc_scratch_bytes(void);
int mm_launch_empty(int grid, int threads, long long smem, void* stream);
int mm_launch_dispatch(const fp8mega::MegaLaunchArgs* a, uint8_t* pool, void* stream);
// fp8mega::read_status (synchronises `stream`).
int mm_read_status(const fp8mega::MegaLaunchArgs* a, int* out, int n, void* stream);
int mm_fill_weights_lane(uint8_t* w, int n_rows, int k_cols, unsigned seed,
                         void* stream);
int mm_pack_weights(uint8_t* dst, const uint8_t* src, int n_mats, int n_rows,
                    int k_cols, void* stream);
int mm_pack_weights_from_reference(uint8_t* dst, const uint8_t* src, int n_mats,
                                   int n_rows, int k_cols, void* stream);
int mm_fill_weights_normal(uint8_t* w, uint8_t* w_sf, int n_mats, int n_rows,
                           int k_cols, unsigned long long seed, float sigma,
                           void* stream);
int mm_quant_act(const uint16_t* x_bf16, int rows, int cols, uint8_t* q,
                 uint8_t* sf, void* stream);
// Element-wise fp32 -> e4m3 / bf16 conversion with the device conversion the
// kernels use (self-test of the rounding; out8/out16 may be null).
int mm_selftest_convert(const float* in, int n, uint8_t* out8, uint16_t* out16,
                        void* stream);
void mm_dump_kernel_resources(void);

// ---- measurement probes (no reference counterpart; nothing on the layer's
// ---- path calls them; they back the numeric design and the measured peaks)
// out[r][n] = sum_k a[r][k] * b[n][k] for 16 rows, fp8 e4m3 operands
// ([16][K] and [N][K] row-major, K % 128 == 0, N % 16 == 0): mode 0 on the
// 16x16x128 fp8 MFMA, mode 1 on the bf16 MFMA after the exact conversion.
int mm_probe_mfma_dot(const uint8_t* a, const uint8_t* b, int K, int N, int mode, float* out,
                      void* stream);
// The layer's L2 recomputed over routed slots, out[s][n] fp32 ([P][H]):
// groups holds ngroups int4 {expert, first slot, end slot, 0} of at most 16
// slots each (an empty group writes nothing); ffn [P][I] + ffn_sf [P][I/128] as L1 writes them, w2 logical
// row-major [E][H][I] + w2_sf [E][H/128][I/128].  mode 0: the 16x16x128 fp8
// MFMA with the UE8M0 bytes as its scale operands; mode 1: the bf16 MFMA
// after the exact conversion, in the L2 GEMM's operand roles and k order.
int mm_probe_l2_rows(const uint8_t* ffn, const uint8_t* ffn_sf, const uint8_t* w2,
                     const uint8_t* w2_sf, const int* groups, int ngroups, int H, int I, int mode,
                     float* out, void* stream);
// Reads `bytes` once with non-temporal 16-byte loads, each of the grid
// workgroups (256 threads) one contiguous bytes / grid chunk; bytes must be a
// multiple of grid * 32 KiB.  sink holds grid * 256 words.
int mm_probe_stream_read(const uint8_t* src, unsigned long long bytes, uint32_t* sink,
                         int grid, void* stream);
// grid workgroups of 4 waves, each running iters x 8 independent MFMAs
// (mode 0: 16x16x32 bf16, mode 1: 16x16x128 fp8); sink holds grid * 4 floats.
int mm_probe_mfma_rate(int mode, int iters, int grid, float* sink, void* stream);
}
