// mm_device.h -- device helpers shared by the gfx950 kernels of the fused
// FP8xFP8 MoE layer: tile layout addressing, fp8 / bf16 / UE8M0 conversions
// and the MFMA wrapper.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace mm {

// ---------------------------------------------------------------------------
// Weight tile layout (this library's own format).
//
// A logical matrix W[n_rows][k_cols] (n = output channel, k = reduction) is
// stored as tiles of 16 rows x 128 k = 2048 bytes, tile (nt, kt) at byte
// (nt * (k_cols/128) + kt) * 2048.  Inside a tile, byte (r, k) (r < 16,
// k < 128) sits at
//     ((k % 32) / 16) * 1024 + (r + 16 * (k / 32)) * 16 + (k % 16)
// so that a wave loading 16 bytes per lane at lane*16 (+1024) reads 1 KiB
// contiguous, and lane L ends up holding row L%16, k in [32*(L/16), +32):
// after an exact fp8 -> bf16 conversion, bytes 8q .. 8q+7 of that range are
// the lane's operand of the q-th of four 16x16x32 bf16 MFMAs per 128 k.
// Activations (x rows, ffn rows) are plain row-major and are loaded with the
// same lane -> (row, k-range) assignment, so both MFMA operands agree on k.
// ---------------------------------------------------------------------------
constexpr int kTileRows = 16;
constexpr int kTileK = 128;
constexpr int kTileBytes = kTileRows * kTileK;  // 2048

__host__ __device__ inline size_t tile_byte(int r, int k, int k_cols) {
    const int nt = r >> 4, kt = k >> 7, rr = r & 15, kk = k & 127;
    return ((size_t)nt * (size_t)(k_cols >> 7) + (size_t)kt) * kTileBytes +
           (size_t)(((kk & 31) >> 4) * 1024 + (rr + 16 * (kk >> 5)) * 16 + (kk & 15));
}

// A wave's weight tiles: each tile row's start, wave-uniform (a scalar
// register pair: the k-step offset arithmetic runs on the scalar unit, and
// a load is a scalar base plus the lane's 16-byte offset); at(t, kt) is the
// lane's 16 bytes of tile t's k-step kt.
template <int WT>
struct WTiles {
    const uint8_t* row[WT];
    int KT;
    uint32_t lane16;
    __device__ __forceinline__ void set(int t, const uint8_t* mat, int nt, int lane) {
        nt = __builtin_amdgcn_readfirstlane(nt);
        row[t] = mat + (size_t)nt * (size_t)KT * kTileBytes;
        lane16 = (uint32_t)lane * 16u;
    }
    __device__ __forceinline__ const uint8_t* at(int t, int kt) const {
        return row[t] + (size_t)kt * kTileBytes + lane16;
    }
};

typedef int v4i __attribute__((ext_vector_type(4)));
typedef float v4f __attribute__((ext_vector_type(4)));
typedef __bf16 v2bf __attribute__((ext_vector_type(2)));
typedef __bf16 v4bf __attribute__((ext_vector_type(4)));
typedef __bf16 v8bf __attribute__((ext_vector_type(8)));

// One 16x16x32 bf16 MFMA (fp32 accumulation): a 16 rows (M) x 32 k, b 32 k x
// 16 columns (N).  Lane L supplies row / column L%16 and 8 consecutive k of
// its k-group L/16, the same for both operands; d lane L holds column L%16,
// rows 4*(L/16) .. +3.  Its sums are fp32-accurate (measured ~1e-8 of
// sum|terms|), unlike gfx950's fp8 MFMAs (truncating, up to ~2^-20).
__device__ __forceinline__ v4f mfma_bf16(const v8bf& a, const v8bf& b, const v4f& c) {
    return __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, b, c, 0, 0, 0);
}

// Eight fp8 e4m3 bytes (two dwords, low byte first) -> eight bf16 values
// multiplied by the power-of-two scale s: exact, since an e4m3 value has at
// most 4 significant bits and bf16 keeps fp32's exponent range.
__device__ __forceinline__ v8bf fp8x8_to_bf16(int d0, int d1, float s) {
    const v2bf a = __builtin_amdgcn_cvt_scalef32_pk_bf16_fp8(d0, s, false);
    const v2bf b = __builtin_amdgcn_cvt_scalef32_pk_bf16_fp8(d0, s, true);
    const v2bf c = __builtin_amdgcn_cvt_scalef32_pk_bf16_fp8(d1, s, false);
    const v2bf d = __builtin_amdgcn_cvt_scalef32_pk_bf16_fp8(d1, s, true);
    const v4bf ab = __builtin_shufflevector(a, b, 0, 1, 2, 3);
    const v4bf cd = __builtin_shufflevector(c, d, 0, 1, 2, 3);
    return __builtin_shufflevector(ab, cd, 0, 1, 2, 3, 4, 5, 6, 7);
}

// UE8M0 exponent byte -> the float 2^(e-127) (e in [1, 254]).
__device__ __forceinline__ float ue8m0_to_f32(int e) { return __uint_as_float((uint32_t)e << 23); }

// fp32 -> OCP e4m3 byte pairs, round to nearest even, saturating at +-448:
// the explicit clamp gives the saturation (the hardware conversion itself is
// RNE), NaN is not clamped and converts to NaN.
__device__ __forceinline__ float sat448(float v) {
    return __builtin_isnan(v) ? v : fminf(fmaxf(v, -448.0f), 448.0f);
}

__device__ __forceinline__ uint32_t pack4_fp8(float a, float b, float c, float d) {
    int r = __builtin_amdgcn_cvt_pk_fp8_f32(sat448(a), sat448(b), 0, false);
    r = __builtin_amdgcn_cvt_pk_fp8_f32(sat448(c), sat448(d), r, true);
    return (uint32_t)r;
}

// fp32 -> bf16 bits, round to nearest even; inf/NaN keep their high half.
__device__ __forceinline__ uint32_t bf16_rne(float v) {
    const uint32_t u = __float_as_uint(v);
    if ((u & 0x7F800000u) == 0x7F800000u) return u >> 16;
    return (u + 0x7FFFu + ((u >> 16) & 1u)) >> 16;
}

// Two fp32 -> packed bf16 (a low, b high) with gfx950's v_cvt_pk_bf16_f32, which
// rounds to nearest even: equal to bf16_rne for every non-NaN input (checked on
// MI355X over all 2^32 bit patterns; a NaN becomes a quiet NaN).  One VALU
// instruction per pair instead of ~5 per value.
__device__ __forceinline__ uint32_t pack2_bf16(float a, float b) {
    typedef float v2f_t __attribute__((ext_vector_type(2)));
    typedef __bf16 v2bf_t __attribute__((ext_vector_type(2)));
    return __builtin_bit_cast(uint32_t, __builtin_convertvector((v2f_t){a, b}, v2bf_t));
}

// SwiGLU's silu(g) * u, with the sigmoid's reciprocal from v_rcp_f32 (1 ulp)
// instead of an IEEE division (a dozen instructions per value).
__device__ __forceinline__ float silu_mul(float g, float u) {
    return g * __builtin_amdgcn_rcpf(1.0f + __expf(-g)) * u;
}

__device__ __forceinline__ float bf16_to_f32(uint32_t h) { return __uint_as_float(h << 16); }

// UE8M0 exponent byte of the power of two >= |x| (ceil), clamped to [1, 254].
__device__ __forceinline__ uint32_t ceil_ue8m0(float x) {
    const uint32_t u = __float_as_uint(x) & 0x7FFFFFFFu;
    int e = (int)(u >> 23) + ((u & 0x7FFFFFu) != 0u);
    e = e < 1 ? 1 : (e > 254 ? 254 : e);
    return (uint32_t)e;
}

// Scale byte for a 128-block with absolute maximum amax (amax.clamp(1e-4)/448).
__device__ __forceinline__ uint32_t block_scale_byte(float amax) {
    return ceil_ue8m0(fmaxf(amax, 1e-4f) / 448.0f);
}

// 2^(127 - e): the exact reciprocal of a UE8M0 scale.
__device__ __forceinline__ float inv_scale(uint32_t e) {
    return __uint_as_float((254u - e) << 23);
}

// Non-temporal / streaming 16-byte load of weight data (read once per launch).
__device__ __forceinline__ v4i load16_stream(const uint8_t* p) {
    return __builtin_nontemporal_load(reinterpret_cast<const v4i*>(p));
}

constexpr int kBufferWord3 = 0x00020000;   // gfx9 buffer resource word 3: 32-bit data format
constexpr int kBufferNT = 2;               // buffer load cache policy bit: nt (non-temporal)
constexpr int kBufferSc1 = 16;             // buffer load cache policy bit: sc1 (device scope)

// The same non-temporal 16-byte weight load through a buffer resource over one
// tile row: base and length in scalar registers, the lane's byte offset `off`
// in a vector register (loop-invariant), the k-step's `soff` in a scalar one,
// so the k-loop spends no vector adds on addresses; lane offsets past
// row_bytes read zeros.  The LDS-staged GEMMs use it: measured on MI355X
// against the global-address form, L2 536-539 vs 546-547 us at T = 512 and
// 645-657 vs 658-666 us at T = 2048, L1 within +-5 us, layer at T = 8192 5061
// vs 5105 us.  With the k-step in soff (and the activation loads below) the
// layer at T = 8192 took 5107-5119 vs 5150-5162 us on one box and 5014 vs
// 5033 us on another, Zipf(1.1) T = 2048 1951 vs 1964 us, T = 512 and
// T = 2048 even.  The sc0 / sc1 scope bits on top of nt changed nothing.
__device__ __forceinline__ v4i load16_row_stream(const uint8_t* row, int row_bytes, int off,
                                                 int soff) {
    const __amdgpu_buffer_rsrc_t r = __builtin_amdgcn_make_buffer_rsrc(
        const_cast<uint8_t*>(row), (short)0, row_bytes, kBufferWord3);
    return __builtin_amdgcn_raw_buffer_load_b128(r, off, soff, kBufferNT);
}

// Cached 16-byte load at base + off + soff through a buffer resource over the
// whole 32-bit range from `base` (wave-uniform): the per-lane row offset in a
// vector register, the k-step in a scalar one.  The callers' offsets stay
// below 2^32 by the capacity limit the host enforces.
// kAux: the load's cache-policy bits (0: cached; kBufferSc1: device-coherent,
// for data another XCD wrote during the same launch).
template <int kAux = 0>
__device__ __forceinline__ v4i load16_rows(const uint8_t* base, uint32_t off, int soff) {
    const __amdgpu_buffer_rsrc_t r = __builtin_amdgcn_make_buffer_rsrc(
        const_cast<uint8_t*>(base), (short)0, -1, kBufferWord3);
    return __builtin_amdgcn_raw_buffer_load_b128(r, (int)off, soff, kAux);
}

__device__ __forceinline__ v4i load16(const uint8_t* p) {
    return *reinterpret_cast<const v4i*>(p);
}

}  // namespace mm
