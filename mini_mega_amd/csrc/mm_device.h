// mm_device.h -- device helpers shared by the gfx950 kernels of the fused
// FP8xFP8 MoE layer: tile layout addressing, fp8 / bf16 / UE8M0 conversions
// and the block-scaled MFMA wrapper.
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
// contiguous, and lane L ends up holding row L%16, k in [32*(L/16), +32): the
// operand of one v_mfma_scale_f32_16x16x128_f8f6f4 for that lane.
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

typedef int v8i __attribute__((ext_vector_type(8)));
typedef int v4i __attribute__((ext_vector_type(4)));
typedef float v4f __attribute__((ext_vector_type(4)));

// One 16x16x128 fp8(e4m3) x fp8(e4m3) MFMA with E8M0 block scales
// (127 = 2^0).  a: 16 rows (M) x 128 k, b: 128 k x 16 columns (N);
// d lane L: column L%16, rows 4*(L/16) .. +3.
__device__ __forceinline__ v4f mfma_fp8(const v8i& a, const v8i& b, const v4f& c,
                                        int sa, int sb) {
    return __builtin_amdgcn_mfma_scale_f32_16x16x128_f8f6f4(a, b, c, 0, 0, 0, sa, 0, sb);
}

__device__ __forceinline__ v8i join8(const v4i& lo, const v4i& hi) {
    v8i r;
    r[0] = lo[0]; r[1] = lo[1]; r[2] = lo[2]; r[3] = lo[3];
    r[4] = hi[0]; r[5] = hi[1]; r[6] = hi[2]; r[7] = hi[3];
    return r;
}

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

__device__ __forceinline__ v4i load16(const uint8_t* p) {
    return *reinterpret_cast<const v4i*>(p);
}

}  // namespace mm
