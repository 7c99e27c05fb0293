// probe.hip -- measurement kernels (no reference counterpart): the
// accumulation precision of gfx950's fp8 and bf16 MFMAs on a dot-product
// block and on the layer's whole L2, a read-only HBM stream of known bytes,
// and MFMA issue-rate loops.
// They back the numeric choice of the GEMMs (bf16 MFMA after an exact fp8 ->
// bf16 conversion) and the measured peaks the benchmark reports beside the
// datasheet ones.  Nothing on the layer's path calls them.
#include "mm_kernels.h"

namespace mm {

typedef int v8i __attribute__((ext_vector_type(8)));

// out[r][n] = sum_k dec(a[r][k]) * dec(b[n][k]) for r < 16, one 64-lane
// workgroup per 16 columns n.  a: [16][K], b: [N][K] fp8 e4m3 row-major,
// K % 128 == 0.  mode 0: v_mfma_scale_f32_16x16x128_f8f6f4 (unit scales),
// one accumulator chained over K; mode 1: v_mfma_f32_16x16x32_bf16 after
// the exact fp8 -> bf16 conversion the layer's GEMMs use.
__global__ void __launch_bounds__(64)
mfma_dot_probe_kernel(const uint8_t* __restrict__ a, const uint8_t* __restrict__ b, int K,
                      int mode, float* __restrict__ out, int N) {
    const int l = threadIdx.x, n0 = blockIdx.x * 16;
    const uint8_t* ar = a + (size_t)(l & 15) * K;
    const uint8_t* br = b + (size_t)(n0 + (l & 15)) * K;
    v4f acc = {0.f, 0.f, 0.f, 0.f};
    for (int kb = 0; kb < K; kb += 128) {
        const int k0 = kb + 32 * (l >> 4);
        const v4i a0 = load16(ar + k0), a1 = load16(ar + k0 + 16);
        const v4i b0 = load16(br + k0), b1 = load16(br + k0 + 16);
        if (mode == 0) {
            const v8i av = {a0[0], a0[1], a0[2], a0[3], a1[0], a1[1], a1[2], a1[3]};
            const v8i bv = {b0[0], b0[1], b0[2], b0[3], b1[0], b1[1], b1[2], b1[3]};
            acc = __builtin_amdgcn_mfma_scale_f32_16x16x128_f8f6f4(av, bv, acc, 0, 0, 0, 127, 0,
                                                                   127);
        } else {
            // lane L holds k in [k0, k0 + 32): bytes 8q .. 8q+7 are its operand
            // of the q-th 16x16x32 MFMA of this 128-k step, as in the GEMMs
            const int aw[8] = {a0[0], a0[1], a0[2], a0[3], a1[0], a1[1], a1[2], a1[3]};
            const int bw[8] = {b0[0], b0[1], b0[2], b0[3], b1[0], b1[1], b1[2], b1[3]};
#pragma unroll
            for (int q = 0; q < 4; ++q)
                acc = mfma_bf16(fp8x8_to_bf16(aw[2 * q], aw[2 * q + 1], 1.0f),
                                fp8x8_to_bf16(bw[2 * q], bw[2 * q + 1], 1.0f), acc);
        }
    }
#pragma unroll
    for (int i = 0; i < 4; ++i) out[(size_t)(4 * (l >> 4) + i) * N + n0 + (l & 15)] = acc[i];
}

// The layer's L2 recomputed over routed slots with either MFMA, for the
// end-to-end effect of the MFMA choice: out[s][n] (fp32) = sum_k
// dec(ffn[s][k]) 2^(ffn_sf[s][k/128] - 127) * dec(w2[e][n][k]) 2^(w2_sf[e][n/128][k/128] - 127)
// for the slots s in [g.y, g.z) of expert g.x, g = groups[blockIdx.y] (at
// most 16 slots; an empty group, g.z <= g.y, computes and writes nothing),
// and the 16 channels n0 = 16 * blockIdx.x ..  w2 is logical
// row-major [E][H][I].  Operand roles and k order are the L2 GEMM's: weights
// are the A operand, ffn rows the B operand, k ascending.  mode 0:
// v_mfma_scale_f32_16x16x128_f8f6f4 with the UE8M0 bytes as its scale
// operands (lane L's 32-k block of its row); mode 1: v_mfma_f32_16x16x32_bf16
// after the exact conversion with the scales folded in, as the GEMM runs it.
__global__ void __launch_bounds__(64)
l2_probe_kernel(const uint8_t* __restrict__ ffn, const uint8_t* __restrict__ ffn_sf,
                const uint8_t* __restrict__ w2, const uint8_t* __restrict__ w2_sf,
                const int4* __restrict__ groups, int H, int I, int mode, float* __restrict__ out) {
    const int l = threadIdx.x, n0 = blockIdx.x * 16;
    const int4 g = groups[blockIdx.y];
    if (g.z <= g.y) return;   // empty group: no row to clamp to
    const int KB = I >> 7;
    const int s = min(g.y + (l & 15), g.z - 1);   // rows past the group's end: loaded, not stored
    const int n = n0 + (l & 15);
    const uint8_t* ar = w2 + ((size_t)g.x * H + n) * I;
    const uint8_t* br = ffn + (size_t)s * I;
    const uint8_t* asf = w2_sf + ((size_t)g.x * (H >> 7) + (n >> 7)) * KB;
    const uint8_t* bsf = ffn_sf + (size_t)s * KB;
    v4f acc = {0.f, 0.f, 0.f, 0.f};
    for (int kb = 0; kb < KB; ++kb) {
        const int k0 = kb * 128 + 32 * (l >> 4);
        const v4i a0 = load16(ar + k0), a1 = load16(ar + k0 + 16);
        const v4i b0 = load16(br + k0), b1 = load16(br + k0 + 16);
        const int ea = asf[kb], eb = bsf[kb];
        if (mode == 0) {
            const v8i av = {a0[0], a0[1], a0[2], a0[3], a1[0], a1[1], a1[2], a1[3]};
            const v8i bv = {b0[0], b0[1], b0[2], b0[3], b1[0], b1[1], b1[2], b1[3]};
            acc = __builtin_amdgcn_mfma_scale_f32_16x16x128_f8f6f4(av, bv, acc, 0, 0, 0, ea, 0,
                                                                   eb);
        } else {
            const int aw[8] = {a0[0], a0[1], a0[2], a0[3], a1[0], a1[1], a1[2], a1[3]};
            const int bw[8] = {b0[0], b0[1], b0[2], b0[3], b1[0], b1[1], b1[2], b1[3]};
            const float sa = ue8m0_to_f32(ea), sb = ue8m0_to_f32(eb);
#pragma unroll
            for (int q = 0; q < 4; ++q)
                acc = mfma_bf16(fp8x8_to_bf16(aw[2 * q], aw[2 * q + 1], sa),
                                fp8x8_to_bf16(bw[2 * q], bw[2 * q + 1], sb), acc);
        }
    }
    // d lane L: column (slot) L%16, rows (channels) 4*(L/16) .. +3
    const int so = g.y + (l & 15);
    if (so < g.z) {
#pragma unroll
        for (int i = 0; i < 4; ++i) out[(size_t)so * H + n0 + 4 * (l >> 4) + i] = acc[i];
    }
}

// Reads `n16` 16-byte words once with non-temporal loads: workgroup b
// streams its own contiguous n16 / gridDim.x words (a multiple of 2048, so
// every load stays in its chunk), eight 4 KiB loads of the 256 threads in
// flight per step, and writes one XOR per thread to sink[global thread id],
// so the loads cannot be dropped.  (Measured on MI355X over 4 GiB: 7.1 TB/s
// at 512 workgroups; a grid-stride walk over the same bytes reached 6.1-6.3.)
__global__ void __launch_bounds__(256)
stream_read_kernel(const uint8_t* __restrict__ src, size_t n16, uint32_t* __restrict__ sink) {
    constexpr int U = 8;
    const size_t per = n16 / gridDim.x;
    const uint8_t* b0 = src + (size_t)blockIdx.x * per * 16;
    uint32_t x = 0;
    for (size_t i = threadIdx.x; i < per; i += 256 * U) {
        v4i r[U];
#pragma unroll
        for (int u = 0; u < U; ++u) r[u] = load16_stream(b0 + (i + 256 * u) * 16);
#pragma unroll
        for (int u = 0; u < U; ++u) x ^= (uint32_t)(r[u][0] ^ r[u][1] ^ r[u][2] ^ r[u][3]);
    }
    sink[(size_t)blockIdx.x * 256 + threadIdx.x] = x;
}

// MFMA issue rate: every wave runs `iters` rounds of 8 independent
// accumulator chains (mode 0: 16x16x32 bf16, mode 1: 16x16x128 fp8 with unit
// scales) from registers; sink[wave] keeps one lane's sum.
__global__ void __launch_bounds__(256)
mfma_rate_kernel(int mode, int iters, float* __restrict__ sink) {
    const int l = threadIdx.x & 63;
    v4f acc[8];
#pragma unroll
    for (int c = 0; c < 8; ++c) acc[c] = v4f{0.f, 0.f, 0.f, 0.f};
    if (mode == 0) {
        v8bf x;
#pragma unroll
        for (int j = 0; j < 8; ++j) x[j] = (__bf16)(0.001f * (float)((l + j) & 7));
        for (int it = 0; it < iters; ++it)
#pragma unroll
            for (int c = 0; c < 8; ++c) acc[c] = mfma_bf16(x, x, acc[c]);
    } else {
        v8i x;
#pragma unroll
        for (int j = 0; j < 8; ++j) x[j] = 0x20202020 + ((l + j) & 7);
        for (int it = 0; it < iters; ++it)
#pragma unroll
            for (int c = 0; c < 8; ++c)
                acc[c] = __builtin_amdgcn_mfma_scale_f32_16x16x128_f8f6f4(x, x, acc[c], 0, 0, 0,
                                                                          127, 0, 127);
    }
    float s = 0.f;
#pragma unroll
    for (int c = 0; c < 8; ++c) s += acc[c][0] + acc[c][1] + acc[c][2] + acc[c][3];
    if (l == 0) sink[(size_t)blockIdx.x * (blockDim.x >> 6) + (threadIdx.x >> 6)] = s;
}

}  // namespace mm

extern "C" {

int mm_probe_mfma_dot(const uint8_t* a, const uint8_t* b, int K, int N, int mode, float* out,
                      void* stream) {
    if (!a || !b || !out) return fp8mega::kErrNullPointer;
    if (K <= 0 || K % 128 || N <= 0 || N % 16 || (mode != 0 && mode != 1))
        return fp8mega::kErrBadDims;
    hipLaunchKernelGGL(mm::mfma_dot_probe_kernel, dim3(N / 16), dim3(64), 0, (hipStream_t)stream,
                       a, b, K, mode, out, N);
    return hipPeekAtLastError() == hipSuccess ? fp8mega::kOk : fp8mega::kErrLaunch;
}

int mm_probe_l2_rows(const uint8_t* ffn, const uint8_t* ffn_sf, const uint8_t* w2,
                     const uint8_t* w2_sf, const int* groups, int ngroups, int H, int I, int mode,
                     float* out, void* stream) {
    if (!ffn || !ffn_sf || !w2 || !w2_sf || !groups || !out) return fp8mega::kErrNullPointer;
    if (H <= 0 || H % 128 || I <= 0 || I % 128 || ngroups <= 0 || ngroups > 65535 ||
        (mode != 0 && mode != 1))
        return fp8mega::kErrBadDims;
    hipLaunchKernelGGL(mm::l2_probe_kernel, dim3(H / 16, ngroups), dim3(64), 0,
                       (hipStream_t)stream, ffn, ffn_sf, w2, w2_sf,
                       reinterpret_cast<const int4*>(groups), H, I, mode, out);
    return hipPeekAtLastError() == hipSuccess ? fp8mega::kOk : fp8mega::kErrLaunch;
}

int mm_probe_stream_read(const uint8_t* src, unsigned long long bytes, uint32_t* sink, int grid,
                         void* stream) {
    if (!src || !sink) return fp8mega::kErrNullPointer;
    if (grid <= 0 || bytes % ((unsigned long long)grid * 32768ull)) return fp8mega::kErrBadDims;
    hipLaunchKernelGGL(mm::stream_read_kernel, dim3(grid), dim3(256), 0, (hipStream_t)stream, src,
                       (size_t)(bytes / 16), sink);
    return hipPeekAtLastError() == hipSuccess ? fp8mega::kOk : fp8mega::kErrLaunch;
}

int mm_probe_mfma_rate(int mode, int iters, int grid, float* sink, void* stream) {
    if (!sink) return fp8mega::kErrNullPointer;
    if ((mode != 0 && mode != 1) || iters <= 0 || grid <= 0) return fp8mega::kErrBadDims;
    hipLaunchKernelGGL(mm::mfma_rate_kernel, dim3(grid), dim3(256), 0, (hipStream_t)stream, mode,
                       iters, sink);
    return hipPeekAtLastError() == hipSuccess ? fp8mega::kOk : fp8mega::kErrLaunch;
}

}  // extern "C"
