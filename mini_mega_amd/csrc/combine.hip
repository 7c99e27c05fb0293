// combine.hip -- top-k weighted reduce of the L2 rows back into token order
// (reference: reduce_tile_body src/combine.cuh:488-641; host model ref_reduce
// src/bench_check.cuh:484-499):
//   y[t][c] = sum_{k = 0..topk-1, in order} bf16->f32(l2[pair_pos[t,k]][c]) * w[t][k]
// in fp32, product then add (no fused multiply-add, so the sum is bitwise the
// reference's sequential loop); pairs without a slot (invalid expert id or
// over the slot cap) contribute nothing.  Each thread owns 8 channels (one
// 16-byte bf16 load per k), no atomics: the output is deterministic.  The
// k-loop runs in groups of 8 whose slot indices, weights and row loads are
// all issued before the group's in-order accumulation, so a thread waits for
// one memory latency per group instead of one per k.
// One workgroup covers a token's H channels when H / 8 <= 1024 threads.  The
// outputs are stored non-temporally (nothing in the layer reads them back);
// the L2 rows are loaded non-temporally when kStreamRows, which the host
// picks when they exceed the Infinity Cache (do_reduce in megakernel.hip
// holds the rule and its measurements).
#include "mm_kernels.h"

namespace mm {

template <bool kStreamRows>
__global__ void __launch_bounds__(1024)
combine_kernel(const uint16_t* __restrict__ l2, const int* __restrict__ pair_pos,
               const float* __restrict__ w, int topk, int H, float* __restrict__ y,
               uint16_t* __restrict__ y_bf16) {
#pragma clang fp contract(off)
    constexpr int kG = 8;
    const int t = blockIdx.x;
    const int c0 = (blockIdx.y * blockDim.x + threadIdx.x) * 8;
    if (c0 >= H) return;
    float acc[8];
#pragma unroll
    for (int i = 0; i < 8; ++i) acc[i] = 0.0f;
    const int* pp = pair_pos + (size_t)t * topk;
    const float* ww = w + (size_t)t * topk;
    for (int k0 = 0; k0 < topk; k0 += kG) {
        int pos[kG];
        float wv[kG];
        v4i raw[kG];
#pragma unroll
        for (int j = 0; j < kG; ++j) {
            pos[j] = k0 + j < topk ? pp[k0 + j] : -1;
            wv[j] = k0 + j < topk ? ww[k0 + j] : 0.0f;
        }
#pragma unroll
        for (int j = 0; j < kG; ++j)
        {
            const uint8_t* row = reinterpret_cast<const uint8_t*>(l2 + (size_t)pos[j] * H + c0);
            raw[j] = pos[j] < 0   ? v4i{0, 0, 0, 0}
                     : kStreamRows ? load16_stream(row)
                                   : load16(row);
        }
#pragma unroll
        for (int j = 0; j < kG; ++j) {
            if (pos[j] < 0) continue;
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                const uint32_t u = (uint32_t)raw[j][i];
                const float lo = bf16_to_f32(u & 0xFFFFu) * wv[j];
                const float hi = bf16_to_f32(u >> 16) * wv[j];
                acc[2 * i] = acc[2 * i] + lo;
                acc[2 * i + 1] = acc[2 * i + 1] + hi;
            }
        }
    }
    if (y) {
        v4f* yo = reinterpret_cast<v4f*>(y + (size_t)t * H + c0);
        __builtin_nontemporal_store(v4f{acc[0], acc[1], acc[2], acc[3]}, yo);
        __builtin_nontemporal_store(v4f{acc[4], acc[5], acc[6], acc[7]}, yo + 1);
    }
    if (y_bf16) {
        v4i o;
#pragma unroll
        for (int i = 0; i < 4; ++i)
            o[i] = (int)(bf16_rne(acc[2 * i]) | (bf16_rne(acc[2 * i + 1]) << 16));
        __builtin_nontemporal_store(o, reinterpret_cast<v4i*>(y_bf16 + (size_t)t * H + c0));
    }
}

template __global__ void combine_kernel<false>(const uint16_t*, const int*, const float*, int, int,
                                               float*, uint16_t*);
template __global__ void combine_kernel<true>(const uint16_t*, const int*, const float*, int, int,
                                              float*, uint16_t*);

}  // namespace mm
