/*
 * moe_oracle.c -- CPU restatement of the reference's host numeric path for the
 * fused FP8xFP8 MoE layer (route -> L1 GEMM+SwiGLU -> fp8 -> L2 GEMM -> bf16 ->
 * top-k weighted reduce).
 *
 * TEST INFRASTRUCTURE ONLY.  This file is the checker: only tests/, the smoke()
 * entry point and bench.py's cpu_baseline leg load it.  The product path
 * (mini_mega_amd/) never links, loads or falls back to it.
 *
 * Every function names the reference file:line it restates (paths relative to
 * the reference repository root).  Weights are taken in LOGICAL row-major form
 * ([rows][k] bytes); the W1 rows are in the reference's gate/up "paired" order
 * with pairing block G (G = 256 in the reference, src/bench_check.cuh:444-445;
 * generalised to G = min(256, I) so that I = 128 is expressible).
 *
 * Scaled variant (an extension the reference kernel does not implement): every
 * operand byte q carries a power-of-two UE8M0 scale s = 2^(e-127); the value is
 * decode(q) * s.  With every scale byte = 127 (2^0) every function reduces
 * exactly to the reference arithmetic.
 *
 * Build: see oracle/Makefile (gcc -O2 -ffp-contract=off, no fast-math).
 */
#include <math.h>
#include <pthread.h>
#include <stdint.h>
#include <stdlib.h>
#include <string.h>

#define ORC_API __attribute__((visibility("default")))

/* Accumulation model of orc_l1_rows / orc_l2_rows: 0 = sequential fp32 (the
 * reference host path), 1 = float64 accumulation rounded once to fp32 (an
 * "exactly summing device" model used only to bound what any device can
 * reach against the fp32 host path). */
static int g_acc64 = 0;
ORC_API void orc_set_acc64(int on) { g_acc64 = on; }

/* Planted mistakes, for the tests that show the oracle's pins are sensitive
 * (0 = none, the only value outside those tests): 1 = the up rows of L1 take
 * their gate rows' 128-row scale block; 2 = the W2 scale block index is
 * transposed ((k/128, n/128) instead of (n/128, k/128)); 3 = the ffn rows
 * take the scale of the next 128-column block; 4 = the 128x128 block cast
 * multiplies by its scale instead of dividing; 5 = the check.cu x bytes use
 * the global token in place of the rank-local one; 6 = the check.cu weights
 * lose their 0.25 * rank term. */
static int g_mutation = 0;
ORC_API void orc_set_mutation(int m) { g_mutation = m; }

/* ------------------------------------------------------------ E4M3 decode --
 * src/bench_check.cuh:327-358: exp=0 -> +-(m/8)*2^-6; exp 1..15 ->
 * +-(1+m/8)*2^(exp-7); 0x7F/0xFF -> NaN; max finite 448 = 0x7E. */
static float g_e4m3[256];
static int g_e4m3_ready = 0;

static void e4m3_init(void) {
    if (g_e4m3_ready) return;
    for (int i = 0; i < 256; ++i) {
        const int sign = (i >> 7) & 1, ex = (i >> 3) & 0xF, man = i & 7;
        float v;
        if (ex == 0xF && man == 7) {
            v = NAN;
        } else {
            const float a = ex == 0 ? (float)man / 8.0f : 1.0f + (float)man / 8.0f;
            v = ldexpf(a, ex == 0 ? -6 : ex - 7);
            if (sign) v = -v;
        }
        g_e4m3[i] = v;
    }
    g_e4m3_ready = 1;
}

ORC_API float orc_e4m3_decode(uint8_t b) {
    e4m3_init();
    return g_e4m3[b];
}

/* ------------------------------------------------------------ E4M3 encode --
 * src/bench_check.cuh:362-380: RNE, saturate to +-448 (0x7E), NaN -> 0x7F,
 * |v| < 2^-6 -> subnormal step 2^-9 (RNE), mantissa carry, overflow after the
 * carry saturates. */
ORC_API uint8_t orc_e4m3_quantize(float v) {
    if (isnan(v)) return 0x7Fu;
    const uint32_t sign = signbit(v) ? 0x80u : 0u;
    const float a = fabsf(v);
    if (a >= 448.0f) return (uint8_t)(sign | 0x7Eu);
    if (a < 1.0f / 64.0f) {
        const int q = (int)nearbyintf(a * 512.0f);
        return (uint8_t)(sign | (uint32_t)q);
    }
    int e2 = 0;
    const float mf = frexpf(a, &e2);
    const float mant = mf * 2.0f;
    const int eu = e2 - 1;
    int q = (int)nearbyintf(mant * 8.0f);
    int enc_e = eu + 7;
    if (q == 16) { q = 8; enc_e += 1; }
    if (enc_e > 15) return (uint8_t)(sign | 0x7Eu);
    return (uint8_t)(sign | ((uint32_t)enc_e << 3) | (uint32_t)(q - 8));
}

/* ------------------------------------------------------------------ BF16 --
 * src/bench_check.cuh:384-400: decode = <<16; encode RNE u += 0x7FFF + lsb,
 * inf/NaN keep their high half. */
ORC_API float orc_bf16_to_f32(uint16_t h) {
    const uint32_t u = (uint32_t)h << 16;
    float v;
    memcpy(&v, &u, 4);
    return v;
}

ORC_API uint16_t orc_f32_to_bf16(float v) {
    uint32_t u;
    memcpy(&u, &v, 4);
    if ((u & 0x7F800000u) == 0x7F800000u) return (uint16_t)(u >> 16);
    u += 0x7FFFu + ((u >> 16) & 1u);
    return (uint16_t)(u >> 16);
}

/* ------------------------------------------------------------------ UE8M0 --
 * torch/mxmegakernel/utils/math.py:13-16 (ceil_to_ue8m0): biased exponent of
 * |x| plus one when the mantissa is non-zero, clamped to [1, 254].  Returned as
 * the exponent byte (scale = 2^(byte-127)). */
ORC_API uint8_t orc_ceil_ue8m0(float x) {
    uint32_t u;
    const float a = fabsf(x);
    memcpy(&u, &a, 4);
    int ex = (int)((u >> 23) & 0xFF) + ((u & 0x7FFFFFu) != 0);
    if (ex < 1) ex = 1;
    if (ex > 254) ex = 254;
    return (uint8_t)ex;
}

static inline float ue8m0_scale(uint8_t e) { return ldexpf(1.0f, (int)e - 127); }

ORC_API float orc_ue8m0_to_f32(uint8_t e) { return ue8m0_scale(e); }

/* Scale byte for one 128-block with absolute maximum amax:
 * utils/math.py:34-37 -- amax.clamp(1e-4) / 448 -> ceil_to_ue8m0. */
ORC_API uint8_t orc_block_scale(float amax) {
    if (!(amax >= 1e-4f)) amax = 1e-4f;
    return orc_ceil_ue8m0(amax / 448.0f);
}

/* Per-row, per-gran-column UE8M0 cast (utils/math.py:23-47, per_token_cast_to_fp8
 * with use_ue8m0=True): q = e4m3(v * (1/sf)), 1/sf exact (power of two).
 * x: [rows][cols] fp32; q: [rows][cols]; sf: [rows][cols/gran] exponent bytes. */
ORC_API void orc_quant_rows_ue8m0(const float* x, int rows, int cols, int gran,
                                  uint8_t* q, uint8_t* sf) {
    const int nb = cols / gran;
    for (int r = 0; r < rows; ++r)
        for (int b = 0; b < nb; ++b) {
            const float* xr = x + (size_t)r * cols + (size_t)b * gran;
            float amax = 0.0f;
            for (int c = 0; c < gran; ++c) amax = fmaxf(amax, fabsf(xr[c]));
            const uint8_t e = orc_block_scale(amax);
            const float inv = ldexpf(1.0f, 127 - (int)e);
            sf[(size_t)r * nb + b] = e;
            for (int c = 0; c < gran; ++c)
                q[(size_t)r * cols + (size_t)b * gran + c] = orc_e4m3_quantize(xr[c] * inv);
        }
}

/* 128x128 block UE8M0 cast (utils/math.py:62-72, per_block_cast_to_fp8).
 * w: [rows][cols] fp32 -> q bytes, sf [rows/gran][cols/gran]. */
ORC_API void orc_quant_blocks_ue8m0(const float* w, int rows, int cols, int gran,
                                    uint8_t* q, uint8_t* sf) {
    const int nbr = rows / gran, nbc = cols / gran;
    for (int br = 0; br < nbr; ++br)
        for (int bc = 0; bc < nbc; ++bc) {
            float amax = 0.0f;
            for (int r = 0; r < gran; ++r)
                for (int c = 0; c < gran; ++c)
                    amax = fmaxf(amax, fabsf(w[(size_t)(br * gran + r) * cols + bc * gran + c]));
            const uint8_t e = orc_block_scale(amax);
            /* mutation 4 (tests only): multiply by the scale instead of its inverse */
            const float inv = ldexpf(1.0f, g_mutation == 4 ? (int)e - 127 : 127 - (int)e);
            sf[(size_t)br * nbc + bc] = e;
            for (int r = 0; r < gran; ++r)
                for (int c = 0; c < gran; ++c) {
                    const size_t i = (size_t)(br * gran + r) * cols + bc * gran + c;
                    q[i] = orc_e4m3_quantize(w[i] * inv);
                }
        }
}

/* ------------------------------------------------------------- generators --
 * src/megakernel.h:46-47 (WPROBE_VAL, WPROBE=0): byte = (seed + row*131 +
 * k*7) & 0x3f, on the logical (paired) row order. */
ORC_API uint8_t orc_wprobe_val(uint32_t seed, uint32_t row, uint32_t k) {
    return (uint8_t)((seed + row * 131u + k * 7u) & 0x3fu);
}

/* test/mega_common.cuh:151-179 (fill_inputs) remapped to one GPU: global token
 * g = r*tpr + t; x byte (r*37 + t*7 + c*3) & 0x3f; weight 1 + 0.25r + 0.01*(i%7)
 * with i = t*topk + k the rank-local pair index. */
ORC_API void orc_checkcu_inputs(int ranks, int tpr, int H, int topk, uint8_t* x,
                                float* w) {
    for (int r = 0; r < ranks; ++r)
        for (int t = 0; t < tpr; ++t) {
            const size_t g = (size_t)r * tpr + t;
            /* mutations 5 / 6 (tests only): the global token in place of the
             * rank-local one in x; the rank term dropped from the weights */
            const int tx = g_mutation == 5 ? (int)g : t;
            for (int c = 0; c < H; ++c)
                x[g * H + c] = (uint8_t)((r * 37 + tx * 7 + c * 3) & 0x3f);
            for (int k = 0; k < topk; ++k) {
                const int i = t * topk + k;
                const float rt = g_mutation == 6 ? 0.0f : (float)r * 0.25f;
                w[g * topk + k] = 1.0f + rt + (float)(i % 7) * 0.01f;
            }
        }
}

/* src/bench_check.cuh:42-69 (make_routes, Balanced pattern) for every source
 * rank, concatenated rank-major: idx[(r*tokens + t)*topk + k] = (i + r*epr +
 * salt) % E with i = t*topk + k. */
ORC_API void orc_balanced_routes(int ranks, int tokens, int topk, int epr, int salt,
                                 int64_t* idx) {
    const int E = ranks * epr;
    for (int r = 0; r < ranks; ++r)
        for (int i = 0; i < tokens * topk; ++i)
            idx[(size_t)r * tokens * topk + i] = (int64_t)((i + r * epr + salt) % E);
}

/* test/mega_common.cuh:460-482 (routes_from_counts): per_expert[R*EPR]
 * rank-major; pair j -> src = j % R, q = j / R, token = q % tokens, k = q /
 * tokens.  Output concatenated rank-major.  Returns 0, or -1 when a token
 * would be routed to the same expert twice (routes_duplicate_free). */
ORC_API int orc_routes_from_counts(const int* per_expert, int R, int epr, int tokens,
                                   int topk, int64_t* idx) {
    memset(idx, 0, sizeof(int64_t) * (size_t)R * tokens * topk);
    long long j = 0;
    for (int r = 0; r < R; ++r)
        for (int e = 0; e < epr; ++e) {
            const int64_t ge = (int64_t)r * epr + e;
            const int c_re = per_expert[r * epr + e];
            for (int c = 0; c < c_re; ++c, ++j) {
                const int src = (int)(j % R);
                const long long q = j / R;
                const int token = (int)(q % tokens);
                const int k = (int)(q / tokens);
                if (k >= topk) return -1;
                idx[((size_t)src * tokens + token) * topk + k] = ge;
            }
        }
    for (int r = 0; r < R; ++r)
        for (int t = 0; t < tokens; ++t) {
            const int64_t* row = idx + ((size_t)r * tokens + t) * topk;
            for (int a = 0; a < topk; ++a)
                for (int b = a + 1; b < topk; ++b)
                    if (row[a] == row[b]) return -1;
        }
    return 0;
}

/* ---------------------------------------------------------------- routing --
 * Semantics of src/prologue.cuh:126-226 (route_build_body) + :269-498
 * (task_setup_body prefix tables) on one GPU: ids outside [0, E) are dropped;
 * each expert keeps its first `cap` pairs; slots are assigned in CANONICAL
 * order = ascending pair index p = t*topk + k (the sorted member of the set
 * the reference's validate_route accepts, src/bench_check.cuh:72-144).
 * counts[E], offsets[E+1] (exclusive prefix of counts), perm[offsets[E]] = pair
 * index per slot, pair_pos[P] = slot of each pair or -1. */
ORC_API void orc_route(const int64_t* topk_idx, int T, int topk, int E, int cap,
                       int32_t* counts, int32_t* offsets, uint32_t* perm,
                       int32_t* pair_pos) {
    const long long P = (long long)T * topk;
    memset(counts, 0, sizeof(int32_t) * (size_t)E);
    for (long long p = 0; p < P; ++p) {
        const int64_t e = topk_idx[p];
        if (e < 0 || e >= E) continue;
        counts[e]++;
    }
    for (int e = 0; e < E; ++e)
        if (counts[e] > cap) counts[e] = cap;
    offsets[0] = 0;
    for (int e = 0; e < E; ++e) offsets[e + 1] = offsets[e] + counts[e];
    int32_t* fill = (int32_t*)calloc((size_t)E, sizeof(int32_t));
    for (long long p = 0; p < P; ++p) {
        const int64_t e = topk_idx[p];
        pair_pos[p] = -1;
        if (e < 0 || e >= E) continue;
        if (fill[e] >= counts[e]) continue;
        const int pos = offsets[e] + fill[e]++;
        perm[pos] = (uint32_t)p;
        pair_pos[p] = pos;
    }
    free(fill);
}

/* --------------------------------------------------------------------- L1 --
 * src/bench_check.cuh:435-455 (ref_l1): for hidden column h the gate row is
 * (h/G)*2G + h%G and the up row is gate + G (paired order, :444-445); g, u are
 * sequential fp32 sums of decode(x_k)*decode(w_k); ffn = silu(g)*u with
 * silu(g) = g/(1+exp(-g)).  Scaled variant: decode(.) is multiplied by the
 * operand's UE8M0 scale (x: per row per 128 columns; w1: per 128x128 block of
 * the paired-order matrix).  Null scale pointers mean scale 1.
 * x: [rows][H]; xsf: [rows][H/128]; w1e: [2I][H] paired order; w1sf: [2I/128][H/128].
 * out: [rows][I] fp32 pre-quantisation values. */
ORC_API void orc_l1_rows(const uint8_t* x, const uint8_t* xsf, int rows, const uint8_t* w1e,
                         const uint8_t* w1sf, int H, int I, int G, float* out) {
    e4m3_init();
    const int kb = H / 128;
    float* xd = (float*)malloc(sizeof(float) * (size_t)rows * H);
    float* wg = (float*)malloc(sizeof(float) * (size_t)H);
    float* wu = (float*)malloc(sizeof(float) * (size_t)H);
    for (int r = 0; r < rows; ++r)
        for (int k = 0; k < H; ++k) {
            float v = g_e4m3[x[(size_t)r * H + k]];
            if (xsf) v *= ue8m0_scale(xsf[(size_t)r * kb + k / 128]);
            xd[(size_t)r * H + k] = v;
        }
    for (int h = 0; h < I; ++h) {
        const int grow = (h / G) * 2 * G + (h % G);
        const int urow = grow + G;
        for (int k = 0; k < H; ++k) {
            wg[k] = g_e4m3[w1e[(size_t)grow * H + k]];
            wu[k] = g_e4m3[w1e[(size_t)urow * H + k]];
        }
        if (w1sf)
            for (int b = 0; b < kb; ++b) {
                const float sg = ue8m0_scale(w1sf[(size_t)(grow / 128) * kb + b]);
                const int ub = g_mutation == 1 ? grow / 128 : urow / 128;
                const float su = ue8m0_scale(w1sf[(size_t)ub * kb + b]);
                for (int k = b * 128; k < b * 128 + 128; ++k) {
                    wg[k] *= sg;
                    wu[k] *= su;
                }
            }
        for (int r = 0; r < rows; ++r) {
            const float* xr = xd + (size_t)r * H;
            float g = 0.0f, u = 0.0f;
            if (g_acc64) {
                double g64 = 0.0, u64 = 0.0;
                for (int k = 0; k < H; ++k) {
                    g64 += (double)xr[k] * wg[k];
                    u64 += (double)xr[k] * wu[k];
                }
                g = (float)g64;
                u = (float)u64;
            } else {
                for (int k = 0; k < H; ++k) {
                    g += xr[k] * wg[k];
                    u += xr[k] * wu[k];
                }
            }
            out[(size_t)r * I + h] = (g / (1.0f + expf(-g))) * u;
        }
    }
    free(xd);
    free(wg);
    free(wu);
}

/* L1 output cast to fp8.  Unscaled (the reference): e4m3 RNE saturating
 * (src/bench_check.cuh:362-380; torch/tests/test_fp8_mega_moe.py:45 clamps to
 * +-448 first).  Scaled: per row per 128 hidden columns UE8M0 recipe
 * (utils/math.py:23-47), sf bytes [rows][I/128]. */
ORC_API void orc_quant_ffn(const float* h, int rows, int I, int scaled, uint8_t* q,
                           uint8_t* sf) {
    if (scaled) {
        orc_quant_rows_ue8m0(h, rows, I, 128, q, sf);
        return;
    }
    for (long long i = 0; i < (long long)rows * I; ++i) q[i] = orc_e4m3_quantize(h[i]);
}

/* --------------------------------------------------------------------- L2 --
 * src/bench_check.cuh:461-476 (ref_l2): o_n = sum_k decode(ffn_k)*decode(W2[n][k])
 * in fp32 (sequential k).  Scaled: ffn per row per 128 k; W2 per 128x128 block.
 * ffn: [rows][I]; w2e: [H][I]; out fp32 [rows][H] (pre-bf16). */
ORC_API void orc_l2_rows(const uint8_t* ffn, const uint8_t* fsf, int rows, const uint8_t* w2e,
                         const uint8_t* w2sf, int H, int I, float* out) {
    e4m3_init();
    const int kb = I / 128;
    float* ad = (float*)malloc(sizeof(float) * (size_t)rows * I);
    float* wr = (float*)malloc(sizeof(float) * (size_t)I);
    for (int r = 0; r < rows; ++r)
        for (int k = 0; k < I; ++k) {
            float v = g_e4m3[ffn[(size_t)r * I + k]];
            const int fb = g_mutation == 3 ? (k / 128 + 1) % kb : k / 128;
            if (fsf) v *= ue8m0_scale(fsf[(size_t)r * kb + fb]);
            ad[(size_t)r * I + k] = v;
        }
    for (int n = 0; n < H; ++n) {
        for (int k = 0; k < I; ++k) wr[k] = g_e4m3[w2e[(size_t)n * I + k]];
        if (w2sf)
            for (int b = 0; b < kb; ++b) {
                const size_t wi = g_mutation == 2 ? (size_t)b * (H / 128) + n / 128
                                                  : (size_t)(n / 128) * kb + b;
                const float sb = ue8m0_scale(w2sf[wi]);
                for (int k = b * 128; k < b * 128 + 128; ++k) wr[k] *= sb;
            }
        for (int r = 0; r < rows; ++r) {
            const float* ar = ad + (size_t)r * I;
            float acc = 0.0f;
            if (g_acc64) {
                double a64 = 0.0;
                for (int k = 0; k < I; ++k) a64 += (double)ar[k] * wr[k];
                acc = (float)a64;
            } else {
                for (int k = 0; k < I; ++k) acc += ar[k] * wr[k];
            }
            out[(size_t)r * H + n] = acc;
        }
    }
    free(ad);
    free(wr);
}

/* ----------------------------------------------------------------- reduce --
 * src/bench_check.cuh:484-499 (ref_reduce) / src/combine.cuh:601-627:
 * y[t][c] = sum over k = 0..topk-1 (in order) of bf16->f32(row_k[c]) * w[t][k],
 * skipping ids outside [0, E) (and pairs without a slot); fp32, product then
 * add.  l2: [slots][H] bf16 bits indexed by pair_pos. */
ORC_API void orc_reduce(const uint16_t* l2, const int32_t* pair_pos, const float* w,
                        int T, int topk, int H, float* y, uint16_t* y_bf16) {
    for (int t = 0; t < T; ++t) {
        float* yr = y + (size_t)t * H;
        for (int c = 0; c < H; ++c) yr[c] = 0.0f;
        for (int k = 0; k < topk; ++k) {
            const int32_t pos = pair_pos[(size_t)t * topk + k];
            if (pos < 0) continue;
            const float wv = w[(size_t)t * topk + k];
            const uint16_t* row = l2 + (size_t)pos * H;
            for (int c = 0; c < H; ++c) {
                const float prod = orc_bf16_to_f32(row[c]) * wv;
                yr[c] = yr[c] + prod;
            }
        }
        if (y_bf16)
            for (int c = 0; c < H; ++c) y_bf16[(size_t)t * H + c] = orc_f32_to_bf16(yr[c]);
    }
}

/* ------------------------------------------------------- full layer (MT) --
 * The check.cu host chain over the whole layer: route -> per slot ref_l1 ->
 * quantise -> ref_l2 -> bf16 -> ref_reduce (src/bench_check.cuh:435-499;
 * threads take whole experts round-robin; test/check.cu:154-165 splits the
 * rows of one expert instead -- the arithmetic per row is the same).
 * w1: [E][2I][H] logical paired order, w2: [E][H][I] logical.  Scales may be
 * null (reference semantics).  Outputs (any may be null except y): ffn
 * [slots][I], ffn_sf [slots][I/128], l2 [slots][H] bf16 bits, y [T][H],
 * y_bf16 [T][H].  Pass expert_mask (E bytes) to restrict the work to a
 * subset of experts (used to time a bounded sample); rows of masked-out
 * experts are left untouched. */
typedef struct {
    const uint8_t *x, *xsf, *w1, *w1sf, *w2, *w2sf;
    const int32_t *offsets;
    const uint32_t* perm;
    const uint8_t* expert_mask;
    int topk, E, H, I, G, scaled;
    uint8_t *ffn, *ffn_sf;
    uint16_t* l2;
    int nthreads, tid;
} LayerJob;

static void* layer_worker(void* arg) {
    LayerJob* j = (LayerJob*)arg;
    const int H = j->H, I = j->I, kbH = H / 128, kbI = I / 128;
    for (int e = j->tid; e < j->E; e += j->nthreads) {
        if (j->expert_mask && !j->expert_mask[e]) continue;
        const int s0 = j->offsets[e], rows = j->offsets[e + 1] - s0;
        if (rows <= 0) continue;
        uint8_t* xr = (uint8_t*)malloc((size_t)rows * H);
        uint8_t* xs = (uint8_t*)malloc((size_t)rows * kbH);
        float* h = (float*)malloc(sizeof(float) * (size_t)rows * I);
        uint8_t* q = (uint8_t*)malloc((size_t)rows * I);
        uint8_t* qs = (uint8_t*)malloc((size_t)rows * kbI);
        float* o = (float*)malloc(sizeof(float) * (size_t)rows * H);
        for (int r = 0; r < rows; ++r) {
            const size_t tok = j->perm[s0 + r] / (uint32_t)j->topk;
            memcpy(xr + (size_t)r * H, j->x + tok * H, (size_t)H);
            if (j->xsf) memcpy(xs + (size_t)r * kbH, j->xsf + tok * kbH, (size_t)kbH);
        }
        orc_l1_rows(xr, j->xsf ? xs : NULL, rows, j->w1 + (size_t)e * 2 * I * H,
                    j->w1sf ? j->w1sf + (size_t)e * (2 * I / 128) * kbH : NULL, H, I, j->G, h);
        orc_quant_ffn(h, rows, I, j->scaled, q, qs);
        orc_l2_rows(q, j->scaled ? qs : NULL, rows, j->w2 + (size_t)e * H * I,
                    j->w2sf ? j->w2sf + (size_t)e * (H / 128) * kbI : NULL, H, I, o);
        if (j->ffn) memcpy(j->ffn + (size_t)s0 * I, q, (size_t)rows * I);
        if (j->ffn_sf && j->scaled) memcpy(j->ffn_sf + (size_t)s0 * kbI, qs, (size_t)rows * kbI);
        if (j->l2)
            for (size_t i = 0; i < (size_t)rows * H; ++i)
                j->l2[(size_t)s0 * H + i] = orc_f32_to_bf16(o[i]);
        free(xr); free(xs); free(h); free(q); free(qs); free(o);
    }
    return NULL;
}

/* Runs L1 -> quant -> L2 -> bf16 for every routed slot (route must be done
 * first with orc_route).  Returns 0. */
ORC_API int orc_layer_slots(const uint8_t* x, const uint8_t* xsf, const uint8_t* w1,
                            const uint8_t* w1sf, const uint8_t* w2, const uint8_t* w2sf,
                            const int32_t* offsets, const uint32_t* perm, int topk, int E,
                            int H, int I, int G, int scaled, const uint8_t* expert_mask,
                            uint8_t* ffn, uint8_t* ffn_sf, uint16_t* l2, int nthreads) {
    e4m3_init();
    if (nthreads < 1) nthreads = 1;
    pthread_t* th = (pthread_t*)malloc(sizeof(pthread_t) * (size_t)nthreads);
    LayerJob* jobs = (LayerJob*)malloc(sizeof(LayerJob) * (size_t)nthreads);
    for (int t = 0; t < nthreads; ++t) {
        LayerJob j = {x, xsf, w1, w1sf, w2, w2sf, offsets, perm, expert_mask, topk, E, H, I,
                      G, scaled, ffn, ffn_sf, l2, nthreads, t};
        jobs[t] = j;
        pthread_create(&th[t], NULL, layer_worker, &jobs[t]);
    }
    for (int t = 0; t < nthreads; ++t) pthread_join(th[t], NULL);
    free(th);
    free(jobs);
    return 0;
}
