/*
 * pkv_oracle.c — CPU oracle for the paged-KV GQA decode path.
 *
 * TEST INFRASTRUCTURE ONLY: loaded by tests/, __graft_entry__.smoke() and the
 * cpu_baseline leg of bench.py, as the checker or the timed CPU baseline.
 * The product (flashatte-hand_amd/) never links or calls it.
 *
 * What each function restates (paths under the reference checkout):
 *   pkv_oracle_decode_f32      submission-oj/best_flashattn_kvcache_decode.cu:233-371
 *   pkv_oracle_decode_f64      submission-oj/diagnostics/diag_integrated.py:49-57 (dense
 *                              softmax(q k^T * scale) v), gathered through block_table as in
 *                              best_flashattn_kvcache_decode.cu:262-272, 313-328
 *   pkv_oracle_split_partials  best_flashattn_kvcache_decode.cu:664-697 (page ranges, empty
 *                              split), 782-833 (exp2 online update), 845-864 (lse2)
 *   pkv_oracle_combine(_f32)   best_flashattn_kvcache_decode.cu:956-1037 and
 *                              v11_best_hybrid/flashattn_kvcache_decode_v11_best_hybrid.cu:604-613
 *   pkv_oracle_attn_f64        the masks the evaluator passes to flash_attn_with_kvcache
 *                              (scripts/evaluate_flashattn_submission.py:242-245: causal,
 *                              window_size, alibi_slopes) with the semantics of the pinned
 *                              flash-attn 2.6.3 (setup/pip_full_list.txt:54): query i of M at
 *                              position i + L - M; causal keeps keys j <= pos; a window keeps
 *                              pos - left <= j <= pos + right; ALiBi adds -slope * |pos - j|
 *                              to the scaled score; a query with no visible key gives 0;
 *                              cache_leftpad (flash-attn 2.6.3's flash_attn_with_kvcache
 *                              argument) hides the keys below it (kv_start)
 *   pkv_oracle_attn8_f64       the same over OCP FP8 e4m3 caches with per-KV-head scales (no
 *                              counterpart in the reference, which keeps 16-bit caches)
 *   pkv_oracle_e4m3_to_f32     the OCP 8-bit floating point specification's E4M3 encoding
 *
 * How each is pinned (tests/test_oracle.py): the dense fp64 result against an
 * independent numpy formula (including the reference's diagnostic seeds),
 * closed forms (K = 0 gives mean(V); one dominant key gives its V row;
 * seqlen 1 copies V), brute-force gathers, page-permutation invariance, and
 * the split algebra against the single-pass result for many split counts;
 * the masked form (tests/test_mask_oracle.py) against the pinned decode over
 * truncated or re-paged rows, and an ALiBi closed form.
 *
 * Two deliberate differences from the reference, both documented in the
 * design notes: the dot product is summed in 8 interleaved fp32 partial sums
 * (the reference sums a 128-thread tree, best:81-106), and a row whose
 * cache_seqlens exceeds block_table_stride * page_size is clamped to that
 * many tokens (the reference reads past its block_table row).
 */
#include "pkv_oracle.h"

#include <math.h>
#include <stdlib.h>
#include <string.h>
#ifdef _OPENMP
#include <omp.h>
#endif

/* ---------------------------------------------------------------- conversions */

static inline uint32_t f32_bits(float f) {
    uint32_t u;
    memcpy(&u, &f, 4);
    return u;
}

static inline float bits_f32(uint32_t u) {
    float f;
    memcpy(&f, &u, 4);
    return f;
}

float pkv_oracle_f16_to_f32(uint16_t h) {
    const uint32_t sign = (uint32_t)(h & 0x8000u) << 16;
    const uint32_t exp = (h >> 10) & 0x1fu;
    const uint32_t man = h & 0x3ffu;
    if (exp == 0) {
        /* zero or subnormal: man * 2^-24, exact in fp32 */
        float v = (float)man * 5.9604644775390625e-08f;
        return sign ? -v : v;
    }
    if (exp == 31) {
        return bits_f32(sign | 0x7f800000u | (man << 13));
    }
    return bits_f32(sign | ((exp + 112u) << 23) | (man << 13));
}

uint16_t pkv_oracle_f32_to_f16(float f) {
    const uint32_t x = f32_bits(f);
    const uint16_t sign = (uint16_t)((x >> 16) & 0x8000u);
    const uint32_t ax = x & 0x7fffffffu;
    if (ax >= 0x7f800000u) {
        return (uint16_t)(sign | (ax > 0x7f800000u ? 0x7e00u : 0x7c00u));
    }
    if (ax >= 0x477ff000u) { /* >= 65520 rounds (to even) past the largest half, 65504 */
        return (uint16_t)(sign | 0x7c00u);
    }
    if (ax < 0x38800000u) { /* below 2^-14: half subnormal or zero, unit 2^-24 */
        if (ax <= 0x33000000u) { /* <= 2^-25: ties to the even value 0 */
            return sign;
        }
        const uint32_t e = ax >> 23;               /* 102 .. 112 */
        const uint32_t shift = 126u - e;           /* 14 .. 24 */
        const uint32_t m = (ax & 0x7fffffu) | 0x800000u;
        uint32_t r = m >> shift;
        const uint32_t rem = m & ((1u << shift) - 1u);
        const uint32_t half = 1u << (shift - 1u);
        if (rem > half || (rem == half && (r & 1u))) {
            ++r;
        }
        return (uint16_t)(sign | r);
    }
    const uint32_t e = (ax >> 23) - 112u;
    const uint32_t m = ax & 0x7fffffu;
    uint32_t r = (e << 10) | (m >> 13);
    const uint32_t rem = m & 0x1fffu;
    if (rem > 0x1000u || (rem == 0x1000u && (r & 1u))) {
        ++r; /* a carry out of the mantissa correctly bumps the exponent */
    }
    return (uint16_t)(sign | r);
}

float pkv_oracle_bf16_to_f32(uint16_t h) {
    return bits_f32((uint32_t)h << 16);
}

uint16_t pkv_oracle_f32_to_bf16(float f) {
    const uint32_t x = f32_bits(f);
    if ((x & 0x7fffffffu) > 0x7f800000u) {
        return (uint16_t)((x >> 16) | 0x40u);
    }
    return (uint16_t)((x + 0x7fffu + ((x >> 16) & 1u)) >> 16);
}

static float g_f16_table[65536];
static int g_f16_table_ready = 0;

static void build_f16_table(void) {
    if (g_f16_table_ready) {
        return;
    }
#ifdef _OPENMP
#pragma omp critical(pkv_oracle_f16_table)
#endif
    {
        if (!g_f16_table_ready) {
            for (uint32_t i = 0; i < 65536u; ++i) {
                g_f16_table[i] = pkv_oracle_f16_to_f32((uint16_t)i);
            }
            g_f16_table_ready = 1;
        }
    }
}

static inline float to_f32(uint16_t h, int32_t dtype) {
    return dtype == 1 ? bits_f32((uint32_t)h << 16) : g_f16_table[h];
}

static inline uint16_t from_f32(float f, int32_t dtype) {
    return dtype == 1 ? pkv_oracle_f32_to_bf16(f) : pkv_oracle_f32_to_f16(f);
}

/* Convert one 16-bit row of n elements to fp32. */
static inline void row_to_f32(const uint16_t* src, int64_t n, int32_t dtype, float* dst) {
    if (dtype == 1) {
        for (int64_t i = 0; i < n; ++i) {
            dst[i] = bits_f32((uint32_t)src[i] << 16);
        }
    } else {
        for (int64_t i = 0; i < n; ++i) {
            dst[i] = g_f16_table[src[i]];
        }
    }
}

/* ---------------------------------------------------------------- indexing */

/* Valid tokens of row b: cache_seqlens[b], clamped to what the block_table row can address. */
static inline int64_t row_seqlen(const pkv_oracle_dims* d, const int32_t* cache_seqlens, int64_t b) {
    int64_t s = cache_seqlens[b];
    const int64_t cap = d->block_table_stride * d->page_size;
    if (s > cap) {
        s = cap;
    }
    return s;
}

/* Element offset of (token t of row b, kv head kvh, dim 0) in k_cache / v_cache:
 * phys = block_table[b * stride + t / P]; offset = (phys * P + t % P) * Hk * D + kvh * D
 * (best_flashattn_kvcache_decode.cu:262-272, 313-328). */
static inline int64_t token_offset(const pkv_oracle_dims* d, const int32_t* block_table, int64_t b,
                                   int64_t t, int64_t kvh) {
    const int64_t phys = block_table[b * d->block_table_stride + t / d->page_size];
    return (phys * d->page_size + t % d->page_size) * d->num_heads_k * d->head_dim + kvh * d->head_dim;
}

static inline float dot_f32(const float* a, const float* b, int64_t n) {
    float s[8] = {0, 0, 0, 0, 0, 0, 0, 0};
    int64_t i = 0;
    for (; i + 8 <= n; i += 8) {
        for (int j = 0; j < 8; ++j) {
            s[j] = fmaf(a[i + j], b[i + j], s[j]);
        }
    }
    for (; i < n; ++i) {
        s[0] = fmaf(a[i], b[i], s[0]);
    }
    return ((s[0] + s[4]) + (s[2] + s[6])) + ((s[1] + s[5]) + (s[3] + s[7]));
}

static void set_threads(const pkv_oracle_dims* d) {
#ifdef _OPENMP
    if (d->num_threads > 0) {
        omp_set_num_threads(d->num_threads);
    }
#else
    (void)d;
#endif
}

/* ---------------------------------------------------------------- fp32 restatement */

void pkv_oracle_decode_f32(const pkv_oracle_dims* d, const uint16_t* q, const uint16_t* k_cache,
                           const uint16_t* v_cache, const int32_t* block_table,
                           const int32_t* cache_seqlens, float softmax_scale, uint16_t* out) {
    build_f16_table();
    set_threads(d);
    const int64_t B = d->batch, H = d->num_heads, D = d->head_dim;
    const int64_t group = H / d->num_heads_k;
    const int32_t dt = d->dtype;

#ifdef _OPENMP
#pragma omp parallel
#endif
    {
        float* qf = (float*)malloc(sizeof(float) * (size_t)D * 3);
        float* kf = qf + D;
        float* acc = kf + D;
#ifdef _OPENMP
#pragma omp for schedule(dynamic, 1)
#endif
        for (int64_t bh = 0; bh < B * H; ++bh) {
            const int64_t b = bh / H;
            const int64_t h = bh % H;
            const int64_t kvh = h / group;
            const int64_t seqlen = row_seqlen(d, cache_seqlens, b);
            uint16_t* o = out + bh * D;
            if (seqlen <= 0) { /* best:256-259 */
                for (int64_t i = 0; i < D; ++i) {
                    o[i] = from_f32(0.0f, dt);
                }
                continue;
            }
            if (seqlen == 1) { /* best:273-283: the single token's V row, copied */
                memcpy(o, v_cache + token_offset(d, block_table, b, 0, kvh), sizeof(uint16_t) * (size_t)D);
                continue;
            }
            row_to_f32(q + bh * D, D, dt, qf);
            for (int64_t i = 0; i < D; ++i) {
                acc[i] = 0.0f;
            }
            float running_max = -INFINITY;
            float running_sum = 0.0f;
            for (int64_t t = 0; t < seqlen; ++t) {
                const int64_t off = token_offset(d, block_table, b, t, kvh);
                row_to_f32(k_cache + off, D, dt, kf);
                const float score = dot_f32(qf, kf, D) * softmax_scale;
                const float new_max = fmaxf(running_max, score);
                const float alpha = running_sum > 0.0f ? expf(running_max - new_max) : 0.0f;
                const float p = expf(score - new_max);
                const uint16_t* vrow = v_cache + off;
                if (dt == 1) {
                    for (int64_t i = 0; i < D; ++i) {
                        acc[i] = fmaf(alpha, acc[i], p * bits_f32((uint32_t)vrow[i] << 16));
                    }
                } else {
                    for (int64_t i = 0; i < D; ++i) {
                        acc[i] = fmaf(alpha, acc[i], p * g_f16_table[vrow[i]]);
                    }
                }
                running_sum = fmaf(alpha, running_sum, p);
                running_max = new_max;
            }
            for (int64_t i = 0; i < D; ++i) {
                o[i] = from_f32(running_sum > 0.0f ? acc[i] / running_sum : 0.0f, dt);
            }
        }
        free(qf);
    }
}

/* ---------------------------------------------------------------- fp64 dense */

void pkv_oracle_decode_f64(const pkv_oracle_dims* d, const uint16_t* q, const uint16_t* k_cache,
                           const uint16_t* v_cache, const int32_t* block_table,
                           const int32_t* cache_seqlens, double softmax_scale, double* out) {
    build_f16_table();
    set_threads(d);
    const int64_t B = d->batch, H = d->num_heads, D = d->head_dim;
    const int64_t group = H / d->num_heads_k;
    const int32_t dt = d->dtype;

#ifdef _OPENMP
#pragma omp parallel
#endif
    {
        int64_t cap = 0;
        double* scores = NULL;
        double* qd = (double*)malloc(sizeof(double) * (size_t)D * 2);
        double* acc = qd + D;
#ifdef _OPENMP
#pragma omp for schedule(dynamic, 1)
#endif
        for (int64_t bh = 0; bh < B * H; ++bh) {
            const int64_t b = bh / H;
            const int64_t h = bh % H;
            const int64_t kvh = h / group;
            const int64_t n = row_seqlen(d, cache_seqlens, b);
            double* o = out + bh * D;
            if (n <= 0) {
                for (int64_t i = 0; i < D; ++i) {
                    o[i] = 0.0;
                }
                continue;
            }
            if (n > cap) {
                free(scores);
                cap = n;
                scores = (double*)malloc(sizeof(double) * (size_t)cap);
            }
            for (int64_t i = 0; i < D; ++i) {
                qd[i] = (double)to_f32(q[bh * D + i], dt);
            }
            double mx = -INFINITY;
            for (int64_t t = 0; t < n; ++t) {
                const uint16_t* krow = k_cache + token_offset(d, block_table, b, t, kvh);
                double s = 0.0;
                for (int64_t i = 0; i < D; ++i) {
                    s += qd[i] * (double)to_f32(krow[i], dt);
                }
                scores[t] = s * softmax_scale;
                if (scores[t] > mx) {
                    mx = scores[t];
                }
            }
            double denom = 0.0;
            for (int64_t i = 0; i < D; ++i) {
                acc[i] = 0.0;
            }
            for (int64_t t = 0; t < n; ++t) {
                const double p = exp(scores[t] - mx);
                denom += p;
                const uint16_t* vrow = v_cache + token_offset(d, block_table, b, t, kvh);
                for (int64_t i = 0; i < D; ++i) {
                    acc[i] += p * (double)to_f32(vrow[i], dt);
                }
            }
            for (int64_t i = 0; i < D; ++i) {
                o[i] = acc[i] / denom;
            }
        }
        free(scores);
        free(qd);
    }
}

/* ---------------------------------------------------------------- OCP FP8 e4m3 */

/* e4m3 (OCP "E4M3FN"): sign, 4 exponent bits (bias 7), 3 mantissa bits; no
 * infinities, S.1111.111 is NaN, max finite 448; exponent 0 is subnormal
 * (m / 8 * 2^-6). */
float pkv_oracle_e4m3_to_f32(uint8_t b) {
    const int sign = b >> 7;
    const int e = (b >> 3) & 15;
    const int m = b & 7;
    float v;
    if (e == 15 && m == 7) {
        v = NAN;
    } else if (e == 0) {
        v = ldexpf((float)m / 8.0f, -6);
    } else {
        v = ldexpf(1.0f + (float)m / 8.0f, e - 7);
    }
    return sign ? -v : v;
}

/* ---------------------------------------------------------------- fp64 dense, several queries, masks */

/* Cache element t (16-bit of dtype dt, or e4m3 byte times scale) as double. */
static inline double kv_elem(const void* cache, int64_t idx, int32_t dt, int kv_fp8, double scale) {
    if (kv_fp8) {
        return (double)pkv_oracle_e4m3_to_f32(((const uint8_t*)cache)[idx]) * scale;
    }
    return (double)to_f32(((const uint16_t*)cache)[idx], dt);
}

static void attn_f64_impl(const pkv_oracle_dims* d, const uint16_t* q, const void* k_cache, const void* v_cache,
                          const int32_t* block_table, const int32_t* cache_seqlens, int64_t seqlen_q, int causal,
                          int64_t window_left, int64_t window_right, const float* alibi_slopes,
                          int64_t alibi_batch_stride, int kv_fp8, const float* k_scale, const float* v_scale,
                          double softmax_scale, double* out, double* lse, double softcap,
                          const int32_t* kv_start) {
    build_f16_table();
    set_threads(d);
    const int64_t B = d->batch, H = d->num_heads, D = d->head_dim, M = seqlen_q;
    const int64_t group = H / d->num_heads_k;
    const int32_t dt = d->dtype;

#ifdef _OPENMP
#pragma omp parallel
#endif
    {
        int64_t cap = 0;
        double* scores = NULL;
        double* qd = (double*)malloc(sizeof(double) * (size_t)D * 2);
        double* acc = qd + D;
#ifdef _OPENMP
#pragma omp for schedule(dynamic, 1)
#endif
        for (int64_t row = 0; row < B * M * H; ++row) {
            /* q / out row (b, i, h) of [B, M, H, D] */
            const int64_t b = row / (M * H);
            const int64_t i = (row / H) % M;
            const int64_t h = row % H;
            const int64_t kvh = h / group;
            const int64_t n = row_seqlen(d, cache_seqlens, b);
            const int64_t pos = i + n - M;
            const int64_t lo = kv_start ? (int64_t)kv_start[b] : 0; /* cache_leftpad: keys below it are hidden */
            const double slope = alibi_slopes ? (double)alibi_slopes[b * alibi_batch_stride + h] : 0.0;
            const double ks = (kv_fp8 && k_scale) ? (double)k_scale[kvh] : 1.0;
            const double vs = (kv_fp8 && v_scale) ? (double)v_scale[kvh] : 1.0;
            double* o = out + row * D;
            /* softmax_lse [B, H, M]: +inf until a visible key sets it (flash-attn's empty-row value) */
            double* l = lse ? lse + (b * H + h) * M + i : NULL;
            if (l) {
                *l = INFINITY;
            }
            for (int64_t c = 0; c < D; ++c) {
                o[c] = 0.0;
                acc[c] = 0.0;
            }
            if (n <= 0) {
                continue;
            }
            if (n > cap) {
                free(scores);
                cap = n;
                scores = (double*)malloc(sizeof(double) * (size_t)cap);
            }
            for (int64_t c = 0; c < D; ++c) {
                qd[c] = (double)to_f32(q[row * D + c], dt);
            }
            double mx = -INFINITY;
            for (int64_t t = 0; t < n; ++t) {
                const int visible = t >= lo && (!causal || t <= pos) && (window_left < 0 || t >= pos - window_left) &&
                                    (window_right < 0 || t <= pos + window_right);
                if (!visible) {
                    scores[t] = -INFINITY;
                    continue;
                }
                const int64_t koff = token_offset(d, block_table, b, t, kvh);
                double s = 0.0;
                for (int64_t c = 0; c < D; ++c) {
                    s += qd[c] * kv_elem(k_cache, koff + c, dt, kv_fp8, ks);
                }
                double x = s * softmax_scale;
                if (softcap > 0.0) {
                    x = softcap * tanh(x / softcap);
                }
                scores[t] = x - slope * fabs((double)(pos - t));
                if (scores[t] > mx) {
                    mx = scores[t];
                }
            }
            if (mx == -INFINITY) {
                continue; /* no visible key */
            }
            double denom = 0.0;
            for (int64_t t = 0; t < n; ++t) {
                if (scores[t] == -INFINITY) {
                    continue;
                }
                const double p = exp(scores[t] - mx);
                denom += p;
                const int64_t voff = token_offset(d, block_table, b, t, kvh);
                for (int64_t c = 0; c < D; ++c) {
                    acc[c] += p * kv_elem(v_cache, voff + c, dt, kv_fp8, vs);
                }
            }
            for (int64_t c = 0; c < D; ++c) {
                o[c] = acc[c] / denom;
            }
            if (l) {
                *l = mx + log(denom);
            }
        }
        free(scores);
        free(qd);
    }
}

void pkv_oracle_attn_f64(const pkv_oracle_dims* d, const uint16_t* q, const uint16_t* k_cache,
                         const uint16_t* v_cache, const int32_t* block_table, const int32_t* cache_seqlens,
                         int64_t seqlen_q, int causal, int64_t window_left, int64_t window_right,
                         const float* alibi_slopes, int64_t alibi_batch_stride, double softmax_scale,
                         double* out, double* lse, double softcap, const int32_t* kv_start) {
    attn_f64_impl(d, q, k_cache, v_cache, block_table, cache_seqlens, seqlen_q, causal, window_left, window_right,
                  alibi_slopes, alibi_batch_stride, 0, NULL, NULL, softmax_scale, out, lse, softcap, kv_start);
}

void pkv_oracle_attn8_f64(const pkv_oracle_dims* d, const uint16_t* q, const uint8_t* k_cache,
                          const uint8_t* v_cache, const int32_t* block_table, const int32_t* cache_seqlens,
                          int64_t seqlen_q, int causal, int64_t window_left, int64_t window_right,
                          const float* alibi_slopes, int64_t alibi_batch_stride, const float* k_scale,
                          const float* v_scale, double softmax_scale, double* out, double* lse,
                          double softcap, const int32_t* kv_start) {
    attn_f64_impl(d, q, k_cache, v_cache, block_table, cache_seqlens, seqlen_q, causal, window_left, window_right,
                  alibi_slopes, alibi_batch_stride, 1, k_scale, v_scale, softmax_scale, out, lse, softcap, kv_start);
}

/* ---------------------------------------------------------------- split-KV algebra */

void pkv_oracle_split_partials(const pkv_oracle_dims* d, const uint16_t* q, const uint16_t* k_cache,
                               const uint16_t* v_cache, const int32_t* block_table,
                               const int32_t* cache_seqlens, float softmax_scale, int splits,
                               float* part_o, float* part_lse) {
    build_f16_table();
    set_threads(d);
    const int64_t B = d->batch, H = d->num_heads, D = d->head_dim, P = d->page_size;
    const int64_t group = H / d->num_heads_k;
    const int32_t dt = d->dtype;
    const float scale_log2 = softmax_scale * 1.4426950408889634074f;

#ifdef _OPENMP
#pragma omp parallel
#endif
    {
        float* qf = (float*)malloc(sizeof(float) * (size_t)D * 3);
        float* kf = qf + D;
        float* vf = kf + D;
#ifdef _OPENMP
#pragma omp for schedule(dynamic, 1)
#endif
        for (int64_t item = 0; item < B * H * splits; ++item) {
            const int64_t bh = item / splits;
            const int64_t s = item % splits;
            const int64_t b = bh / H;
            const int64_t h = bh % H;
            const int64_t kvh = h / group;
            const int64_t seqlen = row_seqlen(d, cache_seqlens, b);
            const int64_t pages = seqlen > 0 ? (seqlen + P - 1) / P : 0;
            const int64_t first = pages * s / splits;
            const int64_t last = pages * (s + 1) / splits;
            float* o = part_o + item * D;
            if (first >= last) { /* best:680-697: both O and LSE are written */
                for (int64_t i = 0; i < D; ++i) {
                    o[i] = 0.0f;
                }
                part_lse[item] = -INFINITY;
                continue;
            }
            row_to_f32(q + bh * D, D, dt, qf);
            for (int64_t i = 0; i < D; ++i) {
                o[i] = 0.0f;
            }
            float m = -INFINITY;
            float sum = 0.0f;
            int64_t t_end = last * P;
            if (t_end > seqlen) {
                t_end = seqlen;
            }
            for (int64_t t = first * P; t < t_end; ++t) {
                const int64_t off = token_offset(d, block_table, b, t, kvh);
                row_to_f32(k_cache + off, D, dt, kf);
                row_to_f32(v_cache + off, D, dt, vf);
                const float score = dot_f32(qf, kf, D) * scale_log2;
                const float new_max = fmaxf(m, score);
                const float alpha = sum > 0.0f ? exp2f(m - new_max) : 0.0f;
                const float p = exp2f(score - new_max);
                for (int64_t i = 0; i < D; ++i) { /* best:817-825: scale, then fma */
                    o[i] = fmaf(vf[i], p, o[i] * alpha);
                }
                sum = fmaf(alpha, sum, p);
                m = new_max;
            }
            const float inv = sum > 0.0f ? 1.0f / sum : 0.0f;
            for (int64_t i = 0; i < D; ++i) {
                o[i] *= inv;
            }
            part_lse[item] = sum > 0.0f ? m + log2f(sum) : -INFINITY;
        }
        free(qf);
    }
}

static void combine_row(const float* part_o, const float* part_lse, int64_t row, int splits,
                        int64_t D, float* acc) {
    const float* lse = part_lse + row * splits;
    float max_lse = -INFINITY;
    for (int s = 0; s < splits; ++s) {
        max_lse = fmaxf(max_lse, lse[s]);
    }
    float denom = 0.0f;
    for (int s = 0; s < splits; ++s) {
        denom += lse[s] == -INFINITY ? 0.0f : exp2f(lse[s] - max_lse);
    }
    const float inv = denom > 0.0f ? 1.0f / denom : 0.0f;
    for (int64_t i = 0; i < D; ++i) {
        acc[i] = 0.0f;
    }
    for (int s = 0; s < splits; ++s) {
        const float w = lse[s] == -INFINITY ? 0.0f : exp2f(lse[s] - max_lse);
        if (w == 0.0f) {
            continue; /* v11:606-610: an empty split's O is never read */
        }
        const float* o = part_o + (row * splits + s) * D;
        for (int64_t i = 0; i < D; ++i) {
            acc[i] = fmaf(w, o[i], acc[i]);
        }
    }
    for (int64_t i = 0; i < D; ++i) {
        acc[i] *= inv;
    }
}

void pkv_oracle_combine_f32(const float* part_o, const float* part_lse, int64_t rows, int splits,
                            int64_t head_dim, float* out) {
    for (int64_t r = 0; r < rows; ++r) {
        combine_row(part_o, part_lse, r, splits, head_dim, out + r * head_dim);
    }
}

void pkv_oracle_combine(const float* part_o, const float* part_lse, int64_t rows, int splits,
                        int64_t head_dim, int32_t dtype, uint16_t* out) {
    float* acc = (float*)malloc(sizeof(float) * (size_t)head_dim);
    for (int64_t r = 0; r < rows; ++r) {
        combine_row(part_o, part_lse, r, splits, head_dim, acc);
        for (int64_t i = 0; i < head_dim; ++i) {
            out[r * head_dim + i] = from_f32(acc[i], dtype);
        }
    }
    free(acc);
}
