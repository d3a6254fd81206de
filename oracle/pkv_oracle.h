/*
 * pkv_oracle.h — CPU oracle for the paged-KV GQA decode path.
 *
 * TEST INFRASTRUCTURE ONLY.  Only tests/, __graft_entry__.smoke() and the
 * cpu_baseline leg of bench.py may load this library, and only as the
 * checker (or as the timed CPU baseline).  The product path never calls it.
 *
 * Layouts are those of include/pkv_decode.h.  16-bit tensors are passed as
 * uint16_t bit patterns; dtype 0 = fp16, 1 = bf16.
 */
#ifndef PKV_ORACLE_H
#define PKV_ORACLE_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

typedef struct pkv_oracle_dims {
    int64_t batch;
    int64_t num_heads;
    int64_t num_heads_k;
    int64_t head_dim;
    int64_t page_size;
    int64_t num_pages;
    int64_t block_table_stride;
    int32_t dtype;
    int32_t num_threads; /* OpenMP threads; <= 0 = runtime default */
} pkv_oracle_dims;

/* 16-bit <-> fp32 conversions written from the IEEE 754 / bfloat16 definitions
 * (round-to-nearest-even, NaN kept quiet). */
float pkv_oracle_f16_to_f32(uint16_t h);
uint16_t pkv_oracle_f32_to_f16(float f);
float pkv_oracle_bf16_to_f32(uint16_t h);
uint16_t pkv_oracle_f32_to_bf16(float f);

/* Restatement of the reference's generic scalar decode
 * (submission-oj/best_flashattn_kvcache_decode.cu:233-371): per (b, h), per
 * token, fp32 online softmax in natural-exp units, output cast RNE.
 * Also the timed CPU baseline. */
void pkv_oracle_decode_f32(const pkv_oracle_dims* d, const uint16_t* q, const uint16_t* k_cache,
                           const uint16_t* v_cache, const int32_t* block_table,
                           const int32_t* cache_seqlens, float softmax_scale, uint16_t* out);

/* Textbook dense attention in fp64 on the gathered K/V rows
 * (the reference's own check formula, submission-oj/diagnostics/diag_integrated.py:49-57).
 * out is fp64 [B, H, D]; rows with seqlen <= 0 give zeros. */
void pkv_oracle_decode_f64(const pkv_oracle_dims* d, const uint16_t* q, const uint16_t* k_cache,
                           const uint16_t* v_cache, const int32_t* block_table,
                           const int32_t* cache_seqlens, double softmax_scale, double* out);

/* Dense fp64 attention with several query tokens per row and masks
 * (flash-attn 2.6.3 semantics for the arguments the reference's evaluator
 * passes, scripts/evaluate_flashattn_submission.py:242-245): q and out are
 * [B, seqlen_q, H, D]; query i of row b sits at position pos = i + L - seqlen_q
 * (L = the row's clamped length) and sees the keys t < L with
 * (!causal || t <= pos), (window_left < 0 || t >= pos - window_left) and
 * (window_right < 0 || t <= pos + window_right); ALiBi (slopes fp32
 * [B, H] at alibi_slopes[b * alibi_batch_stride + h], NULL = none) adds
 * -slope * |pos - t| to the scaled score.  A query without a visible key
 * gives zeros.  out is fp64.  lse (optional, fp64 [B, H, seqlen_q]): each
 * query's log(sum over its visible keys of exp(score)), natural log, +inf for
 * a query without a visible key (flash-attn's softmax_lse).  softcap > 0:
 * each scaled score s becomes softcap * tanh(s / softcap) before the ALiBi
 * term (flash-attn 2.6.3's softcap).  kv_start (optional int32 [B],
 * flash-attn's cache_leftpad): keys t < kv_start[b] are visible to no query
 * of row b; positions are unchanged. */
void pkv_oracle_attn_f64(const pkv_oracle_dims* d, const uint16_t* q, const uint16_t* k_cache,
                         const uint16_t* v_cache, const int32_t* block_table, const int32_t* cache_seqlens,
                         int64_t seqlen_q, int causal, int64_t window_left, int64_t window_right,
                         const float* alibi_slopes, int64_t alibi_batch_stride, double softmax_scale,
                         double* out, double* lse, double softcap, const int32_t* kv_start);

/* OCP FP8 E4M3 ("e4m3fn": no infinities, S.1111.111 = NaN, max 448) to fp32. */
float pkv_oracle_e4m3_to_f32(uint8_t b);

/* pkv_oracle_attn_f64 over FP8 e4m3 caches: element x of KV head kvh stands
 * for e4m3(x) * k_scale[kvh] (v_scale for V; NULL scales = 1). */
void pkv_oracle_attn8_f64(const pkv_oracle_dims* d, const uint16_t* q, const uint8_t* k_cache,
                          const uint8_t* v_cache, const int32_t* block_table, const int32_t* cache_seqlens,
                          int64_t seqlen_q, int causal, int64_t window_left, int64_t window_right,
                          const float* alibi_slopes, int64_t alibi_batch_stride, const float* k_scale,
                          const float* v_scale, double softmax_scale, double* out, double* lse, double softcap,
                          const int32_t* kv_start);

/* Split-KV partition step (best_flashattn_kvcache_decode.cu:664-697, 782-864):
 * split s of row b covers pages [n*s/S, n*(s+1)/S) of its n valid pages;
 * exp2-domain fp32 online softmax; part_o [B*H*S, D] normalised, part_lse
 * [B*H*S] = m2 + log2(sum) or -inf when empty (O = 0 then). */
void pkv_oracle_split_partials(const pkv_oracle_dims* d, const uint16_t* q, const uint16_t* k_cache,
                               const uint16_t* v_cache, const int32_t* block_table,
                               const int32_t* cache_seqlens, float softmax_scale, int splits,
                               float* part_o, float* part_lse);

/* LSE combine (best_flashattn_kvcache_decode.cu:956-1037, v11:604-613):
 * w_s = exp2(lse_s - max) (0 for -inf), out = (sum_s w_s o_s) * (1 / sum_s w_s),
 * o_s never read when w_s == 0.  out is 16-bit [rows, D]. */
void pkv_oracle_combine(const float* part_o, const float* part_lse, int64_t rows, int splits,
                        int64_t head_dim, int32_t dtype, uint16_t* out);

/* Same combine with an fp32 result (for split-invariance checks before the cast). */
void pkv_oracle_combine_f32(const float* part_o, const float* part_lse, int64_t rows, int splits,
                            int64_t head_dim, float* out);

#ifdef __cplusplus
}
#endif

#endif /* PKV_ORACLE_H */
