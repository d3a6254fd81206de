/*
 * pkv_decode.h — C ABI of the MI355X (gfx950) paged-KV GQA flash-attention
 * decode operator.
 *
 * Every entry point takes plain pointers and sizes; nothing here depends on
 * torch or on HIP headers (streams and events are passed as `void*` holding a
 * hipStream_t / hipEvent_t).
 *
 * Tensor layouts (identical to the reference's flash-attn layout,
 * scripts/evaluate_flashattn_submission.py:127-143, 249):
 *   q, out         [B, M, H, D]           16-bit (fp16 or bf16), contiguous (M = seqlen_q, 1 for decode)
 *   k_cache,
 *   v_cache        [num_pages, P, Hk, D]  16-bit like q, or OCP FP8 e4m3 bytes (kv_dtype), contiguous
 *   block_table    [B, block_table_stride] int32 physical page ids
 *   cache_seqlens  [B]                    int32 valid tokens per row
 * Token t of row b lives in page block_table[b][t / P], slot t % P; only
 * t < cache_seqlens[b] is read.  Query head h reads KV head h / (H / Hk).
 */
#ifndef PKV_DECODE_H
#define PKV_DECODE_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* Status codes.  The reference's run_kernel returns void and silently
 * ignores unsupported shapes (submission-oj/best_flashattn_kvcache_decode.cu:1202-1211);
 * every entry point here reports what happened instead. */
#define PKV_OK 0
#define PKV_EINVAL 1           /* null pointer, non-positive or inconsistent dims, misaligned pointer */
#define PKV_EUNSUPPORTED 2     /* dtype / head_dim / page size / path not supported for this shape, or
                                  sizes past the kernels' index range (e.g. 16 * Hk * D * element
                                  bytes >= 2^32: a tile's rows are addressed with 32-bit offsets) */
#define PKV_ENOWORKSPACE 3     /* workspace missing or smaller than pkv_decode_workspace_size() */
#define PKV_ELAUNCH 4          /* a HIP launch or runtime call failed */

#define PKV_DTYPE_F16 0
#define PKV_DTYPE_BF16 1

/* Element type of k_cache / v_cache (pkv_decode_desc.kv_dtype). */
#define PKV_KV_DTYPE_SAME 0     /* desc->dtype, like q and out */
#define PKV_KV_DTYPE_FP8_E4M3 1 /* OCP FP8 e4m3 (1 byte; finite range +-448, no infinities), dequantised as
                                   value * k_scale / v_scale of the KV head; needs the MFMA path */

/* Kernel family selector (pkv_decode_desc.path). */
#define PKV_PATH_AUTO 0        /* measured choice per shape */
#define PKV_PATH_VALU 1        /* VALU dot2 products + DPP row reductions, up to 4 heads per wave */
#define PKV_PATH_MFMA 2        /* gfx950 16x16x32 / 16x16x16 MFMA for QK^T and PV, 16 heads per wave */

/* Work schedules (pkv_decode_schedule). */
#define PKV_SCHED_SINGLE 1     /* one pass per (b, kv head, head group); out written directly */
#define PKV_SCHED_PAGES 2      /* each row's pages cut into num_splits near-equal ranges (the reference's) */
#define PKV_SCHED_WINDOWS 3    /* each row cut into fixed windows of split_tokens tokens */
#define PKV_SCHED_TILES 4      /* the call's 16-token tiles dealt evenly to a fixed set of waves */

/* Masks (pkv_decode_desc.mask), flash-attn 2.6.3 semantics with key positions
 * 0 .. L-1 (L = the row's length) and query i of M at position i + L - M. */
#define PKV_MASK_CAUSAL 1      /* query i sees keys j <= i + L - M (bottom-right aligned) */
#define PKV_MASK_WINDOW 2      /* window_left / window_right apply (each -1 = unbounded) */

/* Largest split count a single call may use (the reference caps at 64,
 * best_flashattn_kvcache_decode.cu:15). */
#define PKV_MAX_SPLITS 256

typedef struct pkv_decode_desc {
    int64_t batch;              /* B */
    int64_t num_heads;          /* H, query heads */
    int64_t num_heads_k;        /* Hk, KV heads; H % Hk == 0 */
    int64_t head_dim;           /* D: 64, 128 or 256 */
    int64_t page_size;          /* P: tokens per page, a power of two in [1, 1024] */
    int64_t num_pages;          /* physical pages held by k_cache / v_cache */
    int64_t block_table_stride; /* int32 elements between consecutive block_table rows */
    int64_t max_seqlen;         /* host-known upper bound of cache_seqlens (flash-attn's seqlen_k);
                                   0 = block_table_stride * page_size.  Used only to choose the
                                   schedule and split count: a row longer than it is still read
                                   whole (every schedule takes row lengths from cache_seqlens,
                                   and the last fixed token window runs to the row's end). */
    int32_t dtype;              /* PKV_DTYPE_F16 or PKV_DTYPE_BF16 (q, caches and out share it) */
    int32_t path;               /* PKV_PATH_* */
    int32_t split_tokens;       /* num_splits == 0 only: tokens per split window (multiple of 16);
                                   0 = the tile-balanced schedule (or, for small or
                                   windowed calls, the single pass) */
    int32_t reserved;           /* must be 0 */
    void* workspace;            /* device memory for split partials; may be NULL when splits == 1 */
    size_t workspace_bytes;
    void* prof_events;          /* optional: hipEvent_t[4] = partition start, partition end, combine
                                   start, combine end, recorded by the kernels' own dispatch packets
                                   (profiling only; NULL in use).  Without a combine, [2] and [3]
                                   are recorded right after the partition. */
    /* Several query tokens per row and masking (a zero-initialised tail = one
     * query token, no mask).  With seqlen_q = M > 1, q and out are
     * [B, M, H, D]; query i of row b sits at position i + L - M, L =
     * cache_seqlens[b] (plus the appended tokens for pkv_decode_append). */
    int64_t seqlen_q;           /* M; 0 or 1 = one query token */
    int32_t mask;               /* PKV_MASK_* bits */
    int32_t window_left;        /* PKV_MASK_WINDOW: keys j >= pos - window_left (-1 = unbounded) */
    int32_t window_right;       /* PKV_MASK_WINDOW: keys j <= pos + window_right (-1 = unbounded);
                                   PKV_MASK_CAUSAL forces 0 */
    int32_t kv_dtype;           /* PKV_KV_DTYPE_*: element type of k_cache / v_cache */
    const float* alibi_slopes;  /* optional fp32 [H] or [B, H]: score -= slope * |pos - j| */
    int64_t alibi_batch_stride; /* 0 for [H] slopes, H for [B, H] */
    const float* k_scale;       /* FP8 caches: optional fp32 [Hk] device array, K = fp8 * k_scale[kv head];
                                   NULL = 1.  The append divides by it before rounding to FP8. */
    const float* v_scale;       /* FP8 caches: the same for V */
    float* softmax_lse;         /* optional fp32 [B, H, M] device array (flash-attn's return_softmax_lse):
                                   log(sum_j exp(softmax_scale * q . k_j + bias_j)) over the keys each
                                   query row attends, natural log; +inf for a row with no visible key
                                   (flash-attn 2.6.3's convention).  NULL = not written. */
    /* Rotary embedding of the appended keys and of q (flash-attn's rotary_cos /
     * rotary_sin / rotary_interleaved; pkv_decode_append only, which then needs
     * seqlen_new >= 1).  New token j of row b is rotated at position
     * max(cache_seqlens[b], 0) + j before it is stored; q token i at that
     * position + i for a causal or windowed call, else at max(cache_seqlens[b], 0)
     * (flash-attn 2.6.3).  Pair (x0, x1) with angle index a becomes
     * (x0 cos[pos][a] - x1 sin[pos][a], x0 sin[pos][a] + x1 cos[pos][a]) in fp32
     * (no fused multiply-add), rounded to the dtype; interleaved pairs are dims
     * (2a, 2a + 1), otherwise (a, a + rotary_dim / 2) (GPT-NeoX); dims from
     * rotary_dim on are unchanged.  V is not rotated. */
    const void* rotary_cos;     /* [rotary_seqlen, rotary_dim / 2], the dtype of q; NULL = no rotary */
    const void* rotary_sin;     /* the same shape and dtype */
    int64_t rotary_seqlen;      /* rows of the tables; at least block_table_stride * page_size */
    int32_t rotary_dim;         /* multiple of 16, at most head_dim */
    int32_t rotary_interleaved; /* 1: pairs (2a, 2a + 1); 0: (a, a + rotary_dim / 2) */
    float softcap;              /* > 0: each scaled score s becomes softcap * tanh(s / softcap) before the
                                   ALiBi bias (flash-attn's softcap, as in Gemma 2); 0 = off.  Needs the
                                   MFMA path. */
    const int32_t* cache_leftpad; /* optional int32 [B] device array (flash-attn's cache_leftpad): row b's
                                   keys at positions below cache_leftpad[b] are padding that no query
                                   sees; the positions of queries, appended tokens and rotary rows do not
                                   change.  Those keys are still read (masked, not skipped).  Needs the
                                   MFMA path; NULL = none. */
} pkv_decode_desc;

/*
 * Paged-KV decode attention:
 *   out[b,h,:] = softmax(softmax_scale * q[b,h,:] . K[b,kvh,t,:]) V[b,kvh,t,:]  over t < cache_seqlens[b]
 * With desc->seqlen_q = M > 1 (speculative-decode verify, chunked prefill
 * over a paged cache), each of the M query tokens of a row attends over the
 * keys its mask leaves (causal, sliding window, ALiBi bias; flash-attn 2.6.3
 * semantics); a query with no visible key gets zeros.  M > 1, masks, ALiBi
 * and a softcap need the MFMA path (PKV_PATH_AUTO or PKV_PATH_MFMA).  With
 * desc->softmax_lse set, each query row's log-sum-exp is written beside it.
 * Replaces the reference's `extern "C" void run_kernel(...)` launch entry
 * (submission-oj/best_flashattn_kvcache_decode.cu:1186-1201) with the
 * north-star argument order and an explicit stream.
 *
 * num_splits follows flash-attn (scripts/evaluate_flashattn_submission.py:246):
 *   0 = heuristic: with desc->split_tokens == 0, the tile-balanced schedule —
 *       all rows' 16-token tiles (times KV heads and head groups) are laid end
 *       to end and dealt in equal shares to one workgroup of waves per CU,
 *       which read cache_seqlens on the device, so every wave streams the same
 *       bytes however ragged the rows are, and a combine merges the rows that
 *       more than one wave touched.  Calls too small to fill the chip
 *       (rows of a few tiles, judged from max_seqlen), and calls whose left
 *       window bounds every row, take the single pass instead when its
 *       longest chain of tiles per wave is no longer: no combine, and no
 *       wave walks several short segments.  With
 *       desc->split_tokens > 0, fixed windows of that many tokens;
 *   1 = single pass writing `out` directly;
 *   n > 1 = forced: each row's valid pages are divided into n near-equal
 *       ranges as the reference does (clamped to [1, min(PKV_MAX_SPLITS,
 *       pages of max_seqlen)]).
 * Rows with cache_seqlens[b] <= 0 produce zeros; a row with one token
 * reproduces that token's V row bit-for-bit (best_flashattn_kvcache_decode.cu:256-283).
 * Asynchronous on `stream` (NULL = the null stream); no host synchronisation.
 * Reentrant when concurrent calls use distinct workspaces.
 */
int pkv_decode(const void* q, const void* k_cache, const void* v_cache,
               const int32_t* block_table, const int32_t* cache_seqlens,
               float softmax_scale, int num_splits, void* out,
               const pkv_decode_desc* desc, void* stream);

/* Bytes of workspace pkv_decode needs for this shape and num_splits (after
 * the same heuristic/clamping pkv_decode applies).  Replaces the reference's
 * hidden grow-only workspace (best_flashattn_kvcache_decode.cu:17-20, 1078-1133). */
size_t pkv_decode_workspace_size(const pkv_decode_desc* desc, int num_splits);

/* Device scratch pkv_decode_noalloc holds on each GPU it runs on: 32 MiB. */
#define PKV_SCRATCH_BYTES ((size_t)32 << 20)

/*
 * pkv_decode for callers that cannot allocate (code under HIP graph capture,
 * tight serving loops, harnesses that forbid allocation).  No counterpart in
 * the reference.  Same arguments and results as pkv_decode, but the split partials go to a
 * scratch buffer of PKV_SCRATCH_BYTES in device memory that the library holds
 * on each GPU for the life of the process (a static device array);
 * desc->workspace and desc->workspace_bytes are ignored.  The call allocates
 * nothing (no hipMalloc, hipFree or allocating library routine); its first
 * call on a GPU looks up that GPU's copy of the buffer, and that is when the
 * GPU commits the buffer's memory: measured on MI355X, loading the library and
 * its first pkv_decode call take 0 and 6 MiB of device memory, the first
 * pkv_decode_noalloc call 34 MiB more; callers that never use this entry point
 * do not pay for the buffer.
 * - A plan that needs more than PKV_SCRATCH_BYTES
 *   (pkv_decode_workspace_size(desc, num_splits) > PKV_SCRATCH_BYTES, e.g.
 *   forced splits over very many rows) returns PKV_ENOWORKSPACE before anything
 *   is enqueued; the heuristic plans of the benchmark configs need at most 21 MB.
 * - `stream` must belong to the current device (PKV_EINVAL otherwise).
 * - Every call on one GPU shares that GPU's buffer: calls that overlap on one
 *   GPU (on other streams, from other host threads) race; serialise them.
 * - The buffer keeps the last call's contents.  No kernel reads a partial the
 *   same call has not written, so nothing needs clearing.
 */
int pkv_decode_noalloc(const void* q, const void* k_cache, const void* v_cache,
                       const int32_t* block_table, const int32_t* cache_seqlens,
                       float softmax_scale, int num_splits, void* out,
                       const pkv_decode_desc* desc, void* stream);

/* Split count pkv_decode will use for `num_splits` (0 = heuristic); for
 * PKV_SCHED_TILES, the number of partition waves sharing the tiles.
 * Replaces choose_splits (best_flashattn_kvcache_decode.cu:1039-1076, 1299-1312).
 * Returns 0 if desc is invalid. */
int pkv_decode_num_splits(const pkv_decode_desc* desc, int num_splits);

/* Schedule (PKV_SCHED_*) pkv_decode will use for `num_splits`; 0 if desc is
 * invalid.  The reference has only single-pass and page-balanced splits
 * (best_flashattn_kvcache_decode.cu:664-671, 1299-1312). */
int pkv_decode_schedule(const pkv_decode_desc* desc, int num_splits);

/* Tokens per split window pkv_decode will use for `num_splits` (0 when the
 * splits are page-balanced or there is a single split).  No counterpart in
 * the reference, which only has page-balanced splits. */
int pkv_decode_split_tokens(const pkv_decode_desc* desc, int num_splits);

/* Kernel family pkv_decode will use for this desc (resolves PKV_PATH_AUTO). */
int pkv_decode_path(const pkv_decode_desc* desc);

/*
 * Paged KV-cache append: writes seqlen_new new tokens per row into the cache,
 * token j of row b at position max(cache_seqlens[b], 0) + j, i.e. slot
 * (pos % P) of page block_table[b][pos / P].
 *   k_new, v_new  [B, seqlen_new, Hk, D]  16-bit (desc->dtype), contiguous, 16-byte aligned
 * FP8 caches (desc->kv_dtype): each value x is stored as the e4m3 value
 * nearest to x * (1 / scale) (fp32 arithmetic, ties to even), saturated to
 * +-448; the scale is the KV head's k_scale / v_scale (1 when NULL).
 * desc is the attention calls' descriptor (it must pass the same checks);
 * the append uses its batch, num_heads_k, head_dim, page_size, num_pages,
 * block_table_stride and dtype, and ignores the workspace.  Positions at or past
 * block_table_stride * P and page ids outside [0, num_pages) are not written.
 * cache_seqlens is read, never updated (the caller advances it, as with
 * flash-attn).  desc->prof_events, when set, are hipEvent_t[2] recorded by
 * the copy kernel's dispatch packet as it starts and completes.  Replaces the in-kernel append of flash-attn 2.6.3's
 * flash_attn_with_kvcache(k=, v=), which the reference's evaluator passes as
 * None (scripts/evaluate_flashattn_submission.py:236-237).
 * Asynchronous on `stream`.
 */
int pkv_append_kv(const void* k_new, const void* v_new, void* k_cache, void* v_cache,
                  const int32_t* block_table, const int32_t* cache_seqlens, int64_t seqlen_new,
                  const pkv_decode_desc* desc, void* stream);

/*
 * Paged KV-cache append by flat slot: token row i of key / value
 * ([num_tokens, Hk, D], 16-bit, contiguous) goes to slot_mapping[i] =
 * page * P + slot of the [num_pages, P, Hk, D] caches; a negative slot is
 * padding and is skipped, a slot >= num_pages * P is not written.  The
 * slot-mapped form of the same copy (vLLM's reshape_and_cache_flash); the
 * reference has no counterpart (its evaluator passes no new tokens,
 * scripts/evaluate_flashattn_submission.py:236-237).  Only desc's
 * num_heads_k, head_dim, page_size, num_pages, dtype and path are read (and
 * checked as pkv_decode checks them); the row-shaped fields may be 0.
 * desc->prof_events as for pkv_append_kv.
 */
int pkv_reshape_and_cache(const void* key, const void* value, void* k_cache, void* v_cache,
                          const int64_t* slot_mapping, int64_t num_tokens, const pkv_decode_desc* desc,
                          void* stream);

/*
 * flash_attn_with_kvcache(q, k_cache, v_cache, k=k_new, v=v_new,
 * cache_seqlens=, block_table=): appends k_new / v_new as pkv_append_kv
 * does, then attends over the first max(cache_seqlens[b], 0) + seqlen_new
 * tokens of each row with the desc's query tokens and masks (flash-attn 2.6.3
 * semantics; the reference's evaluator passes k = v = None,
 * scripts/evaluate_flashattn_submission.py:236-237).  With seqlen_q =
 * seqlen_new and a causal mask this is the speculative-decode verify step.  desc->max_seqlen, when
 * set, bounds cache_seqlens before the append.  The workspace must hold
 * pkv_decode_append_workspace_size(desc, num_splits, seqlen_new) bytes (it
 * always holds the per-row lengths, so it is never NULL); prof_events, when
 * set, time the attention kernels as in pkv_decode.  seqlen_new == 0 is
 * pkv_decode.
 */
int pkv_decode_append(const void* q, const void* k_new, const void* v_new, void* k_cache, void* v_cache,
                      const int32_t* block_table, const int32_t* cache_seqlens, int64_t seqlen_new,
                      float softmax_scale, int num_splits, void* out, const pkv_decode_desc* desc,
                      void* stream);

/* Bytes of workspace pkv_decode_append needs. */
size_t pkv_decode_append_workspace_size(const pkv_decode_desc* desc, int num_splits, int64_t seqlen_new);

/* 1 if pkv_decode_append folds the append into the attention for this call
 * shape (two kernels: the partition attends the cached tokens, the combine
 * adds the new token and stores it in the cache), 0 if it launches the append
 * kernel first and then attends the longer rows (three kernels), -1 if desc
 * is invalid.  Folded: as many new tokens as query tokens, at most 8 (the
 * decode step and the speculative verify step, causal or not), 16-bit or
 * FP8 caches, no window, ALiBi, softcap or rotary tables, the tile schedule
 * with its row-per-wave combine.  The outputs agree within the decode
 * tolerances (the new tokens' scores are summed in a different order); the
 * caches are written identically.  No
 * counterpart in the reference, whose decode never appends
 * (scripts/evaluate_flashattn_submission.py:236-237 passes k = v = None). */
int pkv_decode_append_folds(const pkv_decode_desc* desc, int num_splits, int64_t seqlen_new);

/* Human-readable name of a status code. */
const char* pkv_strerror(int status);

/*
 * Drop-in for the reference's launch entry, same 15 arguments and meaning
 * (submission-oj/best_flashattn_kvcache_decode.cu:1186-1201;
 * scripts/evaluate_flashattn_submission.py:29-44): bf16 tensors,
 * softmax_scale = 1/sqrt(headdim), heuristic splits, null stream,
 * block_table row stride = num_blocks / batch_size, seqlen_k = max seqlen.
 * The reference returns without launching when seqlen_q != 1 or causal != 0
 * (best:1202-1211); here q / output are [B, seqlen_q, H, D] and causal masks
 * bottom-right aligned, as flash-attn does.
 * Like the reference it keeps a grow-only workspace owned by the library
 * and is therefore not reentrant.  Its status is available from
 * pkv_last_status() instead of being dropped.
 */
void run_kernel(const void* q, const void* k_cache_paged, const void* v_cache_paged,
                void* output, const int32_t* cache_seqlens, const int32_t* block_table,
                int64_t batch_size, int64_t seqlen_k, int64_t seqlen_q, int64_t num_heads,
                int64_t num_heads_k, int64_t headdim, int64_t page_block_size,
                int64_t num_blocks, int64_t causal);

/* Status of the calling thread's most recent run_kernel call.  No
 * counterpart in the reference, whose run_kernel discards it. */
int pkv_last_status(void);

#ifdef __cplusplus
}
#endif

#endif /* PKV_DECODE_H */
