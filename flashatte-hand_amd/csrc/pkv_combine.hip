// pkv_combine.hip — LSE combine of split-KV partials on gfx950.
//
// One wave64 per (b, h) row.  The row's non-empty splits are derived from
// cache_seqlens with the same range arithmetic the partition kernel used, so
// slots of empty splits are never read (whatever the workspace holds).  With
// w_s = exp2(lse_s - max_s lse_s), out = (sum_s w_s o_s) * (1 / sum_s w_s),
// cast RNE; a row without tokens gets zeros.  Partial rows are read in
// one batch so their loads are in flight together.
// Reference: submission-oj/best_flashattn_kvcache_decode.cu:956-1037 and
// v11_best_hybrid/flashattn_kvcache_decode_v11_best_hybrid.cu:604-613.
#include "pkv_device.h"
#include "pkv_launch.h"

// Largest split count (PKV_MAX_SPLITS in include/pkv_decode.h).
#define PKV_MAX_SPLITS_DEV 256

namespace pkv {

// Waves (rows) per workgroup; 2, 8 and 16 measured the same.
constexpr int kCombineWaves = 4;

// Waves per output row of combine_row_group_kernel.
constexpr int kRowGroupWaves = 8;

__device__ __forceinline__ bool split_nonempty(const CombineParams& p, int seqlen, int s) {
    const TokenRange r = visible_split_tokens(seqlen, p.q_len, p.win_left, p.page_shift, s, p.splits, p.split_tokens);
    return r.begin < r.end;
}

template <int E>
__device__ __forceinline__ void load_partial(const float* src, float (&x)[E]) {
    if constexpr (E == 4) {
        const float4 t = *reinterpret_cast<const float4*>(src);
        x[0] = t.x; x[1] = t.y; x[2] = t.z; x[3] = t.w;
    } else if constexpr (E == 2) {
        const float2 t = *reinterpret_cast<const float2*>(src);
        x[0] = t.x; x[1] = t.y;
    } else {
#pragma unroll
        for (int e = 0; e < E; ++e) {
            x[e] = src[e];
        }
    }
}

// Two dependent memory round trips per row: cache_seqlens, then the partial
// rows of the first kBatch splits together with the per-split LSEs (lane s
// holds split s + 64k).  Weights reach every lane with readlane; partials are
// folded in with a select, so an unused slot cannot inject NaN.
template <bool BF16, int D>
__global__ __launch_bounds__(64 * kCombineWaves) void combine_kernel(CombineParams p) {
    constexpr int E = D / 64; // output elements per lane
    constexpr int kBatch = 16;
    constexpr int kLseRegs = (PKV_MAX_SPLITS_DEV + 63) / 64;
    static_assert(E >= 1 && E <= 8, "head_dim must be 64..512");
    const int lane = threadIdx.x & 63;
    const int row = blockIdx.x * (blockDim.x >> 6) + (threadIdx.x >> 6);
    if (row >= p.rows) {
        return;
    }
    // Output row (b, i, h) of [B, M, H]; its partials sit at query row
    // sr = (b * Hk + kv head) * M * group + i * group + g (= row when M = 1).
    const int per_b = p.q_len * p.num_heads;
    const int b = row / per_b;
    const int i = (row - b * per_b) / p.num_heads;
    const int h = row - b * per_b - i * p.num_heads;
    const int kvh = h / p.group;
    const int64_t sr = (static_cast<int64_t>(b) * (p.num_heads / p.group) + kvh) * p.q_len * p.group +
                       i * p.group + (h - kvh * p.group);
    const int seqlen = min(p.seqlens[b], p.row_cap);
    // Splits past the last token window are empty in split_tokens mode (the
    // last split runs to the row's end, so a row longer than splits windows
    // has all of them).
    const int n_loop = p.split_tokens > 0
                           ? (seqlen > 0 ? min(p.splits, seqlen / p.split_tokens + (seqlen % p.split_tokens != 0))
                                         : 0)
                           : p.splits;
    const float* __restrict__ lse = p.part_lse + sr * p.splits;
    const float* __restrict__ o = p.part_o + sr * p.splits * D + lane * E;

    // First batch of partial rows, issued before the LSE loads are consumed.
    float x[kBatch][E];
    bool ok[kBatch];
#pragma unroll
    for (int u = 0; u < kBatch; ++u) {
        ok[u] = u < n_loop && split_nonempty(p, seqlen, u);
#pragma unroll
        for (int e = 0; e < E; ++e) {
            x[u][e] = 0.f;
        }
        if (ok[u]) {
            load_partial<E>(o + u * D, x[u]);
        }
    }

    float lw[kLseRegs];
    float mx = kNegInf;
#pragma unroll
    for (int k = 0; k < kLseRegs; ++k) {
        const int s = lane + 64 * k;
        lw[k] = (s < n_loop && split_nonempty(p, seqlen, s)) ? lse[s] : kNegInf;
        mx = fmaxf(mx, lw[k]);
    }
    mx = group_max<64>(mx);
    float den = 0.f;
#pragma unroll
    for (int k = 0; k < kLseRegs; ++k) {
        lw[k] = lw[k] == kNegInf ? 0.f : fast_exp2(lw[k] - mx); // weight of split lane + 64k
        den += lw[k];
    }
    den = group_sum<64>(den);
    const float inv = den > 0.f ? 1.f / den : 0.f;

    float acc[E];
#pragma unroll
    for (int e = 0; e < E; ++e) {
        acc[e] = 0.f;
    }
#pragma unroll
    for (int u = 0; u < kBatch; ++u) {
        const float w = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(lw[0]), u));
#pragma unroll
        for (int e = 0; e < E; ++e) {
            acc[e] = ok[u] ? fmaf(w, x[u][e], acc[e]) : acc[e];
        }
    }
    for (int s = kBatch; s < n_loop; ++s) { // long rows: one split at a time
        if (!split_nonempty(p, seqlen, s)) {
            continue;
        }
        float y[E];
        load_partial<E>(o + static_cast<int64_t>(s) * D, y);
        int wk = 0;
#pragma unroll
        for (int k = 1; k < kLseRegs; ++k) {
            wk = s >= 64 * k ? __float_as_int(lw[k]) : wk;
        }
        const float wsel = s < 64 ? lw[0] : __int_as_float(wk);
        const float w = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(wsel), s & 63));
#pragma unroll
        for (int e = 0; e < E; ++e) {
            acc[e] = fmaf(w, y[e], acc[e]);
        }
    }
    uint16_t* dst = p.out + static_cast<int64_t>(row) * D + lane * E;
#pragma unroll
    for (int e = 0; e < E; ++e) {
        dst[e] = from_f32<BF16>(acc[e] * inv);
    }
    if (p.lse != nullptr && lane == 0) {
        store_lse(p.lse, row, p.q_len, p.num_heads, mx, den);
    }
}

// Row b's tiles, and the stream units of the rows before b and of all rows
// (tile-balanced schedule), from one pass over cache_seqlens: one round trip.
struct RowUnits {
    int32_t nb;
    int64_t before;
    int64_t all;
};

__device__ __forceinline__ RowUnits row_units(const CombineParams& p, int32_t b, int lane) {
    int64_t before = 0;
    int64_t all = 0;
    int32_t nb = 0;
    // The first kScanChunks * 64 rows: every load out before any is used, with no
    // branch around them (lanes past the batch re-read its last row and are
    // dropped), so they cost one round trip, not one per chunk.
    int32_t raw[kScanChunks];
#pragma unroll
    for (int c = 0; c < kScanChunks; ++c) {
        raw[c] = p.seqlens[min(64 * c + lane, p.batch - 1)];
    }
#pragma unroll
    for (int c = 0; c < kScanChunks; ++c) {
        const int32_t bb = 64 * c + lane;
        const int32_t n = bb < p.batch ? tile_span(min(max(raw[c], 0), p.row_cap), p.q_len, p.win_left).n : 0;
        const int32_t t = stream_units(n);
        all += t;
        before += bb < b ? t : 0;
        nb = bb == b ? n : nb;
    }
    for (int32_t bb = lane + 64 * kScanChunks; bb < p.batch; bb += 64) {
        const int32_t n = row_tiles(p.seqlens, bb, p.row_cap, p.q_len, p.win_left);
        const int32_t t = stream_units(n);
        all += t;
        before += bb < b ? t : 0;
        nb = bb == b ? n : nb;
    }
    RowUnits ru;
    ru.nb = __builtin_amdgcn_readlane(nb, b & 63); // lane b % 64 saw row b
    ru.before = uniform(wave_sum_i64(before));
    ru.all = uniform(wave_sum_i64(all));
    return ru;
}

// Where stream u of row b left its partials (tile-balanced schedule, gangs of
// G = 2^gang_shift waves): the gangs g_a .. g_b owning its tiles, found from
// cache_seqlens with the partition's unit arithmetic, and the slot of part 0;
// part k is in slot slot0 + G k.
struct StreamParts {
    int32_t parts; // g_b - g_a + 1
    int64_t slot0;
};

__device__ __forceinline__ StreamParts stream_parts(const CombineParams& p, const RowUnits& ru, int32_t b, int32_t u) {
    const int gs = p.gang_shift;
    const int sps = ((p.num_heads / p.group) * p.head_groups) >> gs;
    const int us = u >> gs; // super-stream of row b
    const int64_t first =
        static_cast<int64_t>(sps) * ru.before + static_cast<int64_t>(us) * stream_units(ru.nb) + kHeaderTiles;
    const TilePlan plan = make_tile_plan(static_cast<int64_t>(sps) * ru.all, p.tile_workers >> gs);
    const int32_t ga = tile_worker_of(first, plan.total, plan.workers);
    const int32_t gb = tile_worker_of(first + ru.nb - 1, plan.total, plan.workers);
    StreamParts sp;
    sp.parts = gb - ga + 1;
    sp.slot0 = ((static_cast<int64_t>(ga) + static_cast<int64_t>(b) * sps + us) << gs) + (u & ((1 << gs) - 1));
    return sp;
}

// Parts [k0, k1) of one query row (lse / po at part 0, parts lse_stride LSEs
// and o_stride floats apart): their wave-uniform LSE max (-inf when there are
// none or all are empty), the sum of their weights exp2(lse - max) and the
// weighted sum of their rows (the lane's E dims).  A part whose rows saw no
// visible key (masks) has lse = -inf and weighs 0.  One round trip for up to
// 64 parts and kBatch rows: the LSEs (lane k holds part k0 + k) and the first
// kBatch partial rows are loaded together; more parts take kBatch rows per
// further round trip.
template <int E, int kBatch>
__device__ __forceinline__ void merge_parts(const float* __restrict__ lse, const float* __restrict__ po,
                                            int64_t lse_stride, int64_t o_stride, int k0, int k1, int lane,
                                            float& mx_out, float& den_out, float (&acc)[E]) {
    static_assert(kBatch <= 64 && 64 % kBatch == 0, "a batch of parts takes its weights from one LSE lane each");
    const int n = k1 - k0;
    lse += k0 * lse_stride;
    po += k0 * o_stride;
    const float l0 = lane < n ? lse[lane * lse_stride] : kNegInf;
    float x[kBatch][E];
#pragma unroll
    for (int v = 0; v < kBatch; ++v) {
#pragma unroll
        for (int e = 0; e < E; ++e) {
            x[v][e] = 0.f;
        }
        if (v < n) {
            load_partial<E>(po + v * o_stride, x[v]);
        }
    }
    float mx = l0;
    for (int k = lane + 64; k < n; k += 64) {
        mx = fmaxf(mx, lse[k * lse_stride]);
    }
    mx = group_max<64>(mx);
#pragma unroll
    for (int e = 0; e < E; ++e) {
        acc[e] = 0.f;
    }
    float wl = (lane < n && l0 != kNegInf) ? fast_exp2(l0 - mx) : 0.f;
    float den = wl;
#pragma unroll
    for (int v = 0; v < kBatch; ++v) {
        const float wv = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(wl), v));
#pragma unroll
        for (int e = 0; e < E; ++e) {
            acc[e] = fmaf(wv, x[v][e], acc[e]); // x = 0 past the last part
        }
    }
#pragma unroll 1
    for (int k = kBatch; k < n; k += kBatch) {
        if ((k & 63) == 0) {
            const int kl = k + lane;
            const float lk = kl < n ? lse[kl * lse_stride] : kNegInf;
            wl = lk != kNegInf ? fast_exp2(lk - mx) : 0.f;
            den += wl;
        }
        float y[kBatch][E];
#pragma unroll
        for (int v = 0; v < kBatch; ++v) {
#pragma unroll
            for (int e = 0; e < E; ++e) {
                y[v][e] = 0.f;
            }
            if (k + v < n) {
                load_partial<E>(po + (k + v) * o_stride, y[v]);
            }
        }
#pragma unroll
        for (int v = 0; v < kBatch; ++v) {
            const float wv = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(wl), (k + v) & 63));
#pragma unroll
            for (int e = 0; e < E; ++e) {
                acc[e] = fmaf(wv, y[v][e], acc[e]);
            }
        }
    }
    mx_out = mx;
    den_out = group_sum<64>(den);
}

// Output row `row` of [B, M, H] in the tile-balanced schedule: query row
// r = i * group + g of stream u = kv head * head_groups + r / heads_per_wave of
// row b, and its index hn among the stream's rows.
struct TileRow {
    int b;
    int u;
    int hn;
};

__device__ __forceinline__ TileRow tile_row(const CombineParams& p, int row) {
    const int per_b = p.q_len * p.num_heads;
    const int b = row / per_b;
    const int i = (row - b * per_b) / p.num_heads;
    const int h = row - b * per_b - i * p.num_heads;
    const int kvh = h / p.group;
    const int r = i * p.group + (h - kvh * p.group);
    const int hg = r / p.heads_per_wave;
    TileRow t;
    t.b = b;
    t.u = kvh * p.head_groups + hg;
    t.hn = r - p.heads_per_wave * hg;
    return t;
}

// The decode step's fold on 16-bit caches (one new token, one query token):
// the general form below with n = 1, written for its registers (the general
// form needs more and drops the kernel to 3 waves per SIMD at head_dim 256).
// Row (b, h) of a decode with a one-token append (fold arguments f): the
// partition attended the row's cache_seqlens[b] cached tokens and left every
// stream's parts in partial slots (force_partial); the new token j = L (its
// position) joins them here as one more part of weight exp2(s - max), s the
// log2-domain score q . k_new, with value v_new.  Its K and V rows go to slot
// L of the row's block table, written by the row of the first query head of
// each KV head.  A position past the block-table row is neither written nor
// attended (the append kernel skips it too); a page id outside
// [0, num_pages) is not written, and the token is attended from k_new.
template <bool BF16, int D, int kBatch>
__device__ __forceinline__ void combine_append_one(const CombineParams& p, const FoldParams& f, const TileRow& t,
                                                   int row, int lane, uint16_t* dst) {
    constexpr int E = D / 64;
    const int h = row - t.b * p.num_heads;
    const int hk = p.num_heads / p.group;
    const int kvh = h / p.group;
    const int64_t new_row = (static_cast<int64_t>(t.b) * hk + kvh) * D + lane * E;
    // Loads that do not wait on cache_seqlens: q, k_new, v_new.
    float qv[E], kv[E], vv[E];
    uint16_t kb[E], vb[E];
#pragma unroll
    for (int e = 0; e < E; ++e) {
        const uint16_t qb = f.q[static_cast<int64_t>(row) * D + lane * E + e];
        kb[e] = f.k[new_row + e];
        vb[e] = f.v[new_row + e];
        float a, b;
        unpack2<BF16>(static_cast<uint32_t>(qb) | (static_cast<uint32_t>(kb[e]) << 16), a, b);
        qv[e] = a;
        kv[e] = b;
        unpack2<BF16>(static_cast<uint32_t>(vb[e]), a, b);
        vv[e] = a;
    }
    const int32_t L = clamped_seqlen(p.seqlens, t.b, p.row_cap);
    const RowUnits ru = row_units(p, t.b, lane);
    float mx = kNegInf;
    float den = 0.f;
    float acc[E];
#pragma unroll
    for (int e = 0; e < E; ++e) {
        acc[e] = 0.f;
    }
    if (ru.nb > 0) {
        const StreamParts sp = stream_parts(p, ru, t.b, t.u);
        const int64_t lse_stride = static_cast<int64_t>(p.part_heads) << p.gang_shift;
        merge_parts<E, kBatch>(p.part_lse + sp.slot0 * p.part_heads + t.hn,
                               p.part_o + (sp.slot0 * p.part_heads + t.hn) * D + lane * E, lse_stride,
                               lse_stride * D, 0, sp.parts, lane, mx, den, acc);
    }
    const int32_t raw = p.seqlens[t.b];
    const bool fits = uniform(max(raw, 0)) < p.row_cap;
    if (fits) {
        // cache_leftpad at or past the new token's position hides it from the query.
        if (f.kv_start == nullptr || L >= uniform(f.kv_start[t.b])) {
            float s = 0.f;
#pragma unroll
            for (int e = 0; e < E; ++e) {
                s = fmaf(qv[e], kv[e], s);
            }
            s = group_sum<64>(s) * f.scale_log2;
            const float m2 = fmaxf(mx, s);
            const float a = mx == kNegInf ? 0.f : fast_exp2(mx - m2);
            const float w = fast_exp2(s - m2);
            den = den * a + w;
            mx = m2;
#pragma unroll
            for (int e = 0; e < E; ++e) {
                acc[e] = fmaf(w, vv[e], acc[e] * a);
            }
        }
        if (h == kvh * p.group) {
            const int32_t page = f.block_table[static_cast<int64_t>(t.b) * f.bt_stride + (L >> p.page_shift)];
            if (page >= 0 && page < f.num_pages) {
                const int64_t slot = (static_cast<int64_t>(page) << p.page_shift) | (L & ((1 << p.page_shift) - 1));
                const int64_t at = (slot * hk + kvh) * D + lane * E;
#pragma unroll
                for (int e = 0; e < E; ++e) {
                    f.k_cache[at + e] = kb[e];
                    f.v_cache[at + e] = vb[e];
                }
            }
        }
    }
    const float inv = den > 0.f ? 1.f / den : 0.f;
#pragma unroll
    for (int e = 0; e < E; ++e) {
        dst[e] = from_f32<BF16>(acc[e] * inv);
    }
    if (p.lse != nullptr && lane == 0) {
        store_lse(p.lse, row, 1, p.num_heads, mx, den);
    }
}

// Most new tokens a folded append adds per row (query tokens per row then).
constexpr int kMaxFold = 8;

// Two OCP e4m3 bytes (bytes 0-1, or 2-3 with HI) to two bf16 values, exactly
// (every e4m3 value is a bf16 value).
template <bool HI>
__device__ __forceinline__ uint32_t fp8x2_to_bf16(uint32_t x) {
    return __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_scalef32_pk_bf16_fp8(x, 1.0f, HI));
}

// E values of the compute dtype to E OCP e4m3 bytes (packed, lane order):
// x * inv in fp32, saturated to +-448, rounded to nearest even, as the append
// kernel stores them; and the bytes' exact values back in fp32.
template <int E>
__device__ __forceinline__ uint32_t quantize_e(const float (&x)[E], float inv, float (&back)[E]) {
    float y[4] = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int e = 0; e < E; ++e) {
        const float v = x[e] * inv;
        y[e] = fabsf(v) > 448.f ? copysignf(448.f, v) : v;
    }
    uint32_t w = static_cast<uint32_t>(__builtin_amdgcn_cvt_pk_fp8_f32(y[0], y[1], 0, false));
    w = static_cast<uint32_t>(__builtin_amdgcn_cvt_pk_fp8_f32(y[2], y[3], static_cast<int>(w), true));
    float a, b;
    unpack2<true>(fp8x2_to_bf16<false>(w), a, b);
    back[0] = a;
    if constexpr (E > 1) {
        back[1] = b;
    }
    if constexpr (E > 2) {
        unpack2<true>(fp8x2_to_bf16<true>(w), a, b);
        back[2] = a;
        back[3] = b;
    }
    return w;
}

// Output row (b, i, h) of a decode whose n = q_len new tokens are folded in
// (fold arguments f; the speculative-decode form: new token j sits at position
// L + j, L = max(cache_seqlens[b], 0), and query i at L + i).  The partition
// attended the row's cached tokens (all of them: every query sits past them)
// and left every stream's parts in partial slots (force_partial); here the new
// tokens query i sees (j <= i when causal, all n otherwise) join as parts of
// weight exp2(s_j - max), s_j the log2-domain score q . k_j, with value v_j.
// FP8 caches: k_j and v_j are quantised as the append stores them and
// attended as those bytes' values (times the KV head's scales).  Token j's K
// and V rows go to slot L + j of the row's block table, written by the wave
// of query j and the first query head of each KV head.  A position past the
// block-table row is neither written nor attended (the append kernel skips
// it too); a page id outside [0, num_pages) is not written, and the token is
// attended from k_new.
template <bool BF16, int D, int kBatch, bool FP8, int NF>
__device__ __forceinline__ void combine_append_row(const CombineParams& p, const FoldParams& f, const TileRow& t,
                                                   int row, int lane, uint16_t* dst) {
    constexpr int E = D / 64;
    const int n = p.q_len;
    const int per_b = n * p.num_heads;
    const int i = (row - t.b * per_b) / p.num_heads;
    const int h = row - t.b * per_b - i * p.num_heads;
    const int hk = p.num_heads / p.group;
    const int kvh = h / p.group;
    const int seen = f.causal ? i + 1 : n; // new tokens query i attends
    // Loads that do not wait on cache_seqlens: q and the new tokens' rows.
    static_assert(NF >= 1 && NF <= kMaxFold, "new tokens per row");
    float qv[E];
    float kv[NF][E];
    float vv[NF][E];
#pragma unroll
    for (int e = 0; e < E; ++e) {
        float a, b;
        unpack2<BF16>(static_cast<uint32_t>(f.q[static_cast<int64_t>(row) * D + lane * E + e]), a, b);
        qv[e] = a;
    }
#pragma unroll
    for (int j = 0; j < NF; ++j) {
        if (j < seen) {
            const int64_t at = ((static_cast<int64_t>(t.b) * n + j) * hk + kvh) * D + lane * E;
#pragma unroll
            for (int e = 0; e < E; ++e) {
                float a, b;
                unpack2<BF16>(static_cast<uint32_t>(f.k[at + e]) | (static_cast<uint32_t>(f.v[at + e]) << 16),
                              a, b);
                kv[j][e] = a;
                vv[j][e] = b;
            }
        }
    }
    const int32_t raw = p.seqlens[t.b];
    const RowUnits ru = row_units(p, t.b, lane);
    float mx = kNegInf;
    float den = 0.f;
    float acc[E];
#pragma unroll
    for (int e = 0; e < E; ++e) {
        acc[e] = 0.f;
    }
    if (ru.nb > 0) {
        const StreamParts sp = stream_parts(p, ru, t.b, t.u);
        const int64_t lse_stride = static_cast<int64_t>(p.part_heads) << p.gang_shift;
        merge_parts<E, kBatch>(p.part_lse + sp.slot0 * p.part_heads + t.hn,
                               p.part_o + (sp.slot0 * p.part_heads + t.hn) * D + lane * E, lse_stride,
                               lse_stride * D, 0, sp.parts, lane, mx, den, acc);
    }
    const int32_t base = uniform(max(raw, 0));
    float score_log2 = f.scale_log2;
    float v_mul = 1.f;
    float inv_k = 1.f;
    float inv_v = 1.f;
    if constexpr (FP8) {
        if (f.k_scale != nullptr) {
            score_log2 *= f.k_scale[kvh];
            inv_k = 1.f / f.k_scale[kvh];
        }
        if (f.v_scale != nullptr) {
            v_mul = f.v_scale[kvh];
            inv_v = 1.f / f.v_scale[kvh];
        }
    }
    // cache_leftpad: new tokens below it are stored but attended by no query.
    const int32_t pad = f.kv_start != nullptr ? uniform(f.kv_start[t.b]) : 0;
#pragma unroll
    for (int j = 0; j < NF; ++j) {
        const int32_t pos = base + j;
        if (j >= seen || pos >= p.row_cap) {
            break;
        }
        uint32_t kq = 0;
        uint32_t vq = 0;
        if constexpr (FP8) {
            kq = quantize_e<E>(kv[j], inv_k, kv[j]);
            vq = quantize_e<E>(vv[j], inv_v, vv[j]);
        }
        if (pos >= pad) {
            float s = 0.f;
#pragma unroll
            for (int e = 0; e < E; ++e) {
                s = fmaf(qv[e], kv[j][e], s);
            }
            s = group_sum<64>(s) * score_log2;
            const float m2 = fmaxf(mx, s);
            const float a = mx == kNegInf ? 0.f : fast_exp2(mx - m2);
            const float w = fast_exp2(s - m2);
            den = den * a + w;
            mx = m2;
#pragma unroll
            for (int e = 0; e < E; ++e) {
                acc[e] = fmaf(w, vv[j][e] * v_mul, acc[e] * a);
            }
        }
        if (i == j && h == kvh * p.group) {
            const int32_t page = f.block_table[static_cast<int64_t>(t.b) * f.bt_stride + (pos >> p.page_shift)];
            if (page >= 0 && page < f.num_pages) {
                const int64_t slot = (static_cast<int64_t>(page) << p.page_shift) | (pos & ((1 << p.page_shift) - 1));
                const int64_t at = (slot * hk + kvh) * D + lane * E;
                if constexpr (FP8) {
                    uint8_t* kc = reinterpret_cast<uint8_t*>(f.k_cache);
                    uint8_t* vc = reinterpret_cast<uint8_t*>(f.v_cache);
                    if constexpr (E == 4) {
                        *reinterpret_cast<uint32_t*>(kc + at) = kq;
                        *reinterpret_cast<uint32_t*>(vc + at) = vq;
                    } else if constexpr (E == 2) {
                        *reinterpret_cast<uint16_t*>(kc + at) = static_cast<uint16_t>(kq);
                        *reinterpret_cast<uint16_t*>(vc + at) = static_cast<uint16_t>(vq);
                    } else {
                        kc[at] = static_cast<uint8_t>(kq);
                        vc[at] = static_cast<uint8_t>(vq);
                    }
                } else {
                    const int64_t src = ((static_cast<int64_t>(t.b) * n + j) * hk + kvh) * D + lane * E;
#pragma unroll
                    for (int e = 0; e < E; ++e) {
                        f.k_cache[at + e] = f.k[src + e];
                        f.v_cache[at + e] = f.v[src + e];
                    }
                }
            }
        }
    }
    const float inv = den > 0.f ? 1.f / den : 0.f;
#pragma unroll
    for (int e = 0; e < E; ++e) {
        dst[e] = from_f32<BF16>(acc[e] * inv);
    }
    if (p.lse != nullptr && lane == 0) {
        store_lse(p.lse, row, p.q_len, p.num_heads, mx, den);
    }
}

// Tile-balanced schedule: row (b, h) belongs to stream u of row b; its parts
// are located by stream_parts.  One part means the partition already wrote
// the row; a row without tokens gets zeros; otherwise the partials in slots
// slot0, slot0 + G, ... are merged with their LSEs, kBatch partial rows in flight
// at a time: 16, or for streams of many parts (long rows) as many as 128
// registers hold, so such a row takes one round trip instead of several.
// LSE: the row's softmax_lse is written when p.lse is set (a kernel without it
// for the calls that ask for none).
template <bool BF16, int D, int kBatch, bool LSE>
__global__ __launch_bounds__(64 * kCombineWaves) void combine_tiles_kernel(CombineParams p) {
    constexpr int E = D / 64;
    const int lane = threadIdx.x & 63;
    const int row = blockIdx.x * (blockDim.x >> 6) + (threadIdx.x >> 6);
    if (row >= p.rows) {
        return;
    }
    const TileRow t = tile_row(p, row);
    uint16_t* dst = p.out + static_cast<int64_t>(row) * D + lane * E;
    const RowUnits ru = row_units(p, t.b, lane);
    if (ru.nb == 0) {
#pragma unroll
        for (int e = 0; e < E; ++e) {
            dst[e] = 0;
        }
        if (LSE && p.lse != nullptr && lane == 0) {
            store_lse(p.lse, row, p.q_len, p.num_heads, 0.f, 0.f);
        }
        return;
    }
    const StreamParts sp = stream_parts(p, ru, t.b, t.u);
    if (sp.parts == 1) {
        return;
    }
    const int64_t lse_stride = static_cast<int64_t>(p.part_heads) << p.gang_shift;
    float mx;
    float den;
    float acc[E];
    merge_parts<E, kBatch>(p.part_lse + sp.slot0 * p.part_heads + t.hn,
                           p.part_o + (sp.slot0 * p.part_heads + t.hn) * D + lane * E, lse_stride, lse_stride * D, 0,
                           sp.parts, lane, mx, den, acc);
    const float inv = den > 0.f ? 1.f / den : 0.f;
#pragma unroll
    for (int e = 0; e < E; ++e) {
        dst[e] = from_f32<BF16>(acc[e] * inv);
    }
    if (LSE && p.lse != nullptr && lane == 0) {
        store_lse(p.lse, row, p.q_len, p.num_heads, mx, den);
    }
}

// The tile combine of a decode with its append folded in (fold arguments f):
// APPEND 1 = 16-bit caches, 2 = FP8 caches; NF new tokens per row at most.
template <bool BF16, int D, int kBatch, int APPEND, int NF>
__global__ __launch_bounds__(64 * kCombineWaves) void combine_fold_kernel(CombineParams p, FoldParams f) {
    constexpr int E = D / 64;
    const int lane = threadIdx.x & 63;
    const int row = blockIdx.x * (blockDim.x >> 6) + (threadIdx.x >> 6);
    if (row >= p.rows) {
        return;
    }
    const TileRow t = tile_row(p, row);
    uint16_t* dst = p.out + static_cast<int64_t>(row) * D + lane * E;
    if constexpr (APPEND == 1 && NF == 1) {
        combine_append_one<BF16, D, kBatch>(p, f, t, row, lane, dst);
    } else {
        combine_append_row<BF16, D, kBatch, APPEND == 2, NF>(p, f, t, row, lane, dst);
    }
}

// Streams of very many parts (a few long rows split over the whole chip: one
// row of 60K tokens has 256 parts per stream): a workgroup of kRowGroupWaves
// waves per output row, wave w merging a contiguous 1/kRowGroupWaves of the
// parts, then wave 0 merging the waves' (max, weight sum, weighted rows)
// through LDS.  Every part's loads are then in flight in the first round trip
// instead of one batch per round trip on one wave.  Exits before the barrier
// depend on the row only, so they are uniform over the workgroup.
template <bool BF16, int D, int kBatch>
__global__ __launch_bounds__(64 * kRowGroupWaves) void combine_row_group_kernel(CombineParams p) {
    constexpr int E = D / 64;
    __shared__ float s_acc[kRowGroupWaves][D];
    __shared__ float s_mx[kRowGroupWaves];
    __shared__ float s_den[kRowGroupWaves];
    const int lane = threadIdx.x & 63;
    const int wave = threadIdx.x >> 6;
    const int row = blockIdx.x;
    const TileRow t = tile_row(p, row);
    uint16_t* dst = p.out + static_cast<int64_t>(row) * D + lane * E;

    const RowUnits ru = row_units(p, t.b, lane);
    if (ru.nb == 0) {
        if (wave == 0) {
#pragma unroll
            for (int e = 0; e < E; ++e) {
                dst[e] = 0;
            }
            if (p.lse != nullptr && lane == 0) {
                store_lse(p.lse, row, p.q_len, p.num_heads, 0.f, 0.f);
            }
        }
        return;
    }
    const StreamParts sp = stream_parts(p, ru, t.b, t.u);
    if (sp.parts == 1) {
        return;
    }
    const int per = (sp.parts + kRowGroupWaves - 1) / kRowGroupWaves;
    const int k0 = min(sp.parts, wave * per);
    const int k1 = min(sp.parts, k0 + per);
    const int64_t lse_stride = static_cast<int64_t>(p.part_heads) << p.gang_shift;
    float mx;
    float den;
    float acc[E];
    merge_parts<E, kBatch>(p.part_lse + sp.slot0 * p.part_heads + t.hn,
                           p.part_o + (sp.slot0 * p.part_heads + t.hn) * D + lane * E, lse_stride, lse_stride * D, k0,
                           k1, lane, mx, den, acc);
#pragma unroll
    for (int e = 0; e < E; ++e) {
        s_acc[wave][lane * E + e] = acc[e];
    }
    if (lane == 0) {
        s_mx[wave] = mx;
        s_den[wave] = den;
    }
    __syncthreads();
    if (wave != 0) {
        return;
    }
    float m = kNegInf;
#pragma unroll
    for (int w = 0; w < kRowGroupWaves; ++w) {
        m = fmaxf(m, s_mx[w]);
    }
    float tot = 0.f;
    float out[E];
#pragma unroll
    for (int e = 0; e < E; ++e) {
        out[e] = 0.f;
    }
    // A wave whose parts are all empty (or that has none) has mx = -inf and
    // weighs 0; so does every wave when all parts are empty (m = -inf).
#pragma unroll
    for (int w = 0; w < kRowGroupWaves; ++w) {
        const float sc = s_mx[w] == kNegInf ? 0.f : fast_exp2(s_mx[w] - m);
        tot = fmaf(sc, s_den[w], tot);
#pragma unroll
        for (int e = 0; e < E; ++e) {
            out[e] = fmaf(sc, s_acc[w][lane * E + e], out[e]);
        }
    }
    const float inv = tot > 0.f ? 1.f / tot : 0.f;
#pragma unroll
    for (int e = 0; e < E; ++e) {
        dst[e] = from_f32<BF16>(out[e] * inv);
    }
    if (p.lse != nullptr && lane == 0) {
        store_lse(p.lse, row, p.q_len, p.num_heads, m, tot);
    }
}

// Tile-balanced schedule, few parts per stream: one wave per block of
// kStreamRows query rows of a stream.  The stream's workers are located once
// for the block, and the LSEs and first partial rows of all its rows are
// loaded together (one round trip for all of them), so the grid has one wave
// per stream block instead of one per output row: 4-8x fewer waves to
// dispatch, the same loads.  Long streams (many parts) use
// combine_tiles_kernel, whose waves take one row each.  (kStreamRows rows per
// wave, pkv_device.h.)

template <bool BF16, int D>
__global__ __launch_bounds__(64 * kCombineWaves) void combine_streams_kernel(CombineParams p) {
    constexpr int E = D / 64;
    constexpr int RB = kStreamRows;
    constexpr int KB = 16 / E; // partial rows per query row and round trip (divides 64)
    const int lane = threadIdx.x & 63;
    const int wid = static_cast<int>(blockIdx.x) * kCombineWaves + static_cast<int>(threadIdx.x >> 6);
    const int spr = (p.num_heads / p.group) * p.head_groups;
    const int blocks = (p.part_heads + RB - 1) / RB;
    const int s = wid / blocks;
    if (s >= p.batch * spr) {
        return;
    }
    const int b = s / spr;
    const int u = s - b * spr;
    const int kvh = u / p.head_groups;
    const int hg = u - kvh * p.head_groups;
    const int r_first = (wid - s * blocks) * RB; // first row of the block within the stream
    const int rows_here = min(RB, min(p.heads_per_wave, p.q_len * p.group - hg * p.heads_per_wave) - r_first);
    if (rows_here <= 0) {
        return;
    }
    // Output row of stream row r: query row qr = i * group + g of (b, kvh).
    auto out_row = [&](int r) -> int64_t {
        const int qr = hg * p.heads_per_wave + r_first + r;
        const int i = qr / p.group;
        const int g = qr - i * p.group;
        return (static_cast<int64_t>(b) * p.q_len + i) * p.num_heads + kvh * p.group + g;
    };

    const RowUnits ru = row_units(p, b, lane);
    const int nb = ru.nb;
    if (nb == 0) {
        for (int r = 0; r < rows_here; ++r) {
            uint16_t* dst = p.out + out_row(r) * D + lane * E;
#pragma unroll
            for (int e = 0; e < E; ++e) {
                dst[e] = 0;
            }
            if (p.lse != nullptr && lane == 0) {
                store_lse(p.lse, out_row(r), p.q_len, p.num_heads, 0.f, 0.f);
            }
        }
        return;
    }
    const StreamParts sp = stream_parts(p, ru, b, u);
    if (sp.parts == 1) {
        return; // one worker: the partition wrote these rows
    }
    const int parts = sp.parts;
    // Row r's part k: LSE at (slot0 + G k) * part_heads + r_first + r, O row likewise.
    const float* __restrict__ lse = p.part_lse + sp.slot0 * p.part_heads + r_first;
    const float* __restrict__ po = p.part_o + (sp.slot0 * p.part_heads + r_first) * D + lane * E;
    const int64_t ls = static_cast<int64_t>(p.part_heads) << p.gang_shift;
    const int64_t os = ls * D;

    // One round trip: every row's first 64 LSEs (lane k: part k) and first KB partial rows.
    float l0[RB];
    float x[RB][KB][E];
#pragma unroll
    for (int r = 0; r < RB; ++r) {
        const bool live = r < rows_here;
        l0[r] = (live && lane < parts) ? lse[lane * ls + r] : kNegInf;
#pragma unroll
        for (int v = 0; v < KB; ++v) {
#pragma unroll
            for (int e = 0; e < E; ++e) {
                x[r][v][e] = 0.f;
            }
            if (live && v < parts) {
                load_partial<E>(po + v * os + r * D, x[r][v]);
            }
        }
    }
    float wl[RB];
    float den[RB];
    float acc[RB][E];
#pragma unroll
    for (int r = 0; r < RB; ++r) {
        float mx = l0[r];
        for (int k = lane + 64; k < parts; k += 64) {
            mx = fmaxf(mx, r < rows_here ? lse[k * ls + r] : kNegInf);
        }
        mx = group_max<64>(mx);
        // A part whose rows saw no visible key (masks) has lse = -inf and
        // weighs 0, also when every part is empty (mx = -inf).
        wl[r] = (lane < parts && l0[r] != kNegInf) ? fast_exp2(l0[r] - mx) : 0.f;
        den[r] = wl[r];
        l0[r] = mx; // keep the row's max for the weights of parts past 64
#pragma unroll
        for (int e = 0; e < E; ++e) {
            acc[r][e] = 0.f;
        }
#pragma unroll
        for (int v = 0; v < KB; ++v) {
            const float wv = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(wl[r]), v));
#pragma unroll
            for (int e = 0; e < E; ++e) {
                acc[r][e] = fmaf(wv, x[r][v][e], acc[r][e]); // x = 0 past the last part
            }
        }
    }
    // Streams with more than KB parts: the rest, KB partial rows of every row per round trip.
#pragma unroll 1
    for (int k = KB; k < parts; k += KB) {
        if ((k & 63) == 0) {
#pragma unroll
            for (int r = 0; r < RB; ++r) {
                const int kl = k + lane;
                const float lk = (r < rows_here && kl < parts) ? lse[kl * ls + r] : kNegInf;
                wl[r] = lk != kNegInf ? fast_exp2(lk - l0[r]) : 0.f;
                den[r] += wl[r];
            }
        }
#pragma unroll
        for (int r = 0; r < RB; ++r) {
#pragma unroll
            for (int v = 0; v < KB; ++v) {
#pragma unroll
                for (int e = 0; e < E; ++e) {
                    x[r][v][e] = 0.f;
                }
                if (r < rows_here && k + v < parts) {
                    load_partial<E>(po + (k + v) * os + r * D, x[r][v]);
                }
            }
        }
#pragma unroll
        for (int r = 0; r < RB; ++r) {
#pragma unroll
            for (int v = 0; v < KB; ++v) {
                const float wv = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(wl[r]), (k + v) & 63));
#pragma unroll
                for (int e = 0; e < E; ++e) {
                    acc[r][e] = fmaf(wv, x[r][v][e], acc[r][e]);
                }
            }
        }
    }
#pragma unroll
    for (int r = 0; r < RB; ++r) {
        const float d = group_sum<64>(den[r]);
        if (r < rows_here) {
            const float inv = d > 0.f ? 1.f / d : 0.f;
            uint16_t* dst = p.out + out_row(r) * D + lane * E;
#pragma unroll
            for (int e = 0; e < E; ++e) {
                dst[e] = from_f32<BF16>(acc[r][e] * inv);
            }
            if (p.lse != nullptr && lane == 0) {
                store_lse(p.lse, out_row(r), p.q_len, p.num_heads, l0[r], d);
            }
        }
    }
}

template <bool BF16, int D>
static hipError_t launch_combine_t(const CombineParams& p, const FoldParams* fold, hipStream_t stream,
                                   const LaunchEvents& ev) {
    constexpr int kWaves = kCombineWaves;
    const int blocks = (p.rows + kWaves - 1) / kWaves;
    if (p.tile_workers > 0 && p.by_stream) {
        const int spr = (p.num_heads / p.group) * p.head_groups;
        const int waves = p.batch * spr * ((p.part_heads + kStreamRows - 1) / kStreamRows);
        launch_kernel(combine_streams_kernel<BF16, D>, dim3((waves + kWaves - 1) / kWaves), dim3(64 * kWaves), 0,
                      stream, ev, p);
    } else if (p.tile_workers > 0 && p.row_groups) {
        constexpr int kGroupBatch = 64 / (D / 64) < 32 ? 64 / (D / 64) : 32;
        launch_kernel(combine_row_group_kernel<BF16, D, kGroupBatch>, dim3(p.rows), dim3(64 * kRowGroupWaves), 0,
                      stream, ev, p);
    } else if (p.tile_workers > 0 && p.long_rows) {
        constexpr int kLong = 128 / (D / 64) < 64 ? 128 / (D / 64) : 64;
        if (p.lse != nullptr) {
            launch_kernel(combine_tiles_kernel<BF16, D, kLong, true>, dim3(blocks), dim3(64 * kWaves), 0, stream, ev,
                          p);
        } else {
            launch_kernel(combine_tiles_kernel<BF16, D, kLong, false>, dim3(blocks), dim3(64 * kWaves), 0, stream, ev,
                          p);
        }
    } else if (p.tile_workers > 0 && fold != nullptr) {
        // One new token (the decode step) or up to kMaxFold (the verify step): the
        // one-token form keeps a single token's registers.
        const dim3 g(blocks);
        const dim3 b(64 * kWaves);
        const FoldParams& f = *fold;
        if (f.kv_fp8) {
            if (p.q_len == 1) {
                launch_kernel(combine_fold_kernel<BF16, D, 16, 2, 1>, g, b, 0, stream, ev, p, f);
            } else {
                launch_kernel(combine_fold_kernel<BF16, D, 16, 2, kMaxFold>, g, b, 0, stream, ev, p, f);
            }
        } else if (p.q_len == 1) {
            launch_kernel(combine_fold_kernel<BF16, D, 16, 1, 1>, g, b, 0, stream, ev, p, f);
        } else {
            launch_kernel(combine_fold_kernel<BF16, D, 16, 1, kMaxFold>, g, b, 0, stream, ev, p, f);
        }
    } else if (p.tile_workers > 0) {
        if (p.lse != nullptr) {
            launch_kernel(combine_tiles_kernel<BF16, D, 16, true>, dim3(blocks), dim3(64 * kWaves), 0, stream, ev, p);
        } else {
            launch_kernel(combine_tiles_kernel<BF16, D, 16, false>, dim3(blocks), dim3(64 * kWaves), 0, stream, ev,
                          p);
        }
    } else {
        launch_kernel(combine_kernel<BF16, D>, dim3(blocks), dim3(64 * kWaves), 0, stream, ev, p);
    }
    return hipGetLastError();
}

hipError_t launch_combine(const CombineParams& p, const FoldParams* fold, bool bf16, int head_dim,
                          hipStream_t stream, const LaunchEvents& ev) {
    if (bf16) {
        switch (head_dim) {
        case 64: return launch_combine_t<true, 64>(p, fold, stream, ev);
        case 128: return launch_combine_t<true, 128>(p, fold, stream, ev);
        case 256: return launch_combine_t<true, 256>(p, fold, stream, ev);
        default: return hipErrorInvalidValue;
        }
    }
    switch (head_dim) {
    case 64: return launch_combine_t<false, 64>(p, fold, stream, ev);
    case 128: return launch_combine_t<false, 128>(p, fold, stream, ev);
    case 256: return launch_combine_t<false, 256>(p, fold, stream, ev);
    default: return hipErrorInvalidValue;
    }
}

} // namespace pkv
