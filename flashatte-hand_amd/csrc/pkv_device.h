// pkv_device.h — device-side building blocks shared by the gfx950 decode kernels.
//
// Layout contract (include/pkv_decode.h): q/out [B,1,H,D], caches
// [num_pages, P, Hk, D], block_table [B, stride] int32, cache_seqlens [B].
// Token t of row b is slot t % P of page block_table[b][t / P]
// (reference: submission-oj/best_flashattn_kvcache_decode.cu:262-272, 313-328).
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace pkv {

// Everything a partition launch needs, passed by value (kernarg segment).
struct PartitionParams {
    const uint16_t* q;
    const uint16_t* k;
    const uint16_t* v;
    const int32_t* block_table;
    const int32_t* seqlens;
    uint16_t* out;        // final output (splits == 1)
    float* part_o;        // [B*H*splits, D] fp32, normalised per split (splits > 1)
    float* part_lse;      // [B*H*splits] log2-domain LSE, -inf for an empty split
    int64_t token_stride; // Hk * D elements
    int64_t page_stride;  // P * Hk * D elements
    int32_t num_heads;    // H
    int32_t num_heads_k;  // Hk
    int32_t group;        // H / Hk
    int32_t head_groups;  // ceil(group / heads per wave)
    int32_t splits;       // split slots per (b, h) row
    int32_t split_tokens; // > 0: split s covers tokens [s*split_tokens, (s+1)*split_tokens);
                          // 0: page-balanced splits of each row (the reference's scheme)
    int32_t page_shift;   // log2(P)
    int32_t bt_stride;
    int32_t num_pages;
    int32_t row_cap;      // tokens a block_table row can address (bt_stride * P, clamped)
    int32_t batch;        // B
    int32_t num_items;    // splits * B * Hk * head_groups
    int32_t num_groups;   // workgroups in the grid
    int32_t item_groups;  // split schedules: a workgroup of waves per item (no more items than CUs,
                          // items of two tiles or more)
    int32_t tile_workers; // > 0: tile-balanced schedule with this many waves
    int32_t part_heads;   // rows per partial slot in the tile-balanced schedule
    int32_t gang_shift;   // tile-balanced schedule: 2^gang_shift waves of a workgroup share a unit share
    int32_t force_partial; // tile-balanced schedule: a stream one worker covers whole still goes to a
                           // partial slot (the combine adds an appended token to every row)
    float scale_log2;     // softmax_scale * log2(e)
    // Query rows: each KV head serves rows = q_len * group query rows,
    // r = i * group + g for query token i and head g of the group.  With
    // q_len == 1 and no mask the kernels take the plain decode path.
    int32_t q_len;        // M: query tokens per row (q, out [B, M, H, D])
    int32_t rows;         // q_len * group
    int32_t win_left;     // keys j >= pos - win_left; -1 = unbounded
    int32_t win_right;    // keys j <= pos + win_right; -1 = unbounded (0 when causal)
    const float* alibi;   // fp32 slopes at alibi[b * alibi_stride + h], or null
    int64_t alibi_stride;
    // Cache element type: 0 = the compute dtype (16-bit), 1 = OCP FP8 e4m3
    // (k / v then point at bytes) with per-KV-head fp32 scales (null = 1).
    int32_t kv_fp8;
    // KV heads per stream: 1, or 2 (FP8 caches, tile schedule): a wave streams
    // KV heads 2m and 2m + 1 together as one head of twice the width, so each
    // token row it loads is 2 D contiguous bytes.  num_heads_k, group and rows
    // then count these pairs (Hk / 2 of them, 2 group query heads each);
    // token_stride and page_stride stay those of the cache.
    int32_t kv_pack;
    const float* k_scale;
    const float* v_scale;
    float* lse;           // optional fp32 [B, H, M]: natural-log LSE of each output row (store_lse)
    float softcap_log2;   // > 0: every score x (log2 units) becomes softcap_log2 * tanh(x / softcap_log2)
    const int32_t* kv_start; // optional [B]: keys below kv_start[b] are visible to no query (cache_leftpad)
};

struct CombineParams {
    const float* part_o;
    const float* part_lse;
    const int32_t* seqlens;
    uint16_t* out;
    int32_t rows;         // B * H
    int32_t num_heads;    // H
    int32_t splits;
    int32_t split_tokens; // as in PartitionParams
    int32_t page_shift;
    int32_t row_cap;
    // Tile-balanced schedule (tile_workers > 0); the fields above that name
    // splits are then unused.
    int32_t tile_workers;
    int32_t part_heads;
    int32_t gang_shift;   // as in PartitionParams
    int32_t batch;
    int32_t group;        // H / Hk
    int32_t head_groups;  // streams per (b, kv head)
    int32_t heads_per_wave; // query rows per stream (16 MFMA, 1/2/4 VALU)
    int32_t q_len;        // as in PartitionParams; rows = B * q_len * H
    int32_t win_left;     // as in PartitionParams (it bounds the tiles a row's streams cover)
    float* lse;           // as in PartitionParams
    int32_t by_stream;    // tile schedule: one wave per block of a stream's rows (few parts per stream)
    int32_t long_rows;    // tile schedule, a row per wave: many parts per stream, all in one round trip
    int32_t row_groups;   // tile schedule, a workgroup per row: very many parts per stream (few long rows)
};

// Decode with its append folded into the combine (tile schedule, q_len new
// tokens for q_len query tokens, no window, ALiBi or softcap): the partition
// attended the cached cache_seqlens[b] tokens and left a partial for every
// stream; the combine adds the new tokens each query sees (all, or j <= i when
// causal) and writes k_new / v_new ([B, q_len, Hk, D]) into slots
// cache_seqlens[b] + j of the row's block table (FP8 caches: quantised).  A
// kernel argument of the fold kernels only, so the plain combine's argument
// block stays as small as it was without the fold.
struct FoldParams {
    const uint16_t* q;
    const uint16_t* k;
    const uint16_t* v;
    uint16_t* k_cache;
    uint16_t* v_cache;
    const int32_t* block_table;
    int32_t bt_stride;
    int32_t num_pages;
    float scale_log2;
    int32_t causal;
    int32_t kv_fp8;
    const float* k_scale; // FP8 caches: per-KV-head scales, or null (1)
    const float* v_scale;
    const int32_t* kv_start; // optional [B] (cache_leftpad): a new token below it is stored, not attended
};

// Query rows per wave of the tile schedule's stream combine.
constexpr int kStreamRows = 4;

// Paged KV-cache append (pkv_append.hip): one 16-byte chunk of K and of V per
// thread.  A token row is Hk * D 16-bit elements, contiguous in the new-token
// tensors ([tokens, Hk, D]) and in its cache slot ([num_pages, P, Hk, D]).
struct AppendParams {
    const uint4* k_new;           // [tokens, Hk, D]: token i = b * n_new + j, or i of the slot mapping
    const uint4* v_new;
    uint4* k_cache;               // [num_pages, P, Hk, D]
    uint4* v_cache;
    const int32_t* block_table;   // block-table form: [B, bt_stride]
    const int32_t* seqlens;       // block-table form: position of token j of row b = max(seqlens[b], 0) + j
    const int64_t* slot_mapping;  // slot form: flat slot page * P + slot of token i; < 0 = padding
    int32_t* seqlens_out;         // optional (block-table form): max(seqlens[b], 0) + n_new per row
    int64_t tokens;               // token rows to write
    int64_t num_slots;            // num_pages * P
    int64_t row_cap;              // positions a block-table row addresses (bt_stride * P)
    int32_t chunks;               // 16-byte chunks per token row (Hk * D / 8)
    int32_t n_new;                // block-table form: new tokens per row
    int32_t page_shift;           // log2(P)
    int32_t bt_stride;
    int32_t num_pages;
    int32_t batch;
    // FP8 caches: each 16-bit input value x is stored as e4m3(sat(x * (1 / scale)))
    // with the chunk's KV head scale (chunk c belongs to head c / head_chunks).
    int32_t kv_fp8;
    int32_t bf16;                 // input dtype: 1 bf16, 0 fp16
    int32_t head_chunks;          // 16-byte input chunks per KV head (D / 8)
    const float* k_scale;         // [Hk] or null (1)
    const float* v_scale;
};

// Block-table append with flash-attn's rotary embedding (flash_attn_with_kvcache
// with rotary_cos / rotary_sin): new token j of row b is rotated at position
// max(seqlens[b], 0) + j before it is stored; V is stored unrotated; q is
// rotated into q_out at max(seqlens[b], 0) + i for query i (q_positions == 1,
// causal or windowed calls) or at max(seqlens[b], 0) for every query.  Pair
// (x0, x1) of angle index a becomes (x0 cos_a - x1 sin_a, x0 sin_a + x1 cos_a)
// in fp32 without fused multiply-adds, rounded to the input dtype; the
// dims from rotary_dim on are copied.
struct RotaryAppendParams {
    AppendParams a;               // block-table form, 16-bit new K / V
    const uint16_t* cos;          // [rotary_seqlen, rotary_dim / 2], the input dtype
    const uint16_t* sin;
    const uint16_t* q;            // [B, M, H, D]
    uint16_t* q_out;              // [B, M, H, D]: q rotated
    int64_t rotary_seqlen;        // rows of cos / sin; positions past the last row use it
    int32_t rotary_dim;           // multiple of 16, <= D
    int32_t interleaved;          // 1: pairs (2p, 2p + 1); 0: (p, p + rotary_dim / 2) (GPT-NeoX)
    int32_t q_len;                // M
    int32_t num_heads;            // H
    int32_t q_positions;
};

constexpr float kNegInf = -__builtin_huge_valf();

// ---------------------------------------------------------------- 16-bit <-> fp32

// bf16 -> fp32 is exact: the bf16 bits are the top half of the fp32 pattern.
__device__ __forceinline__ float bf16_lo(uint32_t w) { return __uint_as_float(w << 16); }
__device__ __forceinline__ float bf16_hi(uint32_t w) { return __uint_as_float(w & 0xffff0000u); }

__device__ __forceinline__ float f16_lo(uint32_t w) {
    return static_cast<float>(__builtin_bit_cast(_Float16, static_cast<uint16_t>(w & 0xffffu)));
}
__device__ __forceinline__ float f16_hi(uint32_t w) {
    return static_cast<float>(__builtin_bit_cast(_Float16, static_cast<uint16_t>(w >> 16)));
}

template <bool BF16>
__device__ __forceinline__ void unpack2(uint32_t w, float& a, float& b) {
    if constexpr (BF16) {
        a = bf16_lo(w);
        b = bf16_hi(w);
    } else {
        a = f16_lo(w);
        b = f16_hi(w);
    }
}

// fp32 -> bf16, round to nearest even, NaN kept quiet (bfloat16 definition).
__device__ __forceinline__ uint16_t f32_to_bf16(float f) {
    const uint32_t x = __float_as_uint(f);
    if ((x & 0x7fffffffu) > 0x7f800000u) {
        return static_cast<uint16_t>((x >> 16) | 0x40u);
    }
    return static_cast<uint16_t>((x + 0x7fffu + ((x >> 16) & 1u)) >> 16);
}

// fp32 -> fp16 with the hardware conversion (round to nearest even in the default mode).
__device__ __forceinline__ uint16_t f32_to_f16(float f) {
    return __builtin_bit_cast(uint16_t, static_cast<_Float16>(f));
}

template <bool BF16>
__device__ __forceinline__ uint16_t from_f32(float f) {
    if constexpr (BF16) {
        return f32_to_bf16(f);
    } else {
        return f32_to_f16(f);
    }
}

template <bool BF16>
__device__ __forceinline__ uint32_t pack2(float a, float b) {
    return static_cast<uint32_t>(from_f32<BF16>(a)) | (static_cast<uint32_t>(from_f32<BF16>(b)) << 16);
}

// Two fp32 -> packed 16-bit with the hardware pack (v_cvt_pk_bf16_f32 /
// v_cvt_pk_f16_f32, round to nearest even).  Used for the softmax
// probabilities fed to MFMA; outputs use the explicit conversions above.
template <bool BF16>
__device__ __forceinline__ uint32_t pack2_hw(float a, float b) {
    typedef float f32x2_t __attribute__((ext_vector_type(2)));
    const f32x2_t v = {a, b};
    if constexpr (BF16) {
        typedef __bf16 bf16x2_t __attribute__((ext_vector_type(2)));
        return __builtin_bit_cast(uint32_t, __builtin_convertvector(v, bf16x2_t));
    } else {
        typedef _Float16 f16x2_t __attribute__((ext_vector_type(2)));
        return __builtin_bit_cast(uint32_t, __builtin_convertvector(v, f16x2_t));
    }
}

// ---------------------------------------------------------------- loads

typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));

// 16-byte load of K/V cache data.  Each cache byte is read exactly once per
// call, so the load is marked non-temporal (streamed past the caches).
__device__ __forceinline__ uint4 load_kv16(const uint16_t* ptr) {
    const u32x4 v = __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(ptr));
    return make_uint4(v.x, v.y, v.z, v.w);
}

// ---------------------------------------------------------------- math

__device__ __forceinline__ float fast_exp2(float x) { return __builtin_amdgcn_exp2f(x); }
__device__ __forceinline__ float fast_log2(float x) { return __builtin_amdgcn_logf(x); }

// tanh x = sign(x) (1 - e) / (1 + e) with e = exp(-2 |x|) from the hardware
// exp2 and reciprocal (about 2 ulp relative, 1e-7 absolute near 0).
__device__ __forceinline__ float tanh_f32(float x) {
    const float e = fast_exp2(-2.8853900817779268f * fabsf(x));
    return copysignf((1.f - e) * __builtin_amdgcn_rcpf(1.f + e), x);
}

// flash-attn's softmax_lse ([B, H, M], natural log) of output row `row` of
// [B, M, H]: (m2 + log2 l) * ln 2 from a log2-domain max m2 and the weight sum
// l of the row's probabilities exp2(s - m2); +inf for a row that saw no key
// (flash-attn 2.6.3 writes +inf there; mathematically log 0 = -inf).
// Rows number B * M * H <= 2^30 (the descriptor check), so the index math is
// 32-bit.
__device__ __forceinline__ void store_lse(float* lse, int64_t row, int32_t q_len, int32_t num_heads, float m2,
                                          float l) {
    uint32_t at = static_cast<uint32_t>(row);
    if (q_len > 1) {
        const uint32_t nh = static_cast<uint32_t>(num_heads);
        const uint32_t per_b = static_cast<uint32_t>(q_len) * nh;
        const uint32_t b = at / per_b;
        const uint32_t rem = at - b * per_b;
        const uint32_t i = rem / nh;
        at = (b * nh + (rem - i * nh)) * static_cast<uint32_t>(q_len) + i;
    }
    lse[at] = l > 0.f ? (m2 + fast_log2(l)) * 0.69314718055994531f : __builtin_huge_valf();
}

// Dot product of two packed 16-bit pairs accumulated into fp32 (v_dot2c_f32_{bf16,f16}).
template <bool BF16>
__device__ __forceinline__ float dot2(uint32_t a, uint32_t b, float c) {
    if constexpr (BF16) {
        typedef __bf16 bf16x2 __attribute__((ext_vector_type(2)));
        return __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(bf16x2, a), __builtin_bit_cast(bf16x2, b), c,
                                               false);
    } else {
        typedef _Float16 f16x2 __attribute__((ext_vector_type(2)));
        return __builtin_amdgcn_fdot2(__builtin_bit_cast(f16x2, a), __builtin_bit_cast(f16x2, b), c, false);
    }
}

// ---------------------------------------------------------------- cross-lane (wave64)

// DPP move within a row of 16 lanes.  Controls: 0xB1 quad_perm[1,0,3,2],
// 0x4E quad_perm[2,3,0,1], 0x141 row_half_mirror, 0x140 row_mirror.
template <int CTRL>
__device__ __forceinline__ float dpp_f32(float x) {
    return __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(x), CTRL, 0xf, 0xf, false));
}

// Value of the lane 8 above within each row of 16 lanes (DPP row_shl:8); 0 in
// lanes 8-15, whose source lies outside the row.
__device__ __forceinline__ float lanes_up8(float x) {
    return __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(x), 0x108, 0xf, 0xf, true));
}

// ds_swizzle in bit mode: lane i reads lane (i & and) | or) ^ xor within each 32-lane half.
template <int XOR_MASK>
__device__ __forceinline__ float swizzle_xor_f32(float x) {
    return __int_as_float(__builtin_amdgcn_ds_swizzle(__float_as_int(x), (XOR_MASK << 10) | 0x1f));
}

// Butterfly all-reduce over aligned groups of N lanes (N = 2..64); every lane of
// a group ends with the bit-identical total (each step adds commutative pairs).
template <int N>
__device__ __forceinline__ float group_sum(float x) {
    if constexpr (N >= 2) x += dpp_f32<0xB1>(x);
    if constexpr (N >= 4) x += dpp_f32<0x4E>(x);
    if constexpr (N >= 8) x += dpp_f32<0x141>(x);
    if constexpr (N >= 16) x += dpp_f32<0x140>(x);
    if constexpr (N >= 32) x += swizzle_xor_f32<16>(x);
    if constexpr (N >= 64) x += __shfl_xor(x, 32, 64);
    return x;
}

template <int N>
__device__ __forceinline__ float group_max(float x) {
    if constexpr (N >= 2) x = fmaxf(x, dpp_f32<0xB1>(x));
    if constexpr (N >= 4) x = fmaxf(x, dpp_f32<0x4E>(x));
    if constexpr (N >= 8) x = fmaxf(x, dpp_f32<0x141>(x));
    if constexpr (N >= 16) x = fmaxf(x, dpp_f32<0x140>(x));
    if constexpr (N >= 32) x = fmaxf(x, swizzle_xor_f32<16>(x));
    if constexpr (N >= 64) x = fmaxf(x, __shfl_xor(x, 32, 64));
    return x;
}

// Reductions across the four 16-lane rows of a wave with the gfx950 row-swap
// instructions (VALU only, no LDS round trip).  permlane16_swap(x, x) returns
// (even-row copy, odd-row copy) of each row pair, permlane32_swap(x, x) the
// (low-half, high-half) copies, so op(first, second) is the pair reduction on
// every lane, with bit-identical results on both partners.
__device__ __forceinline__ float max_rows16(float x) {
    const auto r = __builtin_amdgcn_permlane16_swap(__float_as_uint(x), __float_as_uint(x), false, false);
    return fmaxf(__uint_as_float(r[0]), __uint_as_float(r[1]));
}
__device__ __forceinline__ float sum_rows16(float x) {
    const auto r = __builtin_amdgcn_permlane16_swap(__float_as_uint(x), __float_as_uint(x), false, false);
    return __uint_as_float(r[0]) + __uint_as_float(r[1]);
}
__device__ __forceinline__ float max_halves32(float x) {
    const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x), false, false);
    return fmaxf(__uint_as_float(r[0]), __uint_as_float(r[1]));
}
__device__ __forceinline__ float sum_halves32(float x) {
    const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x), false, false);
    return __uint_as_float(r[0]) + __uint_as_float(r[1]);
}

// Exchange with the lane `STRIDE` away (STRIDE in {8, 16, 32}) — used to merge
// the per-row online-softmax states of a wave.
template <int STRIDE>
__device__ __forceinline__ float xor_lane(float x) {
    if constexpr (STRIDE == 16 || STRIDE == 8 || STRIDE == 4 || STRIDE == 2 || STRIDE == 1) {
        return swizzle_xor_f32<STRIDE>(x);
    } else {
        return __shfl_xor(x, STRIDE, 64);
    }
}

// ---------------------------------------------------------------- indexing

// Token range of split `split` of a row with `seqlen` valid tokens.
// split_tokens > 0: fixed windows of split_tokens tokens, so every work item
// streams the same amount and ragged rows simply own fewer items.
// split_tokens == 0: split s covers pages [n*s/S, n*(s+1)/S) of the row's n
// valid pages (best_flashattn_kvcache_decode.cu:664-671), so any two splits of
// a row differ by at most one page.  Either way the range may be empty, and a
// left window clips it to the keys some query can see (visible_split_tokens,
// after tile_span).
struct TokenRange {
    int32_t begin;
    int32_t end;
};

// Work items of the split schedules: item = (split * B + b) * units + u with
// u = kv head * head_groups + head group, so consecutive waves (and
// workgroups) take the (kv head, head group) units of one row and one split.
struct Item {
    int32_t split;
    int32_t b;
    int32_t kvh;
    int32_t hg;
};

// Waves per workgroup of the split-schedule kernels.
constexpr int kWavesPerGroup = 4;

// Compute units of gfx950 (MI355X): grids are sized against it.
constexpr int kComputeUnits = 256;

// Waves per workgroup (= per CU) of the tile-balanced partition kernel.
// Measured on MI355X over the five workload shapes: 4 (one per SIMD) streams
// faster than 2, 3, 5, 6 or 8, and than 4 with two tiles of prefetch per wave.
constexpr int kTileWaves = 4;

__device__ __forceinline__ int32_t wave_item() {
    return static_cast<int32_t>(blockIdx.x) * kWavesPerGroup + static_cast<int32_t>(threadIdx.x >> 6);
}

__device__ __forceinline__ Item decode_item(int32_t item, const PartitionParams& p) {
    const int32_t units = p.num_heads_k * p.head_groups;
    Item it;
    const int32_t u = item % units;
    const int32_t rest = item / units;
    it.b = rest % p.batch;
    it.split = rest / p.batch;
    it.kvh = u / p.head_groups;
    it.hg = u - it.kvh * p.head_groups;
    return it;
}

// ---------------------------------------------------------------- tile-balanced schedule
//
// A stream is the work of one (b, kv head, head group): the n_b tiles of 16
// tokens of row b that its queries can see (tile_span: every tile of the row
// unless a left window cuts the front).  Streams are numbered r = b * spr + u with
// u = kv head * head_groups + head group (spr streams per row) and laid end to
// end in that order as units_b = stream_units(n_b) balancing units each
// (kHeaderTiles header units, then the tiles), so the call is one sequence of
// T = spr * sum_b units_b units and row b owns units [spr * C_b, spr * C_(b+1))
// with C_b = sum_(b' < b) units_b'.  Worker w of W takes units [lo(w), lo(w + 1)),
// lo(w) = floor(w T / W): every worker gets the same share (+-1) whatever the
// row lengths.  W is the launch's worker count clamped to T, so every worker
// owns a unit.  A worker's share crosses stream boundaries; the tiles of one
// stream it owns are a segment.  A segment that is a whole stream is written
// to the output directly; otherwise it leaves a partial in slot w + r, which
// is unique: the workers owning stream r's tiles are the consecutive
// w_a(r) .. w_b(r), and w_a(r + 1) >= w_b(r).  The combine finds them with
// w(x) = floor(((x + 1) W - 1) / T), the worker owning unit x; tile t of
// stream r is unit spr * C_b + u * units_b + kHeaderTiles + t.
//
// Gangs: with gang_shift = s > 0 a worker is a gang of G = 2^s waves of one
// workgroup and the sequence is laid over super-streams, the G consecutive
// streams u = G q + j (j < G) of a row: sps = spr / G per row, T = sps *
// sum_b units_b, and gang g of W (the launch's waves / G) takes units
// [lo(g), lo(g + 1)) as above.  Member j of gang g streams the tiles of stream
// G q + j for each super-stream q of that share, so the G waves of a CU read
// the same tokens of adjacent KV heads: G head rows next to each other in each
// token row.  A partial of super-stream q' = b * sps + q goes to slot
// G (g + q') + j; the parts of stream r = G q' + j are G slots apart.  s = 0 is
// the schedule above.

// Tiles a row's streams cover: from the tile of the first key any query of the
// row can see to the row's last tile.  Without a left window that is every
// tile of the row; with one, query 0 (at position L - q_len) sees keys from
// L - q_len - win_left on, and no query sees anything earlier.
struct TileSpan {
    int32_t first; // first tile of the span
    int32_t n;     // tiles in the span (0 for an empty row)
};

__device__ __forceinline__ TileSpan tile_span(int32_t sl, int32_t q_len, int32_t win_left) {
    TileSpan t;
    // 64-bit: a window near INT32_MAX (practically unbounded) must not wrap.
    const int64_t lo = static_cast<int64_t>(sl) - q_len - win_left;
    t.first = win_left >= 0 ? static_cast<int32_t>(min(max(lo, int64_t{0}), static_cast<int64_t>(sl)) >> 4) : 0;
    t.n = ((sl + 15) >> 4) - t.first;
    return t;
}

// Tokens of split `split` of a row of seqlen tokens (split schedules), within
// the span some query can see: a left window masks everything before the
// tile of its first key for every query, so no split reads it.  Page-balanced
// splits divide the pages of that span as the reference divides a row's pages
// (best:664-671; the whole row without a window); token windows are clipped
// to it.  With one split the range is the span itself, non-empty for any row
// with tokens.  The partition and the combine both take ranges from here.
__device__ __forceinline__ TokenRange visible_split_tokens(int32_t seqlen, int32_t q_len, int32_t win_left,
                                                           int32_t page_shift, int32_t split, int32_t splits,
                                                           int32_t split_tokens) {
    const int32_t lo = tile_span(seqlen, q_len, win_left).first * 16;
    TokenRange r;
    if (split_tokens > 0) {
        // The window count comes from the host's max_seqlen; the last window
        // runs to the row's end, so a row longer than that bound is still
        // read whole.  (split * split_tokens < max_seqlen: no overflow.)
        r.begin = max(split * split_tokens, lo);
        const int32_t stop = split + 1 == splits ? seqlen : min(split * split_tokens + split_tokens, seqlen);
        r.end = max(r.begin, stop);
        return r;
    }
    const int32_t p0 = lo >> page_shift;
    const int32_t pages = seqlen > 0 ? ((seqlen - 1) >> page_shift) + 1 - p0 : 0;
    const int32_t first = p0 + static_cast<int32_t>((static_cast<int64_t>(pages) * split) / splits);
    const int32_t last = p0 + static_cast<int32_t>((static_cast<int64_t>(pages) * (split + 1)) / splits);
    r.begin = max(first << page_shift, lo);
    r.end = first < last ? min(last << page_shift, seqlen) : r.begin;
    return r;
}

__device__ __forceinline__ int32_t clamped_seqlen(const int32_t* __restrict__ seqlens, int32_t b, int32_t row_cap) {
    return min(max(seqlens[b], 0), row_cap);
}

__device__ __forceinline__ int32_t row_tiles(const int32_t* __restrict__ seqlens, int32_t b, int32_t row_cap,
                                             int32_t q_len, int32_t win_left) {
    return tile_span(clamped_seqlen(seqlens, b, row_cap), q_len, win_left).n;
}

// Balancing units of a stream with n tiles: its tiles plus kHeaderTiles for
// the dependent loads that start every segment (page window, first tile),
// which cost about as much as a tile each.  A worker that starts a new stream
// inside its share is charged for them, so workers with an extra segment do
// not end up last.  The header units precede the stream's tiles and are never
// processed.
constexpr int32_t kHeaderTiles = 2;

__device__ __forceinline__ int32_t stream_units(int32_t n) { return n > 0 ? n + kHeaderTiles : 0; }

__device__ __forceinline__ int64_t wave_sum_i64(int64_t x) {
#pragma unroll
    for (int d = 32; d >= 1; d >>= 1) {
        x += __shfl_xor(x, d, 64);
    }
    return x;
}


// Worker owning tile x: floor(((x + 1) W - 1) / T), in 32 bits when it fits.
__device__ __forceinline__ int32_t tile_worker_of(int64_t x, int64_t total, int32_t workers) {
    const uint64_t n = static_cast<uint64_t>(x + 1) * static_cast<uint64_t>(workers) - 1;
    if (n < (1ull << 32) && total < (int64_t{1} << 32)) {
        return static_cast<int32_t>(static_cast<uint32_t>(n) / static_cast<uint32_t>(total));
    }
    return static_cast<int32_t>(n / static_cast<uint64_t>(total));
}

// Row holding stream-unit index y (0 <= y < sum_b units_b): b, its clamped
// seqlen, n_b and C_b.  Rows without tokens own no units and are never returned.
struct RowTiles {
    int32_t b;
    int32_t seqlen;
    int32_t n;
    int64_t before;
};

__device__ __forceinline__ RowTiles locate_row(const int32_t* __restrict__ seqlens, int32_t batch, int32_t row_cap,
                                               int32_t q_len, int32_t win_left, int64_t y, int32_t lane) {
    int64_t carry = 0;
    for (int32_t base = 0; base < batch; base += 64) {
        const int32_t b = base + lane;
        const int32_t sl = b < batch ? clamped_seqlen(seqlens, b, row_cap) : 0;
        const int32_t n = tile_span(sl, q_len, win_left).n;
        const int32_t un = stream_units(n);
        int64_t incl = un;
#pragma unroll
        for (int d = 1; d < 64; d <<= 1) {
            const int64_t t = __shfl_up(incl, d, 64);
            incl += lane >= d ? t : 0;
        }
        incl += carry;
        const uint64_t hit = __ballot(b < batch && incl > y);
        if (hit != 0) {
            const int32_t l = __builtin_ctzll(hit);
            RowTiles r;
            r.b = base + l;
            r.seqlen = __shfl(sl, l, 64);
            r.n = __shfl(n, l, 64);
            r.before = __shfl(incl, l, 64) - stream_units(r.n);
            return r;
        }
        carry = __shfl(incl, 63, 64);
    }
    RowTiles r; // not reached for y < sum_b n_b
    r.b = batch - 1;
    r.seqlen = 0;
    r.n = 0;
    r.before = carry;
    return r;
}

// Inclusive prefix sum over the wave's lanes in 32 bits with DPP: Hillis-Steele
// within each row of 16 lanes (row_shr 1, 2, 4, 8; lanes shifted in from
// outside the row read 0), then the running totals of rows 0 and 2 are added
// to rows 1 and 3 (row_bcast:15), and of row 1 to rows 2 and 3 (row_bcast:31).
template <int CTRL, int ROW_MASK>
__device__ __forceinline__ uint32_t dpp_u32(uint32_t x) {
    return static_cast<uint32_t>(__builtin_amdgcn_update_dpp(0, static_cast<int>(x), CTRL, ROW_MASK, 0xf, true));
}

__device__ __forceinline__ uint32_t wave_inclusive_scan_u32(uint32_t x) {
    x += dpp_u32<0x111, 0xf>(x);
    x += dpp_u32<0x112, 0xf>(x);
    x += dpp_u32<0x114, 0xf>(x);
    x += dpp_u32<0x118, 0xf>(x);
    x += dpp_u32<0x142, 0xa>(x);
    x += dpp_u32<0x143, 0xc>(x);
    return x;
}

// Inclusive prefix sum over the wave's lanes.
__device__ __forceinline__ int64_t wave_inclusive_scan(int64_t x, int32_t lane) {
#pragma unroll
    for (int d = 1; d < 64; d <<= 1) {
        const int64_t t = __shfl_up(x, d, 64);
        x += lane >= d ? t : 0;
    }
    return x;
}

// Units per row of the call, as a wave-wide prefix.  Up to kScanChunks * 64
// rows are read once (one load per lane and chunk, all issued together) and
// kept in registers, each chunk scanned in 32 bits with DPP and the chunks
// chained by uniform carries, so locating a unit is a ballot per chunk with no
// further memory access.  Larger batches add a sum over the remaining rows,
// and locating a unit in them takes a chunked pass that reads cache_seqlens
// again (locate_row).
constexpr int kScanChunks = 4;

struct RowScan {
    int64_t rows_total;           // sum over rows of stream_units(n_b)
    bool fast;                    // the chunks hold every row (batch <= 256, row_cap <= 2^24)
    uint32_t incl[kScanChunks];   // lane: units of rows 64c .. 64c + lane (inclusive), within chunk c
    int64_t carry[kScanChunks];   // units of the rows before chunk c (uniform)
    int32_t sl[kScanChunks];      // lane: clamped seqlen of row 64c + lane
    int32_t n[kScanChunks];       // lane: tiles of that row
};

__device__ __forceinline__ RowScan scan_rows(const int32_t* __restrict__ seqlens, int32_t batch, int32_t row_cap,
                                             int32_t q_len, int32_t win_left, int32_t lane) {
    RowScan rs;
    // Units of one stream are below 2^27 (row_cap < 2^31 tokens), so a chunk
    // of 64 rows of them fits 32 bits when row_cap <= 2^24.
    rs.fast = batch <= 64 * kScanChunks && row_cap <= (1 << 24);
    // Every chunk's load goes out before any is used, with no branch around it
    // (lanes past the batch re-read its last row; a select drops them): a load
    // under a branch would make the compiler wait for each chunk in turn.
    int32_t raw[kScanChunks];
#pragma unroll
    for (int c = 0; c < kScanChunks; ++c) {
        raw[c] = seqlens[min(64 * c + lane, batch - 1)];
    }
#pragma unroll
    for (int c = 0; c < kScanChunks; ++c) {
        const int32_t b = 64 * c + lane;
        rs.sl[c] = b < batch ? min(max(raw[c], 0), row_cap) : 0;
        rs.n[c] = tile_span(rs.sl[c], q_len, win_left).n;
    }
    if (rs.fast) {
        int64_t carry = 0;
#pragma unroll
        for (int c = 0; c < kScanChunks; ++c) {
            rs.carry[c] = carry;
            rs.incl[c] = 0;
            if (c == 0 || 64 * c < batch) {
                rs.incl[c] = wave_inclusive_scan_u32(static_cast<uint32_t>(stream_units(rs.n[c])));
                carry += __builtin_amdgcn_readlane(rs.incl[c], 63);
            }
        }
        rs.rows_total = carry;
        return rs;
    }
#pragma unroll
    for (int c = 0; c < kScanChunks; ++c) {
        rs.incl[c] = 0;
        rs.carry[c] = 0;
    }
    int64_t sum = 0;
#pragma unroll
    for (int c = 0; c < kScanChunks; ++c) {
        sum += stream_units(rs.n[c]);
    }
    for (int32_t b = lane + 64 * kScanChunks; b < batch; b += 64) {
        sum += stream_units(row_tiles(seqlens, b, row_cap, q_len, win_left));
    }
    rs.rows_total = wave_sum_i64(sum);
    return rs;
}

// Clamped seqlen of row b (wave-uniform b): from the scan's registers when
// they hold every row, else from cache_seqlens (one dependent load).
__device__ __forceinline__ int32_t scanned_seqlen(const RowScan& rs, const int32_t* __restrict__ seqlens, int32_t b,
                                                  int32_t row_cap) {
    if (rs.fast) {
        int32_t v = 0;
#pragma unroll
        for (int c = 0; c < kScanChunks; ++c) {
            if ((b >> 6) == c) {
                v = __builtin_amdgcn_readlane(rs.sl[c], b & 63);
            }
        }
        return v;
    }
    return __builtin_amdgcn_readfirstlane(clamped_seqlen(seqlens, b, row_cap));
}

// Row holding stream-unit index y (0 <= y < rows_total).
__device__ __forceinline__ RowTiles locate_unit_row(const RowScan& rs, const int32_t* __restrict__ seqlens,
                                                    int32_t batch, int32_t row_cap, int32_t q_len, int32_t win_left,
                                                    int64_t y, int32_t lane) {
    if (rs.fast) {
#pragma unroll
        for (int c = 0; c < kScanChunks; ++c) {
            const int64_t yc = y - rs.carry[c];
            const uint64_t hit = __ballot(64 * c + lane < batch && yc >= 0 && yc < (int64_t{1} << 32) &&
                                          rs.incl[c] > static_cast<uint32_t>(yc));
            if (hit != 0) {
                const int32_t l = __builtin_ctzll(hit);
                RowTiles r;
                r.b = 64 * c + l;
                r.seqlen = __shfl(rs.sl[c], l, 64);
                r.n = __shfl(rs.n[c], l, 64);
                r.before = rs.carry[c] + static_cast<int64_t>(__builtin_amdgcn_readlane(rs.incl[c], l)) -
                           stream_units(r.n);
                return r;
            }
        }
    }
    return locate_row(seqlens, batch, row_cap, q_len, win_left, y, lane);
}

// floor(a * b / c) for a, b >= 0, c > 0, a * b < 2^63; 32-bit when it fits.
__device__ __forceinline__ int64_t muldiv(int64_t a, int64_t b, int64_t c) {
    const uint64_t ab = static_cast<uint64_t>(a) * static_cast<uint64_t>(b);
    if (ab < (1ull << 32) && c < (int64_t{1} << 32)) {
        return static_cast<uint32_t>(ab) / static_cast<uint32_t>(c);
    }
    return static_cast<int64_t>(ab / static_cast<uint64_t>(c));
}

// Shares of the tile-balanced schedule: worker w of W = min(launched workers,
// T) takes units [floor(w T / W), floor((w + 1) T / W)).
struct TilePlan {
    int64_t total;   // T: units of the call
    int32_t workers; // W
};

__device__ __forceinline__ TilePlan make_tile_plan(int64_t total, int32_t launch_workers) {
    TilePlan pl;
    pl.total = total;
    pl.workers = static_cast<int32_t>(min(static_cast<int64_t>(launch_workers), total));
    return pl;
}

__device__ __forceinline__ int64_t share_start(int64_t w, const TilePlan& pl) { return muldiv(w, pl.total, pl.workers); }

__device__ __forceinline__ int32_t uniform(int32_t x) { return __builtin_amdgcn_readfirstlane(x); }
__device__ __forceinline__ int64_t uniform(int64_t x) {
    const uint32_t lo = __builtin_amdgcn_readfirstlane(static_cast<uint32_t>(x));
    const uint32_t hi = __builtin_amdgcn_readfirstlane(static_cast<uint32_t>(static_cast<uint64_t>(x) >> 32));
    return static_cast<int64_t>((static_cast<uint64_t>(hi) << 32) | lo);
}

// Page-id window: lane l holds the physical id of logical page base + l of the
// row (64 pages per window).  Kernels read ids from it with readlane /
// ds_bpermute, so the K/V address of a tile never waits on a global load —
// a dependent global load would force the wave to drain (vmcnt is in order)
// every K/V load it has in flight.  Out-of-range ids are clamped to page 0 so a
// corrupt table cannot fault the GPU; entries past the row's last page are 0
// and never used.  Every lane loads (lanes past the last page re-read it) and a
// select drops the extra entries: a load under a branch would make the
// compiler's later waits count every load issued since as outstanding work to
// drain, so the first tile's addresses would also wait for q.
__device__ __forceinline__ int32_t load_page_window(const int32_t* __restrict__ bt_row, int32_t base,
                                                    int32_t last_page, int32_t lane, int32_t num_pages) {
    const int32_t idx = base + lane;
    const int32_t e = bt_row[min(idx, last_page)];
    const int32_t v = idx <= last_page ? e : 0;
    return static_cast<uint32_t>(v) < static_cast<uint32_t>(num_pages) ? v : 0;
}

// Element offset of (token t, kv head base) given the row's block_table.
// Out-of-range page ids are clamped so a corrupt table cannot fault the GPU.
__device__ __forceinline__ int64_t token_elem_offset(const int32_t* __restrict__ bt_row, int32_t t,
                                                     const PartitionParams& p) {
    int32_t phys = bt_row[t >> p.page_shift];
    phys = static_cast<uint32_t>(phys) < static_cast<uint32_t>(p.num_pages) ? phys : 0;
    return static_cast<int64_t>(phys) * p.page_stride +
           static_cast<int64_t>(t & ((1 << p.page_shift) - 1)) * p.token_stride;
}

} // namespace pkv
