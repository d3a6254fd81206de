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
    int32_t splits;
    int32_t page_shift;   // log2(P)
    int32_t bt_stride;
    int32_t num_pages;
    int32_t row_cap;      // tokens a block_table row can address (bt_stride * P, clamped)
    int32_t num_items;    // B * Hk * head_groups * splits
    float scale_log2;     // softmax_scale * log2(e)
};

struct CombineParams {
    const float* part_o;
    const float* part_lse;
    uint16_t* out;
    int32_t rows;   // B * H
    int32_t splits;
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

// Split s of S covers pages [n*s/S, n*(s+1)/S) of the row's n valid pages
// (best_flashattn_kvcache_decode.cu:664-671): any two splits differ by at most one page.
struct TokenRange {
    int32_t begin;
    int32_t end;
};

__device__ __forceinline__ TokenRange split_tokens(int32_t seqlen, int32_t page_shift, int32_t split,
                                                   int32_t splits) {
    const int32_t pages = seqlen > 0 ? ((seqlen - 1) >> page_shift) + 1 : 0;
    const int32_t first = static_cast<int32_t>((static_cast<int64_t>(pages) * split) / splits);
    const int32_t last = static_cast<int32_t>((static_cast<int64_t>(pages) * (split + 1)) / splits);
    TokenRange r;
    r.begin = first << page_shift;
    r.end = min(last << page_shift, seqlen);
    if (first >= last) {
        r.end = r.begin; // empty split
    }
    return r;
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
