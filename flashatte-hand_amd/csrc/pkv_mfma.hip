// pkv_mfma.hip — MFMA partition kernel for paged-KV GQA decode on gfx950.
//
// One wave64 owns one work item (b, kv head, group of up to 16 query heads,
// split) and walks its token range in tiles of 16 tokens.  Lane l is
// (n = l & 15, j = l >> 4).
//
//   S^T[16 tok x 16 heads] = K[16 tok x D] . Q^T[D x 16 heads]
//       v_mfma_f32_16x16x32_{bf16,f16}, D/32 steps.  A = K: lane loads token n,
//       dims 8(4kk + j) .. +7 straight from HBM (16 B/lane, 64 contiguous bytes
//       per token per step).  B = Q^T: head n, same dims, held in VGPRs for the
//       whole item (heads beyond the group are zero columns).
//       Result: lane holds head n, tokens 4j + i (i = 0..3).
//   softmax: fp32, log2 domain, one max/rescale per tile; the 4 scores a lane
//       holds become the B operand of PV after one 16-bit pack (p <= 1).
//   O^T[D x 16 heads] += V^T[D x 16 tok] . P^T[16 tok x 16 heads]
//       v_mfma_f32_16x16x16{bf16_1k,f16}, D/16 output tiles.  A = V^T needs
//       4 tokens of one dim per lane, so the V tile (loaded with the same
//       addresses as K) is written to a per-wave LDS tile whose 16-byte chunks
//       are XOR-swizzled by token (chunk c of token t sits at c ^ t), which
//       keeps both the row writes and the column gathers free of bank conflicts.
//   The next tile's K and V are loaded into a second register set before the
//   current tile is computed.
// The per-wave LDS tile is private to the wave and LDS operations of a wave
// complete in order, so no barrier is needed.
//
// Reference semantics followed: submission-oj/best_flashattn_kvcache_decode.cu
// 595-954 (partition, page ranges 664-671, empty split 680-697, exp2 online
// update 782-833, lse2 845-864); the MMA-QK idea of packing the GQA heads into
// the M/N dimension is the reference's flashattn_kvcache_decode_mma_v2.cu:685-1001,
// re-tiled here for 64-lane MFMA with PV also on MFMA.
#include "pkv_device.h"
#include "pkv_launch.h"

namespace pkv {

typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef short s16x8 __attribute__((ext_vector_type(8)));
typedef short s16x4 __attribute__((ext_vector_type(4)));
typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));
typedef _Float16 f16x4 __attribute__((ext_vector_type(4)));
typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));

template <bool BF16>
__device__ __forceinline__ f32x4 mfma_qk(const uint4& a, const uint4& b, f32x4 c) {
    if constexpr (BF16) {
        return __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8, a), __builtin_bit_cast(bf16x8, b), c,
                                                       0, 0, 0);
    } else {
        return __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(f16x8, a), __builtin_bit_cast(f16x8, b), c,
                                                      0, 0, 0);
    }
}

template <bool BF16>
__device__ __forceinline__ f32x4 mfma_pv(const uint2& a, const uint2& b, f32x4 c) {
    if constexpr (BF16) {
        return __builtin_amdgcn_mfma_f32_16x16x16bf16_1k(__builtin_bit_cast(s16x4, a), __builtin_bit_cast(s16x4, b), c,
                                                         0, 0, 0);
    } else {
        return __builtin_amdgcn_mfma_f32_16x16x16f16(__builtin_bit_cast(f16x4, a), __builtin_bit_cast(f16x4, b), c, 0,
                                                     0, 0);
    }
}

template <int D>
struct TileRegs {
    uint4 k[D / 32];
    uint4 v[D / 32];
};

template <int D>
__device__ __forceinline__ void load_tile(TileRegs<D>& r, const PartitionParams& p, const int32_t* __restrict__ bt_row,
                                          int t0, int end, int n, int64_t lane_off) {
    const int t = min(t0 + n, end - 1); // clamp: never touch unowned slots
    const int64_t off = token_elem_offset(bt_row, t, p) + lane_off;
#pragma unroll
    for (int kk = 0; kk < D / 32; ++kk) {
        r.k[kk] = load_kv16(p.k + off + 32 * kk);
        r.v[kk] = load_kv16(p.v + off + 32 * kk);
    }
}

template <bool BF16, int D>
__device__ __forceinline__ void process_tile(const TileRegs<D>& r, const uint4 (&qop)[D / 32], f32x4 (&o)[D / 16],
                                             float& m, float& l, uint16_t* lds, int t0, int end, int n, int j,
                                             float scale_log2) {
    constexpr int KS = D / 32;
    constexpr int DT = D / 16;
    constexpr int CHM = D / 8 - 1; // 16-byte chunks per token row, minus one

    // V tile -> LDS, row n, logical chunk 4kk + j stored at chunk (4kk + j) ^ n.
#pragma unroll
    for (int kk = 0; kk < KS; ++kk) {
        *reinterpret_cast<uint4*>(lds + n * D + 8 * ((4 * kk + j) ^ (n & CHM))) = r.v[kk];
    }

    f32x4 s = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int kk = 0; kk < KS; ++kk) {
        s = mfma_qk<BF16>(r.k[kk], qop[kk], s);
    }

    float sc[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        sc[i] = (t0 + 4 * j + i) < end ? s[i] * scale_log2 : kNegInf;
    }
    float tmax = fmaxf(fmaxf(sc[0], sc[1]), fmaxf(sc[2], sc[3]));
    tmax = fmaxf(tmax, swizzle_xor_f32<16>(tmax));
    tmax = fmaxf(tmax, __shfl_xor(tmax, 32, 64));
    const float m_new = fmaxf(m, tmax);
    const float m_use = m_new == kNegInf ? 0.f : m_new;
    const float alpha = fast_exp2(m - m_use);
    m = m_new;
    if (__any(alpha != 1.f)) {
#pragma unroll
        for (int dt = 0; dt < DT; ++dt) {
            o[dt] *= alpha;
        }
    }
    float pr[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        pr[i] = fast_exp2(sc[i] - m_use);
    }
    l = l * alpha + ((pr[0] + pr[1]) + (pr[2] + pr[3]));
    uint2 pb;
    pb.x = pack2<BF16>(pr[0], pr[1]);
    pb.y = pack2<BF16>(pr[2], pr[3]);

    // O^T tile dt: A = V^T, lane gathers V[4j + i][16 dt + n] for i = 0..3.
#pragma unroll
    for (int dt = 0; dt < DT; ++dt) {
        const int c = 2 * dt + (n >> 3);
        const int e = n & 7;
        uint16_t x[4];
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const int tok = 4 * j + i;
            x[i] = lds[tok * D + 8 * (c ^ (tok & CHM)) + e];
        }
        uint2 a;
        a.x = static_cast<uint32_t>(x[0]) | (static_cast<uint32_t>(x[1]) << 16);
        a.y = static_cast<uint32_t>(x[2]) | (static_cast<uint32_t>(x[3]) << 16);
        o[dt] = mfma_pv<BF16>(a, pb, o[dt]);
    }
}

template <bool BF16, int D>
__global__ __launch_bounds__(256) void partition_mfma_kernel(PartitionParams p) {
    constexpr int KS = D / 32;
    constexpr int DT = D / 16;
    constexpr int kWaves = 4;
    __shared__ __attribute__((aligned(16))) uint16_t lds_tiles[kWaves][16 * D];

    const int wave = threadIdx.x >> 6;
    const int lane = threadIdx.x & 63;
    const int item = blockIdx.x * kWaves + wave;
    if (item >= p.num_items) {
        return;
    }
    const int split = item % p.splits;
    int rest = item / p.splits;
    const int hg = rest % p.head_groups;
    rest /= p.head_groups;
    const int kvh = rest % p.num_heads_k;
    const int b = rest / p.num_heads_k;

    const int n = lane & 15;
    const int j = lane >> 4;
    const int g_first = hg * 16;
    const int heads_here = min(16, p.group - g_first);
    const int64_t bh_first = static_cast<int64_t>(b) * p.num_heads + kvh * p.group + g_first;

    const int seqlen = min(p.seqlens[b], p.row_cap);
    const TokenRange range = split_tokens(seqlen, p.page_shift, split, p.splits);

    if (range.begin >= range.end) {
        constexpr int CH = D / 8; // 16-byte output chunks per head
        for (int idx = lane; idx < heads_here * CH; idx += 64) {
            const int g = idx / CH;
            const int c = idx % CH;
            if (p.splits == 1) {
                uint4 z = {0u, 0u, 0u, 0u};
                *reinterpret_cast<uint4*>(p.out + (bh_first + g) * D + c * 8) = z;
            } else {
                const int64_t pi = (bh_first + g) * p.splits + split;
                float4 z = {0.f, 0.f, 0.f, 0.f};
                float4* dst = reinterpret_cast<float4*>(p.part_o + pi * D + c * 8);
                dst[0] = z;
                dst[1] = z;
            }
        }
        if (p.splits > 1 && lane < heads_here) {
            p.part_lse[(bh_first + lane) * p.splits + split] = kNegInf;
        }
        return;
    }

    // B operand of QK: head n, dims 8(4kk + j) .. +7; zero columns past the group.
    uint4 qop[KS];
#pragma unroll
    for (int kk = 0; kk < KS; ++kk) {
        if (n < heads_here) {
            qop[kk] = *reinterpret_cast<const uint4*>(p.q + (bh_first + n) * D + 8 * (4 * kk + j));
        } else {
            qop[kk] = make_uint4(0u, 0u, 0u, 0u);
        }
    }

    f32x4 o[DT];
#pragma unroll
    for (int dt = 0; dt < DT; ++dt) {
        o[dt] = f32x4{0.f, 0.f, 0.f, 0.f};
    }
    float m = kNegInf;
    float l = 0.f;

    const int32_t* __restrict__ bt_row = p.block_table + static_cast<int64_t>(b) * p.bt_stride;
    const int64_t lane_off = static_cast<int64_t>(kvh) * D + 8 * j;
    uint16_t* lds = lds_tiles[wave];
    const int end = range.end;

    TileRegs<D> ra, rb;
    int t = range.begin;
    load_tile<D>(ra, p, bt_row, t, end, n, lane_off);
    while (true) {
        if (t + 16 < end) {
            load_tile<D>(rb, p, bt_row, t + 16, end, n, lane_off);
        }
        process_tile<BF16, D>(ra, qop, o, m, l, lds, t, end, n, j, p.scale_log2);
        t += 16;
        if (t >= end) {
            break;
        }
        if (t + 16 < end) {
            load_tile<D>(ra, p, bt_row, t + 16, end, n, lane_off);
        }
        process_tile<BF16, D>(rb, qop, o, m, l, lds, t, end, n, j, p.scale_log2);
        t += 16;
        if (t >= end) {
            break;
        }
    }

    // l holds this lane's 4-token partial sums; total over the 4 lanes of head n.
    l += swizzle_xor_f32<16>(l);
    l += __shfl_xor(l, 32, 64);

    if (n >= heads_here) {
        return;
    }
    const float inv = l > 0.f ? 1.f / l : 0.f;
    const int64_t bh = bh_first + n;
    if (p.splits == 1) {
        uint16_t* dst = p.out + bh * D + 4 * j;
#pragma unroll
        for (int dt = 0; dt < DT; ++dt) {
            uint2 w;
            w.x = pack2<BF16>(o[dt][0] * inv, o[dt][1] * inv);
            w.y = pack2<BF16>(o[dt][2] * inv, o[dt][3] * inv);
            *reinterpret_cast<uint2*>(dst + 16 * dt) = w;
        }
    } else {
        const int64_t pi = bh * p.splits + split;
        float* dst = p.part_o + pi * D + 4 * j;
#pragma unroll
        for (int dt = 0; dt < DT; ++dt) {
            *reinterpret_cast<float4*>(dst + 16 * dt) =
                make_float4(o[dt][0] * inv, o[dt][1] * inv, o[dt][2] * inv, o[dt][3] * inv);
        }
        if (j == 0) {
            p.part_lse[pi] = l > 0.f ? m + fast_log2(l) : kNegInf;
        }
    }
}

template <bool BF16, int D>
static hipError_t launch_mfma_t(const PartitionParams& p, hipStream_t stream) {
    constexpr int kWaves = 4;
    const int blocks = (p.num_items + kWaves - 1) / kWaves;
    hipLaunchKernelGGL((partition_mfma_kernel<BF16, D>), dim3(blocks), dim3(64 * kWaves), 0, stream, p);
    return hipGetLastError();
}

hipError_t launch_partition_mfma(const PartitionParams& p, bool bf16, int head_dim, hipStream_t stream) {
    if (bf16) {
        switch (head_dim) {
        case 64: return launch_mfma_t<true, 64>(p, stream);
        case 128: return launch_mfma_t<true, 128>(p, stream);
        case 256: return launch_mfma_t<true, 256>(p, stream);
        default: return hipErrorInvalidValue;
        }
    }
    switch (head_dim) {
    case 64: return launch_mfma_t<false, 64>(p, stream);
    case 128: return launch_mfma_t<false, 128>(p, stream);
    case 256: return launch_mfma_t<false, 256>(p, stream);
    default: return hipErrorInvalidValue;
    }
}

} // namespace pkv
