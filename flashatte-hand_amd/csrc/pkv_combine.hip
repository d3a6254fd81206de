// pkv_combine.hip — LSE combine of split-KV partials on gfx950.
//
// One wave64 per (b, h) row.  The row's non-empty splits are derived from
// cache_seqlens with the same range arithmetic the partition kernel used, so
// slots of empty splits are never read (whatever the workspace holds).  With
// w_s = exp2(lse_s - max_s lse_s), out = (sum_s w_s o_s) * (1 / sum_s w_s),
// cast RNE; a row without tokens gets zeros.  Partial rows are read in
// batches of 8 splits so their loads are in flight together.
// Reference: submission-oj/best_flashattn_kvcache_decode.cu:956-1037 and
// v11_best_hybrid/flashattn_kvcache_decode_v11_best_hybrid.cu:604-613.
#include "pkv_device.h"
#include "pkv_launch.h"

namespace pkv {

__device__ __forceinline__ bool split_nonempty(const CombineParams& p, int seqlen, int s) {
    const TokenRange r = split_tokens_of(seqlen, p.page_shift, s, p.splits, p.split_tokens);
    return r.begin < r.end;
}

template <bool BF16, int D>
__global__ __launch_bounds__(256) void combine_kernel(CombineParams p) {
    constexpr int E = D / 64; // output elements per lane
    constexpr int kBatch = 8;
    static_assert(E >= 1 && E <= 8, "head_dim must be 64..512");
    const int lane = threadIdx.x & 63;
    const int row = blockIdx.x * (blockDim.x >> 6) + (threadIdx.x >> 6);
    if (row >= p.rows) {
        return;
    }
    const int seqlen = min(p.seqlens[row / p.num_heads], p.row_cap);
    // Splits past the last token window are empty in split_tokens mode.
    const int n_loop = p.split_tokens > 0
                           ? (seqlen > 0 ? min(p.splits, (seqlen + p.split_tokens - 1) / p.split_tokens) : 0)
                           : p.splits;
    const float* __restrict__ lse = p.part_lse + static_cast<int64_t>(row) * p.splits;

    float mx = kNegInf;
    for (int s = lane; s < n_loop; s += 64) {
        if (split_nonempty(p, seqlen, s)) {
            mx = fmaxf(mx, lse[s]);
        }
    }
    mx = group_max<64>(mx);
    float den = 0.f;
    for (int s = lane; s < n_loop; s += 64) {
        if (split_nonempty(p, seqlen, s)) {
            den += fast_exp2(lse[s] - mx);
        }
    }
    den = group_sum<64>(den);
    const float inv = den > 0.f ? 1.f / den : 0.f;

    float acc[E];
#pragma unroll
    for (int e = 0; e < E; ++e) {
        acc[e] = 0.f;
    }
    const float* __restrict__ o = p.part_o + static_cast<int64_t>(row) * p.splits * D + lane * E;
    for (int s0 = 0; s0 < n_loop; s0 += kBatch) {
        float w[kBatch];
        float x[kBatch][E];
#pragma unroll
        for (int u = 0; u < kBatch; ++u) {
            const int s = s0 + u;
            const bool use = s < n_loop && split_nonempty(p, seqlen, s);
            w[u] = use ? fast_exp2(lse[s] - mx) : 0.f;
#pragma unroll
            for (int e = 0; e < E; ++e) {
                x[u][e] = 0.f;
            }
            if (use) {
                const float* src = o + static_cast<int64_t>(s) * D;
                if constexpr (E == 4) {
                    const float4 t = *reinterpret_cast<const float4*>(src);
                    x[u][0] = t.x; x[u][1] = t.y; x[u][2] = t.z; x[u][3] = t.w;
                } else if constexpr (E == 2) {
                    const float2 t = *reinterpret_cast<const float2*>(src);
                    x[u][0] = t.x; x[u][1] = t.y;
                } else {
#pragma unroll
                    for (int e = 0; e < E; ++e) {
                        x[u][e] = src[e];
                    }
                }
            }
        }
#pragma unroll
        for (int u = 0; u < kBatch; ++u) {
#pragma unroll
            for (int e = 0; e < E; ++e) {
                acc[e] = fmaf(w[u], x[u][e], acc[e]);
            }
        }
    }
    uint16_t* dst = p.out + static_cast<int64_t>(row) * D + lane * E;
#pragma unroll
    for (int e = 0; e < E; ++e) {
        dst[e] = from_f32<BF16>(acc[e] * inv);
    }
}

template <bool BF16, int D>
static hipError_t launch_combine_t(const CombineParams& p, hipStream_t stream) {
    constexpr int kWaves = 4;
    const int blocks = (p.rows + kWaves - 1) / kWaves;
    hipLaunchKernelGGL((combine_kernel<BF16, D>), dim3(blocks), dim3(64 * kWaves), 0, stream, p);
    return hipGetLastError();
}

hipError_t launch_combine(const CombineParams& p, bool bf16, int head_dim, hipStream_t stream) {
    if (bf16) {
        switch (head_dim) {
        case 64: return launch_combine_t<true, 64>(p, stream);
        case 128: return launch_combine_t<true, 128>(p, stream);
        case 256: return launch_combine_t<true, 256>(p, stream);
        default: return hipErrorInvalidValue;
        }
    }
    switch (head_dim) {
    case 64: return launch_combine_t<false, 64>(p, stream);
    case 128: return launch_combine_t<false, 128>(p, stream);
    case 256: return launch_combine_t<false, 256>(p, stream);
    default: return hipErrorInvalidValue;
    }
}

} // namespace pkv
