// pkv_combine.hip — LSE combine of split-KV partials on gfx950.
//
// One wave64 per (b, h) row.  With w_s = exp2(lse_s - max_s lse_s) (0 when the
// split is empty, lse = -inf), out = (sum_s w_s o_s) / sum_s w_s, cast RNE.
// An empty split's O is never read (its weight is 0), so stale workspace
// contents cannot reach the output.
// Reference: submission-oj/best_flashattn_kvcache_decode.cu:956-1037 and
// v11_best_hybrid/flashattn_kvcache_decode_v11_best_hybrid.cu:604-613.
#include "pkv_device.h"
#include "pkv_launch.h"

namespace pkv {

template <bool BF16, int D>
__global__ __launch_bounds__(256) void combine_kernel(CombineParams p) {
    constexpr int E = D / 64; // output elements per lane
    static_assert(E >= 1 && E <= 8, "head_dim must be 64..512");
    const int lane = threadIdx.x & 63;
    const int row = blockIdx.x * (blockDim.x >> 6) + (threadIdx.x >> 6);
    if (row >= p.rows) {
        return;
    }
    const int splits = p.splits;
    const float* __restrict__ lse = p.part_lse + static_cast<int64_t>(row) * splits;

    float mx = kNegInf;
    for (int s = lane; s < splits; s += 64) {
        mx = fmaxf(mx, lse[s]);
    }
    mx = group_max<64>(mx);

    float den = 0.f;
    for (int s = lane; s < splits; s += 64) {
        const float v = lse[s];
        den += v == kNegInf ? 0.f : fast_exp2(v - mx);
    }
    den = group_sum<64>(den);
    const float inv = den > 0.f ? 1.f / den : 0.f;

    float acc[E];
#pragma unroll
    for (int e = 0; e < E; ++e) {
        acc[e] = 0.f;
    }
    const float* __restrict__ o = p.part_o + static_cast<int64_t>(row) * splits * D + lane * E;
#pragma unroll 4
    for (int s = 0; s < splits; ++s) {
        const float v = lse[s];
        if (v == kNegInf) {
            continue;
        }
        const float w = fast_exp2(v - mx);
        float x[E];
        if constexpr (E == 4) {
            const float4 t = *reinterpret_cast<const float4*>(o + static_cast<int64_t>(s) * D);
            x[0] = t.x; x[1] = t.y; x[2] = t.z; x[3] = t.w;
        } else if constexpr (E == 2) {
            const float2 t = *reinterpret_cast<const float2*>(o + static_cast<int64_t>(s) * D);
            x[0] = t.x; x[1] = t.y;
        } else {
#pragma unroll
            for (int e = 0; e < E; ++e) {
                x[e] = o[static_cast<int64_t>(s) * D + e];
            }
        }
#pragma unroll
        for (int e = 0; e < E; ++e) {
            acc[e] = fmaf(w, x[e], acc[e]);
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
