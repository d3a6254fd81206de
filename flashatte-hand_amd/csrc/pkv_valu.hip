// pkv_valu.hip — VALU partition kernel for paged-KV GQA decode on gfx950.
//
// One wave64 owns one work item (b, kv head, head group, split).  The 64 lanes
// form R = 64 / L rows of L = D / 8 lanes; a row holds one token at a time,
// each lane 8 consecutive dims (16 bytes), so one vector load per lane moves R
// whole token rows and every load of the wave is a coalesced 16 B/lane access.
// The heads of the group that share the KV head (GQA) reuse each K/V load:
//   scores   v_dot2c_f32_{bf16,f16} on packed 16-bit q and k (no unpacking of K),
//            then a DPP butterfly over the L lanes of the row,
//   softmax  fp32, log2 domain, updated once per chunk of NT tokens per row,
//   PV       fp32 FMAs into 8 accumulators per head per lane.
// At the end the R per-row states are merged (max / rescale / add) and the wave
// writes either the final output (splits == 1) or a normalised partial O plus
// its log2 LSE for the combine kernel.
//
// Reference semantics followed: submission-oj/best_flashattn_kvcache_decode.cu
// 595-954 (partition: page ranges 664-671, empty split 680-697, exp2 online
// update 782-833, lse2 845-864), 256-283 (seqlen 0 and 1), 410-413 (GQA map).
#include "pkv_device.h"
#include "pkv_launch.h"

namespace pkv {

template <bool BF16, int D, int GT, int NT>
__global__ __launch_bounds__(64 * kWavesPerGroup) void partition_valu_kernel(PartitionParams p) {
    constexpr int L = D / 8;   // lanes per token row
    constexpr int R = 64 / L;  // token rows per wave
    static_assert(L * R == 64, "head_dim must be 64, 128, 256 or 512");

    const int lane = threadIdx.x & 63;
    const int item = wave_item();
    if (item >= p.num_items) {
        return;
    }
    const Item it = decode_item(item, p);
    const int split = it.split;
    const int b = it.b;
    const int kvh = it.kvh;
    const int hg = it.hg;

    const int row = lane / L;
    const int sub = lane % L;
    const int g_first = hg * GT;
    const int heads_here = min(GT, p.group - g_first);
    const int h_first = kvh * p.group + g_first;          // first query head of this wave
    const int64_t bh_first = static_cast<int64_t>(b) * p.num_heads + h_first;

    const int seqlen = min(p.seqlens[b], p.row_cap);
    const TokenRange range = split_tokens_of(seqlen, p.page_shift, split, p.splits, p.split_tokens);

    if (range.begin >= range.end) {
        // Empty range: zeros for a row without tokens (one split); with several
        // splits the combine skips this slot (it derives them from cache_seqlens).
        if (p.splits == 1) {
            for (int g = row; g < heads_here; g += R) {
                *reinterpret_cast<uint4*>(p.out + (bh_first + g) * D + sub * 8) = make_uint4(0u, 0u, 0u, 0u);
            }
        }
        return;
    }

    // q of every head in the group, packed 16-bit, this lane's 8 dims.
    uint4 qv[GT];
#pragma unroll
    for (int g = 0; g < GT; ++g) {
        const int gg = g < heads_here ? g : 0;
        qv[g] = *reinterpret_cast<const uint4*>(p.q + (bh_first + gg) * D + sub * 8);
    }

    const int32_t* __restrict__ bt_row = p.block_table + static_cast<int64_t>(b) * p.bt_stride;
    const int64_t head_off = static_cast<int64_t>(kvh) * D + sub * 8;

    float m[GT], l[GT], acc[GT][8];
#pragma unroll
    for (int g = 0; g < GT; ++g) {
        m[g] = kNegInf;
        l[g] = 0.f;
#pragma unroll
        for (int j = 0; j < 8; ++j) {
            acc[g][j] = 0.f;
        }
    }

    for (int tc = range.begin; tc < range.end; tc += R * NT) {
        uint4 kr[NT], vr[NT];
        bool valid[NT];
#pragma unroll
        for (int i = 0; i < NT; ++i) {
            const int t = tc + row + R * i;
            valid[i] = t < range.end;
            const int tt = valid[i] ? t : range.end - 1; // clamp: never touch unowned slots
            const int64_t off = token_elem_offset(bt_row, tt, p) + head_off;
            kr[i] = load_kv16(p.k + off);
            vr[i] = load_kv16(p.v + off);
        }

        float s[NT][GT];
#pragma unroll
        for (int i = 0; i < NT; ++i) {
#pragma unroll
            for (int g = 0; g < GT; ++g) {
                float d = dot2<BF16>(qv[g].x, kr[i].x, 0.f);
                d = dot2<BF16>(qv[g].y, kr[i].y, d);
                d = dot2<BF16>(qv[g].z, kr[i].z, d);
                d = dot2<BF16>(qv[g].w, kr[i].w, d);
                d = group_sum<L>(d);
                s[i][g] = valid[i] ? d * p.scale_log2 : kNegInf;
            }
        }

#pragma unroll
        for (int g = 0; g < GT; ++g) {
            float cmax = s[0][g];
#pragma unroll
            for (int i = 1; i < NT; ++i) {
                cmax = fmaxf(cmax, s[i][g]);
            }
            const float m_new = fmaxf(m[g], cmax);
            const float m_use = m_new == kNegInf ? 0.f : m_new; // keeps exp2 away from -inf - -inf
            const float alpha = fast_exp2(m[g] - m_use);
            m[g] = m_new;
            l[g] *= alpha;
#pragma unroll
            for (int j = 0; j < 8; ++j) {
                acc[g][j] *= alpha;
            }
#pragma unroll
            for (int i = 0; i < NT; ++i) {
                s[i][g] = fast_exp2(s[i][g] - m_use);
                l[g] += s[i][g];
            }
        }

#pragma unroll
        for (int i = 0; i < NT; ++i) {
            float vf[8];
            unpack2<BF16>(vr[i].x, vf[0], vf[1]);
            unpack2<BF16>(vr[i].y, vf[2], vf[3]);
            unpack2<BF16>(vr[i].z, vf[4], vf[5]);
            unpack2<BF16>(vr[i].w, vf[6], vf[7]);
#pragma unroll
            for (int g = 0; g < GT; ++g) {
#pragma unroll
                for (int j = 0; j < 8; ++j) {
                    acc[g][j] = fmaf(s[i][g], vf[j], acc[g][j]);
                }
            }
        }
    }

    // Merge the R row states: every lane ends with the wave total for its 8 dims.
#pragma unroll
    for (int g = 0; g < GT; ++g) {
        float mw = m[g];
#pragma unroll
        for (int stride = L; stride < 64; stride *= 2) {
            mw = fmaxf(mw, __shfl_xor(mw, stride, 64));
        }
        const float sc = m[g] == kNegInf ? 0.f : fast_exp2(m[g] - mw);
        float lw = l[g] * sc;
#pragma unroll
        for (int j = 0; j < 8; ++j) {
            acc[g][j] *= sc;
        }
#pragma unroll
        for (int stride = L; stride < 64; stride *= 2) {
            lw += __shfl_xor(lw, stride, 64);
#pragma unroll
            for (int j = 0; j < 8; ++j) {
                acc[g][j] += __shfl_xor(acc[g][j], stride, 64);
            }
        }
        m[g] = mw;
        l[g] = lw;
    }

#pragma unroll
    for (int g = 0; g < GT; ++g) {
        if (g >= heads_here || (g % R) != row) {
            continue;
        }
        const float inv = l[g] > 0.f ? 1.f / l[g] : 0.f;
        if (p.splits == 1) {
            uint4 o;
            o.x = pack2<BF16>(acc[g][0] * inv, acc[g][1] * inv);
            o.y = pack2<BF16>(acc[g][2] * inv, acc[g][3] * inv);
            o.z = pack2<BF16>(acc[g][4] * inv, acc[g][5] * inv);
            o.w = pack2<BF16>(acc[g][6] * inv, acc[g][7] * inv);
            *reinterpret_cast<uint4*>(p.out + (bh_first + g) * D + sub * 8) = o;
        } else {
            const int64_t pi = (bh_first + g) * p.splits + split;
            float4* dst = reinterpret_cast<float4*>(p.part_o + pi * D + sub * 8);
            dst[0] = make_float4(acc[g][0] * inv, acc[g][1] * inv, acc[g][2] * inv, acc[g][3] * inv);
            dst[1] = make_float4(acc[g][4] * inv, acc[g][5] * inv, acc[g][6] * inv, acc[g][7] * inv);
            if (sub == 0) {
                p.part_lse[pi] = l[g] > 0.f ? m[g] + fast_log2(l[g]) : kNegInf;
            }
        }
    }
}

// ---------------------------------------------------------------- launchers

template <bool BF16, int D, int GT>
static hipError_t launch_valu_t(const PartitionParams& p, hipStream_t stream, const LaunchEvents& ev) {
    constexpr int NT = GT <= 2 ? 8 : (GT <= 4 ? 8 : (GT <= 8 ? 4 : 2));
    constexpr int kWaves = kWavesPerGroup;
    const int blocks = p.num_groups;
    launch_kernel(partition_valu_kernel<BF16, D, GT, NT>, dim3(blocks), dim3(64 * kWaves), 0, stream, ev, p);
    return hipGetLastError();
}

template <bool BF16, int D>
static hipError_t launch_valu_d(const PartitionParams& p, int gt, hipStream_t stream, const LaunchEvents& ev) {
    switch (gt) {
    case 1: return launch_valu_t<BF16, D, 1>(p, stream, ev);
    case 2: return launch_valu_t<BF16, D, 2>(p, stream, ev);
    case 4: return launch_valu_t<BF16, D, 4>(p, stream, ev);
    case 8: return launch_valu_t<BF16, D, 8>(p, stream, ev);
    case 16: return launch_valu_t<BF16, D, 16>(p, stream, ev);
    default: return hipErrorInvalidValue;
    }
}

hipError_t launch_partition_valu(const PartitionParams& p, bool bf16, int head_dim, int heads_per_wave,
                                 hipStream_t stream, const LaunchEvents& ev) {
    if (bf16) {
        switch (head_dim) {
        case 64: return launch_valu_d<true, 64>(p, heads_per_wave, stream, ev);
        case 128: return launch_valu_d<true, 128>(p, heads_per_wave, stream, ev);
        case 256: return launch_valu_d<true, 256>(p, heads_per_wave, stream, ev);
        default: return hipErrorInvalidValue;
        }
    }
    switch (head_dim) {
    case 64: return launch_valu_d<false, 64>(p, heads_per_wave, stream, ev);
    case 128: return launch_valu_d<false, 128>(p, heads_per_wave, stream, ev);
    case 256: return launch_valu_d<false, 256>(p, heads_per_wave, stream, ev);
    default: return hipErrorInvalidValue;
    }
}

} // namespace pkv
