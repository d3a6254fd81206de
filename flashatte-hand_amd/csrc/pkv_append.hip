// pkv_append.hip — paged KV-cache append on gfx950.
//
// Writes new tokens' K and V rows into their page slots.  A pure copy: every
// byte of the new-token tensors is read once and written once into the cache,
// so the kernel is HBM-bound at 4 bytes moved per 16-bit element of K and V
// each.  One 16-byte chunk of K and one of V per thread, grid-strided.
//
// Two index sources for the destination slot of token row i:
//  - block table (flash-attn 2.6.3 flash_attn_with_kvcache with k / v given;
//    the reference's evaluator passes them as None,
//    scripts/evaluate_flashattn_submission.py:236-237): token j of row b goes to
//    position pos = max(cache_seqlens[b], 0) + j of the row, i.e. slot pos % P of
//    page block_table[b][pos / P];
//  - slot mapping (vLLM's reshape_and_cache_flash over the same
//    [num_pages, P, Hk, D] layout): token i goes to flat slot slot_mapping[i] =
//    page * P + slot; a negative slot is padding and is skipped.
// Positions past the block-table row, page ids outside [0, num_pages) and slots
// outside the cache are not written, so a bad index never writes out of bounds.
#include <algorithm>

#include "pkv_device.h"
#include "pkv_launch.h"

namespace pkv {

constexpr int kAppendThreads = 256;

// Grid cap: enough workgroups to keep every CU's memory pipeline full; larger
// copies loop.
constexpr int64_t kAppendMaxGroups = int64_t{kComputeUnits} * 32;

template <bool SLOTS>
__global__ __launch_bounds__(kAppendThreads) void append_kernel(AppendParams p) {
    const int64_t total = p.tokens * p.chunks;
    const int64_t step = static_cast<int64_t>(gridDim.x) * kAppendThreads;
    for (int64_t x = static_cast<int64_t>(blockIdx.x) * kAppendThreads + threadIdx.x; x < total; x += step) {
        const int64_t i = x / p.chunks;
        const int32_t c = static_cast<int32_t>(x - i * p.chunks);
        int64_t slot;
        if constexpr (SLOTS) {
            slot = p.slot_mapping[i];
            if (slot < 0 || slot >= p.num_slots) {
                continue;
            }
        } else {
            const int32_t b = static_cast<int32_t>(i / p.n_new);
            const int32_t j = static_cast<int32_t>(i - static_cast<int64_t>(b) * p.n_new);
            const int64_t base = max(p.seqlens[b], 0);
            if (p.seqlens_out != nullptr && j == 0 && c == 0) {
                p.seqlens_out[b] = static_cast<int32_t>(min(base + p.n_new, static_cast<int64_t>(INT32_MAX)));
            }
            const int64_t pos = base + j;
            if (pos >= p.row_cap) {
                continue;
            }
            const int32_t page =
                p.block_table[static_cast<int64_t>(b) * p.bt_stride + static_cast<int32_t>(pos >> p.page_shift)];
            if (page < 0 || page >= p.num_pages) {
                continue;
            }
            slot = (static_cast<int64_t>(page) << p.page_shift) | (pos & ((int64_t{1} << p.page_shift) - 1));
        }
        const u32x4 kx = __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(p.k_new) + x);
        const u32x4 vx = __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(p.v_new) + x);
        const int64_t dst = slot * p.chunks + c;
        reinterpret_cast<u32x4*>(p.k_cache)[dst] = kx;
        reinterpret_cast<u32x4*>(p.v_cache)[dst] = vx;
    }
}

hipError_t launch_append(const AppendParams& p, hipStream_t stream, const LaunchEvents& ev) {
    const int64_t total = p.tokens * p.chunks;
    if (total <= 0) {
        return hipSuccess;
    }
    const int64_t groups = std::min<int64_t>((total + kAppendThreads - 1) / kAppendThreads, kAppendMaxGroups);
    if (p.slot_mapping != nullptr) {
        launch_kernel(append_kernel<true>, dim3(static_cast<uint32_t>(groups)), dim3(kAppendThreads), 0, stream, ev,
                      p);
    } else {
        launch_kernel(append_kernel<false>, dim3(static_cast<uint32_t>(groups)), dim3(kAppendThreads), 0, stream, ev,
                      p);
    }
    return hipGetLastError();
}

} // namespace pkv
