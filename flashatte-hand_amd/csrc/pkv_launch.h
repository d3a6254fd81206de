// pkv_launch.h — host-side launchers of the device kernels (internal to the library).
#pragma once

#include <hip/hip_ext.h>
#include <hip/hip_runtime.h>

#include "pkv_device.h"

namespace pkv {

// Optional profiling events.  When set, the launch's own dispatch packet
// records them as the kernel starts and completes (hipExtLaunchKernelGGL), so
// their difference is the kernel's execution time without extra marker packets
// on the stream.
struct LaunchEvents {
    hipEvent_t start = nullptr;
    hipEvent_t stop = nullptr;
};

template <typename... KArgs, typename... Args>
inline void launch_kernel(void (*kernel)(KArgs...), dim3 grid, dim3 block, size_t lds, hipStream_t stream,
                          const LaunchEvents& ev, Args... args) {
    if (ev.start != nullptr) {
        hipExtLaunchKernelGGL(kernel, grid, block, static_cast<uint32_t>(lds), stream, ev.start, ev.stop, 0u,
                              args...);
    } else {
        hipLaunchKernelGGL(kernel, grid, block, static_cast<uint32_t>(lds), stream, args...);
    }
}

// Partition kernels (pkv_partition_impl.h, one translation unit per head_dim):
// MFMA math (heads_per_wave 16 or 32 query rows, zero-padded; several query
// tokens, masks and FP8 caches) or VALU math (heads_per_wave in {1, 2, 4};
// one query token, 16-bit caches); head_dim in {64, 128, 256}; the
// tile-balanced kernel when p.tile_workers > 0, else the split-schedule kernels.
hipError_t launch_partition(const PartitionParams& p, bool mfma, bool bf16, int head_dim, int heads_per_wave,
                            hipStream_t stream, const LaunchEvents& ev);

// LSE combine of split partials into the 16-bit output; with `fold` (tile
// schedule only) the combine also adds and stores the appended tokens.
hipError_t launch_combine(const CombineParams& p, const FoldParams* fold, bool bf16, int head_dim,
                          hipStream_t stream, const LaunchEvents& ev);

// Paged KV-cache append: slot-mapping form when p.slot_mapping is set, else
// the block-table form.
hipError_t launch_append(const AppendParams& p, hipStream_t stream, const LaunchEvents& ev);

// Block-table append with rotary embedding of the new keys, and q rotated
// into p.q_out (RotaryAppendParams).
hipError_t launch_rotary_append(const RotaryAppendParams& p, hipStream_t stream);

} // namespace pkv
