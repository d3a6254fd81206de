// pkv_launch.h — host-side launchers of the device kernels (internal to the library).
#pragma once

#include <hip/hip_runtime.h>

#include "pkv_device.h"

namespace pkv {

// VALU partition kernel; heads_per_wave in {1, 2, 4, 8, 16}, head_dim in {64, 128, 256}.
hipError_t launch_partition_valu(const PartitionParams& p, bool bf16, int head_dim, int heads_per_wave,
                                 hipStream_t stream);

// MFMA partition kernel; 16 heads per wave (zero-padded), head_dim in {64, 128, 256}.
hipError_t launch_partition_mfma(const PartitionParams& p, bool bf16, int head_dim, hipStream_t stream);

// LSE combine of split partials into the 16-bit output.
hipError_t launch_combine(const CombineParams& p, bool bf16, int head_dim, hipStream_t stream);

} // namespace pkv
