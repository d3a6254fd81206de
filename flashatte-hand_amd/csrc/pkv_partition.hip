// pkv_partition.hip — head_dim dispatch of the partition kernels (their
// templates are in pkv_partition_impl.h, instantiated by pkv_part_d*.hip).
#include "pkv_launch.h"

namespace pkv {

hipError_t launch_partition_d64(const PartitionParams& p, bool mfma, bool bf16, int heads_per_wave,
                                hipStream_t stream, const LaunchEvents& ev);
hipError_t launch_partition_d128(const PartitionParams& p, bool mfma, bool bf16, int heads_per_wave,
                                 hipStream_t stream, const LaunchEvents& ev);
hipError_t launch_partition_d256(const PartitionParams& p, bool mfma, bool bf16, int heads_per_wave,
                                 hipStream_t stream, const LaunchEvents& ev);

hipError_t launch_partition(const PartitionParams& p, bool mfma, bool bf16, int head_dim, int heads_per_wave,
                            hipStream_t stream, const LaunchEvents& ev) {
    switch (head_dim) {
    case 64: return launch_partition_d64(p, mfma, bf16, heads_per_wave, stream, ev);
    case 128: return launch_partition_d128(p, mfma, bf16, heads_per_wave, stream, ev);
    case 256: return launch_partition_d256(p, mfma, bf16, heads_per_wave, stream, ev);
    default: return hipErrorInvalidValue;
    }
}

} // namespace pkv
