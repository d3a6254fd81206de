// pkv_part_d128.hip — the partition kernels for head_dim 128 (one translation
// unit per head_dim so the library builds in parallel).
#include "pkv_partition_impl.h"

namespace pkv {

hipError_t launch_partition_d128(const PartitionParams& p, bool mfma, bool bf16, int heads_per_wave,
                                 hipStream_t stream, const LaunchEvents& ev) {
    return launch_partition_for_d<128>(p, mfma, bf16, heads_per_wave, stream, ev);
}

} // namespace pkv
