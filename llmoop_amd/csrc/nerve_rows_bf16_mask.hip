// nerve_rows_bf16_mask.hip -- slice kernels for 16-byte loads of 8 bf16, with an allowed-token mask.
// One translation unit per variant so the kernels compile in parallel.
#include "nerve_sampler_device.h"

namespace nerve {

hipError_t launch_rows_bf16_mask(const StepArgs &a, hipStream_t stream) { return launch_vec<uint16_t, 8, true>(a, stream); }

}  // namespace nerve
