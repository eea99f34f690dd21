// nerve_rows_scalar_bf16_mask.hip -- slice kernels for one bf16 per load (unaligned rows), with an allowed-token mask.
// One translation unit per variant so the kernels compile in parallel.
#include "nerve_sampler_device.h"

namespace nerve {

hipError_t launch_rows_scalar_bf16_mask(const StepArgs &a, hipStream_t stream) { return launch_scalar<uint16_t, true>(a, stream); }

}  // namespace nerve
