// nerve_rows_scalar_f32_plain.hip -- slice kernels for one f32 per load (unaligned rows), without an allowed-token mask.
// One translation unit per variant so the kernels compile in parallel.
#include "nerve_sampler_device.h"

namespace nerve {

hipError_t launch_rows_scalar_f32_plain(const StepArgs &a, hipStream_t stream) { return launch_scalar<float, false>(a, stream); }

}  // namespace nerve
