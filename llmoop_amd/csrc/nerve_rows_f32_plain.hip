// nerve_rows_f32_plain.hip -- slice kernels for 16-byte loads of 4 f32, without an allowed-token mask.
// One translation unit per variant so the kernels compile in parallel.
#include "nerve_sampler_device.h"

namespace nerve {

hipError_t launch_rows_f32_plain(const StepArgs &a, hipStream_t stream) { return launch_vec<float, 4, false>(a, stream); }

}  // namespace nerve
