// nerve_sampler_kernels.hip -- launch dispatch, launch-shape helpers and the
// seen-token recording kernel. The slice kernels are instantiated per variant
// in nerve_rows_*.hip (device code in nerve_sampler_device.h).
#include <mutex>

#include "nerve_sampler_device.h"

namespace nerve {

// Cross-workgroup scratch of nerve_sampler_step_static_scratch: one array per
// GPU, held until the process ends. In host code `scratch` names a host-side
// stand-in, so launches use the device address hipGetSymbolAddress returns,
// taken once per device with that device current.
static __device__ __align__(256) uint8_t scratch[kStaticScratchBytes];

hipError_t static_scratch(int device, void **ptr) {
    static std::mutex mu;
    static void *addr[kMaxDevices] = {};
    if (device < 0 || device >= kMaxDevices) return hipErrorInvalidDevice;
    std::lock_guard<std::mutex> lock(mu);
    if (!addr[device]) {
        void *p = nullptr;
        const hipError_t e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
        if (e != hipSuccess) return e;
        addr[device] = p;
    }
    *ptr = addr[device];
    return hipSuccess;
}

__global__ void record_tokens_kernel(uint32_t *seen, uint32_t seen_stride, uint32_t rows, const uint32_t *ids,
                                     uint32_t ids_stride, const uint32_t *counts, uint32_t max_count,
                                     uint32_t vocab) {
    // record_seen_tokens_batch64.comp.template:19-28, one row per workgroup
    const uint32_t row = blockIdx.x;
    if (row >= rows) return;
    uint32_t n = counts[row];
    n = n > max_count ? max_count : n;
    n = n > ids_stride ? ids_stride : n;
    for (uint32_t i = threadIdx.x; i < n; i += blockDim.x) {
        const uint32_t id = ids[(uint64_t)row * ids_stride + i];
        if (id < vocab) atomicOr(&seen[(uint64_t)row * seen_stride + (id >> 5)], 1u << (id & 31u));
    }
}

template <size_t N>
static uint32_t pick_nv(const uint32_t (&list)[N], uint32_t need) {
    for (uint32_t nv : list)
        if (need <= nv) return nv;
    return 0u;
}
uint32_t max_vectors_per_lane(uint32_t variant) {
    switch (variant) {
        case kVariantBf16Vec: return kBf16NV[4];
        case kVariantF32Vec: return kF32NV[3];
        default: return kScalarNV[1];
    }
}

uint32_t vectors_per_lane(uint32_t variant, uint32_t need) {
    switch (variant) {
        case kVariantBf16Vec: return pick_nv(kBf16NV, need);
        case kVariantF32Vec: return pick_nv(kF32NV, need);
        default: return pick_nv(kScalarNV, need);
    }
}

uint32_t bitmap_words_for(uint32_t variant, uint32_t nv) {
    // every lane of the 512 holding nv lane-vectors: the flag reads of
    // lane-vectors past the slice stay inside the bitmaps
    const uint32_t epv = elems_per_vector(variant);
    return slice_bitmap_words((uint32_t)kBlock * nv * epv, epv);
}

uint32_t elems_per_vector(uint32_t variant) {
    switch (variant) {
        case kVariantF32Vec: return 4u;
        case kVariantBf16Vec: return 8u;
        default: return 1u;
    }
}

uint32_t block_threads() { return (uint32_t)kBlock; }
uint32_t merge_capacity() { return kCandCap; }
uint32_t kernel_merge_capacity() { return kStreamCandCap; }

// LDS of the slice kernel, in its layout order: staged lane-vectors and their
// slots, candidates, the sorted list, the history table, the penalty bitmap
// and the mask bitmap.
uint32_t stream_lds_bytes(uint32_t variant, bool mask, bool pen, uint32_t hash_slots, uint32_t bitmap_words,
                          uint32_t kcap) {
    uint32_t stage = 0;
    switch (variant) {
        case kVariantF32Vec: stage = stage_area_bytes<float, 4>(); break;
        case kVariantBf16Vec: stage = stage_area_bytes<uint16_t, 8>(); break;
        case kVariantF32Scalar: stage = stage_area_bytes<float, 1>(); break;
        default: stage = stage_area_bytes<uint16_t, 1>(); break;
    }
    return stage + kStreamCandCap * 8u + kcap * 8u + hash_slots * 4u + bitmap_words * 4u * ((pen ? 1u : 0u) + (mask ? 1u : 0u));
}

hipError_t launch_sample_rows(uint32_t variant, const StepArgs &a, hipStream_t stream) {
    const bool mask = a.allowed != nullptr;
    switch (variant) {
        case kVariantF32Vec: return mask ? launch_rows_f32_mask(a, stream) : launch_rows_f32_plain(a, stream);
        case kVariantBf16Vec: return mask ? launch_rows_bf16_mask(a, stream) : launch_rows_bf16_plain(a, stream);
        case kVariantF32Scalar:
            return mask ? launch_rows_scalar_f32_mask(a, stream) : launch_rows_scalar_f32_plain(a, stream);
        case kVariantBf16Scalar:
            return mask ? launch_rows_scalar_bf16_mask(a, stream) : launch_rows_scalar_bf16_plain(a, stream);
        default: return hipErrorInvalidValue;
    }
}

hipError_t launch_record_tokens(uint32_t *seen, uint32_t seen_stride, uint32_t rows, const uint32_t *ids,
                                uint32_t ids_stride, const uint32_t *counts, uint32_t max_count, uint32_t vocab,
                                hipStream_t stream) {
    hipLaunchKernelGGL(record_tokens_kernel, dim3(rows), dim3(64), 0, stream, seen, seen_stride, rows, ids,
                       ids_stride, counts, max_count, vocab);
    return hipGetLastError();
}

}  // namespace nerve
