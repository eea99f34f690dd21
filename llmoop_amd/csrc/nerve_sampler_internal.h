// nerve_sampler_internal.h -- launch arguments shared by the API and the kernels.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "nerve_sampler.h"

namespace nerve {

enum : uint32_t {
    kVariantF32Vec = 0,     // 16-byte loads, 4 f32 per load
    kVariantBf16Vec = 1,    // 16-byte loads, 8 bf16 per load
    kVariantF32Scalar = 2,  // unaligned rows: one element per load
    kVariantBf16Scalar = 3,
};

struct StepArgs {
    const void *logits;
    uint64_t ld;
    const nerve_sampler_row_params *params;
    uint32_t *history;
    uint32_t *history_len;
    uint32_t history_stride;
    uint32_t *seen;
    uint32_t seen_stride;
    const uint32_t *allowed;
    uint32_t allowed_stride;
    const uint32_t *seeds;
    const uint64_t *steps;
    uint32_t *stream_control;
    uint32_t *ring;
    uint32_t ring_stride;
    nerve_sampler_output *out;
    uint32_t *topk_ids;
    float *topk_logits;
    float *topk_probs;
    uint2 *scratch_lists;    // [max_batch][slices][kcap] sorted slice survivors
    uint32_t *scratch_meta;  // [max_batch][slices]: count | flags << 16
    uint32_t *scratch_counts;  // [max_batch] slices of the row that have arrived (zero between steps)
    uint32_t merge_in_kernel;  // the last slice of a row merges and finishes it
    uint32_t vocab;
    uint32_t batch;
    uint32_t slices;
    uint32_t kcap;
    uint32_t rng;
    uint32_t eos;
    uint32_t nvec;           // full vector slots per row (vocab / elements per slot)
    uint32_t vec_per_slice;  // <= kBlock * nv
    uint32_t nv;             // lane-vectors per lane of the launched kernel
    uint32_t hash_slots;     // power of two, 0 without a history
    uint32_t log2_slots;
    uint32_t bitmap_words;   // LDS words of each slice bitmap (penalty state, mask)
    uint32_t big_entries;    // uint2 entries of the candidate / merge area
    uint32_t dyn_lds_bytes;     // slice kernel
    uint32_t finish_lds_bytes;  // finish kernel (slices > 1)
    int device;                 // HIP ordinal the launch runs on
    uint32_t flags;             // NERVE_BATCH_*
    uint64_t tick_base;
    const uint32_t *prefix_ids;
    const uint32_t *prefix_counts;
    uint32_t prefix_stride;
    uint32_t *feedback_control;
    uint32_t feedback_stride;
    const uint32_t *stop_tokens;
    uint32_t stop_stride;
    const uint2 *tile_records;  // [batch][tile_stride] {largest order key, NaN count} per 64 columns
    uint32_t tile_stride;
};

// Bytes of the static scratch array of nerve_sampler_step_static_scratch
// (per GPU): slice lists of batch x slices x top_k_capacity entries of 8 bytes
// plus 4 bytes of metadata per (row, slice).
constexpr size_t kStaticScratchBytes = (size_t)4 << 20;
// The static array starts with the per-row arrival counts (zero at load,
// reset by each step), then the lists and metadata.
constexpr uint32_t kStaticMaxRows = 16384;
constexpr int kMaxDevices = 64;
// Device address of this GPU's static scratch array (the current device must
// be `device`); taken once per device.
hipError_t static_scratch(int device, void **ptr);

uint32_t elems_per_vector(uint32_t variant);
uint32_t block_threads();
uint32_t merge_capacity();
uint32_t kernel_merge_capacity();  // slice-list entries the slice kernel itself can merge
uint32_t stream_lds_bytes(uint32_t variant, bool mask, bool pen, uint32_t hash_slots, uint32_t bitmap_words,
                          uint32_t kcap);
uint32_t max_vectors_per_lane(uint32_t variant);
uint32_t vectors_per_lane(uint32_t variant, uint32_t need);  // 0 when need exceeds every kernel
uint32_t bitmap_words_for(uint32_t variant, uint32_t nv);  // LDS words of each slice bitmap
hipError_t launch_sample_rows(uint32_t variant, const StepArgs &a, hipStream_t stream);
// per-variant slice-kernel launchers (nerve_rows_*.hip)
hipError_t launch_rows_bf16_plain(const StepArgs &a, hipStream_t stream);
hipError_t launch_rows_bf16_mask(const StepArgs &a, hipStream_t stream);
hipError_t launch_rows_f32_plain(const StepArgs &a, hipStream_t stream);
hipError_t launch_rows_f32_mask(const StepArgs &a, hipStream_t stream);
hipError_t launch_rows_scalar_bf16_plain(const StepArgs &a, hipStream_t stream);
hipError_t launch_rows_scalar_bf16_mask(const StepArgs &a, hipStream_t stream);
hipError_t launch_rows_scalar_f32_plain(const StepArgs &a, hipStream_t stream);
hipError_t launch_rows_scalar_f32_mask(const StepArgs &a, hipStream_t stream);
// sampling from tile records (nerve_tiles.hip)
hipError_t launch_sample_tiles(bool bf16, const StepArgs &a, hipStream_t stream);
uint32_t sample_tiles_lds_bytes(uint32_t hash_slots, uint32_t vocab, bool pen, uint32_t kcap);
uint32_t tile_columns();
uint32_t max_tiles();
hipError_t launch_tile_records(bool bf16, const void *logits, uint64_t ld, uint32_t batch, uint32_t vocab, uint2 *records,
                               uint32_t rec_stride, hipStream_t stream);
// LM-head projection with the tile-record epilogue (nerve_lm_head.hip)
hipError_t launch_lm_head(const uint16_t *frames, uint64_t frames_ld, const uint16_t *weight, uint64_t weight_ld,
                          uint32_t batch, uint32_t input_size, uint32_t vocab, float scale, float *logits, uint64_t logits_ld,
                          uint2 *records, uint32_t rec_stride, hipStream_t stream);
hipError_t launch_record_tokens(uint32_t *seen, uint32_t seen_stride, uint32_t rows, const uint32_t *ids,
                                uint32_t ids_stride, const uint32_t *counts, uint32_t max_count, uint32_t vocab,
                                hipStream_t stream);

}  // namespace nerve
