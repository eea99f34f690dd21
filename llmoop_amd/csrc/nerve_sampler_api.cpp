// nerve_sampler_api.cpp -- host side of the C ABI declared in include/nerve_sampler.h.
//
// Spec and runtime-override logic restate the reference's Rust runner
// (runtime-rs/src/vulkan_stream_circuit/sampler.rs); the device handle owns
// only the cross-workgroup scratch of the fused kernel. Every failure is
// reported as a status code; nothing falls back to a CPU path.
#include <hip/hip_runtime.h>

#include <cmath>
#include <cstdio>
#include <cstring>
#include <new>
#include <string>

#include "nerve_sampler.h"
#include "nerve_sampler_internal.h"

namespace {

thread_local std::string g_last_error;

int hip_fail(hipError_t e, const char *what) {
    g_last_error = std::string(what) + ": " + hipGetErrorString(e);
    return NERVE_ERR_HIP;
}

int fail(int code, const std::string &msg) {
    g_last_error = msg;
    return code;
}

bool is_finite(float v) { return std::isfinite(v); }

const char *method_name(uint32_t m) {
    return m == NERVE_METHOD_GREEDY ? "greedy"
           : m == NERVE_METHOD_TEMPERATURE_TOP_K_TOP_P ? "temperature_top_k_top_p"
                                                        : "unknown";
}

uint32_t next_pow2(uint32_t v) {
    uint32_t p = 1;
    while (p < v) p <<= 1;
    return p;
}

// Automatic slices per row: rows of 256 KiB or more in batches below 128
// rows split three ways at most (enough workgroups to use more CUs, each
// slice merged by the row's last one), measured on MI355X: B=64 x V=151936
// bf16 15.7 us with 3 slices against 17.2 with 1; B=32 x V=32000 and B=1
// stay fastest with one.
uint32_t auto_slices(const nerve_sampler_desc &d, uint32_t batch) {
    const uint64_t row_bytes = (uint64_t)d.vocab_size * (d.dtype == NERVE_DTYPE_F32 ? 4u : 2u);
    if (row_bytes < (256u << 10) || batch >= 128u || batch == 0u) return 1u;
    const uint32_t s = (192u + batch - 1u) / batch;
    return s < 3u ? s : 3u;
}

uint32_t log2u(uint32_t v) {
    uint32_t l = 0;
    while ((1u << l) < v) ++l;
    return l;
}

}  // namespace

struct nerve_sampler {
    nerve_sampler_desc desc;
    int device;
    uint32_t slices;           // requested workgroups per row (raised per step if the slice would not fit)
    uint32_t slices_capacity;  // scratch sized for this many
    uint32_t last_slices;      // workgroups per row of the last step
    uint2 *scratch_lists;
    uint32_t *scratch_meta;
    uint32_t *scratch_counts;  // [max_batch] arrival counts of the in-kernel merge, zero between steps
    size_t lds_per_block;      // hipDeviceProp_t::sharedMemPerBlock
};

extern "C" {

uint32_t nerve_sampler_abi_version(void) { return NERVE_SAMPLER_ABI_VERSION; }

const char *nerve_sampler_last_error(void) { return g_last_error.c_str(); }

// sampler.rs:144-160
int nerve_sampler_kernel_role_matches(const char *role, uint32_t runtime_parameterized, uint32_t method) {
    if (!role) return 0;
    const std::string r(role);
    if (method == NERVE_METHOD_GREEDY) return runtime_parameterized ? r == "runtime_sample_logits" : r == "sample_logits";
    if (method == NERVE_METHOD_TEMPERATURE_TOP_K_TOP_P) {
        if (runtime_parameterized) return r == "runtime_partition_top_k" || r == "runtime_sample_candidates";
        return r == "partition_top_k" || r == "sample_candidates";
    }
    return 0;
}

// sampler.rs:66-141
int nerve_sampler_apply_runtime_config(const nerve_sampler_spec *compiled, const nerve_sampler_runtime_config *cfg,
                                       nerve_sampler_spec *out, char *message, size_t message_capacity) {
    if (!compiled || !cfg || !out) return fail(NERVE_ERR_INVALID_ARGUMENT, "null argument");
    const bool empty = !cfg->has_temperature && !cfg->has_top_k && !cfg->has_top_p && !cfg->has_min_p &&
                       !cfg->has_presence_penalty && !cfg->has_repetition_penalty;
    if (empty) {
        *out = *compiled;
        return NERVE_OK;
    }
    nerve_sampler_spec e = *compiled;
    const bool sampled_request = cfg->has_temperature || cfg->has_top_k || cfg->has_top_p || cfg->has_min_p;
    if (compiled->method == NERVE_METHOD_GREEDY && sampled_request) {
        std::snprintf(e.sampler_id, sizeof(e.sampler_id), "%s", "runtime_temperature_top_k_top_p_sampler");
        e.method = NERVE_METHOD_TEMPERATURE_TOP_K_TOP_P;
        e.temperature = 1.0f;
        e.top_k = e.top_k_capacity < 50u ? e.top_k_capacity : 50u;
        e.top_p = 1.0f;
        e.min_p = 0.0f;
    }
    if (cfg->has_temperature) e.temperature = cfg->temperature;
    if (cfg->has_top_k) e.top_k = cfg->top_k;
    if (cfg->has_top_p) e.top_p = cfg->top_p;
    if (cfg->has_min_p) e.min_p = cfg->min_p;
    if (cfg->has_presence_penalty) e.presence_penalty = cfg->presence_penalty;
    if (cfg->has_repetition_penalty) e.repetition_penalty = cfg->repetition_penalty;
    const bool valid_common =
        is_finite(e.presence_penalty) && is_finite(e.repetition_penalty) && e.repetition_penalty > 0.0f;
    bool valid = false;
    if (e.method == NERVE_METHOD_GREEDY) {
        valid = e.min_p == 0.0f && valid_common;
    } else if (e.method == NERVE_METHOD_TEMPERATURE_TOP_K_TOP_P) {
        valid = is_finite(e.temperature) && e.temperature > 0.0f && e.top_k > 0u && e.top_k <= e.top_k_capacity &&
                is_finite(e.top_p) && e.top_p > 0.0f && e.top_p <= 1.0f && is_finite(e.min_p) && e.min_p >= 0.0f &&
                e.min_p <= 1.0f && valid_common;
    }
    if (!valid) {
        char buf[512];
        std::snprintf(buf, sizeof(buf),
                      "runtime sampler override is invalid for method \"%s\": temperature=%g, top_k=%u (capacity %u), "
                      "top_p=%g, min_p=%g, presence_penalty=%g, repetition_penalty=%g",
                      method_name(e.method), (double)e.temperature, e.top_k, e.top_k_capacity, (double)e.top_p,
                      (double)e.min_p, (double)e.presence_penalty, (double)e.repetition_penalty);
        if (message && message_capacity) std::snprintf(message, message_capacity, "%s", buf);
        return fail(NERVE_ERR_UNSUPPORTED_RUNTIME_SAMPLING_OVERRIDE, buf);
    }
    e.runtime_parameterized = 1u;
    *out = e;
    return NERVE_OK;
}

// Construction-time checks of sampler.rs:259-382 that do not concern SPIR-V
// kernel artifacts: logits capacity, history capacity, method parameters and
// the partition scratch size (G * k * 8 bytes).
int nerve_sampler_validate_spec(const nerve_sampler_spec *s, uint64_t logits_byte_capacity,
                                uint32_t history_capacity_activations, uint32_t partition_count) {
    if (!s) return fail(NERVE_ERR_INVALID_ARGUMENT, "null spec");
    if (logits_byte_capacity != s->logits_byte_capacity) {
        char buf[160];
        std::snprintf(buf, sizeof(buf), "sampler logits buffer has %llu bytes, expected %llu",
                      (unsigned long long)logits_byte_capacity, (unsigned long long)s->logits_byte_capacity);
        return fail(NERVE_ERR_INVALID_LOGITS_BYTE_CAPACITY, buf);
    }
    if (history_capacity_activations == 0u) return fail(NERVE_ERR_ZERO_HISTORY_CAPACITY, "sampler history capacity must be nonzero");
    const uint64_t vocab = logits_byte_capacity / 4u;
    const uint32_t per_partition = s->runtime_parameterized ? s->top_k_capacity : s->top_k;
    bool ok = false;
    if (s->method == NERVE_METHOD_GREEDY) {
        ok = s->min_p == 0.0f && is_finite(s->presence_penalty) && is_finite(s->repetition_penalty) &&
             s->repetition_penalty > 0.0f;
    } else if (s->method == NERVE_METHOD_TEMPERATURE_TOP_K_TOP_P) {
        const uint64_t required = (uint64_t)partition_count * per_partition * 8u;
        ok = is_finite(s->temperature) && s->temperature > 0.0f && s->top_k > 0u && s->top_k <= vocab &&
             is_finite(s->top_p) && s->top_p > 0.0f && s->top_p <= 1.0f && is_finite(s->min_p) && s->min_p >= 0.0f &&
             s->min_p <= 1.0f && is_finite(s->presence_penalty) && is_finite(s->repetition_penalty) &&
             s->repetition_penalty > 0.0f && s->top_k <= s->top_k_capacity && partition_count > 0u &&
             required <= s->scratch_byte_capacity;
    }
    if (!ok) {
        char buf[320];
        std::snprintf(buf, sizeof(buf),
                      "invalid resident sampling spec method=\"%s\" temperature=%g top_k=%u top_p=%g min_p=%g "
                      "presence_penalty=%g repetition_penalty=%g",
                      method_name(s->method), (double)s->temperature, s->top_k, (double)s->top_p, (double)s->min_p,
                      (double)s->presence_penalty, (double)s->repetition_penalty);
        return fail(NERVE_ERR_INVALID_SAMPLING_SPEC, buf);
    }
    const uint64_t history_bytes = (uint64_t)history_capacity_activations * 16u + s->output_byte_capacity;
    if (history_bytes < s->output_byte_capacity) return fail(NERVE_ERR_HISTORY_CAPACITY_OVERFLOW, "sampler history byte capacity overflowed");
    return NERVE_OK;
}

int nerve_sampler_create(const nerve_sampler_desc *desc, nerve_sampler **out) {
    if (!desc || !out) return fail(NERVE_ERR_INVALID_ARGUMENT, "null argument");
    *out = nullptr;
    const nerve_sampler_desc d = *desc;
    if (d.vocab_size == 0u || d.vocab_size > NERVE_MAX_VOCAB)
        return fail(NERVE_ERR_INVALID_ARGUMENT, "vocab_size must be in 1..1048575");
    if (d.max_batch == 0u) return fail(NERVE_ERR_INVALID_ARGUMENT, "max_batch must be nonzero");
    if (d.dtype != NERVE_DTYPE_F32 && d.dtype != NERVE_DTYPE_BF16) return fail(NERVE_ERR_INVALID_ARGUMENT, "dtype must be f32 or bf16");
    if (d.top_k_capacity == 0u || d.top_k_capacity > NERVE_MAX_TOP_K_CAPACITY)
        return fail(NERVE_ERR_INVALID_SAMPLING_SPEC, "top_k_capacity must be in 1..1024");
    if (d.history_capacity > NERVE_MAX_HISTORY_CAPACITY)
        return fail(NERVE_ERR_HISTORY_CAPACITY_OVERFLOW, "history_capacity must be <= 4095");
    int ndev = 0;
    hipError_t e = hipGetDeviceCount(&ndev);
    if (e != hipSuccess) return hip_fail(e, "hipGetDeviceCount");
    if ((int)d.device >= ndev) return fail(NERVE_ERR_INVALID_ARGUMENT, "device ordinal out of range");
    hipDeviceProp_t prop;
    e = hipGetDeviceProperties(&prop, (int)d.device);
    if (e != hipSuccess) return hip_fail(e, "hipGetDeviceProperties");
    if (std::strncmp(prop.gcnArchName, "gfx950", 6) != 0)
        return fail(NERVE_ERR_HIP, std::string("the sampler kernels are built for gfx950 only, device is ") + prop.gcnArchName);

    // Workgroups per row: a workgroup holds its slice of the row in VGPRs, so
    // a slice is at most block_threads() * max_vectors_per_lane() lane-vectors
    // (raised per step to what the row needs). Automatic (slices_per_row 0):
    // auto_slices() per step.
    const uint32_t threads = nerve::block_threads();
    uint32_t want = d.slices_per_row;
    if (want == 0u) want = 1u;
    // Slices the scratch holds: what 16-byte aligned rows of this dtype need
    // (or more when asked), the automatic split of large rows, and the more
    // slices of the one-element-per-load kernels for unaligned rows when the
    // merge area allows them (otherwise such steps are rejected).
    const uint32_t vvar = d.dtype == NERVE_DTYPE_F32 ? nerve::kVariantF32Vec : nerve::kVariantBf16Vec;
    const uint32_t vec_tokens = threads * nerve::max_vectors_per_lane(vvar) * nerve::elems_per_vector(vvar);
    const uint32_t vec_need = (d.vocab_size + vec_tokens - 1u) / vec_tokens;
    uint32_t capacity = want > vec_need ? want : vec_need;
    if (d.slices_per_row == 0u && auto_slices(d, 1u) > capacity) capacity = auto_slices(d, 1u);
    if ((uint64_t)capacity * d.top_k_capacity > 12288u)
        return fail(NERVE_ERR_INVALID_SAMPLING_SPEC, "slices_per_row * top_k_capacity exceeds the 12288-entry merge area");
    if (capacity > 64u) return fail(NERVE_ERR_INVALID_ARGUMENT, "slices_per_row must be at most 64");
    const uint32_t scalar_tokens = threads * nerve::max_vectors_per_lane(nerve::kVariantF32Scalar);
    const uint32_t scalar_need = (d.vocab_size + scalar_tokens - 1u) / scalar_tokens;
    if (scalar_need > capacity && (uint64_t)scalar_need * d.top_k_capacity <= 12288u && scalar_need <= 64u)
        capacity = scalar_need;

    nerve_sampler *s = new (std::nothrow) nerve_sampler();
    if (!s) return fail(NERVE_ERR_INVALID_ARGUMENT, "out of host memory");
    s->desc = d;
    s->device = (int)d.device;
    s->slices = want;
    s->slices_capacity = capacity;
    {
        // before the first step: the count of an aligned step of this dtype
        const uint32_t v = d.dtype == NERVE_DTYPE_F32 ? nerve::kVariantF32Vec : nerve::kVariantBf16Vec;
        const uint32_t per = threads * nerve::max_vectors_per_lane(v);
        const uint32_t nvec = d.vocab_size / nerve::elems_per_vector(v);
        const uint32_t need_v = nvec ? (nvec + per - 1u) / per : 1u;
        const uint32_t w = d.slices_per_row ? want : auto_slices(d, d.max_batch);
        s->last_slices = w > need_v ? w : need_v;
    }
    s->lds_per_block = prop.sharedMemPerBlock;
    int prev = 0;
    (void)hipGetDevice(&prev);
    (void)hipSetDevice(s->device);
    const size_t lists_bytes = (size_t)d.max_batch * capacity * d.top_k_capacity * sizeof(uint2);
    const size_t meta_bytes = (size_t)d.max_batch * capacity * sizeof(uint32_t);
    if (!(d.flags & NERVE_DESC_NO_SCRATCH)) {
        e = hipMalloc((void **)&s->scratch_lists, lists_bytes);
        if (e == hipSuccess) e = hipMalloc((void **)&s->scratch_meta, meta_bytes);
        if (e == hipSuccess) e = hipMalloc((void **)&s->scratch_counts, (size_t)d.max_batch * sizeof(uint32_t));
        if (e == hipSuccess) e = hipMemset(s->scratch_counts, 0, (size_t)d.max_batch * sizeof(uint32_t));
        if (e == hipSuccess) e = hipDeviceSynchronize();
    }
    (void)hipSetDevice(prev);
    if (e != hipSuccess) {
        int rc = hip_fail(e, "nerve_sampler_create scratch");
        nerve_sampler_destroy(s);
        return rc;
    }
    *out = s;
    return NERVE_OK;
}

int nerve_sampler_destroy(nerve_sampler *s) {
    if (!s) return NERVE_OK;
    int prev = 0;
    (void)hipGetDevice(&prev);
    (void)hipSetDevice(s->device);
    if (s->scratch_lists) (void)hipFree(s->scratch_lists);
    if (s->scratch_meta) (void)hipFree(s->scratch_meta);
    if (s->scratch_counts) (void)hipFree(s->scratch_counts);
    (void)hipSetDevice(prev);
    delete s;
    return NERVE_OK;
}

uint32_t nerve_sampler_slices_per_row(const nerve_sampler *s) { return s ? s->last_slices : 0u; }

namespace {

// One step; `static_scratch` takes the cross-workgroup scratch (used only when
// a row has several slices) from the library's static per-GPU array instead
// of the handle's allocation.
int step_impl(nerve_sampler *s, const nerve_sampler_batch *b, void *stream, bool static_scratch,
              const uint32_t *tile_records = nullptr, uint32_t tile_stride = 0u) {
    if (!s || !b) return fail(NERVE_ERR_INVALID_ARGUMENT, "null argument");
    const nerve_sampler_desc &d = s->desc;
    if (b->batch == 0u) return NERVE_OK;
    if (b->batch > d.max_batch) return fail(NERVE_ERR_BATCH_CAPACITY_EXCEEDED, "batch exceeds max_batch");
    if (!b->logits || !b->params || !b->out) return fail(NERVE_ERR_INVALID_ARGUMENT, "logits, params and out are required");
    if (b->logits_row_stride < d.vocab_size) return fail(NERVE_ERR_INVALID_LOGITS_BYTE_CAPACITY, "logits_row_stride < vocab_size");
    if (b->rng != NERVE_RNG_REFERENCE_HASH && b->rng != NERVE_RNG_PHILOX) return fail(NERVE_ERR_INVALID_ARGUMENT, "unknown rng");
    if (b->history && b->seen) return fail(NERVE_ERR_INVALID_ARGUMENT, "pass a history list or a seen bitmap, not both");
    const uint32_t words = (d.vocab_size + 31u) / 32u;
    if (b->history) {
        if (!b->history_len) return fail(NERVE_ERR_INVALID_ARGUMENT, "history_len is required with history");
        if (b->history_stride == 0u || b->history_stride > d.history_capacity)
            return fail(NERVE_ERR_HISTORY_CAPACITY_OVERFLOW, "history_stride must be in 1..history_capacity");
    }
    if (b->seen && b->seen_stride != 0u && b->seen_stride < words)
        return fail(NERVE_ERR_INVALID_ARGUMENT, "seen_stride must be 0 (one shared bitmap) or >= ceil(vocab/32)");
    if (b->flags & ~(uint32_t)(NERVE_BATCH_APPEND_HISTORY | NERVE_BATCH_CONSECUTIVE_TICKS))
        return fail(NERVE_ERR_INVALID_ARGUMENT, "unknown batch flags");
    if ((b->flags & NERVE_BATCH_APPEND_HISTORY) && !b->history && !b->seen)
        return fail(NERVE_ERR_INVALID_ARGUMENT, "NERVE_BATCH_APPEND_HISTORY needs a history list or a seen bitmap");
    if (b->prefix_ids && !b->seen)
        return fail(NERVE_ERR_INVALID_ARGUMENT, "prefix_ids extend a seen bitmap (set semantics)");
    if (b->prefix_ids && !b->prefix_counts && b->batch > NERVE_TOKEN_BATCH_CAPACITY) {
        char buf[128];
        std::snprintf(buf, sizeof(buf), "sampler repetition-state batch requests %u tokens, capacity is %u", b->batch,
                      NERVE_TOKEN_BATCH_CAPACITY);
        return fail(NERVE_ERR_TOKEN_BATCH_CAPACITY_EXCEEDED, buf);
    }
    if (b->stop_tokens && !b->feedback_control)
        return fail(NERVE_ERR_INVALID_ARGUMENT, "stop_tokens need a feedback_control block");
    if (b->allowed && b->allowed_stride < words) return fail(NERVE_ERR_INVALID_ARGUMENT, "allowed_stride < ceil(vocab/32)");
    if (b->output_ring && !b->stream_control) return fail(NERVE_ERR_INVALID_ARGUMENT, "output_ring requires stream_control");
    if (b->output_ring && b->ring_stride < 4u) return fail(NERVE_ERR_INVALID_ARGUMENT, "ring_stride must hold the 4-word record");

    const bool tiles = tile_records != nullptr;
    if (tiles) {
        const uint32_t ntiles = (d.vocab_size + nerve::tile_columns() - 1u) / nerve::tile_columns();
        if (ntiles > nerve::max_tiles()) return fail(NERVE_ERR_INVALID_ARGUMENT, "vocabulary too large for tile records");
        if (tile_stride < ntiles) return fail(NERVE_ERR_INVALID_ARGUMENT, "tile_stride < ceil(vocab/64)");
        if ((uintptr_t)tile_records % 8u) return fail(NERVE_ERR_INVALID_ARGUMENT, "tile_records must be 8-byte aligned");
    }
    const size_t esize = d.dtype == NERVE_DTYPE_F32 ? 4u : 2u;
    const bool aligned = ((uintptr_t)b->logits % 16u == 0u) && ((b->logits_row_stride * esize) % 16u == 0u);
    // 16-byte loads need an aligned row base and stride and at least one full slot.
    const bool vec_ok = aligned && d.vocab_size >= (d.dtype == NERVE_DTYPE_F32 ? 4u : 8u);
    uint32_t variant;
    if (d.dtype == NERVE_DTYPE_F32) variant = vec_ok ? nerve::kVariantF32Vec : nerve::kVariantF32Scalar;
    else variant = vec_ok ? nerve::kVariantBf16Vec : nerve::kVariantBf16Scalar;

    const uint32_t epv = nerve::elems_per_vector(variant);
    const uint32_t nvec = d.vocab_size / epv;  // full slots; the V % epv tail goes to the last slice
    const uint32_t per_slice_max = nerve::block_threads() * nerve::max_vectors_per_lane(variant);
    uint32_t slices = tiles ? 1u : (d.slices_per_row ? s->slices : auto_slices(d, b->batch));
    const uint32_t slices_need = (nvec + per_slice_max - 1u) / per_slice_max;
    if (slices < slices_need && !tiles) slices = slices_need;
    if (slices > s->slices_capacity) {
        char buf[200];
        std::snprintf(buf, sizeof(buf),
                      "rows of this vocabulary need %u slices with %s logits rows; the handle holds %u (pass "
                      "16-byte aligned rows and strides)",
                      slices, vec_ok ? "aligned" : "unaligned", s->slices_capacity);
        return fail(NERVE_ERR_INVALID_ARGUMENT, buf);
    }
    const uint32_t vec_per_slice = (nvec + slices - 1u) / slices;
    const uint32_t nv = tiles ? 1u : nerve::vectors_per_lane(variant, (vec_per_slice + nerve::block_threads() - 1u) / nerve::block_threads());
    if (nv == 0u) return fail(NERVE_ERR_INVALID_ARGUMENT, "slice exceeds the kernel's register capacity");

    nerve::StepArgs a;
    std::memset(&a, 0, sizeof(a));
    a.logits = b->logits;
    a.ld = b->logits_row_stride;
    a.params = b->params;
    a.history = b->history;
    a.history_len = b->history_len;
    a.history_stride = b->history ? b->history_stride : 0u;
    a.seen = b->seen;
    a.seen_stride = b->seen_stride;
    a.allowed = b->allowed;
    a.allowed_stride = b->allowed_stride;
    a.seeds = b->seeds;
    a.steps = b->steps;
    a.stream_control = b->stream_control;
    a.ring = b->output_ring;
    a.ring_stride = b->ring_stride;
    a.out = b->out;
    a.topk_ids = b->topk_ids;
    a.topk_logits = b->topk_logits;
    a.topk_probs = b->topk_probs;
    a.scratch_lists = s->scratch_lists;
    a.scratch_meta = s->scratch_meta;
    a.scratch_counts = s->scratch_counts;
    a.merge_in_kernel = slices * d.top_k_capacity <= nerve::kernel_merge_capacity() ? 1u : 0u;
    a.vocab = d.vocab_size;
    a.batch = b->batch;
    a.slices = slices;
    a.kcap = d.top_k_capacity;
    a.rng = b->rng;
    a.eos = b->eos_token_id;
    a.nvec = nvec;
    a.vec_per_slice = vec_per_slice;
    a.nv = nv;
    if (b->history) {
        a.hash_slots = next_pow2(2u * b->history_stride);
        if (a.hash_slots < 64u) a.hash_slots = 64u;
        a.log2_slots = log2u(a.hash_slots);
    }
    const bool pen = b->history != nullptr || b->seen != nullptr;
    if (pen || b->allowed) a.bitmap_words = nerve::bitmap_words_for(variant, nv);
    uint32_t big = nerve::merge_capacity();
    if (slices * d.top_k_capacity > big) big = slices * d.top_k_capacity;
    if (d.top_k_capacity + 32u > big) big = d.top_k_capacity + 32u;  // weights + running sums of the finish step
    a.big_entries = big;
    a.finish_lds_bytes = a.hash_slots * 4u + big * 8u + d.top_k_capacity * 8u + (d.top_k_capacity + 64u) * 4u;
    const uint32_t stream_lds = nerve::stream_lds_bytes(variant, b->allowed != nullptr, pen, a.hash_slots,
                                                        a.bitmap_words, d.top_k_capacity);
    a.dyn_lds_bytes = stream_lds;
    a.device = s->device;
    a.flags = b->flags;
    a.tick_base = b->tick_base;
    a.prefix_ids = b->prefix_ids;
    a.prefix_counts = b->prefix_counts;
    a.prefix_stride = b->prefix_stride;
    a.feedback_control = b->feedback_control;
    a.feedback_stride = b->feedback_stride;
    a.stop_tokens = b->stop_tokens;
    a.stop_stride = b->stop_stride;
    const size_t static_lds = 2u * 1024u;  // reduction scratch
    if (tiles) {
        a.tile_records = (const uint2 *)tile_records;
        a.tile_stride = tile_stride;
        a.dyn_lds_bytes = nerve::sample_tiles_lds_bytes(a.hash_slots, d.vocab_size, pen, d.top_k_capacity);
        if (a.dyn_lds_bytes + static_lds + 6u * 1024u > s->lds_per_block)
            return fail(NERVE_ERR_INVALID_ARGUMENT, "LDS need of the tile step (vocabulary, history, top_k_capacity) exceeds the device");
        s->last_slices = 1u;
        int prev_t = 0;
        (void)hipGetDevice(&prev_t);
        if (prev_t != s->device) (void)hipSetDevice(s->device);
        const hipError_t et = nerve::launch_sample_tiles(d.dtype == NERVE_DTYPE_BF16, a, (hipStream_t)stream);
        if (prev_t != s->device) (void)hipSetDevice(prev_t);
        if (et != hipSuccess) return hip_fail(et, "sample_tiles launch");
        return NERVE_OK;
    }
    s->last_slices = slices;
    if (stream_lds + static_lds > s->lds_per_block || a.finish_lds_bytes + static_lds > s->lds_per_block)
        return fail(NERVE_ERR_INVALID_ARGUMENT, "LDS need of this top_k_capacity / history / slice count exceeds the device");

    int prev = 0;
    (void)hipGetDevice(&prev);
    if (prev != s->device) (void)hipSetDevice(s->device);
    struct Restore {
        int prev, dev;
        ~Restore() {
            if (prev != dev) (void)hipSetDevice(prev);
        }
    } restore{prev, s->device};
    if (slices > 1u) {
        const size_t lists = (size_t)b->batch * slices * d.top_k_capacity * sizeof(uint2);
        const size_t meta = (size_t)b->batch * slices * sizeof(uint32_t);
        const size_t counts = (size_t)nerve::kStaticMaxRows * sizeof(uint32_t);
        if (static_scratch) {
            if (counts + lists + meta > nerve::kStaticScratchBytes || b->batch > nerve::kStaticMaxRows) {
                char buf[200];
                std::snprintf(buf, sizeof(buf),
                              "step needs %zu bytes of scratch (batch x slices x top_k_capacity), the static array "
                              "holds %zu",
                              counts + lists + meta, nerve::kStaticScratchBytes);
                return fail(NERVE_ERR_INVALID_ARGUMENT, buf);
            }
            void *base = nullptr;
            const hipError_t e = nerve::static_scratch(s->device, &base);
            if (e != hipSuccess) return hip_fail(e, "hipGetSymbolAddress(scratch)");
            a.scratch_counts = (uint32_t *)base;
            a.scratch_lists = (uint2 *)((uint8_t *)base + counts);
            a.scratch_meta = (uint32_t *)((uint8_t *)base + counts + lists);
        } else if (!s->scratch_lists) {
            return fail(NERVE_ERR_INVALID_ARGUMENT,
                        "this handle was created with NERVE_DESC_NO_SCRATCH: steps with several slices per row go "
                        "through nerve_sampler_step_static_scratch");
        }
    }
    hipError_t e = nerve::launch_sample_rows(variant, a, (hipStream_t)stream);
    if (e != hipSuccess) return hip_fail(e, "sample_rows launch");
    return NERVE_OK;
}

}  // namespace

int nerve_sampler_step(nerve_sampler *s, const nerve_sampler_batch *b, void *stream) {
    return step_impl(s, b, stream, false);
}

int nerve_sampler_step_static_scratch(nerve_sampler *s, const nerve_sampler_batch *b, void *stream) {
    return step_impl(s, b, stream, true);
}

int nerve_sampler_step_tiles(nerve_sampler *s, const nerve_sampler_batch *b, const uint32_t *tile_records,
                             uint32_t tile_stride, void *stream) {
    if (!tile_records) return fail(NERVE_ERR_INVALID_ARGUMENT, "tile_records is required");
    return step_impl(s, b, stream, false, tile_records, tile_stride);
}

int nerve_tile_records(const void *logits, uint32_t dtype, uint32_t logits_row_stride, uint32_t batch, uint32_t vocab_size,
                       uint32_t *tile_records, uint32_t tile_stride, void *stream) {
    if (batch == 0u) return NERVE_OK;
    if (!logits || !tile_records) return fail(NERVE_ERR_INVALID_ARGUMENT, "null argument");
    if (dtype != NERVE_DTYPE_F32 && dtype != NERVE_DTYPE_BF16) return fail(NERVE_ERR_INVALID_ARGUMENT, "dtype must be f32 or bf16");
    if (vocab_size == 0u || logits_row_stride < vocab_size)
        return fail(NERVE_ERR_INVALID_LOGITS_BYTE_CAPACITY, "logits_row_stride < vocab_size");
    const uint32_t ntiles = (vocab_size + nerve::tile_columns() - 1u) / nerve::tile_columns();
    if (tile_stride < ntiles) return fail(NERVE_ERR_INVALID_ARGUMENT, "tile_stride < ceil(vocab/64)");
    if ((uintptr_t)tile_records % 8u) return fail(NERVE_ERR_INVALID_ARGUMENT, "tile_records must be 8-byte aligned");
    const hipError_t e = nerve::launch_tile_records(dtype == NERVE_DTYPE_BF16, logits, logits_row_stride, batch, vocab_size,
                                                    (uint2 *)tile_records, tile_stride, (hipStream_t)stream);
    return e == hipSuccess ? NERVE_OK : hip_fail(e, "tile_records launch");
}

int nerve_lm_head_project(const void *frames, uint32_t frames_row_stride, const void *weight, uint32_t weight_row_stride,
                          uint32_t batch, uint32_t input_size, uint32_t vocab_size, float output_scale, float *logits,
                          uint32_t logits_row_stride, uint32_t *tile_records, uint32_t tile_stride, void *stream) {
    if (batch == 0u || vocab_size == 0u) return NERVE_OK;
    if (!frames || !weight || !logits) return fail(NERVE_ERR_INVALID_ARGUMENT, "null argument");
    if (input_size == 0u || input_size % 64u)
        return fail(NERVE_ERR_INVALID_ARGUMENT, "input_size must be a positive multiple of 64");
    if (frames_row_stride < input_size || weight_row_stride < input_size || frames_row_stride % 8u || weight_row_stride % 8u)
        return fail(NERVE_ERR_INVALID_ARGUMENT, "frame and weight row strides must be >= input_size and multiples of 8");
    if ((uintptr_t)frames % 16u || (uintptr_t)weight % 16u)
        return fail(NERVE_ERR_INVALID_ARGUMENT, "frames and weight must be 16-byte aligned");
    if (logits_row_stride < vocab_size) return fail(NERVE_ERR_INVALID_LOGITS_BYTE_CAPACITY, "logits_row_stride < vocab_size");
    if ((uint64_t)(batch < 256u ? batch : 256u) * frames_row_stride * 2u >= (1ull << 31) ||
        (uint64_t)256u * weight_row_stride * 2u >= (1ull << 31))
        return fail(NERVE_ERR_INVALID_ARGUMENT, "row strides too large");
    const uint32_t ntiles = (vocab_size + nerve::tile_columns() - 1u) / nerve::tile_columns();
    if (tile_records && tile_stride < ntiles) return fail(NERVE_ERR_INVALID_ARGUMENT, "tile_stride < ceil(vocab/64)");
    if (tile_records && (uintptr_t)tile_records % 8u) return fail(NERVE_ERR_INVALID_ARGUMENT, "tile_records must be 8-byte aligned");
    if (!(output_scale - output_scale == 0.0f)) return fail(NERVE_ERR_INVALID_ARGUMENT, "output_scale must be finite");
    const hipError_t e = nerve::launch_lm_head((const uint16_t *)frames, frames_row_stride, (const uint16_t *)weight,
                                               weight_row_stride, batch, input_size, vocab_size, output_scale, logits,
                                               logits_row_stride, (uint2 *)tile_records, tile_stride, (hipStream_t)stream);
    return e == hipSuccess ? NERVE_OK : hip_fail(e, "lm_head launch");
}

int nerve_sampler_record_tokens(nerve_sampler *s, uint32_t *seen, uint32_t seen_stride, uint32_t rows,
                                const uint32_t *ids, uint32_t ids_stride, const uint32_t *counts, uint32_t max_count,
                                void *stream) {
    if (!s || !seen || !ids || !counts) return fail(NERVE_ERR_INVALID_ARGUMENT, "null argument");
    if (max_count == 0u || max_count > NERVE_TOKEN_BATCH_CAPACITY) {
        char buf[128];
        std::snprintf(buf, sizeof(buf), "sampler repetition-state batch requests %u tokens, capacity is %u", max_count,
                      NERVE_TOKEN_BATCH_CAPACITY);
        return fail(NERVE_ERR_TOKEN_BATCH_CAPACITY_EXCEEDED, buf);
    }
    if (rows == 0u) return NERVE_OK;
    if (seen_stride < (s->desc.vocab_size + 31u) / 32u) return fail(NERVE_ERR_INVALID_ARGUMENT, "seen_stride < ceil(vocab/32)");
    int prev = 0;
    (void)hipGetDevice(&prev);
    if (prev != s->device) (void)hipSetDevice(s->device);
    hipError_t e = nerve::launch_record_tokens(seen, seen_stride, rows, ids, ids_stride, counts, max_count,
                                               s->desc.vocab_size, (hipStream_t)stream);
    if (prev != s->device) (void)hipSetDevice(prev);
    if (e != hipSuccess) return hip_fail(e, "record_tokens launch");
    return NERVE_OK;
}

int nerve_sampler_copy_token_state(nerve_sampler *s, uint32_t *dst, const uint32_t *src, uint32_t rows,
                                   uint32_t seen_stride, void *stream) {
    if (!s || !dst || !src) return fail(NERVE_ERR_INVALID_ARGUMENT, "null argument");
    if (rows == 0u) return NERVE_OK;
    int prev = 0;
    (void)hipGetDevice(&prev);
    if (prev != s->device) (void)hipSetDevice(s->device);
    hipError_t e = hipMemcpyAsync(dst, src, (size_t)rows * seen_stride * sizeof(uint32_t), hipMemcpyDeviceToDevice,
                                  (hipStream_t)stream);
    if (prev != s->device) (void)hipSetDevice(prev);
    if (e != hipSuccess) return hip_fail(e, "copy_token_state");
    return NERVE_OK;
}

}  // extern "C"
