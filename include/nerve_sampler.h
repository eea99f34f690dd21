/*
 * nerve_sampler.h -- C ABI of the MI355X (gfx950) token-sampling stage.
 *
 * One fused HIP launch samples every row of a decode batch: allowed-token
 * mask, repetition / frequency / presence penalties, temperature, top-k,
 * min-p, top-p and an argmax or seeded multinomial draw. Plain C types only;
 * device pointers are HIP device addresses owned by the caller, the library
 * owns only its scratch. Everything is asynchronous on the stream passed in.
 * Calls on one handle are not thread-safe; distinct handles may be used
 * concurrently (each owns its scratch).
 *
 * Reference surface each entry point replaces (paths under the reference root,
 * runtime-rs/src/vulkan_stream_circuit/):
 *   nerve_sampler_spec / nerve_sampler_runtime_config  <- VulkanResidentSamplerSpec
 *        and VulkanResidentSamplerRuntimeConfig (sampler.rs:29-54)
 *   nerve_sampler_apply_runtime_config                 <- RuntimeConfig::apply_to (sampler.rs:66-141)
 *   nerve_sampler_validate_spec                        <- spec checks in
 *        from_logits_buffer_with_feedback_control (sampler.rs:259-382)
 *   nerve_sampler_kernel_role_matches                  <- sampler_kernel_role_matches (sampler.rs:144-160)
 *   nerve_sampler_create / nerve_sampler_destroy       <- VulkanResidentSamplerRunner construction / Drop
 *        (sampler.rs:245-727), batched over B lanes
 *   nerve_sampler_step                                 <- VulkanResidentBatchedOutputProjectionRunner::sample_lanes
 *        (batched_output_projection.rs:316-371) and VulkanResidentSamplerRunner::run (sampler.rs:748-759):
 *        one launch for all rows instead of B two-dispatch sequences
 *   nerve_sampler_record_tokens                        <- record_input_tokens (sampler.rs:773-814) and
 *        VulkanResidentSamplerLogitsView::prepare_token_state (sampler.rs:1146-1193)
 *   nerve_sampler_copy_token_state                     <- capture_token_state / restore_token_state
 *        (sampler.rs:816-828)
 *   nerve_sampler_output / stream-control ring         <- VulkanResidentSamplerRun (sampler.rs:1221-1230),
 *        completed_run_at (sampler.rs:852-873), output record of greedy_sampler_f32.comp.template:85-107
 *   nerve_status codes                                 <- VulkanResidentSamplerRunnerError (sampler.rs:1232-1258)
 */
#ifndef NERVE_SAMPLER_H
#define NERVE_SAMPLER_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define NERVE_SAMPLER_ABI_VERSION 2u

typedef enum {
    NERVE_OK = 0,
    NERVE_ERR_INVALID_LOGITS_BYTE_CAPACITY = 1,
    NERVE_ERR_ZERO_HISTORY_CAPACITY = 2,
    NERVE_ERR_HISTORY_CAPACITY_OVERFLOW = 3,
    NERVE_ERR_TOKEN_BATCH_CAPACITY_EXCEEDED = 4,
    NERVE_ERR_INVALID_KERNEL_ROLE = 5,
    NERVE_ERR_UNSUPPORTED_RUNTIME_SAMPLING_OVERRIDE = 6,
    NERVE_ERR_INVALID_SAMPLING_SPEC = 7,
    NERVE_ERR_HIP = 8,
    NERVE_ERR_INVALID_ARGUMENT = 9,
    NERVE_ERR_BATCH_CAPACITY_EXCEEDED = 10
} nerve_status;

enum { NERVE_DTYPE_F32 = 0, NERVE_DTYPE_BF16 = 1 };
enum { NERVE_METHOD_GREEDY = 0, NERVE_METHOD_TEMPERATURE_TOP_K_TOP_P = 1 };
enum { NERVE_RNG_REFERENCE_HASH = 0, NERVE_RNG_PHILOX = 1 };
enum { NERVE_FLAG_SAMPLED = 1u, NERVE_FLAG_EOS_FALLBACK = 2u };

/* nerve_sampler_batch.flags */
enum {
    /* Append each row's sampled token to its penalty state after the step:
     * history ids (count semantics): history[row][history_len[row] % history_stride] = token,
     * history_len[row] += 1 (the rows then read the last history_stride ids);
     * seen bitmap (set semantics): seen bit of the token set.
     * Replaces the per-lane record_token_batch dispatch of the decode loop
     * (multi_stream_batch_runner.rs:235-240; record_input_tokens, sampler.rs:773-814). */
    NERVE_BATCH_APPEND_HISTORY = 1u,
    /* The tick of row r is tick_base + r (steps and stream_control ignored for the tick):
     * consecutive_component_batch_stream_ticks (stream_control_bytes.rs:54-67). */
    NERVE_BATCH_CONSECUTIVE_TICKS = 2u
};

/* Feedback-control block (resident_feedback_control.rs:1-6, 397-424): words[0] flags
 * (bit 0 enabled, bit 1 cancel requested), words[2] stop reason (0 none, 1 EOS,
 * 2 cancelled), words[8] drain state, words[9] sampled ticks; the stop-token mask is
 * its own array (the reference keeps it at word 12 of the same buffer). */
enum { NERVE_FEEDBACK_ENABLED = 1u, NERVE_FEEDBACK_CANCEL_REQUESTED = 2u };
enum { NERVE_STOP_REASON_NONE = 0u, NERVE_STOP_REASON_EOS = 1u, NERVE_STOP_REASON_CANCELLED = 2u };

/* nerve_sampler_desc.flags */
enum {
    /* The handle allocates no device memory; steps whose rows need more than one
     * slice (the only ones that use cross-workgroup scratch) must then go through
     * nerve_sampler_step_static_scratch. */
    NERVE_DESC_NO_SCRATCH = 1u
};

/* Up to this many token ids per row per record call
 * (VULKAN_BACKEND_LOOP_MAX_WINDOW, vulkan_stream_circuit.rs:82). */
#define NERVE_TOKEN_BATCH_CAPACITY 64u
#define NERVE_MAX_TOP_K_CAPACITY 1024u
#define NERVE_MAX_HISTORY_CAPACITY 4095u
#define NERVE_MAX_VOCAB 1048575u

/* ---- Host-side spec surface (no device work) ---------------------------- */

#define NERVE_SAMPLER_ID_CAPACITY 64

typedef struct {
    char sampler_id[NERVE_SAMPLER_ID_CAPACITY];
    uint32_t method; /* NERVE_METHOD_* */
    float temperature;
    uint32_t top_k;
    float top_p;
    float min_p;
    float presence_penalty;
    float repetition_penalty;
    uint32_t top_k_capacity;
    uint32_t runtime_parameterized;
    uint64_t logits_byte_capacity;
    uint64_t output_byte_capacity;
    uint64_t scratch_byte_capacity;
} nerve_sampler_spec;

/* Each field applies only when its has_* flag is nonzero (Rust Option<_>). */
typedef struct {
    uint32_t has_temperature, has_top_k, has_top_p, has_min_p, has_presence_penalty, has_repetition_penalty;
    float temperature;
    uint32_t top_k;
    float top_p;
    float min_p;
    float presence_penalty;
    float repetition_penalty;
} nerve_sampler_runtime_config;

/* Greedy -> sampled promotion and validation; writes `out` on success.
 * On failure returns NERVE_ERR_UNSUPPORTED_RUNTIME_SAMPLING_OVERRIDE and, if
 * `message` is non-null, the reason (contains "capacity <n>"). */
int nerve_sampler_apply_runtime_config(const nerve_sampler_spec *compiled,
                                       const nerve_sampler_runtime_config *config,
                                       nerve_sampler_spec *out, char *message, size_t message_capacity);

/* Spec checks at runner construction; vocab_size = logits_byte_capacity / 4. */
int nerve_sampler_validate_spec(const nerve_sampler_spec *spec, uint64_t logits_byte_capacity,
                                uint32_t history_capacity_activations, uint32_t partition_count);

/* Kernel-role table of the reference; kept for callers that select roles. */
int nerve_sampler_kernel_role_matches(const char *role, uint32_t runtime_parameterized, uint32_t method);

/* ---- Device sampler ----------------------------------------------------- */

typedef struct nerve_sampler nerve_sampler;

typedef struct {
    uint32_t vocab_size;        /* V, 1..NERVE_MAX_VOCAB */
    uint32_t max_batch;         /* rows per step */
    uint32_t dtype;             /* NERVE_DTYPE_* of the logits */
    uint32_t top_k_capacity;    /* 1..NERVE_MAX_TOP_K_CAPACITY */
    uint32_t history_capacity;  /* max history ids per row, 0..NERVE_MAX_HISTORY_CAPACITY */
    uint32_t slices_per_row;    /* workgroups cooperating on one row; 0 = automatic: one, or the
                                   fewest whose registers hold the row (raised per step as needed) */
    uint32_t device;            /* HIP device ordinal */
    uint32_t flags;             /* NERVE_DESC_* */
} nerve_sampler_desc;

/* Per-row sampling parameters (device array [batch], 32 bytes each). */
typedef struct {
    uint32_t method;            /* NERVE_METHOD_* */
    float temperature;          /* > 0 */
    uint32_t top_k;             /* 1..top_k_capacity (clamped on device) */
    float top_p;                /* (0, 1] */
    float min_p;                /* [0, 1] */
    float repetition_penalty;   /* > 0 */
    float frequency_penalty;    /* finite; subtracts penalty * count */
    float presence_penalty;     /* finite */
} nerve_sampler_row_params;

/* Output record: words 0-3 of the reference sampler output buffer. */
typedef struct {
    uint32_t token_id;
    uint32_t selected_logit_bits; /* penalised, pre-temperature logit */
    uint32_t flags;               /* NERVE_FLAG_* */
    uint32_t reserved;
} nerve_sampler_output;

typedef struct {
    uint32_t batch;                        /* rows this step, <= max_batch */
    uint32_t rng;                          /* NERVE_RNG_* */
    const void *logits;                    /* [batch][logits_row_stride] of dtype */
    uint64_t logits_row_stride;            /* elements, >= vocab_size */
    const nerve_sampler_row_params *params;/* [batch] */
    /* Penalty state, at most one of: */
    uint32_t *history;                     /* [batch][history_stride] token ids (count semantics) */
    uint32_t *history_len;                 /* [batch] ids per row; the last min(len, history_stride) count */
    uint32_t history_stride;               /* <= history_capacity */
    uint32_t *seen;                        /* [batch][seen_stride] packed bitmap (set semantics) */
    uint32_t seen_stride;                  /* words, >= ceil(V/32), or 0: one bitmap for all rows */
    /* Allowed-token bitmask (optional); an all-zero row samples eos_token_id. */
    const uint32_t *allowed;               /* [batch][allowed_stride] */
    uint32_t allowed_stride;
    uint32_t eos_token_id;
    /* Draw key: seeds[row] and the stream tick (from stream_control when set, else steps[row]). */
    const uint32_t *seeds;                 /* [batch] */
    const uint64_t *steps;                 /* [batch] */
    /* Optional reference stream control: [batch][5] words {token, tick_lo, tick_hi, flags,
     * history_capacity}; the step writes the token and advances the 64-bit tick. */
    uint32_t *stream_control;
    /* Optional reference output ring: [batch][ring_stride] words; record at words 0-3 and at
     * 4 + (tick_lo % history_capacity) * 4. Requires stream_control. */
    uint32_t *output_ring;
    uint32_t ring_stride;
    nerve_sampler_output *out;             /* [batch] (required) */
    /* Optional survivors: [batch][top_k_capacity]; padding id 0xffffffff, logit -FLT_MAX, prob 0. */
    uint32_t *topk_ids;
    float *topk_logits;
    float *topk_probs;
    /* ---- ABI 2 ---- */
    uint32_t flags;                        /* NERVE_BATCH_* */
    uint32_t prefix_stride;                /* words between rows of prefix_ids (0: one list for all rows) */
    uint64_t tick_base;                    /* with NERVE_BATCH_CONSECUTIVE_TICKS */
    /* Per-lane token prefix added to the seen state (set semantics; requires seen): row r
     * samples with seen[r] | {prefix_ids[r * prefix_stride + i] : i < count_r}, count_r =
     * prefix_counts[r] (<= NERVE_TOKEN_BATCH_CAPACITY), or r + 1 when prefix_counts is null (the
     * [..=r] prefixes of sample_batch, batched_output_projection.rs:277-298). seen_stride 0
     * shares one base bitmap among all rows, like the lanes' copies of the runner's bitmap
     * (prepare_token_state, sampler.rs:1146-1193); the seen arrays are not modified. */
    const uint32_t *prefix_ids;
    const uint32_t *prefix_counts;
    /* Optional feedback-control commit of each row's token (commit_feedback_control,
     * greedy_sampler_f32.comp.template:35-50): with words[0] bit 0 set, words[9] += 1; on a
     * cancel request or a stop token, words[2] 0 -> 1 (EOS) or 2 (cancelled) by
     * compare-and-swap, and words[8] = 2 by the row that won it. */
    uint32_t *feedback_control;            /* [batch][feedback_stride] words (stride 0: one shared block) */
    const uint32_t *stop_tokens;           /* [batch][stop_stride] packed bitmask (stride 0: one mask) */
    uint32_t feedback_stride;
    uint32_t stop_stride;
} nerve_sampler_batch;

int nerve_sampler_create(const nerve_sampler_desc *desc, nerve_sampler **out);
int nerve_sampler_destroy(nerve_sampler *sampler);

/* One decode step for every row of `batch`, asynchronous on `stream`
 * (a hipStream_t; NULL = the device's null stream). */
int nerve_sampler_step(nerve_sampler *sampler, const nerve_sampler_batch *batch, void *stream);

/* nerve_sampler_step that allocates nothing. No counterpart in the reference: it is
 * for callers that cannot allocate device memory (HIP graph capture, tight serving
 * loops, harnesses that forbid hipMalloc). Steps whose rows need several slices take
 * their cross-workgroup scratch (64 KiB of per-row arrival counts, then batch x slices x
 * top_k_capacity x 8 bytes + 4 bytes per (row, slice)) from one static array of 4 MiB per
 * GPU instead of the handle's; larger needs return NERVE_ERR_INVALID_ARGUMENT. Every call
 * on a GPU shares that array, so calls that overlap on one GPU (other streams, other
 * handles) race. The counts start at zero when the library loads and every step leaves
 * them at zero; nothing else needs clearing between calls. Results equal
 * nerve_sampler_step's. */
int nerve_sampler_step_static_scratch(nerve_sampler *sampler, const nerve_sampler_batch *batch, void *stream);

/* ---- LM head fused with the step (the projection's tile records) ----------------------
 * A tile record is two words per batch row and per 64 vocabulary columns t:
 * records[row*tile_stride + 2*t] = the largest order key of logits [64 t, 64 t + 64) (the
 * float's bits mapped so that larger values give larger unsigned keys: non-negative x ->
 * bits | 0x80000000, negative -> ~bits, +-0 -> 0x80000000, NaN excluded), and word
 * 2*t + 1 = the count of NaNs among them. tile_stride counts records (>= ceil(vocab/64));
 * the array holds batch x tile_stride x 8 bytes, 8-byte aligned. */

/* logits[b*logits_row_stride + v] = output_scale * sum_d frames[b][d] * weight[v][d] for
 * b < batch, v < vocab_size: bf16 frames [batch][frames_row_stride] and weight
 * [vocab][weight_row_stride] (16-byte aligned, strides multiples of 8, input_size a
 * multiple of 64), f32 accumulation and output; with tile_records, also the tile record of
 * every row and 64 columns. Replaces tied_output_projection_batch_bf16.comp.template
 * (dispatched by batched_output_projection.rs:162-206), whose per-lane summation order
 * this does not reproduce (f32 sums of the same products in another order). */
int nerve_lm_head_project(const void *frames, uint32_t frames_row_stride, const void *weight,
                          uint32_t weight_row_stride, uint32_t batch, uint32_t input_size,
                          uint32_t vocab_size, float output_scale, float *logits, uint32_t logits_row_stride,
                          uint32_t *tile_records, uint32_t tile_stride, void *stream);

/* The tile records of existing logits (dtype NERVE_DTYPE_F32 or NERVE_DTYPE_BF16), as the
 * projection's epilogue writes them. No counterpart in the reference: for logits that
 * another producer wrote. */
int nerve_tile_records(const void *logits, uint32_t dtype, uint32_t logits_row_stride, uint32_t batch,
                       uint32_t vocab_size, uint32_t *tile_records, uint32_t tile_stride, void *stream);

/* nerve_sampler_step given the tile records of batch->logits: reads the records and only
 * the tiles that can hold a survivor instead of every logit (sample_lanes,
 * batched_output_projection.rs:316-371, after the projection). Results equal
 * nerve_sampler_step's on the same logits; rows the records cannot narrow (fewer than
 * top_k clean tiles, constant rows) read their whole row. One workgroup per row. */
int nerve_sampler_step_tiles(nerve_sampler *sampler, const nerve_sampler_batch *batch,
                             const uint32_t *tile_records, uint32_t tile_stride, void *stream);

/* Sets bits for token ids < vocab_size into per-row seen bitmaps:
 * seen[row*seen_stride + id/32] |= 1 << (id%32) for ids[row*ids_stride + i], i < min(counts[row], max_count).
 * ids and counts are device arrays; max_count is the host-side bound of the call and must be
 * 1..NERVE_TOKEN_BATCH_CAPACITY (else NERVE_ERR_TOKEN_BATCH_CAPACITY_EXCEEDED), like the reference. */
int nerve_sampler_record_tokens(nerve_sampler *sampler, uint32_t *seen, uint32_t seen_stride, uint32_t rows,
                                const uint32_t *ids, uint32_t ids_stride, const uint32_t *counts,
                                uint32_t max_count, void *stream);

/* Device-to-device copy of `rows` seen bitmaps (capture: live -> snapshot; restore: snapshot -> live). */
int nerve_sampler_copy_token_state(nerve_sampler *sampler, uint32_t *dst, const uint32_t *src, uint32_t rows,
                                   uint32_t seen_stride, void *stream);

/* Last HIP error text for this thread, or "" */
const char *nerve_sampler_last_error(void);
uint32_t nerve_sampler_abi_version(void);
/* Workgroups per row that the next step of this handle will use. */
uint32_t nerve_sampler_slices_per_row(const nerve_sampler *sampler);

#ifdef __cplusplus
}
#endif
#endif
