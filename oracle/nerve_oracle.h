/*
 * nerve_oracle.h -- CPU restatement of NERVE's token-sampling semantics.
 *
 * TEST INFRASTRUCTURE ONLY. This library is the parity checker for the HIP
 * sampler in llmoop_amd/csrc and the CPU baseline timed by bench.py. Only
 * tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg may load it.
 * The product path never calls into it.
 *
 * Reference files restated (paths relative to the reference root):
 *   runtime-rs/shaders/greedy_sampler_f32.comp.template:52-108          (greedy)
 *   runtime-rs/shaders/greedy_sampler_repetition_f32.comp.template:42-50 (penalty)
 *   runtime-rs/shaders/temperature_top_k_candidates_repetition_f32.comp.template:63-127
 *   runtime-rs/shaders/temperature_top_k_top_p_sampler_f32.comp.template:56-216
 *   runtime-rs/shaders/record_seen_tokens_batch64.comp.template:19-28
 *   runtime-rs/src/vulkan_stream_circuit/sampler.rs:56-141 (apply_to / validation)
 *   runtime-rs/src/vulkan_stream_circuit/tests/fixture_model_helpers.rs:679-686 (hash)
 *
 * Pinning (what checks each function, see tests/test_oracle_*.py):
 *   nro_hash_u32            reference test vectors (ref tests restated in tests/golden)
 *   nro_philox4x32_10       Random123 known-answer vectors (Salmon et al., SC'11)
 *   nro_expf / nro_logf     libm expf/logf within 2 ulp over dense sweeps, exp(0)==1
 *   nro_sample_batch        brute force on tiny V, the literal partition/merge
 *                           restatement (nro_sample_row_literal), the reference's
 *                           six sampler tests, closed forms (equal-weight nuclei)
 * Parity with the reference GPU's own exp()/division rounding for non-uniform
 * draws is unpinned: no reference test exercises it, and the reference shaders
 * cannot run here (no Vulkan); this library defines that rounding.
 */
#ifndef NERVE_ORACLE_H
#define NERVE_ORACLE_H

#include <stdint.h>
#include <stddef.h>

#ifdef __cplusplus
extern "C" {
#endif

#define NRO_DTYPE_F32 0u
#define NRO_DTYPE_BF16 1u
#define NRO_METHOD_GREEDY 0u
#define NRO_METHOD_TOP_K_TOP_P 1u
#define NRO_RNG_REFERENCE_HASH 0u
#define NRO_RNG_PHILOX 1u
#define NRO_FLAG_SAMPLED 1u
#define NRO_FLAG_EOS_FALLBACK 2u
#define NRO_PAD_ID 0xffffffffu

typedef struct {
    uint32_t method;
    float temperature;
    uint32_t top_k;
    float top_p;
    float min_p;
    float repetition_penalty;
    float frequency_penalty;
    float presence_penalty;
} nro_row_params;

typedef struct {
    uint32_t token_id;
    uint32_t selected_logit_bits;
    uint32_t flags;
    uint32_t reserved;
} nro_output;

typedef struct {
    uint32_t batch;
    uint32_t vocab_size;
    uint32_t dtype;
    uint32_t top_k_capacity;
    const void *logits;
    uint64_t logits_row_stride;          /* elements */
    const nro_row_params *params;        /* [batch] */
    const uint32_t *history;             /* [batch][history_stride] or NULL */
    const uint32_t *history_len;         /* [batch] */
    uint32_t history_stride;
    const uint32_t *seen;                /* [batch][seen_stride] words or NULL */
    uint32_t seen_stride;
    const uint32_t *allowed;             /* [batch][allowed_stride] words or NULL */
    uint32_t allowed_stride;
    const uint32_t *seeds;               /* [batch] */
    const uint64_t *steps;               /* [batch] */
    uint32_t rng;
    uint32_t eos_token_id;
    nro_output *out;                     /* [batch] */
    uint32_t *topk_ids;                  /* [batch][top_k_capacity] or NULL */
    float *topk_logits;                  /* same shape or NULL */
    float *topk_probs;                   /* same shape or NULL */
} nro_batch;

uint32_t nro_hash_u32(uint32_t value);
void nro_philox4x32_10(const uint32_t ctr[4], const uint32_t key[2], uint32_t out[4]);
float nro_expf(float x);
float nro_logf(float x);
float nro_bf16_to_f32(uint16_t raw);
uint32_t nro_order_key(float value);

/* Random unit float in [0,1) with 24 bits, as the reference draw. */
float nro_random_unit(uint32_t rng, uint32_t seed, uint64_t step, uint32_t row);

/* Configured (masked + penalised) logit for one token, given its count. */
float nro_configured_logit(float x, uint32_t allowed, uint32_t count, const nro_row_params *p);

/* Fast exact restatement; rows in parallel over `threads` OpenMP threads. */
int nro_sample_batch(const nro_batch *b, int threads);

/* Literal restatement of the reference kernel structure for one row:
 * `partitions` partition top-k lists built by k strict-worse passes, then the
 * k-round G-way cursor merge; greedy rows run the 1024-lane strided argmax and
 * LDS tree. Used only to pin nro_sample_batch. */
int nro_sample_row_literal(const nro_batch *b, uint32_t row, uint32_t partitions);

/* Seen-bitmap recording: record_seen_tokens_batch64.comp.template:19-28. */
void nro_record_tokens(uint32_t *seen, uint32_t vocab_size, const uint32_t *ids, uint32_t n);

#ifdef __cplusplus
}
#endif
#endif
