/*
 * nerve_oracle.c -- CPU restatement of NERVE's token-sampling semantics.
 *
 * TEST INFRASTRUCTURE ONLY: the parity checker and the reported CPU baseline.
 * It is never linked into or called by the product library. Citations point
 * into the reference tree; the header lists which check pins each function.
 *
 * Build: see oracle/Makefile (-O3 -ffp-contract=off: the arithmetic below is
 * plain IEEE-754 binary32 with one rounding per operation, the same sequence
 * the HIP kernels execute).
 */
#include "nerve_oracle.h"

#include <math.h>
#include <stdlib.h>
#include <string.h>

#ifdef _OPENMP
#include <omp.h>
#endif

#define LOWEST_FLOAT (-3.4028234663852886e38f)

static inline uint32_t f2u(float f) { uint32_t u; memcpy(&u, &f, 4); return u; }
static inline float u2f(uint32_t u) { float f; memcpy(&f, &u, 4); return f; }

/* fixture_model_helpers.rs:679-686 and temperature_top_k_top_p_sampler_f32:56-63 */
uint32_t nro_hash_u32(uint32_t value) {
    value ^= value >> 16;
    value *= 0x7feb352du;
    value ^= value >> 15;
    value *= 0x846ca68bu;
    value ^= value >> 16;
    return value;
}

/* Philox4x32-10 (Salmon, Moraes, Dror, Shaw; SC'11 "Parallel Random Numbers:
 * As Easy as 1, 2, 3"): ten rounds of two 32x32->64 multiplies with the
 * published multipliers, key bumped by the published Weyl constants. */
void nro_philox4x32_10(const uint32_t ctr[4], const uint32_t key[2], uint32_t out[4]) {
    uint32_t c0 = ctr[0], c1 = ctr[1], c2 = ctr[2], c3 = ctr[3];
    uint32_t k0 = key[0], k1 = key[1];
    for (int round = 0; round < 10; ++round) {
        uint64_t p0 = (uint64_t)0xD2511F53u * c0;
        uint64_t p1 = (uint64_t)0xCD9E8D57u * c2;
        uint32_t n0 = (uint32_t)(p1 >> 32) ^ c1 ^ k0;
        uint32_t n1 = (uint32_t)p1;
        uint32_t n2 = (uint32_t)(p0 >> 32) ^ c3 ^ k1;
        uint32_t n3 = (uint32_t)p0;
        c0 = n0; c1 = n1; c2 = n2; c3 = n3;
        k0 += 0x9E3779B9u;
        k1 += 0xBB67AE85u;
    }
    out[0] = c0; out[1] = c1; out[2] = c2; out[3] = c3;
}

/* exp(x) in binary32, the sampler's one definition of exp:
 *   k  = rint(x * log2(e))
 *   r  = (x - k*LN2_HI) - k*LN2_LO       (Cody-Waite; LN2_HI has 16 significant
 *                                        bits so k*LN2_HI is exact for |k|<256)
 *   p  = Horner form of the degree-7 Taylor polynomial of e^r (|r| <= 0.35,
 *        truncation error < 6e-9 relative)
 *   result = p * 2^k, built from exponent bits; results below 2^-126 are
 *            scaled in two steps so the only rounding is the final one.
 * No fused multiply-add anywhere: each operation rounds once. */
float nro_expf(float x) {
    if (x != x) return x;
    if (x > 88.72283935546875f) return INFINITY;
    if (x < -103.972084045410156f) return 0.0f;
    const float log2e = 1.44269502162933349609375f;       /* binary32 nearest log2(e) */
    const float ln2_hi = 0.693145751953125f;               /* 0x3f317200 */
    const float ln2_lo = 1.428606765330187045e-06f;        /* ln2 - ln2_hi */
    float t = x * log2e;
    float kf = rintf(t);
    int k = (int)kf;
    float hi = kf * ln2_hi;
    float r = x - hi;
    float lo = kf * ln2_lo;
    r = r - lo;
    float p = 1.0f / 5040.0f;
    p = p * r; p = p + (1.0f / 720.0f);
    p = p * r; p = p + (1.0f / 120.0f);
    p = p * r; p = p + (1.0f / 24.0f);
    p = p * r; p = p + (1.0f / 6.0f);
    p = p * r; p = p + 0.5f;
    p = p * r; p = p + 1.0f;
    p = p * r; p = p + 1.0f;
    if (k > 127) {
        p = p * 2.0f;
        k -= 1;
    }
    if (k >= -126) {
        return p * u2f((uint32_t)(k + 127) << 23);
    }
    p = p * u2f((uint32_t)(k + 64 + 127) << 23);
    return p * u2f((uint32_t)(-64 + 127) << 23);
}

/* ln(x) in binary32 for x > 0 (min_p arguments):
 *   x = m * 2^e with m in [sqrt(1/2), sqrt(2)), s = (m-1)/(m+1),
 *   ln(m) = 2*atanh(s) = 2s(1 + s^2/3 + s^4/5 + ... + s^14/15) (|s| <= 0.1716,
 *   truncation error < 1e-13), ln(x) = e*LN2_HI + (e*LN2_LO + ln(m)). */
float nro_logf(float x) {
    if (x != x || x < 0.0f) return NAN;
    if (x == 0.0f) return -INFINITY;
    if (x == INFINITY) return INFINITY;
    uint32_t bits = f2u(x);
    int e = 0;
    if ((bits >> 23) == 0) {                 /* subnormal: scale by 2^32 */
        x = x * 4294967296.0f;
        bits = f2u(x);
        e = -32;
    }
    e += (int)(bits >> 23) - 127;
    float m = u2f((bits & 0x007fffffu) | 0x3f800000u);
    if (m > 1.41421353816986083984375f) {
        m = m * 0.5f;
        e += 1;
    }
    float num = m - 1.0f;
    float den = m + 1.0f;
    float s = num / den;
    float s2 = s * s;
    float q = 1.0f / 15.0f;
    q = q * s2; q = q + (1.0f / 13.0f);
    q = q * s2; q = q + (1.0f / 11.0f);
    q = q * s2; q = q + (1.0f / 9.0f);
    q = q * s2; q = q + (1.0f / 7.0f);
    q = q * s2; q = q + (1.0f / 5.0f);
    q = q * s2; q = q + (1.0f / 3.0f);
    q = q * s2; q = q + 1.0f;
    float two_s = s + s;
    float lnm = two_s * q;
    float ef = (float)e;
    float lo = ef * 1.428606765330187045e-06f;
    lo = lo + lnm;
    float hi = ef * 0.693145751953125f;
    return hi + lo;
}

float nro_bf16_to_f32(uint16_t raw) { return u2f((uint32_t)raw << 16); }

/* Ordered key: larger float -> larger key, -0.0 and +0.0 share one key (the
 * reference compares with ==, so they tie and the smaller id wins). NaN maps to
 * 0 and is never selected by the top-k path (candidates_f32:68-70). */
uint32_t nro_order_key(float value) {
    if (value != value) return 0u;
    uint32_t bits = value == 0.0f ? 0u : f2u(value);
    return (bits & 0x80000000u) ? ~bits : (bits | 0x80000000u);
}

float nro_random_unit(uint32_t rng, uint32_t seed, uint64_t step, uint32_t row) {
    uint32_t bits;
    if (rng == NRO_RNG_PHILOX) {
        uint32_t ctr[4] = {(uint32_t)step, (uint32_t)(step >> 32), 0u, 0u};
        uint32_t key[2] = {seed, row};
        uint32_t out[4];
        nro_philox4x32_10(ctr, key, out);
        bits = out[0];
    } else {
        /* temperature_top_k_top_p_sampler_f32:65-72 */
        bits = nro_hash_u32(seed ^ (uint32_t)step ^ ((uint32_t)(step >> 32) * 0x9e3779b9u));
    }
    return (float)(bits >> 8) * (1.0f / 16777216.0f);
}

/* greedy_sampler_repetition_f32:42-50 (repetition then presence), with the
 * frequency term between them and the allowed-token mask applied first. */
float nro_configured_logit(float x, uint32_t allowed, uint32_t count, const nro_row_params *p) {
    if (!allowed) return -INFINITY;
    if (count == 0u) return x;
    float v = x < 0.0f ? x * p->repetition_penalty : x / p->repetition_penalty;
    float f = p->frequency_penalty * (float)count;
    v = v - f;
    return v - p->presence_penalty;
}

static inline float load_logit(const nro_batch *b, uint32_t row, uint32_t t) {
    const uint64_t off = (uint64_t)row * b->logits_row_stride + t;
    if (b->dtype == NRO_DTYPE_BF16) return nro_bf16_to_f32(((const uint16_t *)b->logits)[off]);
    return ((const float *)b->logits)[off];
}

static inline int candidate_is_better(float cl, uint32_t cid, float bl, uint32_t bid) {
    return cl > bl || (cl == bl && cid < bid);
}

static inline int candidate_is_worse(float cl, uint32_t cid, float bl, uint32_t bid) {
    return cl < bl || (cl == bl && cid > bid);
}

typedef struct {
    float value;
    uint32_t id;
} entry;

/* Per-row penalty counts. Histories are short (<= a few thousand ids), so a
 * sorted copy plus binary search keeps the per-thread state O(H). */
typedef struct {
    uint32_t *ids;
    uint32_t *counts;
    uint32_t n;
} count_table;

static int cmp_u32(const void *a, const void *b) {
    uint32_t x = *(const uint32_t *)a, y = *(const uint32_t *)b;
    return x < y ? -1 : x > y;
}

static void build_counts(const nro_batch *b, uint32_t row, count_table *ct) {
    ct->n = 0;
    if (!b->history) return;
    uint32_t len = b->history_len[row];
    if (len > b->history_stride) len = b->history_stride;
    const uint32_t *h = b->history + (uint64_t)row * b->history_stride;
    uint32_t *tmp = (uint32_t *)malloc(sizeof(uint32_t) * (len ? len : 1));
    uint32_t m = 0;
    for (uint32_t i = 0; i < len; ++i)
        if (h[i] < b->vocab_size) tmp[m++] = h[i];
    qsort(tmp, m, sizeof(uint32_t), cmp_u32);
    ct->ids = (uint32_t *)malloc(sizeof(uint32_t) * (m ? m : 1));
    ct->counts = (uint32_t *)malloc(sizeof(uint32_t) * (m ? m : 1));
    for (uint32_t i = 0; i < m; ++i) {
        if (ct->n && ct->ids[ct->n - 1] == tmp[i]) {
            ct->counts[ct->n - 1]++;
        } else {
            ct->ids[ct->n] = tmp[i];
            ct->counts[ct->n] = 1;
            ct->n++;
        }
    }
    free(tmp);
}

static void free_counts(count_table *ct) {
    if (ct->n || ct->ids) {
        free(ct->ids);
        free(ct->counts);
    }
    ct->ids = ct->counts = NULL;
    ct->n = 0;
}

static inline uint32_t token_count(const nro_batch *b, uint32_t row, const count_table *ct, uint32_t t) {
    if (b->history) {
        uint32_t lo = 0, hi = ct->n;
        while (lo < hi) {
            uint32_t mid = (lo + hi) >> 1;
            if (ct->ids[mid] < t) lo = mid + 1; else hi = mid;
        }
        return (lo < ct->n && ct->ids[lo] == t) ? ct->counts[lo] : 0u;
    }
    if (b->seen) {
        const uint32_t *w = b->seen + (uint64_t)row * b->seen_stride;
        return (w[t >> 5] >> (t & 31u)) & 1u;
    }
    return 0u;
}

static inline uint32_t token_allowed(const nro_batch *b, uint32_t row, uint32_t t) {
    if (!b->allowed) return 1u;
    const uint32_t *w = b->allowed + (uint64_t)row * b->allowed_stride;
    return (w[t >> 5] >> (t & 31u)) & 1u;
}

static int row_mask_empty(const nro_batch *b, uint32_t row) {
    if (!b->allowed) return 0;
    const uint32_t *w = b->allowed + (uint64_t)row * b->allowed_stride;
    uint32_t words = (b->vocab_size + 31u) / 32u;
    for (uint32_t i = 0; i < words; ++i) {
        uint32_t bits = w[i];
        if (i == words - 1 && (b->vocab_size & 31u)) bits &= (1u << (b->vocab_size & 31u)) - 1u;
        if (bits) return 0;
    }
    return 1;
}

static inline float configured(const nro_batch *b, uint32_t row, const count_table *ct, uint32_t t) {
    return nro_configured_logit(load_logit(b, row, t), token_allowed(b, row, t),
                                token_count(b, row, ct, t), &b->params[row]);
}

/* greedy_sampler_f32:52-83: 1024 lanes stride the vocabulary, then a 1024->1
 * tree with strides 512..1. NaN never wins a comparison but a lane whose first
 * value is NaN keeps it, exactly as the shader does. */
static void greedy_row(const nro_batch *b, uint32_t row, const count_table *ct, entry *result) {
    static const uint32_t lanes = 1024u;
    entry slot[1024];
    const uint32_t V = b->vocab_size;
    for (uint32_t lane = 0; lane < lanes; ++lane) {
        uint32_t best_id = lane;
        float best = lane < V ? configured(b, row, ct, lane) : LOWEST_FLOAT;
        for (uint32_t t = lane + lanes; t < V; t += lanes) {
            float c = configured(b, row, ct, t);
            if (candidate_is_better(c, t, best, best_id)) {
                best = c;
                best_id = t;
            }
        }
        slot[lane].value = best;
        slot[lane].id = best_id;
    }
    for (uint32_t stride = 512u; stride > 0u; stride >>= 1) {
        for (uint32_t lane = 0; lane < stride; ++lane) {
            if (candidate_is_better(slot[lane + stride].value, slot[lane + stride].id,
                                    slot[lane].value, slot[lane].id))
                slot[lane] = slot[lane + stride];
        }
    }
    *result = slot[0];
}

/* temperature_top_k_top_p_sampler_f32:157-194 over the k survivors `top`.
 * The three sequential loops of the shader sum the same weights in the same
 * order, so their running sums are one prefix array. */
static uint32_t top_p_draw(const entry *top, uint32_t k, const nro_row_params *p, float u,
                           float *probs_out) {
    const float T = p->temperature;
    const float m = top[0].value / T;
    float minimum = LOWEST_FLOAT;
    if (p->min_p > 0.0f) {
        float lg = nro_logf(p->min_p);
        float d = T * lg;
        minimum = top[0].value + d;
    }
    float *prefix = (float *)malloc(sizeof(float) * k);
    float *w = (float *)malloc(sizeof(float) * k);
    uint32_t n_valid = 0;
    float total = 0.0f;
    for (uint32_t i = 0; i < k; ++i) {
        if (top[i].value < minimum) break;
        float s = top[i].value / T;
        w[i] = nro_expf(s - m);
        total = total + w[i];
        prefix[i] = total;
        n_valid = i + 1;
    }
    float threshold = p->top_p * total;
    uint32_t nucleus_count = 0;
    for (uint32_t i = 0; i < n_valid; ++i) {
        nucleus_count = i + 1;
        if (prefix[i] >= threshold) break;
    }
    if (nucleus_count == 0) nucleus_count = 1; /* unreachable: top[0] is never below minimum */
    float nucleus_weight = prefix[nucleus_count - 1 < n_valid ? nucleus_count - 1 : 0];
    if (n_valid == 0) nucleus_weight = 0.0f;
    float target = u * nucleus_weight;
    uint32_t selected = nucleus_count - 1;
    for (uint32_t i = 0; i < nucleus_count && i < n_valid; ++i) {
        if (target < prefix[i]) {
            selected = i;
            break;
        }
    }
    if (probs_out) {
        for (uint32_t i = 0; i < k; ++i)
            probs_out[i] = (i < nucleus_count && i < n_valid) ? w[i] / nucleus_weight : 0.0f;
    }
    free(prefix);
    free(w);
    return selected;
}

/* Binary min-heap on "worst first" for the running top-k. */
static inline int heap_worse(const entry *a, const entry *b) {
    return candidate_is_worse(a->value, a->id, b->value, b->id);
}

static void heap_sift_down(entry *h, uint32_t n, uint32_t i) {
    for (;;) {
        uint32_t l = 2 * i + 1, r = l + 1, w = i;
        if (l < n && heap_worse(&h[l], &h[w])) w = l;
        if (r < n && heap_worse(&h[r], &h[w])) w = r;
        if (w == i) return;
        entry t = h[i]; h[i] = h[w]; h[w] = t;
        i = w;
    }
}

static void heap_sift_up(entry *h, uint32_t i) {
    while (i) {
        uint32_t p = (i - 1) / 2;
        if (!heap_worse(&h[i], &h[p])) return;
        entry t = h[i]; h[i] = h[p]; h[p] = t;
        i = p;
    }
}

static int cmp_entry_desc(const void *a, const void *b) {
    const entry *x = (const entry *)a, *y = (const entry *)b;
    if (candidate_is_better(x->value, x->id, y->value, y->id)) return -1;
    if (candidate_is_better(y->value, y->id, x->value, x->id)) return 1;
    return 0;
}

static void write_row(const nro_batch *b, uint32_t row, uint32_t token, float value,
                      uint32_t flags, const entry *top, uint32_t k, const float *probs) {
    b->out[row].token_id = token;
    b->out[row].selected_logit_bits = f2u(value);
    b->out[row].flags = flags;
    b->out[row].reserved = 0u;
    const uint32_t cap = b->top_k_capacity;
    for (uint32_t i = 0; i < cap; ++i) {
        uint64_t o = (uint64_t)row * cap + i;
        if (b->topk_ids) b->topk_ids[o] = i < k ? top[i].id : NRO_PAD_ID;
        if (b->topk_logits) b->topk_logits[o] = i < k ? top[i].value : LOWEST_FLOAT;
        if (b->topk_probs) b->topk_probs[o] = (i < k && probs) ? probs[i] : 0.0f;
    }
}

static uint32_t effective_k(const nro_batch *b, uint32_t row) {
    uint32_t k = b->params[row].top_k;
    if (k > b->top_k_capacity) k = b->top_k_capacity;
    if (k == 0u) k = 1u;
    return k;
}

static int eos_fallback(const nro_batch *b, uint32_t row) {
    if (!row_mask_empty(b, row)) return 0;
    entry e = {LOWEST_FLOAT, b->eos_token_id};
    float one = 1.0f;
    uint32_t flags = NRO_FLAG_EOS_FALLBACK |
                     (b->params[row].method == NRO_METHOD_GREEDY ? 0u : NRO_FLAG_SAMPLED);
    write_row(b, row, b->eos_token_id, -INFINITY, flags, &e, 1, &one);
    return 1;
}

static void sample_row_fast(const nro_batch *b, uint32_t row) {
    if (eos_fallback(b, row)) return;
    count_table ct = {0};
    build_counts(b, row, &ct);
    const nro_row_params *p = &b->params[row];
    if (p->method == NRO_METHOD_GREEDY) {
        entry best;
        greedy_row(b, row, &ct, &best);
        float one = 1.0f;
        write_row(b, row, best.id, best.value, 0u, &best, 1, &one);
        free_counts(&ct);
        return;
    }
    const uint32_t k = effective_k(b, row);
    entry *heap = (entry *)malloc(sizeof(entry) * k);
    uint32_t n = 0;
    for (uint32_t t = 0; t < b->vocab_size; ++t) {
        float v = configured(b, row, &ct, t);
        if (v != v || v == -INFINITY) continue;
        entry e = {v, t};
        if (n < k) {
            heap[n] = e;
            heap_sift_up(heap, n);
            ++n;
        } else if (heap_worse(&heap[0], &e)) {
            heap[0] = e;
            heap_sift_down(heap, n, 0);
        }
    }
    qsort(heap, n, sizeof(entry), cmp_entry_desc);
    entry *top = (entry *)malloc(sizeof(entry) * k);
    for (uint32_t i = 0; i < k; ++i) {
        if (i < n) top[i] = heap[i];
        else { top[i].value = LOWEST_FLOAT; top[i].id = NRO_PAD_ID; }
    }
    float *probs = (float *)malloc(sizeof(float) * k);
    float u = nro_random_unit(b->rng, b->seeds[row], b->steps[row], row);
    uint32_t sel = top_p_draw(top, k, p, u, probs);
    write_row(b, row, top[sel].id, top[sel].value, NRO_FLAG_SAMPLED, top, k, probs);
    free(probs);
    free(top);
    free(heap);
    free_counts(&ct);
}

int nro_sample_batch(const nro_batch *b, int threads) {
    if (!b || !b->out || !b->params || !b->logits) return 1;
    if (b->top_k_capacity == 0u) return 1;
#ifdef _OPENMP
    if (threads < 1) threads = 1;
#pragma omp parallel for schedule(dynamic, 1) num_threads(threads)
#endif
    for (uint32_t row = 0; row < b->batch; ++row) sample_row_fast(b, row);
    (void)threads;
    return 0;
}

/* Literal restatement for one row: candidates_repetition_f32:63-127 then
 * temperature_top_k_top_p_sampler_f32:90-194, serialised lane by lane. */
int nro_sample_row_literal(const nro_batch *b, uint32_t row, uint32_t partitions) {
    if (row >= b->batch || partitions == 0u) return 1;
    if (eos_fallback(b, row)) return 0;
    count_table ct = {0};
    build_counts(b, row, &ct);
    const nro_row_params *p = &b->params[row];
    if (p->method == NRO_METHOD_GREEDY) {
        entry best;
        greedy_row(b, row, &ct, &best);
        float one = 1.0f;
        write_row(b, row, best.id, best.value, 0u, &best, 1, &one);
        free_counts(&ct);
        return 0;
    }
    const uint32_t V = b->vocab_size;
    const uint32_t K = effective_k(b, row);
    const uint32_t part_size = (V + partitions - 1u) / partitions;
    entry *cand = (entry *)malloc(sizeof(entry) * (size_t)partitions * K);
    for (uint32_t g = 0; g < partitions; ++g) {
        uint32_t start = g * part_size;
        uint32_t end = start + part_size < V ? start + part_size : V;
        float prev = 0.0f;
        uint32_t prev_id = 0u;
        for (uint32_t rank = 0; rank < K; ++rank) {
            float best = LOWEST_FLOAT;
            uint32_t best_id = 0xffffffffu;
            for (uint32_t t = start; t < end; ++t) {
                float c = configured(b, row, &ct, t);
                if (c != c) continue;
                if (rank != 0u && !candidate_is_worse(c, t, prev, prev_id)) continue;
                if (candidate_is_better(c, t, best, best_id)) {
                    best = c;
                    best_id = t;
                }
            }
            cand[(size_t)g * K + rank].value = best;
            cand[(size_t)g * K + rank].id = best_id;
            prev = best;
            prev_id = best_id;
        }
    }
    uint32_t *cursor = (uint32_t *)calloc(partitions, sizeof(uint32_t));
    entry *top = (entry *)malloc(sizeof(entry) * K);
    for (uint32_t rank = 0; rank < K; ++rank) {
        float best = LOWEST_FLOAT;
        uint32_t best_id = 0xffffffffu, best_g = 0xffffffffu;
        for (uint32_t g = 0; g < partitions; ++g) {
            entry e = cand[(size_t)g * K + cursor[g]];
            if (best_g == 0xffffffffu || candidate_is_better(e.value, e.id, best, best_id)) {
                best = e.value;
                best_id = e.id;
                best_g = g;
            }
        }
        top[rank].value = best;
        top[rank].id = best_id;
        cursor[best_g] += 1u;
        if (cursor[best_g] >= K) cursor[best_g] = K - 1u; /* list exhausted; never read again */
    }
    /* The shader's three loops, literally, with exp recomputed each time. */
    const float T = p->temperature;
    const float m = top[0].value / T;
    float minimum = LOWEST_FLOAT;
    if (p->min_p > 0.0f) {
        float lg = nro_logf(p->min_p);
        float d = T * lg;
        minimum = top[0].value + d;
    }
    float total = 0.0f;
    for (uint32_t i = 0; i < K; ++i) {
        if (top[i].value < minimum) break;
        float s = top[i].value / T;
        total = total + nro_expf(s - m);
    }
    float threshold = p->top_p * total;
    float nucleus_weight = 0.0f;
    uint32_t nucleus_count = 0;
    for (uint32_t i = 0; i < K; ++i) {
        if (top[i].value < minimum) break;
        float s = top[i].value / T;
        nucleus_weight = nucleus_weight + nro_expf(s - m);
        nucleus_count = i + 1;
        if (nucleus_weight >= threshold) break;
    }
    float u = nro_random_unit(b->rng, b->seeds[row], b->steps[row], row);
    float target = u * nucleus_weight;
    float cumulative = 0.0f;
    uint32_t sel = nucleus_count - 1u;
    for (uint32_t i = 0; i < nucleus_count; ++i) {
        float s = top[i].value / T;
        cumulative = cumulative + nro_expf(s - m);
        if (target < cumulative) {
            sel = i;
            break;
        }
    }
    float *probs = (float *)malloc(sizeof(float) * K);
    for (uint32_t i = 0; i < K; ++i) {
        float s = top[i].value / T;
        probs[i] = i < nucleus_count ? nro_expf(s - m) / nucleus_weight : 0.0f;
    }
    write_row(b, row, top[sel].id, top[sel].value, NRO_FLAG_SAMPLED, top, K, probs);
    free(probs);
    free(top);
    free(cursor);
    free(cand);
    free_counts(&ct);
    return 0;
}

void nro_record_tokens(uint32_t *seen, uint32_t vocab_size, const uint32_t *ids, uint32_t n) {
    for (uint32_t i = 0; i < n; ++i)
        if (ids[i] < vocab_size) seen[ids[i] >> 5] |= 1u << (ids[i] & 31u);
}
