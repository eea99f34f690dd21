// nerve_sampler_kernels.hip -- the fused gfx950 sampling kernel and its launcher.
//
// One launch samples every row of a decode batch. Each row is split into S
// vocabulary slices, one 512-lane workgroup per slice (S*B workgroups in all,
// mapped so the slices of one row land on one XCD and share its L2):
//
//   1. history ids of the row that fall in the slice go into an LDS bitmap and
//      an LDS id->count hash (penalties are looked up only where a bit is set);
//   2. the slice streams from HBM once with 16-byte loads, all loads of a lane
//      issued before the first is consumed, and stays in VGPRs as order keys
//      (mask, penalties, NaN and -inf exclusion applied on the fly);
//   3. top-k: an 8+8-bit LDS radix select over the 512 per-lane maxima gives a
//      threshold t with at least k keys >= t; for iid logits about k+3 keys
//      pass it. They are compacted to LDS and rank-sorted (value desc, id asc).
//      A skewed slice (more than kCandCap survivors) falls back to an exact
//      4-pass radix select on all keys plus an id-ordered tie cut;
//   4. the sorted slice list goes to scratch; the last workgroup of the row
//      (device-scope counter) merges the S lists by binary-search ranks, then
//      one wave runs min-p / top-p over the k survivors and the draw, and
//      writes the output record (and, if asked, survivors, probabilities,
//      stream control and the output ring).
//
// Semantics follow the reference shaders (paths under runtime-rs/shaders/):
//   greedy_sampler_f32.comp.template:31-34, 52-108       tie-break, argmax, record, tick carry
//   temperature_top_k_candidates_f32.comp.template:59-126 exact top-k, NaN skipped, -inf never enters
//   temperature_top_k_top_p_sampler_f32.comp.template:90-216 merge, min-p, top-p, draw, record
// The greedy path reproduces the reference's NaN behaviour (a lane that starts
// on a NaN keeps it through the 1024-lane tree) by re-running that exact lane
// structure for the rare rows that contain a NaN.
#include <hip/hip_runtime.h>
#include <stdint.h>

#include "nerve_device_math.h"
#include "nerve_sampler_internal.h"

namespace nerve {

constexpr int kBlock = 512;
constexpr int kWaves = kBlock / 64;
constexpr uint32_t kCandCap = 1024;
constexpr uint32_t kHashEmpty = 0xffffffffu;

__device__ __forceinline__ uint32_t lane_id() { return __lane_id(); }

__device__ __forceinline__ uint32_t wave_inclusive_scan(uint32_t v) {
    const uint32_t lane = lane_id();
#pragma unroll
    for (int o = 1; o < 64; o <<= 1) {
        uint32_t t = __shfl_up(v, o, 64);
        if (lane >= (uint32_t)o) v += t;
    }
    return v;
}

__device__ __forceinline__ uint32_t wave_sum(uint32_t v) {
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) v += __shfl_xor(v, o, 64);
    return v;
}

__device__ __forceinline__ uint64_t wave_max_u64(uint64_t v) {
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) {
        uint32_t lo = __shfl_xor((uint32_t)v, o, 64);
        uint32_t hi = __shfl_xor((uint32_t)(v >> 32), o, 64);
        uint64_t t = ((uint64_t)hi << 32) | lo;
        v = t > v ? t : v;
    }
    return v;
}

// Exclusive prefix over the block in thread order; `total` gets the block sum.
__device__ __forceinline__ uint32_t block_exclusive_scan(uint32_t v, uint32_t *s_tmp, uint32_t &total) {
    const uint32_t tid = threadIdx.x, wave = tid >> 6;
    uint32_t inc = wave_inclusive_scan(v);
    if (lane_id() == 63) s_tmp[wave] = inc;
    __syncthreads();
    uint32_t base = 0, tot = 0;
#pragma unroll
    for (int w = 0; w < kWaves; ++w) {
        uint32_t t = s_tmp[w];
        base += (uint32_t)w < wave ? t : 0u;
        tot += t;
    }
    __syncthreads();
    total = tot;
    return base + inc - v;
}

__device__ __forceinline__ uint32_t block_sum(uint32_t v, uint32_t *s_tmp) {
    uint32_t total;
    (void)block_exclusive_scan(v, s_tmp, total);
    return total;
}

__device__ __forceinline__ uint64_t block_max_u64(uint64_t v, uint64_t *s_tmp) {
    v = wave_max_u64(v);
    if (lane_id() == 0) s_tmp[threadIdx.x >> 6] = v;
    __syncthreads();
    uint64_t m = s_tmp[0];
#pragma unroll
    for (int w = 1; w < kWaves; ++w) m = s_tmp[w] > m ? s_tmp[w] : m;
    __syncthreads();
    return m;
}

__device__ __forceinline__ bool entry_better(uint2 a, uint2 b) {
    return a.x > b.x || (a.x == b.x && (a.y & kIdMask) < (b.y & kIdMask));
}

__device__ __forceinline__ float entry_value(uint2 e) {
    return (e.x == kZeroKey && (e.y & kNegZeroFlag)) ? -0.0f : key_to_float(e.x);
}

// ---- LDS id -> count table (linear probing, insert-only) ------------------

__device__ __forceinline__ uint32_t hash_slot(uint32_t id, uint32_t log2_slots) {
    return (id * 0x9E3779B1u) >> (32u - log2_slots);
}

__device__ void hash_insert(uint32_t *h, uint32_t log2_slots, uint32_t id) {
    const uint32_t mask = (1u << log2_slots) - 1u;
    uint32_t slot = hash_slot(id, log2_slots);
    for (uint32_t probe = 0; probe <= mask; ++probe) {
        uint32_t cur = h[slot];
        if (cur == kHashEmpty) {
            uint32_t old = atomicCAS(&h[slot], kHashEmpty, (id << 12) | 1u);
            if (old == kHashEmpty) return;
            cur = old;
        }
        if ((cur >> 12) == id) {
            atomicAdd(&h[slot], 1u);
            return;
        }
        slot = (slot + 1u) & mask;
    }
}

__device__ __forceinline__ uint32_t hash_lookup(const uint32_t *h, uint32_t log2_slots, uint32_t id) {
    const uint32_t mask = (1u << log2_slots) - 1u;
    uint32_t slot = hash_slot(id, log2_slots);
    for (uint32_t probe = 0; probe <= mask; ++probe) {
        uint32_t cur = h[slot];
        if (cur == kHashEmpty) return 0u;
        if ((cur >> 12) == id) return cur & 0xfffu;
        slot = (slot + 1u) & mask;
    }
    return 0u;
}

// ---- element access ---------------------------------------------------------

template <typename Elem>
__device__ __forceinline__ float load_elem(const Elem *row, uint32_t t);

template <>
__device__ __forceinline__ float load_elem<float>(const float *row, uint32_t t) {
    return row[t];
}

template <>
__device__ __forceinline__ float load_elem<uint16_t>(const uint16_t *row, uint32_t t) {
    return u2f((uint32_t)row[t] << 16);
}

// Raw words of one EPV-element vector slot: W = EPV*sizeof(Elem)/4 words (min 1).
template <typename Elem, int EPV>
struct VecTraits {
    static constexpr int W = (EPV * (int)sizeof(Elem) + 3) / 4;
};

template <typename Elem, int EPV>
__device__ __forceinline__ float raw_elem(const uint32_t (&r)[VecTraits<Elem, EPV>::W], int e) {
    if constexpr (sizeof(Elem) == 4) {
        return u2f(r[e]);
    } else {
        if constexpr (EPV == 1) {
            return u2f(r[0] << 16);
        } else {
            uint32_t w = r[e >> 1];
            return u2f((e & 1) ? (w & 0xffff0000u) : (w << 16));
        }
    }
}

// Row state shared by the helpers that recompute a single configured value.
struct RowCtx {
    const void *logits_row;
    const uint32_t *allowed_row;
    const uint32_t *seen_row;
    const uint32_t *hash;      // LDS
    const uint32_t *bitmap;    // LDS (slice-relative) or null: probe the hash directly
    uint32_t log2_slots;
    uint32_t tok0;
    float rep, freq, pres;
    bool history;
};

template <typename Elem>
__device__ float configured_at(const RowCtx &c, uint32_t t) {
    float x = load_elem<Elem>((const Elem *)c.logits_row, t);
    bool allowed = c.allowed_row ? ((c.allowed_row[t >> 5] >> (t & 31u)) & 1u) : true;
    uint32_t count = 0;
    if (c.history) {
        bool bit = true;
        if (c.bitmap) {
            uint32_t o = t - c.tok0;
            bit = (c.bitmap[o >> 5] >> (o & 31u)) & 1u;
        }
        if (bit) count = hash_lookup(c.hash, c.log2_slots, t);
    } else if (c.seen_row) {
        count = (c.seen_row[t >> 5] >> (t & 31u)) & 1u;
    }
    return configured_logit(x, allowed, count, c.rep, c.freq, c.pres);
}

__device__ __forceinline__ bool float_better(float cl, uint32_t cid, float bl, uint32_t bid) {
    return cl > bl || (cl == bl && cid < bid);
}

// ---- radix select over per-lane key arrays --------------------------------
//
// Returns a key threshold t: the first `passes` bytes of the k-th largest
// nonzero key (lower bytes zero), so #{key >= t} >= k. Returns 1 ("every
// nonzero key") when fewer than k keys are nonzero. `count_ge` receives the
// number of keys >= t when passes == 4 or the fewer-than-k case applies.
template <int N>
__device__ uint32_t radix_threshold(const uint32_t (&v)[N], uint32_t k, int passes, uint32_t *s_hist,
                                    uint32_t *s_sel, uint32_t &count_ge) {
    const uint32_t tid = threadIdx.x;
    uint32_t prefix = 0, remaining = k, above_total = 0;
    count_ge = 0;
    for (int p = 0; p < passes; ++p) {
        const int shift = 24 - 8 * p;
        const uint32_t hmask = p == 0 ? 0u : (0xffffffffu << (shift + 8));
        for (uint32_t i = tid; i < 256u; i += kBlock) s_hist[i] = 0u;
        __syncthreads();
#pragma unroll
        for (int i = 0; i < N; ++i) {
            uint32_t x = v[i];
            if (x != 0u && (x & hmask) == prefix) atomicAdd(&s_hist[(x >> shift) & 255u], 1u);
        }
        __syncthreads();
        if (tid < 64) {
            const uint32_t lane = tid;
            uint32_t c[4], sum = 0;
#pragma unroll
            for (int q = 0; q < 4; ++q) {
                c[q] = s_hist[255u - 4u * lane - (uint32_t)q];
                sum += c[q];
            }
            uint32_t incl = wave_inclusive_scan(sum);
            uint32_t excl = incl - sum;
            if (excl < remaining && remaining <= incl) {
                uint32_t acc = excl;
#pragma unroll
                for (int q = 0; q < 4; ++q) {
                    if (acc < remaining && acc + c[q] >= remaining) {
                        s_sel[0] = 255u - 4u * lane - (uint32_t)q;
                        s_sel[1] = acc;
                        s_sel[2] = c[q];
                    }
                    acc += c[q];
                }
            }
            if (lane == 63 && incl < remaining) {
                s_sel[0] = 0xffffffffu;
                s_sel[1] = incl;
            }
        }
        __syncthreads();
        const uint32_t d = s_sel[0], above = s_sel[1], in_bin = s_sel[2];
        __syncthreads();
        if (d == 0xffffffffu) {
            count_ge = above_total + above;
            return 1u;
        }
        remaining -= above;
        above_total += above;
        prefix |= d << shift;
        count_ge = above_total + in_bin;
    }
    return prefix;
}

// Same contract as radix_threshold (all four bytes), over the tokens
// [t0, t1) of a slice with keys produced by `key_of(t)`; used by the rare
// exact path, which recomputes keys from memory instead of holding them.
template <typename KeyFn>
__device__ uint32_t radix_threshold_fn(uint32_t t0, uint32_t t1, uint32_t k, uint32_t *s_hist, uint32_t *s_sel,
                                       uint32_t &count_ge, KeyFn key_of) {
    const uint32_t tid = threadIdx.x;
    uint32_t prefix = 0, remaining = k, above_total = 0;
    count_ge = 0;
    for (int p = 0; p < 4; ++p) {
        const int shift = 24 - 8 * p;
        const uint32_t hmask = p == 0 ? 0u : (0xffffffffu << (shift + 8));
        for (uint32_t i = tid; i < 256u; i += kBlock) s_hist[i] = 0u;
        __syncthreads();
        for (uint32_t t = t0 + tid; t < t1; t += kBlock) {
            const uint32_t x = key_of(t);
            if (x != 0u && (x & hmask) == prefix) atomicAdd(&s_hist[(x >> shift) & 255u], 1u);
        }
        __syncthreads();
        if (tid < 64) {
            const uint32_t lane = tid;
            uint32_t c[4], sum = 0;
#pragma unroll
            for (int q = 0; q < 4; ++q) {
                c[q] = s_hist[255u - 4u * lane - (uint32_t)q];
                sum += c[q];
            }
            const uint32_t incl = wave_inclusive_scan(sum);
            const uint32_t excl = incl - sum;
            if (excl < remaining && remaining <= incl) {
                uint32_t acc = excl;
#pragma unroll
                for (int q = 0; q < 4; ++q) {
                    if (acc < remaining && acc + c[q] >= remaining) {
                        s_sel[0] = 255u - 4u * lane - (uint32_t)q;
                        s_sel[1] = acc;
                        s_sel[2] = c[q];
                    }
                    acc += c[q];
                }
            }
            if (lane == 63 && incl < remaining) {
                s_sel[0] = 0xffffffffu;
                s_sel[1] = incl;
            }
        }
        __syncthreads();
        const uint32_t d = s_sel[0], above = s_sel[1], in_bin = s_sel[2];
        __syncthreads();
        if (d == 0xffffffffu) {
            count_ge = above_total + above;
            return 1u;
        }
        remaining -= above;
        above_total += above;
        prefix |= d << shift;
        count_ge = above_total + in_bin;
    }
    return prefix;
}

// ---- the fused kernel -------------------------------------------------------

struct SharedSmall {
    uint32_t hist[256];
    uint32_t sel[4];
    uint32_t scan[kWaves];
    uint64_t red[kWaves];
    uint32_t flag[4];
};

__device__ __forceinline__ uint32_t xcd_remap(uint32_t b, uint32_t n) {
    // Workgroups are dispatched round-robin over the 8 XCDs; give each XCD a
    // contiguous run of logical ids so the slices of a row share one L2.
    const uint32_t q = n / 8u, rem = n % 8u;
    const uint32_t xcd = b % 8u, idx = b / 8u;
    return xcd < rem ? xcd * (q + 1u) + idx : rem * (q + 1u) + (xcd - rem) * q + idx;
}

// PEN: 0 = no penalty state, 1 = seen bitmap (set semantics), 2 = history ids (count semantics).
template <typename Elem, int EPV, int NV, bool MASK, int PEN>
__global__ __launch_bounds__(kBlock) void sample_rows_kernel(StepArgs a) {
    constexpr int E = NV * EPV;
    constexpr int W = VecTraits<Elem, EPV>::W;
    __shared__ SharedSmall sm;
    __shared__ uint32_t s_bitmap[kBlock * E / 32];
    extern __shared__ uint32_t s_dyn[];
    uint32_t *s_hash = s_dyn;                                        // [hash_slots]
    uint2 *s_big = (uint2 *)(s_dyn + a.hash_slots);                   // [big_entries]
    uint2 *s_sorted = s_big + a.big_entries;                          // [kcap]

    const uint32_t tid = threadIdx.x;
    const uint32_t logical = xcd_remap(blockIdx.x, gridDim.x);
    const uint32_t row = logical / a.slices;
    const uint32_t slice = logical % a.slices;

    const nerve_sampler_row_params P = a.params[row];
    const bool sampled = P.method != NERVE_METHOD_GREEDY;
    uint32_t k = sampled ? P.top_k : 1u;
    k = k < 1u ? 1u : (k > a.kcap ? a.kcap : k);
    const uint32_t valid_min = sampled ? kMinFiniteKey : kNegInfKey;

    const uint32_t v0 = slice * a.vec_per_slice;
    const uint32_t v1 = min(v0 + a.vec_per_slice, a.nvec);
    const uint32_t tok0 = v0 * EPV;
    const uint32_t tok1 = min(v1 * EPV, a.vocab);

    const Elem *lrow = (const Elem *)a.logits + (uint64_t)row * a.ld;
    const uint32_t *arow = MASK ? a.allowed + (uint64_t)row * a.allowed_stride : nullptr;
    const uint32_t *srow = PEN == 1 ? a.seen + (uint64_t)row * a.seen_stride : nullptr;
    constexpr bool history = PEN == 2;

    // 1. penalty tables for this slice
    if constexpr (history) {
        const uint32_t nslots = a.hash_slots;
        for (uint32_t i = tid; i < nslots; i += kBlock) s_hash[i] = kHashEmpty;
        const uint32_t nbw = (tok1 - tok0 + 31u) / 32u;
        for (uint32_t i = tid; i < nbw; i += kBlock) s_bitmap[i] = 0u;
        __syncthreads();
        uint32_t len = a.history_len[row];
        len = len > a.history_stride ? a.history_stride : len;
        const uint32_t *hrow = a.history + (uint64_t)row * a.history_stride;
        for (uint32_t i = tid; i < len; i += kBlock) {
            uint32_t id = hrow[i];
            if (id >= tok0 && id < tok1) {
                uint32_t o = id - tok0;
                atomicOr(&s_bitmap[o >> 5], 1u << (o & 31u));
                hash_insert(s_hash, a.log2_slots, id);
            }
        }
        __syncthreads();
    }

    // 2. stream the slice once into registers
    uint32_t raw[NV][W];
    uint32_t mword[MASK ? NV : 1], sword[PEN == 1 ? NV : 1];
#pragma unroll
    for (int j = 0; j < NV; ++j) {
        const uint32_t slot = v0 + (uint32_t)j * kBlock + tid;
        const uint32_t id0 = slot * EPV;
#pragma unroll
        for (int w = 0; w < W; ++w) raw[j][w] = 0u;
        if (slot < v1) {
            if constexpr (EPV > 1) {
                if (id0 + EPV <= a.vocab) {
                    uint4 q = *(const uint4 *)(lrow + id0);
                    raw[j][0] = q.x; raw[j][1] = q.y; raw[j][2] = q.z; raw[j][3] = q.w;
                } else {
#pragma unroll
                    for (int e = 0; e < EPV; ++e) {
                        if (id0 + e < a.vocab) {
                            uint32_t bits = sizeof(Elem) == 4 ? f2u(load_elem<Elem>(lrow, id0 + e))
                                                              : (f2u(load_elem<Elem>(lrow, id0 + e)) >> 16);
                            if constexpr (sizeof(Elem) == 4) raw[j][e] = bits;
                            else raw[j][e >> 1] |= (e & 1) ? (bits << 16) : bits;
                        }
                    }
                }
            } else {
                if constexpr (sizeof(Elem) == 4) raw[j][0] = f2u(lrow[id0]);
                else raw[j][0] = (uint32_t)lrow[id0];
            }
        }
        if constexpr (MASK) mword[j] = slot < v1 ? arow[id0 >> 5] : 0u;
        if constexpr (PEN == 1) sword[j] = slot < v1 ? srow[id0 >> 5] : 0u;
    }

    // keys, per-lane max (sampled) or best (greedy), slice flags
    uint32_t keys[E];
    uint32_t tmax = 0, best_id = kPadId;
    uint32_t any_allowed = 0, has_nan = 0;
#pragma unroll
    for (int j = 0; j < NV; ++j) {
        const uint32_t slot = v0 + (uint32_t)j * kBlock + tid;
        const uint32_t id0 = slot * EPV;
        uint32_t hb = 0u;
        if constexpr (history) hb = slot < v1 ? s_bitmap[(id0 - tok0) >> 5] >> ((id0 - tok0) & 31u) : 0u;
#pragma unroll
        for (int e = 0; e < EPV; ++e) {
            const uint32_t id = id0 + (uint32_t)e;
            const bool valid = slot < v1 && id < a.vocab;
            const float x = raw_elem<Elem, EPV>(raw[j], e);
            bool allowed = true;
            if constexpr (MASK) allowed = (mword[j] >> (id & 31u)) & 1u;
            uint32_t count = 0;
            if constexpr (history) {
                if ((hb >> e) & 1u) count = hash_lookup(s_hash, a.log2_slots, id);
            } else if constexpr (PEN == 1) {
                count = (sword[j] >> (id & 31u)) & 1u;
            }
            const float v = configured_logit(x, allowed, count, P.repetition_penalty, P.frequency_penalty,
                                             P.presence_penalty);
            uint32_t key = order_key(v);
            if (valid && allowed) any_allowed = 1u;
            if (valid && v != v) has_nan = 1u;
            if (!valid || key < valid_min) key = 0u;
            keys[j * EPV + e] = key;
            if (key > tmax) {
                tmax = key;
                best_id = id;
            }
        }
    }

    RowCtx ctx;
    ctx.logits_row = lrow;
    ctx.allowed_row = arow;
    ctx.seen_row = srow;
    ctx.hash = s_hash;
    ctx.bitmap = s_bitmap;
    ctx.log2_slots = a.log2_slots;
    ctx.tok0 = tok0;
    ctx.rep = P.repetition_penalty;
    ctx.freq = P.frequency_penalty;
    ctx.pres = P.presence_penalty;
    ctx.history = history;

    // slice flags: bit 0 = some token allowed, bit 1 = some configured value is NaN
    const uint32_t fsum = block_sum(any_allowed | (has_nan << 16), sm.scan);
    const uint32_t flags_slice = ((fsum & 0xffffu) ? 1u : 0u) | ((fsum >> 16) ? 2u : 0u);

    // 3. selection -> s_sorted[0 .. n_out)
    uint32_t n_out = 0;
    if (!sampled) {
        uint64_t packed = tmax ? (((uint64_t)tmax << 32) | (uint64_t)(~best_id)) : 0ull;
        uint64_t m = block_max_u64(packed, sm.red);
        if (m != 0ull) {
            if (tid == 0) s_sorted[0] = make_uint2((uint32_t)(m >> 32), ~(uint32_t)m);
            n_out = 1;
        }
        __syncthreads();
    } else {
        uint32_t cnt_unused;
        const uint32_t tm[1] = {tmax};
        uint32_t t = radix_threshold<1>(tm, k, 2, sm.hist, sm.sel, cnt_unused);
        uint32_t c = 0;
#pragma unroll
        for (int i = 0; i < E; ++i) c += keys[i] >= t ? 1u : 0u;
        uint32_t C;
        uint32_t base = block_exclusive_scan(c, sm.scan, C);
        uint2 *s_cand = s_big;
        if (C <= kCandCap) {
            uint32_t pos = base;
#pragma unroll
            for (int i = 0; i < E; ++i) {
                if (keys[i] >= t) {
                    const uint32_t id = (v0 + (uint32_t)(i / EPV) * kBlock + tid) * EPV + (uint32_t)(i % EPV);
                    s_cand[pos++] = make_uint2(keys[i], id);
                }
            }
        } else {
            // Skewed slice: exact selection recomputed from memory (rare). The
            // k-th largest key kv, then the `need` smallest ids among keys == kv.
            auto key_at = [&](uint32_t t) -> uint32_t {
                uint32_t key = order_key(configured_at<Elem>(ctx, t));
                return key < valid_min ? 0u : key;
            };
            uint32_t count_ge;
            const uint32_t kv = radix_threshold_fn(tok0, tok1, k, sm.hist, sm.sel, count_ge, key_at);
            uint32_t gt = 0;
            for (uint32_t t = tok0 + tid; t < tok1; t += kBlock) gt += key_at(t) > kv ? 1u : 0u;
            const uint32_t G = block_sum(gt, sm.scan);
            const uint32_t need = k - G;  // count_ge >= k > G here
            auto tie_at = [&](uint32_t t) -> uint32_t { return key_at(t) == kv ? ~t : 0u; };
            uint32_t ties_ge;
            const uint32_t id_cut = ~radix_threshold_fn(tok0, tok1, need, sm.hist, sm.sel, ties_ge, tie_at);
            if (tid == 0) sm.flag[1] = 0u;
            __syncthreads();
            for (uint32_t t = tok0 + tid; t < tok1; t += kBlock) {
                const uint32_t key = key_at(t);
                if (key > kv || (key == kv && t <= id_cut)) {
                    const uint32_t pos = atomicAdd(&sm.flag[1], 1u);
                    if (pos < kCandCap) s_cand[pos] = make_uint2(key, t);
                }
            }
            __syncthreads();
            C = min(sm.flag[1], kCandCap);
        }
        __syncthreads();
        // rank sort (ids are distinct, so ranks are a permutation)
        for (uint32_t i = tid; i < C; i += kBlock) {
            const uint2 e = s_cand[i];
            uint32_t r = 0;
            for (uint32_t j = 0; j < C; ++j) r += entry_better(s_cand[j], e) ? 1u : 0u;
            if (r < k) s_sorted[r] = e;
        }
        n_out = C < k ? C : k;
        __syncthreads();
    }

    // the sign of a zero survivor comes from its own configured value
    for (uint32_t i = tid; i < n_out; i += kBlock) {
        uint2 e = s_sorted[i];
        if (e.x == kZeroKey) {
            float v = configured_at<Elem>(ctx, e.y);
            if (f2u(v) == 0x80000000u) s_sorted[i].y = e.y | kNegZeroFlag;
        }
    }
    __syncthreads();

    // 4. publish / merge
    uint32_t n = n_out;
    uint32_t row_flags = flags_slice;
    if (a.slices > 1) {
        uint2 *lists = a.scratch_lists + (uint64_t)(row * a.slices + slice) * a.kcap;
        for (uint32_t i = tid; i < n_out; i += kBlock) lists[i] = s_sorted[i];
        if (tid == 0) a.scratch_meta[row * a.slices + slice] = n_out | (flags_slice << 16);
        __threadfence();
        __syncthreads();
        if (tid == 0) {
            uint32_t old = atomicAdd(&a.counters[row], 1u);
            sm.flag[0] = old == a.slices - 1u ? 1u : 0u;
        }
        __syncthreads();
        if (!sm.flag[0]) return;
        __threadfence();
        if (tid == 0) a.counters[row] = 0u;
        const uint2 *all = a.scratch_lists + (uint64_t)row * a.slices * a.kcap;
        const uint32_t *meta = a.scratch_meta + row * a.slices;
        uint32_t total = 0;
        row_flags = 0;
        for (uint32_t s = 0; s < a.slices; ++s) {
            uint32_t m = meta[s];
            total += m & 0xffffu;
            row_flags |= m >> 16;
        }
        const uint32_t ne = a.slices * a.kcap;
        for (uint32_t i = tid; i < ne; i += kBlock) {
            const uint32_t s = i / a.kcap, pos = i % a.kcap;
            const uint32_t ns = meta[s] & 0xffffu;
            if (pos < ns) s_big[i] = all[i];
        }
        __syncthreads();
        for (uint32_t i = tid; i < ne; i += kBlock) {
            const uint32_t s = i / a.kcap, pos = i % a.kcap;
            const uint32_t ns = meta[s] & 0xffffu;
            if (pos >= ns) continue;
            const uint2 e = s_big[i];
            uint32_t r = pos;
            for (uint32_t o = 0; o < a.slices && r < k; ++o) {
                if (o == s) continue;
                const uint2 *lo = s_big + o * a.kcap;
                uint32_t lo_i = 0, hi_i = meta[o] & 0xffffu;
                while (lo_i < hi_i) {
                    uint32_t mid = (lo_i + hi_i) >> 1;
                    if (entry_better(lo[mid], e)) lo_i = mid + 1; else hi_i = mid;
                }
                r += lo_i;
            }
            if (r < k) s_sorted[r] = e;
        }
        n = total < k ? total : k;
        __syncthreads();
    }

    // 5. final step for the row
    float *s_w = (float *)s_big;               // [kcap] weights
    float *s_p = (float *)s_big + a.kcap;      // [kcap] running sums
    uint32_t token = 0, sel_bits = 0, out_flags = 0;
    uint32_t kout = 1;                         // survivors to report
    __shared__ uint32_t s_res[4];

    const bool eos = a.allowed && !(row_flags & 1u);
    if (eos) {
        token = a.eos;
        sel_bits = 0xff800000u;
        out_flags = NERVE_FLAG_EOS_FALLBACK | (sampled ? NERVE_FLAG_SAMPLED : 0u);
        if (tid == 0) {
            s_sorted[0] = make_uint2(0u, a.eos);  // reported as (LOWEST_FLOAT, eos), prob 1
            s_p[0] = 1.0f;
        }
        kout = 1;
    } else if (!sampled) {
        if (row_flags & 2u) {
            // NaN present: replay the reference lane structure exactly.
            if (history) {
                for (uint32_t i = tid; i < a.hash_slots; i += kBlock) s_hash[i] = kHashEmpty;
                __syncthreads();
                uint32_t len = a.history_len[row];
                len = len > a.history_stride ? a.history_stride : len;
                const uint32_t *hrow = a.history + (uint64_t)row * a.history_stride;
                for (uint32_t i = tid; i < len; i += kBlock)
                    if (hrow[i] < a.vocab) hash_insert(s_hash, a.log2_slots, hrow[i]);
                __syncthreads();
            }
            RowCtx full = ctx;
            full.bitmap = nullptr;
            uint2 *slots = s_big;  // 1024 entries of (float bits, id)
            for (uint32_t L = tid; L < 1024u; L += kBlock) {
                uint32_t bid = L;
                float best = L < a.vocab ? configured_at<Elem>(full, L) : u2f(kLowestBits);
                for (uint32_t t = L + 1024u; t < a.vocab; t += 1024u) {
                    float c = configured_at<Elem>(full, t);
                    if (float_better(c, t, best, bid)) {
                        best = c;
                        bid = t;
                    }
                }
                slots[L] = make_uint2(f2u(best), bid);
            }
            __syncthreads();
            for (uint32_t stride = 512u; stride > 0u; stride >>= 1) {
                for (uint32_t L = tid; L < stride; L += kBlock) {
                    uint2 c = slots[L + stride], b = slots[L];
                    if (float_better(u2f(c.x), c.y, u2f(b.x), b.y)) slots[L] = c;
                }
                __syncthreads();
            }
            token = slots[0].y;
            sel_bits = slots[0].x;
        } else {
            uint2 e = s_sorted[0];
            if (e.x == kNegInfKey && a.vocab < 1024u) {
                token = a.vocab;
                sel_bits = kLowestBits;
            } else {
                token = e.y & kIdMask;
                sel_bits = f2u(entry_value(e));
            }
        }
        out_flags = 0u;
        kout = 1;
        __syncthreads();
        if (tid == 0) s_p[0] = 1.0f;
    } else {
        // pad to k with (LOWEST_FLOAT, 0xffffffff)
        for (uint32_t i = n + tid; i < k; i += kBlock) s_sorted[i] = make_uint2(kMinFiniteKey, kPadId);
        __syncthreads();
        if (tid < 64) {
            const uint32_t lane = tid;
            const float T = P.temperature;
            const float l0 = entry_value(s_sorted[0]);
            const float m = l0 / T;
            float minimum = u2f(kLowestBits);
            if (P.min_p > 0.0f) {
                const float lg = nerve_logf(P.min_p);
                const float d = T * lg;
                minimum = l0 + d;
            }
            // n_valid: leading survivors not below the min-p floor
            uint32_t n_valid = k;
            for (uint32_t c0 = 0; c0 < k; c0 += 64u) {
                const uint32_t i = c0 + lane;
                const bool below = i < k && entry_value(s_sorted[i]) < minimum;
                const uint64_t b = __ballot(below);
                if (b) {
                    n_valid = c0 + (uint32_t)__builtin_ctzll(b);
                    break;
                }
            }
            // weights and their sequential running sums (the reference's loop order)
            float acc = 0.0f;
            for (uint32_t c0 = 0; c0 < n_valid; c0 += 64u) {
                const uint32_t i = c0 + lane;
                float w = 0.0f;
                if (i < n_valid) {
                    const float s = entry_value(s_sorted[i]) / T;
                    w = nerve_expf(s - m);
                    s_w[i] = w;
                }
                const uint32_t cnt = min(64u, n_valid - c0);
                float mine = 0.0f;
                for (uint32_t j = 0; j < cnt; ++j) {
                    const float wj = __shfl(w, (int)j, 64);
                    acc = acc + wj;
                    if (lane == j) mine = acc;
                }
                if (i < n_valid) s_p[i] = mine;
            }
            const float total = n_valid ? s_p[n_valid - 1] : 0.0f;
            const float threshold = P.top_p * total;
            uint32_t nucleus = n_valid;
            for (uint32_t c0 = 0; c0 < n_valid; c0 += 64u) {
                const uint32_t i = c0 + lane;
                const uint64_t b = __ballot(i < n_valid && s_p[i] >= threshold);
                if (b) {
                    nucleus = c0 + (uint32_t)__builtin_ctzll(b) + 1u;
                    break;
                }
            }
            if (nucleus == 0u) nucleus = 1u;
            const float nucleus_weight = n_valid ? s_p[nucleus - 1u] : 0.0f;
            uint64_t tick;
            uint32_t *sc = a.stream_control ? a.stream_control + (uint64_t)row * 5u : nullptr;
            if (sc) tick = (uint64_t)sc[1] | ((uint64_t)sc[2] << 32);
            else tick = a.steps ? a.steps[row] : 0ull;
            const uint32_t seed = a.seeds ? a.seeds[row] : 0u;
            const float u = random_unit(a.rng, seed, tick, row);
            const float target = u * nucleus_weight;
            uint32_t selected = nucleus - 1u;
            for (uint32_t c0 = 0; c0 < nucleus && c0 < n_valid; c0 += 64u) {
                const uint32_t i = c0 + lane;
                const uint64_t b = __ballot(i < nucleus && i < n_valid && target < s_p[i]);
                if (b) {
                    selected = c0 + (uint32_t)__builtin_ctzll(b);
                    break;
                }
            }
            // post-filter probabilities overwrite the running sums
            for (uint32_t i = lane; i < k; i += 64u) {
                const float pw = (i < nucleus && i < n_valid) ? s_w[i] / nucleus_weight : 0.0f;
                s_p[i] = pw;
            }
            if (lane == 0) {
                const uint2 e = s_sorted[selected];
                s_res[0] = e.y & kIdMask;
                s_res[1] = f2u(entry_value(e));
            }
        }
        __syncthreads();
        token = s_res[0];
        sel_bits = s_res[1];
        out_flags = NERVE_FLAG_SAMPLED;
        kout = k;
    }
    __syncthreads();

    // outputs
    if (tid == 0) {
        nerve_sampler_output o;
        o.token_id = token;
        o.selected_logit_bits = sel_bits;
        o.flags = out_flags;
        o.reserved = 0u;
        a.out[row] = o;
        uint32_t *sc = a.stream_control ? a.stream_control + (uint64_t)row * 5u : nullptr;
        if (sc) {
            const uint32_t lo = sc[1];
            if (a.ring) {
                uint32_t *ring = a.ring + (uint64_t)row * a.ring_stride;
                const uint32_t cap = sc[4];
                ring[0] = token; ring[1] = sel_bits; ring[2] = out_flags; ring[3] = 0u;
                if (cap) {
                    const uint64_t w = 4ull + (uint64_t)(lo % cap) * 4ull;
                    if (w + 4ull <= a.ring_stride) {
                        ring[w] = token; ring[w + 1] = sel_bits; ring[w + 2] = out_flags; ring[w + 3] = 0u;
                    }
                }
            }
            sc[0] = token;
            const uint32_t next = lo + 1u;
            if (next == 0u) sc[2] = sc[2] + 1u;
            sc[1] = next;
        }
    }
    if (a.topk_ids || a.topk_logits || a.topk_probs) {
        for (uint32_t i = tid; i < a.kcap; i += kBlock) {
            const uint64_t o = (uint64_t)row * a.kcap + i;
            const bool live = i < kout;
            uint2 e = live ? s_sorted[i] : make_uint2(kMinFiniteKey, kPadId);
            float value;
            uint32_t id;
            if (eos && i == 0) {
                value = u2f(kLowestBits);
                id = a.eos;
            } else if (!sampled && !eos && i == 0) {
                value = u2f(sel_bits);
                id = token;
            } else {
                value = live ? entry_value(e) : u2f(kLowestBits);
                id = e.y == kPadId ? kPadId : (e.y & kIdMask);
            }
            if (a.topk_ids) a.topk_ids[o] = id;
            if (a.topk_logits) a.topk_logits[o] = value;
            if (a.topk_probs) a.topk_probs[o] = live ? s_p[i] : 0.0f;
        }
    }
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

// ---- launch ------------------------------------------------------------------

template <typename Elem, int EPV, int NV, bool MASK, int PEN>
static hipError_t launch_one(const StepArgs &a, hipStream_t stream) {
    const size_t dyn = a.dyn_lds_bytes;
    auto kern = sample_rows_kernel<Elem, EPV, NV, MASK, PEN>;
    if (dyn > 48u * 1024u) {
        hipError_t e = hipFuncSetAttribute((const void *)kern, hipFuncAttributeMaxDynamicSharedMemorySize, (int)dyn);
        if (e != hipSuccess) return e;
    }
    hipLaunchKernelGGL(kern, dim3(a.batch * a.slices), dim3(kBlock), dyn, stream, a);
    return hipGetLastError();
}

template <typename Elem, int EPV, int NV>
static hipError_t launch_variant(const StepArgs &a, hipStream_t stream) {
    const bool mask = a.allowed != nullptr;
    const int pen = a.history ? 2 : (a.seen ? 1 : 0);
    if (mask) {
        if (pen == 2) return launch_one<Elem, EPV, NV, true, 2>(a, stream);
        if (pen == 1) return launch_one<Elem, EPV, NV, true, 1>(a, stream);
        return launch_one<Elem, EPV, NV, true, 0>(a, stream);
    }
    if (pen == 2) return launch_one<Elem, EPV, NV, false, 2>(a, stream);
    if (pen == 1) return launch_one<Elem, EPV, NV, false, 1>(a, stream);
    return launch_one<Elem, EPV, NV, false, 0>(a, stream);
}

uint32_t elems_per_thread(uint32_t variant) {
    switch (variant) {
        case kVariantF32Vec: return 4u * 8u;
        case kVariantBf16Vec: return 8u * 8u;
        default: return 16u;
    }
}

uint32_t elems_per_vector(uint32_t variant) {
    switch (variant) {
        case kVariantF32Vec: return 4u;
        case kVariantBf16Vec: return 8u;
        default: return 1u;
    }
}

uint32_t block_threads() { return (uint32_t)kBlock; }
uint32_t cand_capacity() { return kCandCap; }

hipError_t launch_sample_rows(uint32_t variant, const StepArgs &a, hipStream_t stream) {
    switch (variant) {
        case kVariantF32Vec: return launch_variant<float, 4, 8>(a, stream);
        case kVariantBf16Vec: return launch_variant<uint16_t, 8, 8>(a, stream);
        case kVariantF32Scalar: return launch_variant<float, 1, 16>(a, stream);
        case kVariantBf16Scalar: return launch_variant<uint16_t, 1, 16>(a, stream);
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
