// nerve_sampler_device.h -- the gfx950 sampling kernels (device code shared by
// the per-variant translation units that instantiate them).
//
// One step samples every row of a decode batch with at most two launches.
// sample_rows_kernel: each row is split into S vocabulary slices, one 512-lane
// workgroup per slice (mapped so the slices of a row share one XCD's L2). A
// workgroup streams its slice from HBM once, in chunks of 8 x 16-byte loads per
// lane, double-buffered in VGPRs so the loads of chunk c+1 are in flight while
// chunk c is processed:
//   - history ids of the slice go into an LDS bitmap and an id -> count hash;
//     a token with penalty state leaves the stream and re-enters as a patch
//     entry carrying its configured (masked + penalised) value;
//   - every other element becomes an order key straight from its raw bits;
//   - greedy rows keep a per-lane best; sampled rows take a threshold from the
//     first chunk (the k-th largest per-lane maximum, 16-bit LDS radix select:
//     at least k keys are >= it) and append every later key >= it to an LDS
//     candidate list with wave-ballot compaction (about k + a few per chunk
//     for iid logits). A list that would overflow switches the slice to an
//     exact radix selection recomputed from memory;
//   - the candidates are rank-sorted (value desc, id asc) into the slice's
//     top-k list.
// With S = 1 the workgroup finishes the row itself; otherwise it writes the
// list to scratch and finish_rows_kernel (one workgroup per row, same stream,
// so no cross-workgroup fence) merges the S lists by binary-search ranks, then
// one wave runs min-p / top-p over the k survivors and the draw.
//
// Semantics follow the reference shaders (paths under runtime-rs/shaders/):
//   greedy_sampler_f32.comp.template:31-34, 52-108       tie-break, argmax, record, tick carry
//   temperature_top_k_candidates_f32.comp.template:59-126 exact top-k, NaN skipped, -inf never enters
//   temperature_top_k_top_p_sampler_f32.comp.template:90-216 merge, min-p, top-p, draw, record
// The greedy path reproduces the reference's NaN behaviour (a lane that starts
// on a NaN keeps it through the 1024-lane tree) by re-running that exact lane
// structure for the rare rows that contain a NaN.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include <atomic>
#include <utility>

#include "nerve_device_math.h"
#include "nerve_sampler_internal.h"

namespace nerve {


constexpr int kBlock = 512;
constexpr int kWaves = kBlock / 64;
constexpr int kFinishBlock = 256;
constexpr uint32_t kCandCap = 1024;
constexpr uint32_t kRankPad = 128;  // candidate counts the unrolled rank sort handles
constexpr uint32_t kHashEmpty = 0xffffffffu;
constexpr uint32_t kMaxHistory = NERVE_MAX_HISTORY_CAPACITY;

__device__ __forceinline__ uint32_t lane_id() { return __lane_id(); }

// Calls f(std::integral_constant<int, J>) for J = B .. E-1 in order: indices
// into register arrays stay compile-time however large the body grows.
template <int B, typename F, int... Js>
__device__ __forceinline__ void static_for_impl(F &&f, std::integer_sequence<int, Js...>) {
    (f(std::integral_constant<int, B + Js>{}), ...);
}
template <int B, int E, typename F>
__device__ __forceinline__ void static_for(F &&f) {
    if constexpr (E > B) static_for_impl<B>(f, std::make_integer_sequence<int, E - B>{});
}

// Workgroup barrier that orders LDS only: waits for this wave's LDS traffic,
// not for its global loads, so prefetched chunks stay in flight across it.
__device__ __forceinline__ void lds_sync() {
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup", "local");
    __builtin_amdgcn_s_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "workgroup", "local");
}

// The largest t (top B bits significant, the rest zero) with at least `need`
// of the wave's keys v[] >= t: an MSB-first search with ballot counts. 0 when
// fewer than `need` keys are nonzero.
template <int N, int B>
__device__ __forceinline__ uint32_t wave_kth(const uint32_t (&v)[N], uint32_t need) {
    uint32_t prefix = 0u;
#pragma unroll
    for (int b = 31; b >= 32 - B; --b) {
        const uint32_t cand = prefix | (1u << b);
        uint32_t cnt = 0u;
#pragma unroll
        for (int i = 0; i < N; ++i) cnt += (uint32_t)__popcll(__ballot(v[i] >= cand));
        prefix = cnt >= need ? cand : prefix;
    }
    return prefix;
}

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
    lds_sync();
    uint32_t base = 0, tot = 0;
#pragma unroll
    for (int w = 0; w < kWaves; ++w) {
        uint32_t t = s_tmp[w];
        base += (uint32_t)w < wave ? t : 0u;
        tot += t;
    }
    lds_sync();
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
    lds_sync();
    uint64_t m = s_tmp[0];
#pragma unroll
    for (int w = 1; w < kWaves; ++w) m = s_tmp[w] > m ? s_tmp[w] : m;
    lds_sync();
    return m;
}

// Order key of a binary32 bit pattern (same mapping as order_key()).
__device__ __forceinline__ uint32_t raw_order_key(uint32_t bits) {
    const uint32_t mag = bits & 0x7fffffffu;
    const uint32_t b = mag == 0u ? 0u : bits;
    const uint32_t key = (b & 0x80000000u) ? ~b : (b | 0x80000000u);
    return mag > 0x7f800000u ? 0u : key;
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

__device__ __forceinline__ void hash_insert(uint32_t *h, uint32_t log2_slots, uint32_t id) {
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

// One EPV-element slot as loaded from HBM (16 bytes for the vector variants).
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));

template <typename Elem, int EPV>
struct VecTraits;

// bits(): the binary32 bit pattern of element e (bf16 widens exactly by a shift).
// upper(): an upper bound of the canonical order keys of the lane-vector's raw
// values (exact except that -0.0 is lifted to +0.0's key), computed with packed
// integer ops; has_nan(): whether any raw value is a NaN.
typedef unsigned short u16x2 __attribute__((ext_vector_type(2)));
typedef short i16x2 __attribute__((ext_vector_type(2)));

// Order keys of two bf16 values at once: negative -> ~h, else h | 0x8000.
__device__ __forceinline__ uint32_t bf16x2_keys(uint32_t w) {
    const i16x2 s = __builtin_bit_cast(i16x2, w) >> (i16x2){15, 15};
    return w ^ (__builtin_bit_cast(uint32_t, s) | 0x80008000u);
}

__device__ __forceinline__ uint32_t u16x2_max(uint32_t a, uint32_t b) {
    return __builtin_bit_cast(uint32_t, __builtin_elementwise_max(__builtin_bit_cast(u16x2, a), __builtin_bit_cast(u16x2, b)));
}

__device__ __forceinline__ uint32_t f32_key_upper(uint32_t w) {
    const uint32_t key = w ^ ((uint32_t)((int32_t)w >> 31) | 0x80000000u);
    return key == 0x7fffffffu ? 0x80000000u : key;
}
__device__ __forceinline__ uint32_t i32_max(uint32_t a, uint32_t b) { return (uint32_t)max((int32_t)a, (int32_t)b); }

__device__ __forceinline__ uint32_t i16x2_max(uint32_t a, uint32_t b) {
    return __builtin_bit_cast(uint32_t, __builtin_elementwise_max(__builtin_bit_cast(i16x2, a), __builtin_bit_cast(i16x2, b)));
}

// Raw-bit maxima. Read as signed integers, the bit patterns of non-negative
// values order like the values and sit above every negative one, so the
// signed maximum of a set is its largest value whenever that is >= +0 (and
// otherwise still one of its elements). vmax() reduces one lane-vector into
// the accumulator form (packed i16 pairs for bf16, one i32 for f32); merge()
// folds two accumulators; report_bits() gives the binary32 pattern of report r
// (0x80000000, the bits of -0.0, is the empty marker); ge_pos(vm, thr) tests
// whether a vmax() value holds a key >= thr, valid when thr > kZeroKey.
template <>
struct VecTraits<float, 4> {
    using load_t = u32x4;
    static constexpr int kReports = 1;
    static constexpr uint32_t kAccInit = 0x80000000u;
    __device__ static __forceinline__ uint32_t vmax(const load_t &r) { return i32_max(i32_max(r[0], r[1]), i32_max(r[2], r[3])); }
    __device__ static __forceinline__ uint32_t merge(uint32_t a, uint32_t b) { return i32_max(a, b); }
    __device__ static __forceinline__ uint32_t report_bits(uint32_t acc, int) { return acc; }
    __device__ static __forceinline__ bool ge_pos(uint32_t vm, uint32_t thr) { return (int32_t)vm >= (int32_t)(thr & 0x7fffffffu); }
    __device__ static __forceinline__ uint32_t staged_bits(const load_t *v, uint32_t i, uint32_t e) { return ((const uint32_t *)(v + i))[e]; }
    __device__ static __forceinline__ uint32_t upper(const load_t &r) {
        const uint32_t a = max(f32_key_upper(r[0]), f32_key_upper(r[1]));
        const uint32_t b = max(f32_key_upper(r[2]), f32_key_upper(r[3]));
        return max(a, b);
    }
    __device__ static __forceinline__ bool has_nan(const load_t &r) {
        const uint32_t m = max(max(r[0] & 0x7fffffffu, r[1] & 0x7fffffffu), max(r[2] & 0x7fffffffu, r[3] & 0x7fffffffu));
        return m > 0x7f800000u;
    }
    __device__ static __forceinline__ uint32_t bits(const load_t &r, int e) { return r[e]; }
    __device__ static __forceinline__ uint32_t bits_dyn(const load_t &r, uint32_t e) {
        const uint32_t lo = (e & 1u) ? r[1] : r[0], hi = (e & 1u) ? r[3] : r[2];
        return (e & 2u) ? hi : lo;
    }
};

template <>
struct VecTraits<uint16_t, 8> {
    using load_t = u32x4;
    static constexpr int kReports = 2;
    static constexpr uint32_t kAccInit = 0x80008000u;
    __device__ static __forceinline__ uint32_t vmax(const load_t &r) { return i16x2_max(i16x2_max(r[0], r[1]), i16x2_max(r[2], r[3])); }
    __device__ static __forceinline__ uint32_t merge(uint32_t a, uint32_t b) { return i16x2_max(a, b); }
    __device__ static __forceinline__ uint32_t report_bits(uint32_t acc, int r) { return r == 0 ? acc << 16 : acc & 0xffff0000u; }
    __device__ static __forceinline__ bool ge_pos(uint32_t vm, uint32_t thr) {
        const int32_t m = max((int32_t)(int16_t)(vm & 0xffffu), (int32_t)(int16_t)(vm >> 16));
        return m >= (int32_t)(((thr & 0x7fffffffu) + 0xffffu) >> 16);
    }
    __device__ static __forceinline__ uint32_t staged_bits(const load_t *v, uint32_t i, uint32_t e) {
        const uint32_t w = ((const uint32_t *)(v + i))[e >> 1];
        return (e & 1u) ? (w & 0xffff0000u) : (w << 16);
    }
    __device__ static __forceinline__ uint32_t upper(const load_t &r) {
        const uint32_t m2 = u16x2_max(u16x2_max(bf16x2_keys(r[0]), bf16x2_keys(r[1])),
                                      u16x2_max(bf16x2_keys(r[2]), bf16x2_keys(r[3])));
        const uint32_t m16 = max(m2 & 0xffffu, m2 >> 16);
        return m16 == 0x7fffu ? 0x80000000u : ((m16 << 16) | 0xffffu);
    }
    __device__ static __forceinline__ bool has_nan(const load_t &r) {
        const uint32_t t = ((r[0] & 0x7fff7fffu) + 0x007f007fu) | ((r[1] & 0x7fff7fffu) + 0x007f007fu) |
                           ((r[2] & 0x7fff7fffu) + 0x007f007fu) | ((r[3] & 0x7fff7fffu) + 0x007f007fu);
        return (t & 0x80008000u) != 0u;
    }
    __device__ static __forceinline__ uint32_t bits(const load_t &r, int e) {
        const uint32_t w = r[e >> 1];
        return (e & 1) ? (w & 0xffff0000u) : (w << 16);
    }
    __device__ static __forceinline__ uint32_t bits_dyn(const load_t &r, uint32_t e) {
        const uint32_t lo = (e & 2u) ? r[1] : r[0], hi = (e & 2u) ? r[3] : r[2];
        const uint32_t w = (e & 4u) ? hi : lo;
        return (e & 1u) ? (w & 0xffff0000u) : (w << 16);
    }
};

template <>
struct VecTraits<float, 1> {
    using load_t = float;
    static constexpr int kReports = 1;
    static constexpr uint32_t kAccInit = 0x80000000u;
    __device__ static __forceinline__ uint32_t vmax(const load_t &r) { return f2u(r); }
    __device__ static __forceinline__ uint32_t merge(uint32_t a, uint32_t b) { return i32_max(a, b); }
    __device__ static __forceinline__ uint32_t report_bits(uint32_t acc, int) { return acc; }
    __device__ static __forceinline__ bool ge_pos(uint32_t vm, uint32_t thr) { return (int32_t)vm >= (int32_t)(thr & 0x7fffffffu); }
    __device__ static __forceinline__ uint32_t staged_bits(const load_t *v, uint32_t i, uint32_t) { return f2u(v[i]); }
    __device__ static __forceinline__ uint32_t upper(const load_t &r) { return f32_key_upper(f2u(r)); }
    __device__ static __forceinline__ bool has_nan(const load_t &r) { return (f2u(r) & 0x7fffffffu) > 0x7f800000u; }
    __device__ static __forceinline__ uint32_t bits(const load_t &r, int) { return f2u(r); }
    __device__ static __forceinline__ uint32_t bits_dyn(const load_t &r, uint32_t) { return f2u(r); }
};

template <>
struct VecTraits<uint16_t, 1> {
    using load_t = uint16_t;
    static constexpr int kReports = 1;
    static constexpr uint32_t kAccInit = 0x80000000u;
    __device__ static __forceinline__ uint32_t vmax(const load_t &r) { return (uint32_t)r << 16; }
    __device__ static __forceinline__ uint32_t merge(uint32_t a, uint32_t b) { return i32_max(a, b); }
    __device__ static __forceinline__ uint32_t report_bits(uint32_t acc, int) { return acc; }
    __device__ static __forceinline__ bool ge_pos(uint32_t vm, uint32_t thr) { return (int32_t)vm >= (int32_t)(thr & 0x7fffffffu); }
    __device__ static __forceinline__ uint32_t staged_bits(const load_t *v, uint32_t i, uint32_t) { return (uint32_t)v[i] << 16; }
    __device__ static __forceinline__ uint32_t upper(const load_t &r) { return f32_key_upper((uint32_t)r << 16); }
    __device__ static __forceinline__ bool has_nan(const load_t &r) { return ((uint32_t)r & 0x7fffu) > 0x7f80u; }
    __device__ static __forceinline__ uint32_t bits(const load_t &r, int) { return (uint32_t)r << 16; }
    __device__ static __forceinline__ uint32_t bits_dyn(const load_t &r, uint32_t) { return (uint32_t)r << 16; }
};

// Tokens of row `row`'s seen-state prefix: prefix_counts[row] (at most the
// token-batch capacity), or row + 1 for the [..=row] prefixes of a batch.
__device__ __forceinline__ uint32_t prefix_count(const StepArgs &a, uint32_t row) {
    if (!a.prefix_ids) return 0u;
    const uint32_t n = a.prefix_counts ? a.prefix_counts[row] : row + 1u;
    return n < NERVE_TOKEN_BATCH_CAPACITY ? n : NERVE_TOKEN_BATCH_CAPACITY;
}

// Row state shared by the helpers that recompute a single configured value.
struct RowCtx {
    const void *logits_row;
    const uint32_t *allowed_row;
    const uint32_t *seen_row;
    const uint32_t *hash;      // LDS
    // LDS bitmap of the slice's history ids (from tok0) with `hash` holding
    // the occurrences beyond the first; or null, and `hash` holds full counts
    const uint32_t *bitmap;
    uint32_t log2_slots;
    uint32_t tok0;
    float rep, freq, pres;
    bool history;
    const uint32_t *prefix;  // seen-state prefix of the row (set semantics), prefix_n ids
    uint32_t prefix_n;
    bool whole_row;  // `bitmap` (from token 0) and `hash` cover every token of the row
};

// The configured value of token t whose raw logit x the caller has loaded.
__device__ __forceinline__ float configured_from(const RowCtx &c, uint32_t t, float x) {
    bool allowed = c.allowed_row ? ((c.allowed_row[t >> 5] >> (t & 31u)) & 1u) : true;
    uint32_t count = 0;
    if (c.history) {
        if (c.bitmap) {
            const uint32_t o = t - c.tok0;
            if ((c.bitmap[o >> 5] >> (o & 31u)) & 1u) count = 1u + hash_lookup(c.hash, c.log2_slots, t);
        } else {
            count = hash_lookup(c.hash, c.log2_slots, t);
        }
    } else if (c.bitmap) {
        // the slice's LDS copy of the seen words, prefix included
        const uint32_t o = t - c.tok0;
        count = (c.bitmap[o >> 5] >> (o & 31u)) & 1u;
    } else if (c.seen_row) {
        count = (c.seen_row[t >> 5] >> (t & 31u)) & 1u;
        for (uint32_t i = 0; i < c.prefix_n && count == 0u; ++i) count = c.prefix[i] == t ? 1u : 0u;
    }
    return configured_logit(x, allowed, count, c.rep, c.freq, c.pres);
}

template <typename Elem>
__device__ __forceinline__ float configured_at(const RowCtx &c, uint32_t t) {
    return configured_from(c, t, load_elem<Elem>((const Elem *)c.logits_row, t));
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
__device__ __forceinline__ uint32_t radix_threshold(const uint32_t (&v)[N], uint32_t k, int passes, uint32_t *s_hist,
                                    uint32_t *s_sel, uint32_t &count_ge) {
    const uint32_t tid = threadIdx.x;
    uint32_t prefix = 0, remaining = k, above_total = 0;
    count_ge = 0;
    for (int p = 0; p < passes; ++p) {
        const int shift = 24 - 8 * p;
        const uint32_t hmask = p == 0 ? 0u : (0xffffffffu << (shift + 8));
        for (uint32_t i = tid; i < 256u; i += kBlock) s_hist[i] = 0u;
        lds_sync();
#pragma unroll
        for (int i = 0; i < N; ++i) {
            uint32_t x = v[i];
            if (x != 0u && (x & hmask) == prefix) atomicAdd(&s_hist[(x >> shift) & 255u], 1u);
        }
        lds_sync();
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
        lds_sync();
        const uint32_t d = s_sel[0], above = s_sel[1], in_bin = s_sel[2];
        lds_sync();
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
// visit(fn) calls fn(key) for every key this thread holds (0: no key).
template <typename VisitFn>
__device__ __forceinline__ uint32_t radix_threshold_visit(uint32_t k, uint32_t *s_hist, uint32_t *s_sel, uint32_t &count_ge,
                                                          VisitFn visit, uint32_t *count_gt = nullptr) {
    const uint32_t tid = threadIdx.x;
    uint32_t prefix = 0, remaining = k, above_total = 0;
    count_ge = 0;
    for (int p = 0; p < 4; ++p) {
        const int shift = 24 - 8 * p;
        const uint32_t hmask = p == 0 ? 0u : (0xffffffffu << (shift + 8));
        for (uint32_t i = tid; i < 256u; i += kBlock) s_hist[i] = 0u;
        lds_sync();
        visit([&](uint32_t x) __attribute__((always_inline)) {
            if (x != 0u && (x & hmask) == prefix) atomicAdd(&s_hist[(x >> shift) & 255u], 1u);
        });
        lds_sync();
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
        lds_sync();
        const uint32_t d = s_sel[0], above = s_sel[1], in_bin = s_sel[2];
        lds_sync();
        if (d == 0xffffffffu) {
            count_ge = above_total + above;
            if (count_gt) *count_gt = count_ge;
            return 1u;
        }
        remaining -= above;
        above_total += above;
        prefix |= d << shift;
        count_ge = above_total + in_bin;
    }
    if (count_gt) *count_gt = above_total;
    return prefix;
}

// The same over the tokens [t0, t1) of a slice with keys key_of(t).
template <typename KeyFn>
__device__ __forceinline__ uint32_t radix_threshold_fn(uint32_t t0, uint32_t t1, uint32_t k, uint32_t *s_hist, uint32_t *s_sel,
                                       uint32_t &count_ge, KeyFn key_of, uint32_t *count_gt = nullptr) {
    const uint32_t tid = threadIdx.x;
    auto visit = [&](auto &&fn) __attribute__((always_inline)) {
        // 8 keys per lane and round, all computed before any count
        for (uint32_t t = t0 + tid; t < t1; t += 8u * kBlock) {
            uint32_t x[8];
#pragma unroll
            for (int u = 0; u < 8; ++u) {
                const uint32_t tt = t + (uint32_t)u * kBlock;
                x[u] = tt < t1 ? key_of(tt) : 0u;
            }
#pragma unroll
            for (int u = 0; u < 8; ++u) fn(x[u]);
        }
    };
    return radix_threshold_visit(k, s_hist, s_sel, count_ge, visit, count_gt);
}

// ---- the fused kernel -------------------------------------------------------

struct SharedSmall {
    uint32_t hist[256];
    uint32_t sel[4];
    uint32_t scan[kWaves];
    uint64_t red[kWaves];
    uint32_t flag[4];
    uint32_t ones[1];  // all-ones mask word of rows without a mask
    uint32_t io[4];                  // the row's RowIo, stored during the set-up
    uint32_t ukeys[2][kWaves * 64];  // report unions of the two threshold passes
    uint32_t ucount[2][kWaves];
    uint32_t uthr[2];
    float u;  // the row's uniform draw
};

__device__ __forceinline__ uint32_t xcd_remap(uint32_t b, uint32_t n) {
    // Workgroups are dispatched round-robin over the 8 XCDs; give each XCD a
    // contiguous run of logical ids so the slices of a row share one L2.
    const uint32_t q = n / 8u, rem = n % 8u;
    const uint32_t xcd = b % 8u, idx = b / 8u;
    return xcd < rem ? xcd * (q + 1u) + idx : rem * (q + 1u) + (xcd - rem) * q + idx;
}

// Per-row draw inputs, read at kernel start so their latency hides behind
// the stream: the seed, the tick (stream control words 1-2, else the step),
// and the output ring capacity (stream control word 4).
struct RowIo {
    uint32_t seed, tick_lo, tick_hi, ring_cap;
};

// Per-row inputs are read with vector buffer loads: their completion is
// tracked by the in-order vector-memory counter, so waiting for them never
// waits for the logits issued after them (scalar or flat loads share a
// counter with the kernel-argument loads and would be waited for before the
// stream starts), and a null pointer becomes a zero-size buffer that reads 0
// with no branch.
__device__ __forceinline__ __amdgpu_buffer_rsrc_t small_rsrc(const void *p, uint32_t bytes) {
    return __builtin_amdgcn_make_buffer_rsrc((void *)p, (short)0, p ? (int)bytes : 0, 0x00020000);
}

// The per-row inputs as issued at kernel start: lane i of each word holds
// word i of its record, so nothing is uniform for the compiler to move into
// scalar registers at once (which would wait for the loads before the logits
// are issued); lane_word() takes the words out after the stream has started.
struct RowLoads {
    uint32_t params;  // lanes 0-7: nerve_sampler_row_params
    uint32_t sc;      // lanes 0-4: stream control words
    uint32_t steps;   // lanes 0-1: steps[row] (low, high)
    uint32_t seed;    // lane 0
    uint32_t hlen;    // lane 0: history_len[row]
};

__device__ __forceinline__ RowLoads issue_row_loads(const StepArgs &a, uint32_t row, uint32_t lane) {
    RowLoads l;
    const uint32_t w8 = (lane & 7u) * 4u, w2 = (lane & 1u) * 4u;
    l.params = __builtin_amdgcn_raw_buffer_load_b32(small_rsrc(a.params + row, 32u), w8, 0, 0);
    l.sc = __builtin_amdgcn_raw_buffer_load_b32(
        small_rsrc(a.stream_control ? a.stream_control + (uint64_t)row * 5u : nullptr, 20u), w8, 0, 0);
    l.steps = __builtin_amdgcn_raw_buffer_load_b32(small_rsrc(a.steps ? a.steps + row : nullptr, 8u), w2, 0, 0);
    l.seed = __builtin_amdgcn_raw_buffer_load_b32(small_rsrc(a.seeds ? a.seeds + row : nullptr, 4u), w2, 0, 0);
    l.hlen = __builtin_amdgcn_raw_buffer_load_b32(small_rsrc(a.history_len ? a.history_len + row : nullptr, 4u), w2, 0, 0);
    return l;
}

__device__ __forceinline__ uint32_t lane_word(uint32_t v, int i) { return (uint32_t)__builtin_amdgcn_readlane((int)v, i); }

__device__ __forceinline__ nerve_sampler_row_params row_params_of(const RowLoads &l) {
    nerve_sampler_row_params p;
    p.method = lane_word(l.params, 0);
    p.temperature = u2f(lane_word(l.params, 1));
    p.top_k = lane_word(l.params, 2);
    p.top_p = u2f(lane_word(l.params, 3));
    p.min_p = u2f(lane_word(l.params, 4));
    p.repetition_penalty = u2f(lane_word(l.params, 5));
    p.frequency_penalty = u2f(lane_word(l.params, 6));
    p.presence_penalty = u2f(lane_word(l.params, 7));
    return p;
}

// Draw inputs: the seed, the tick (stream control words 1-2, else the
// step), and the output ring capacity (stream control word 4).
__device__ __forceinline__ RowIo row_io_of(const StepArgs &a, const RowLoads &l, uint32_t row) {
    RowIo io;
    io.seed = lane_word(l.seed, 0);
    io.tick_lo = a.stream_control ? lane_word(l.sc, 1) : lane_word(l.steps, 0);
    io.tick_hi = a.stream_control ? lane_word(l.sc, 2) : lane_word(l.steps, 1);
    if (a.flags & NERVE_BATCH_CONSECUTIVE_TICKS) {
        // consecutive ticks of sample_batch: tick_base + row
        const uint64_t t = a.tick_base + row;
        io.tick_lo = (uint32_t)t;
        io.tick_hi = (uint32_t)(t >> 32);
    }
    io.ring_cap = lane_word(l.sc, 4);
    return io;
}

__device__ __forceinline__ RowIo load_row_io(const StepArgs &a, uint32_t row) {
    return row_io_of(a, issue_row_loads(a, row, lane_id()), row);
}

// Finishes one row from its sorted survivors s_sorted[0 .. n) (value desc,
// id asc): EOS fallback for an all-zero mask, the greedy record (replaying the
// reference's 1024-lane argmax when the row holds a NaN), or min-p / top-p over
// the k survivors and the draw (temperature_top_k_top_p_sampler_f32:157-216).
// Writes the output record, optional survivors / probabilities, the stream
// control tick and the output ring. Runs on NT threads; wave 0 does the
// sequential running sums.
// A candidate (order key, token id) as one unsigned 64-bit value, key in the
// high word and the complemented id in the low word: a larger value is a
// better entry (larger key, then smaller id), and 0 ranks below every
// candidate (candidate keys are nonzero).
__device__ __forceinline__ uint64_t cand_pack(uint32_t key, uint32_t id) { return ((uint64_t)key << 32) | (uint64_t)(~id); }
__device__ __forceinline__ uint2 cand_entry(uint64_t p) { return make_uint2((uint32_t)(p >> 32), ~(uint32_t)p); }

// Sum of r over each aligned group of 8 lanes, valid in the group's first
// lane (row shifts toward lower lanes: dpp_ctrl 0x101/0x102/0x104 are
// row_shl:1/2/4; lanes past a row's end read 0).
__device__ __forceinline__ uint32_t group8_sum(uint32_t r) {
    r += (uint32_t)__builtin_amdgcn_update_dpp(0, (int)r, 0x101, 0xf, 0xf, true);
    r += (uint32_t)__builtin_amdgcn_update_dpp(0, (int)r, 0x102, 0xf, 0xf, true);
    r += (uint32_t)__builtin_amdgcn_update_dpp(0, (int)r, 0x104, 0xf, 0xf, true);
    return r;
}

// Running sums of one wave's lane values in sequential order: lane l gets
// (((c + w_0) + w_1) + ... + w_l), rounded after every add exactly as a
// sequential loop rounds. Each step adds a lane's own value to the sum of its
// left neighbour (a wavefront shift by one lane; lane 0 reads c), so the sum
// of lane l is final after l steps and unchanged by later ones. Lanes at or
// past `len` hold partial sums.
__device__ __forceinline__ float sequential_prefix(float w, float c, uint32_t len) {
    float acc = c + w;
    // steps in groups of 8 (steps past len - 1 change no final sum)
    for (uint32_t step = 1; step < len; step += 8u) {
        static_for<0, 8>([&](auto) __attribute__((always_inline)) {
            // dpp_ctrl 0x138: wave_shr:1 (lane l reads lane l - 1; lane 0 keeps `old`)
            const float left = u2f((uint32_t)__builtin_amdgcn_update_dpp((int)f2u(c), (int)f2u(acc), 0x138, 0xf, 0xf, false));
            acc = left + w;
        });
    }
    return acc;
}

template <typename Elem, int PEN, int NT>
__device__ __forceinline__ void finish_row(const StepArgs &a, uint32_t row, const RowIo &io, const nerve_sampler_row_params &P, uint32_t k,
                           bool sampled, uint32_t n, uint32_t row_flags, uint2 *s_sorted, uint2 *s_big,
                           float *s_w, float *s_p, uint32_t *s_hash, const RowCtx &ctx, float u) {
    // s_w [kcap]: weights, zero past the min-p cut (more than 64 survivors)
    // s_p [kcap]: running sums, then probabilities.
    const uint32_t tid = threadIdx.x;
    uint32_t token = 0, sel_bits = 0, out_flags = 0, kout = 1;
    uint32_t *sc = a.stream_control ? a.stream_control + (uint64_t)row * 5u : nullptr;

    const bool eos = a.allowed && !(row_flags & 1u);
    if (eos) {
        token = a.eos;
        sel_bits = 0xff800000u;  // -inf: every token was masked
        out_flags = NERVE_FLAG_EOS_FALLBACK | (sampled ? NERVE_FLAG_SAMPLED : 0u);
        if (tid == 0) s_p[0] = 1.0f;
    } else if (!sampled) {
        if (row_flags & 2u) {
            // A NaN in the row: replay the reference lane structure exactly
            // (greedy_sampler_f32:52-83), with penalties for the whole row:
            // the caller's state when it covers the row (a bitmap probe per
            // token, the table only for penalised ones), else the history's
            // full counts rebuilt in the table.
            RowCtx full = ctx;
            if (!ctx.whole_row) {
                if constexpr (PEN == 2) {
                    for (uint32_t i = tid; i < a.hash_slots; i += NT) s_hash[i] = kHashEmpty;
                    __syncthreads();
                    uint32_t len = a.history_len[row];
                    len = len > a.history_stride ? a.history_stride : len;
                    const uint32_t *hrow = a.history + (uint64_t)row * a.history_stride;
                    for (uint32_t i = tid; i < len; i += NT)
                        if (hrow[i] < a.vocab) hash_insert(s_hash, a.log2_slots, hrow[i]);
                }
                full.bitmap = nullptr;
            }
            __syncthreads();
            uint2 *slots = s_big;  // 1024 entries of (float bits, id)
            // The thread's reference lanes L = tid + NT q advance together,
            // 8 strides of each loaded before any is compared. A lane whose
            // first value is NaN keeps it (no comparison with NaN succeeds);
            // the others visit their values in order.
            constexpr int Q = 1024 / NT;
            float best[Q];
            uint32_t bid[Q];
#pragma unroll
            for (int q = 0; q < Q; ++q) {
                const uint32_t L = tid + (uint32_t)q * NT;
                bid[q] = L;
                best[q] = L < a.vocab ? configured_at<Elem>(full, L) : u2f(kLowestBits);
            }
            for (uint32_t t0 = 1024u; t0 < a.vocab; t0 += 8u * 1024u) {
                // raw values first (no control flow between the loads), then
                // the penalties from registers
                float c[Q][8];
#pragma unroll
                for (int q = 0; q < Q; ++q)
#pragma unroll
                    for (int u = 0; u < 8; ++u) {
                        const uint32_t t = t0 + tid + (uint32_t)q * NT + (uint32_t)u * 1024u;
                        c[q][u] = load_elem<Elem>((const Elem *)full.logits_row, t < a.vocab ? t : 0u);
                    }
#pragma unroll
                for (int q = 0; q < Q; ++q)
#pragma unroll
                    for (int u = 0; u < 8; ++u) {
                        const uint32_t t = t0 + tid + (uint32_t)q * NT + (uint32_t)u * 1024u;
                        c[q][u] = t < a.vocab ? configured_from(full, t, c[q][u]) : u2f(kLowestBits);
                    }
#pragma unroll
                for (int q = 0; q < Q; ++q)
#pragma unroll
                    for (int u = 0; u < 8; ++u) {
                        const uint32_t t = t0 + tid + (uint32_t)q * NT + (uint32_t)u * 1024u;
                        if (t < a.vocab && float_better(c[q][u], t, best[q], bid[q])) {
                            best[q] = c[q][u];
                            bid[q] = t;
                        }
                    }
            }
#pragma unroll
            for (int q = 0; q < Q; ++q) slots[tid + (uint32_t)q * NT] = make_uint2(f2u(best[q]), bid[q]);
            __syncthreads();
            for (uint32_t stride = 512u; stride > 0u; stride >>= 1) {
                for (uint32_t L = tid; L < stride; L += NT) {
                    const uint2 c = slots[L + stride], b = slots[L];
                    if (float_better(u2f(c.x), c.y, u2f(b.x), b.y)) slots[L] = c;
                }
                __syncthreads();
            }
            token = slots[0].y;
            sel_bits = slots[0].x;
        } else {
            const uint2 e = s_sorted[0];
            if (e.x == kNegInfKey && a.vocab < 1024u) {
                // every token is -inf: the shader's padded lane V (LOWEST_FLOAT) wins
                token = a.vocab;
                sel_bits = kLowestBits;
            } else {
                token = e.y & kIdMask;
                sel_bits = f2u(entry_value(e));
            }
        }
        if (tid == 0) s_p[0] = 1.0f;
    } else if (tid < 64) {
        // Sampled rows: wave 0 finishes alone (no block barriers). Entries
        // past the n candidates are padding (the lowest finite value, an
        // invalid id).
        const uint32_t lane = tid;
        const uint2 pad = make_uint2(kMinFiniteKey, kPadId);
        const float T = P.temperature;
        const float l0 = entry_value(n ? s_sorted[0] : pad);
        const float m = l0 / T;
        float minimum = u2f(kLowestBits);
        if (P.min_p > 0.0f) {
            const float lg = nerve_logf(P.min_p);
            const float d = T * lg;
            minimum = l0 + d;
        }
        // The min-p cut (the first survivor below the floor ends the list),
        // then running sums in the reference's sequential order.
        uint32_t n_valid = k, nucleus, selected;
        float nucleus_weight;
        if (k <= 64u) {
            // one survivor per lane: values, weights and sums in registers
            const bool live = lane < k;
            const uint2 ev = lane < n ? s_sorted[lane] : pad;
            const float v = live ? entry_value(ev) : 0.0f;
            const uint64_t below = __ballot(live && v < minimum);
            if (below) n_valid = (uint32_t)__builtin_ctzll(below);
            float w = 0.0f;
            if (lane < n_valid) w = nerve_expf(v / T - m);
            const float acc = sequential_prefix(w, 0.0f, n_valid);
            const float total = n_valid ? u2f(__builtin_amdgcn_readlane(f2u(acc), (int)(n_valid - 1u))) : 0.0f;
            const float threshold = P.top_p * total;
            const uint64_t bn = __ballot(lane < n_valid && acc >= threshold);
            nucleus = bn ? (uint32_t)__builtin_ctzll(bn) + 1u : n_valid;
            if (nucleus == 0u) nucleus = 1u;
            nucleus_weight = n_valid ? u2f(__builtin_amdgcn_readlane(f2u(acc), (int)(nucleus - 1u))) : 0.0f;
            const float target = u * nucleus_weight;
            const uint64_t bs = __ballot(lane < nucleus && lane < n_valid && target < acc);
            selected = bs ? (uint32_t)__builtin_ctzll(bs) : nucleus - 1u;
            if (a.topk_probs && live) s_p[lane] = (lane < nucleus && lane < n_valid) ? w / nucleus_weight : 0.0f;
            // the selected survivor is in lane `selected`
            const uint32_t sid = __builtin_amdgcn_readlane(ev.y, (int)selected);
            token = sid == kPadId ? kPadId : (sid & kIdMask);
            sel_bits = __builtin_amdgcn_readlane(f2u(v), (int)selected);
        } else {
            // chunks of 64 survivors: s_w holds the weights (zero past the
            // cut), s_p the running sums
            for (uint32_t i = n + lane; i < k; i += 64u) s_sorted[i] = pad;
            float carry = 0.0f;  // P_(c0 - 1)
            for (uint32_t c0 = 0; c0 < n_valid; c0 += 64u) {
                const uint32_t i = c0 + lane;
                const float v = i < k ? entry_value(s_sorted[i]) : 0.0f;
                const uint64_t below = __ballot(i < k && v < minimum);
                if (below) n_valid = min(n_valid, c0 + (uint32_t)__builtin_ctzll(below));
                if (c0 >= n_valid) break;
                const bool in = i < n_valid;
                float w = 0.0f;
                if (in) w = nerve_expf(v / T - m);
                if (i < k) s_w[i] = w;
                const uint32_t len = min(64u, n_valid - c0);
                const float acc = sequential_prefix(w, carry, len);
                s_p[i] = acc;
                carry = u2f(__builtin_amdgcn_readlane(f2u(acc), (int)(len - 1u)));
            }
            const float total = n_valid ? carry : 0.0f;
            const float threshold = P.top_p * total;
            nucleus = n_valid;
            for (uint32_t c0 = 0; c0 < n_valid; c0 += 64u) {
                const uint32_t i = c0 + lane;
                const uint64_t b = __ballot(i < n_valid && s_p[i] >= threshold);
                if (b) {
                    nucleus = c0 + (uint32_t)__builtin_ctzll(b) + 1u;
                    break;
                }
            }
            if (nucleus == 0u) nucleus = 1u;
            nucleus_weight = n_valid ? s_p[nucleus - 1u] : 0.0f;
            const float target = u * nucleus_weight;
            selected = nucleus - 1u;
            for (uint32_t c0 = 0; c0 < nucleus && c0 < n_valid; c0 += 64u) {
                const uint32_t i = c0 + lane;
                const uint64_t b = __ballot(i < nucleus && i < n_valid && target < s_p[i]);
                if (b) {
                    selected = c0 + (uint32_t)__builtin_ctzll(b);
                    break;
                }
            }
            for (uint32_t i = lane; i < k; i += 64u)
                s_p[i] = (i < nucleus && i < n_valid) ? s_w[i] / nucleus_weight : 0.0f;
            const uint2 e = s_sorted[selected];
            token = e.y == kPadId ? kPadId : (e.y & kIdMask);
            sel_bits = f2u(entry_value(e));
        }
        out_flags = NERVE_FLAG_SAMPLED;
        kout = k;
    }

    if (tid == 0) {
        nerve_sampler_output o;
        o.token_id = token;
        o.selected_logit_bits = sel_bits;
        o.flags = out_flags;
        o.reserved = 0u;
        a.out[row] = o;
        if (sc) {
            const uint32_t lo = io.tick_lo;
            if (a.ring) {
                uint32_t *ring = a.ring + (uint64_t)row * a.ring_stride;
                const uint32_t cap = io.ring_cap;
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
            if (next == 0u) sc[2] = io.tick_hi + 1u;
            sc[1] = next;
        }
        if ((a.flags & NERVE_BATCH_APPEND_HISTORY) && token < a.vocab) {
            // the sampled token joins the row's penalty state for the next step
            if (a.history) {
                const uint32_t len = a.history_len[row];
                a.history[(uint64_t)row * a.history_stride + len % a.history_stride] = token;
                a.history_len[row] = len + 1u;
            } else if (a.seen) {
                atomicOr(&a.seen[(uint64_t)row * a.seen_stride + (token >> 5)], 1u << (token & 31u));
            }
        }
        if (a.feedback_control) {
            // commit_feedback_control (greedy_sampler_f32.comp.template:35-50)
            uint32_t *fc = a.feedback_control + (uint64_t)row * a.feedback_stride;
            const uint32_t fl = __hip_atomic_load(&fc[0], __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            if (fl & NERVE_FEEDBACK_ENABLED) {
                atomicAdd(&fc[9], 1u);
                const bool cancelled = (fl & NERVE_FEEDBACK_CANCEL_REQUESTED) != 0u;
                const uint32_t *stop = a.stop_tokens ? a.stop_tokens + (uint64_t)row * a.stop_stride : nullptr;
                const bool eos = stop && token < a.vocab && ((stop[token >> 5] >> (token & 31u)) & 1u);
                if (cancelled || eos) {
                    if (atomicCAS(&fc[2], 0u, cancelled ? NERVE_STOP_REASON_CANCELLED : NERVE_STOP_REASON_EOS) == 0u)
                        __hip_atomic_store(&fc[8], 2u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
                }
            }
        }
    }
    if (a.topk_ids || a.topk_logits || a.topk_probs) {
        if (sampled && !eos) kout = k;  // set by wave 0 only
        __syncthreads();                // s_p is written by wave 0
        for (uint32_t i = tid; i < a.kcap; i += NT) {
            const uint64_t o = (uint64_t)row * a.kcap + i;
            const bool live = i < kout;
            float value = u2f(kLowestBits);
            uint32_t id = kPadId;
            if (live && i == 0 && (eos || !sampled)) {
                value = eos ? u2f(kLowestBits) : u2f(sel_bits);
                id = token;
            } else if (live) {
                const uint2 e = i < n ? s_sorted[i] : make_uint2(kMinFiniteKey, kPadId);
                value = entry_value(e);
                id = e.y == kPadId ? kPadId : (e.y & kIdMask);
            }
            if (a.topk_ids) a.topk_ids[o] = id;
            if (a.topk_logits) a.topk_logits[o] = value;
            if (a.topk_probs) a.topk_probs[o] = live ? s_p[i] : 0.0f;
        }
    }
}

// Defined after the slice kernel, which uses them for the last slice of a row.
template <int NT, typename LoadEntry, typename LoadMeta>
__device__ __forceinline__ uint32_t merge_slices(const StepArgs &a, uint32_t k, uint2 *s_big, uint2 *s_sorted,
                                                 uint32_t *s_meta, uint32_t &row_flags, LoadEntry load_entry,
                                                 LoadMeta load_meta);
template <typename Elem, int PEN>
__device__ __forceinline__ RowCtx row_ctx(const StepArgs &a, uint32_t row, const nerve_sampler_row_params &P,
                                          uint32_t *s_hash);

constexpr uint32_t kStageCap = 1024;       // lane-vectors staged for exact work per slice

constexpr uint32_t kStreamCandCap = 2048;  // candidate entries per slice

// Bytes of the staging area (lane-vectors and their slots).
template <typename Elem, int EPV>
__host__ __device__ constexpr uint32_t stage_area_bytes() {
    return kStageCap * ((uint32_t)sizeof(typename VecTraits<Elem, EPV>::load_t) + 4u);
}

// Bitmap words of a slice: its tokens [tok0, tok1) rounded out to 32-token
// words, plus slack; the host sizes the LDS bitmaps with the same bound.
__host__ __device__ constexpr uint32_t slice_bitmap_words(uint32_t tokens, uint32_t epv) {
    return (tokens + epv + 62u) / 32u + 1u;
}

// PEN: 0 = no penalty state, 1 = seen bitmap (set semantics), 2 = history ids
// (count semantics). EPV elements per lane-vector, NV lane-vectors per lane.
//
// The slice [v0, v1) of full lane-vectors lives in VGPRs: wave w owns a run
// of `span` slots, and lane-vector j of lane l is the slot 64 * j + l of that
// run. Loads run D lane-vectors ahead of the processing:
//   pass 1  as the loads land, two signed-integer maxima per lane over the raw
//           values of fully allowed lane-vectors; each report is a real
//           element of the slice;
//   select  after the first half: every wave's top reports go to an LDS union
//           and its k-th largest key becomes thr;
//   pass 2  lane-vectors whose raw maximum reaches thr are staged in LDS;
//   exact   four lanes per staged lane-vector compute the configured keys
//           (mask, penalties) and append keys >= thr to the candidate list;
//   rank    a rank sort of the candidates writes the top k in order;
//   finish  wave 0: weights, sequential running sums, nucleus, draw, record.
// The top k are all candidates exactly when at least k configured keys reach
// thr; a slice where penalties pushed too many reported values below thr
// takes the exact selection from memory instead. Penalties that never raise
// a logit (repetition >= 1, frequency and presence >= 0) keep configured <=
// raw, so the raw test of pass 2 is conservative for penalised tokens too.
// Other settings take penalised tokens out of the vector passes and evaluate
// each one from the history state instead (one gather per id).
template <typename Elem, int EPV, int NV, int PEN, bool MASK, int AUX>
__global__ __launch_bounds__(kBlock) void sample_rows_kernel(StepArgs a) {
    constexpr int HPT = (kMaxHistory + kBlock - 1) / kBlock;  // history ids per lane
    constexpr int BW = (int)((slice_bitmap_words((uint32_t)kBlock * NV * EPV, EPV) + kBlock - 1u) / kBlock);
    constexpr int LW = (NV + 31) / 32;
    constexpr uint32_t kFull = EPV == 32 ? 0xffffffffu : ((1u << EPV) - 1u);
    constexpr bool history = PEN == 2;
    using VT = VecTraits<Elem, EPV>;
    using vec_t = typename VT::load_t;
    constexpr uint32_t kVecBytes = (uint32_t)sizeof(vec_t);
    __shared__ SharedSmall sm;
    extern __shared__ __align__(16) uint32_t s_dyn[];
    uint32_t *s_hash = s_dyn;                                      // [hash_slots], a multiple of 64
    vec_t *s_svec = (vec_t *)(s_hash + a.hash_slots);              // [kStageCap]
    uint32_t *s_sslot = (uint32_t *)(s_svec + kStageCap);          // [kStageCap]
    uint64_t *s_cand = (uint64_t *)(s_sslot + kStageCap);          // [kStreamCandCap] packed, later finish scratch
    uint2 *s_sorted = (uint2 *)(s_cand + kStreamCandCap);          // [kcap]
    uint32_t *s_pen = (uint32_t *)(s_sorted + a.kcap);             // [bitmap_words] when PEN != 0
    uint32_t *s_allow = s_pen + (PEN != 0 ? a.bitmap_words : 0u);  // [bitmap_words] with a mask
    uint2 *s_big = (uint2 *)s_cand;

    const uint32_t tid = threadIdx.x;
    const uint32_t logical = xcd_remap(blockIdx.x, gridDim.x);
    const uint32_t row = logical / a.slices;
    const uint32_t slice = logical % a.slices;

    const uint32_t nfull = a.nvec;
    const uint32_t v0 = min(slice * a.vec_per_slice, nfull);
    const uint32_t v1 = min(v0 + a.vec_per_slice, nfull);
    const bool last_slice = slice == a.slices - 1u;
    const uint32_t tok0 = v0 * EPV;
    const uint32_t tok1 = last_slice ? a.vocab : v1 * EPV;
    const uint32_t bm_base = tok0 & ~31u;
    const uint32_t bm_n = tok1 > tok0 ? ((tok1 - 1u) >> 5) - (bm_base >> 5) + 1u : 0u;
    const uint32_t tail_id = nfull * EPV + tid;
    const bool has_tail = last_slice && tail_id < a.vocab;

    const Elem *lrow = (const Elem *)a.logits + (uint64_t)row * a.ld;
    // 1. loads. The small per-row inputs first (parameters, draw inputs,
    // history ids and the slice's bitmap words), so the set-up finds them
    // landed, and without any wait before the logits are issued; then the
    // first D lane-vectors through a buffer resource bounded by the wave's
    // valid run. A wave owns a run of consecutive slots, so the loads of a
    // lane sit 64 slots apart and share one offset register per 4 KiB.
    const uint32_t lane = lane_id();
    const RowLoads rl = issue_row_loads(a, row, lane);
    const uint32_t wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    // the slice is spread evenly: wave w owns `span` slots from w * span
    const uint32_t span = ((a.vec_per_slice + (uint32_t)kBlock - 1u) / (uint32_t)kBlock) * 64u;
    const uint32_t wslots = v1 - v0 > wave * span ? min(span, v1 - v0 - wave * span) : 0u;  // valid slots of the wave
    const uint32_t wbase = wave * span + lane;  // slot of lane-vector 0, relative to v0
    // per-wave buffer resource: a load past the wave's valid run reads zero
    // and costs no memory traffic
    const __amdgpu_buffer_rsrc_t rsrc = __builtin_amdgcn_make_buffer_rsrc(
        (void *)(lrow + (uint64_t)(v0 + wave * span) * EPV), (short)0, (int)(wslots * kVecBytes), 0x00020000);
    constexpr bool mask = MASK;  // an allowed-token bitmask is present
    const uint32_t *arow = mask ? a.allowed + (uint64_t)row * a.allowed_stride : nullptr;
    const uint32_t *srow = PEN == 1 ? a.seen + (uint64_t)row * a.seen_stride : nullptr;
    uint32_t hist[history ? HPT : 1];
    uint32_t hlen = 0;
    if constexpr (history) {
        const uint32_t *hrow = a.history + (uint64_t)row * a.history_stride;
        const uint32_t hlast = a.history_stride - 1u;
#pragma unroll
        for (int h = 0; h < HPT; ++h) hist[h] = hrow[min(tid + (uint32_t)h * kBlock, hlast)];
    }
    const uint32_t bm_last = bm_n ? bm_n - 1u : 0u;
    uint32_t mw[BW];
    if (mask) {
#pragma unroll
        for (int i = 0; i < BW; ++i) mw[i] = arow[(bm_base >> 5) + min(tid + (uint32_t)i * kBlock, bm_last)];
    }
    uint32_t sw[PEN == 1 ? BW : 1];
    uint32_t pid = 0xffffffffu;  // seen-state prefix token of this lane (wave 0), if any
    if constexpr (PEN == 1) {
#pragma unroll
        for (int i = 0; i < BW; ++i) sw[i] = srow[(bm_base >> 5) + min(tid + (uint32_t)i * kBlock, bm_last)];
        if (a.prefix_ids && tid < prefix_count(a, row)) pid = a.prefix_ids[(uint64_t)row * a.prefix_stride + tid];
    }

    vec_t data[NV];
    // AUX: cache policy of the stream's loads (kLoadNT or 0)
    auto load = [&](int j) __attribute__((always_inline)) {
        const uint32_t off = (lane + (uint32_t)j * 64u) * kVecBytes;
        if constexpr (kVecBytes == 16) data[j] = __builtin_amdgcn_raw_buffer_load_b128(rsrc, off, 0, AUX);
        else if constexpr (kVecBytes == 4) data[j] = u2f(__builtin_amdgcn_raw_buffer_load_b32(rsrc, off, 0, AUX));
        else data[j] = __builtin_amdgcn_raw_buffer_load_b16(rsrc, off, 0, AUX);
    };
    // lane-vectors in flight ahead of the one being processed
#ifndef NERVE_LOOKAHEAD
#define NERVE_LOOKAHEAD 5
#endif
    constexpr int D = NV < NERVE_LOOKAHEAD ? NV : NERVE_LOOKAHEAD;
    static_for<0, D>([&](auto J) __attribute__((always_inline)) { load(J); });

    const nerve_sampler_row_params P = row_params_of(rl);
    const RowIo io = row_io_of(a, rl, row);
    if constexpr (history) hlen = min(lane_word(rl.hlen, 0), a.history_stride);
    const bool sampled = P.method != NERVE_METHOD_GREEDY;
    uint32_t k = sampled ? P.top_k : 1u;
    k = k < 1u ? 1u : (k > a.kcap ? a.kcap : k);
    const uint32_t valid_min = sampled ? kMinFiniteKey : kNegInfKey;
    const uint32_t masked_key = sampled ? 0u : kNegInfKey;
    const bool lowering = P.repetition_penalty >= 1.0f && P.frequency_penalty >= 0.0f && P.presence_penalty >= 0.0f;

    // 2. LDS state: counters, mask / seen words of the slice (bits outside
    // [tok0, tok1) cleared); history ids -> bitmap, and repeats -> a table of
    // occurrences beyond the first
    if constexpr (history) {
        const uint4 empty4 = make_uint4(kHashEmpty, kHashEmpty, kHashEmpty, kHashEmpty);
        for (uint32_t i = tid; i < a.hash_slots / 4u; i += kBlock) ((uint4 *)s_hash)[i] = empty4;
        // the bitmap is 8-byte aligned: zero it in pairs of words
        for (uint32_t i = tid; i < bm_n / 2u; i += kBlock) ((uint2 *)s_pen)[i] = make_uint2(0u, 0u);
        if ((bm_n & 1u) && tid == 0) s_pen[bm_n - 1u] = 0u;
    }
    // the candidate list reads as zero past its end (the rank sort's padding)
    if (tid < kRankPad) s_cand[tid] = 0u;
    if (tid == 0) {
        sm.flag[1] = 0u;  // candidates
        sm.flag[2] = 0u;  // staged lane-vectors
        sm.flag[3] = 0u;  // slice flags
        sm.ones[0] = 0xffffffffu;
        sm.io[0] = io.seed;
        sm.io[1] = io.tick_lo;
        sm.io[2] = io.tick_hi;
        sm.io[3] = io.ring_cap;
    }
    auto range_bits = [&](uint32_t w) __attribute__((always_inline)) -> uint32_t {
        const uint32_t t = bm_base + w * 32u;
        uint32_t m = 0xffffffffu;
        if (t < tok0) m &= 0xffffffffu << (tok0 - t);
        if (t + 32u > tok1) m &= (tok1 - t) >= 32u ? 0xffffffffu : ((1u << (tok1 - t)) - 1u);
        return m;
    };
    uint32_t any_allowed = mask ? 0u : (tok1 > tok0 ? 1u : 0u);
    if (mask) {
#pragma unroll
        for (int i = 0; i < BW; ++i) {
            const uint32_t w = tid + (uint32_t)i * kBlock;
            if (w < bm_n) {
                const uint32_t v = mw[i] & range_bits(w);
                s_allow[w] = v;
                any_allowed |= v ? 1u : 0u;
            }
        }
    }
    lds_sync();
    // the uniform draw depends only on the seed and tick: one wave computes it
    // now, off the finish's critical path
    if (sampled && wave == 1u) {
        const float uu = random_unit(a.rng, io.seed, (uint64_t)io.tick_lo | ((uint64_t)io.tick_hi << 32), row);
        if (lane == 0u) sm.u = uu;
    }
    // The penalty state (seen words, or history ids -> bitmap + repeat table)
    // is needed only by the exact pass after the stream, so it is built at the
    // midpoint of the stream, when its loads have long landed.
    auto build_penalty_state = [&]() __attribute__((always_inline)) {
        if constexpr (PEN == 1) {
#pragma unroll
            for (int i = 0; i < BW; ++i) {
                const uint32_t w = tid + (uint32_t)i * kBlock;
                if (w < bm_n) s_pen[w] = sw[i] & range_bits(w);
            }
            if (a.prefix_ids) {
                // the lane's prefix token, after every word is stored (the
                // barrier before the exact pass makes it visible)
                lds_sync();
                if (pid >= tok0 && pid < tok1) atomicOr(&s_pen[(pid - bm_base) >> 5], 1u << ((pid - bm_base) & 31u));
            }
        }
    };
    // history id h of this lane -> bitmap; a repeat (its bit already set) ->
    // the table of occurrences beyond the first. One id per first-half step,
    // so the LDS round trips overlap the loads in flight.
    auto insert_history = [&](int h) __attribute__((always_inline)) {
        if constexpr (history) {
            const uint32_t id = hist[h];
            if (tid + (uint32_t)h * kBlock < hlen && id >= tok0 && id < tok1) {
                const uint32_t o = id - bm_base, bit = 1u << (o & 31u);
                if (atomicOr(&s_pen[o >> 5], bit) & bit) hash_insert(s_hash, a.log2_slots, id);
            }
        }
    };

    // 3. the stream. Lane-vector j is processed as it lands while lane-vector
    // j + D is issued. With a mask, per group of 8: the flags from the mask
    // bitmap (ok = every element valid and allowed; live = some element valid
    // and allowed); without one, every valid lane-vector is ok and live. Pass
    // 1 folds the raw values of ok lane-vectors into the lane reports. After
    // the first half, thr is set from the reports so far and pass 2 stages
    // every lane-vector that can hold a key >= thr, first-half ones included.
    // Raw reports ignore penalties, so thr is a guess, checked after the exact
    // pass: the top k are all candidates exactly when at least k keys reach
    // thr; otherwise the slice takes the exact selection from memory.
    const uint32_t nval = wslots > lane ? (wslots - lane + 63u) / 64u : 0u;  // valid lane-vectors of this lane
    uint32_t okm[LW], live[LW], vmask[LW];
#pragma unroll
    for (int i = 0; i < LW; ++i) {
        const uint32_t lo = (uint32_t)i * 32u;
        const uint32_t n = nval > lo ? min(nval - lo, 32u) : 0u;
        vmask[i] = n >= 32u ? 0xffffffffu : ((1u << n) - 1u);  // valid lane-vectors
        okm[i] = vmask[i];
        live[i] = vmask[i];
    }
    // Lane-vector j of this lane starts at bitmap bit tok_base + 64 * EPV * j:
    // the word moves by a constant (an immediate offset) and the bit position
    // stays put. The bitmaps are sized for NV full lane-vectors per lane, so
    // the reads of invalid ones stay inside them (their flags are masked).
    const uint32_t tok_base = (v0 + wbase) * EPV - bm_base;
    const uint32_t wsh = tok_base & 31u;
    const uint32_t *allow_w = s_allow + (tok_base >> 5);
    constexpr uint32_t kWordsPerJ = 64u * EPV / 32u;
    auto flags_group = [&](auto J0) __attribute__((always_inline)) {
        constexpr int j0 = decltype(J0)::value;
        uint32_t aw[8];
#pragma unroll
        for (int q = 0; q < 8; ++q) aw[q] = allow_w[(uint32_t)(j0 + q) * kWordsPerJ];
        uint32_t okg = 0u, lvg = 0u;
#pragma unroll
        for (int q = 0; q < 8; ++q) {
            const uint32_t ab = (aw[q] >> wsh) & kFull;
            okg |= ab == kFull ? (1u << q) : 0u;
            lvg |= ab != 0u ? (1u << q) : 0u;
        }
        const int sh = j0 & 31;
        okm[j0 >> 5] &= ~(0xffu << sh) | (okg << sh);
        live[j0 >> 5] &= ~(0xffu << sh) | (lvg << sh);
    };
    auto flags_at = [&](auto J0) __attribute__((always_inline)) {
        if constexpr (MASK) flags_group(J0);
    };
    uint32_t acc0 = VT::kAccInit, acc1 = VT::kAccInit;
    // vmx[j]: the raw signed-integer maximum of lane-vector j, computed once
    // by pass 1 and reused by pass 2
    uint32_t vmx[NV];
    auto pass1 = [&](int j) __attribute__((always_inline)) {
        vmx[j] = VT::vmax(data[j]);
        // branch-free: a lane-vector that is not ok contributes the empty marker
        const uint32_t sel = 0u - ((okm[j >> 5] >> (j & 31)) & 1u);
        const uint32_t vm = (vmx[j] & sel) | (VT::kAccInit & ~sel);
        if (j & 1) acc1 = VT::merge(acc1, vm);
        else acc0 = VT::merge(acc0, vm);
    };
    // Threshold from the reports. A lane reports the largest key among its
    // accumulated elements (itself an element of the slice). Every wave finds
    // the min(k, 64)-th largest report of its lanes by an MSB-first ballot
    // search over the top key bits and appends the reports at or above it to
    // an LDS union (at most 64 per wave); wave 0 takes the k-th largest of the
    // union the same way and publishes it. At least k elements of the slice
    // reach the result, and for k <= 64 it is the k-th largest report (to the
    // searched bits). 1 when the union has fewer than k.
    auto report_threshold = [&](int call) __attribute__((always_inline)) -> uint32_t {
        constexpr int kBits = sizeof(Elem) == 2 ? 16 : 24;
        uint32_t best[1] = {0u};
#pragma unroll
        for (int r = 0; r < VT::kReports; ++r) {
            const uint32_t b0 = VT::report_bits(acc0, r), b1 = VT::report_bits(acc1, r);
            uint32_t k0 = b0 == 0x80000000u ? 0u : raw_order_key(b0);
            uint32_t k1 = b1 == 0x80000000u ? 0u : raw_order_key(b1);
            k0 = k0 < valid_min ? 0u : k0;
            k1 = k1 < valid_min ? 0u : k1;
            best[0] = max(best[0], max(k0, k1));
        }
        const uint32_t tw = wave_kth<1, kBits>(best, min(k, 64u));
        const bool in = best[0] != 0u && best[0] >= tw;
        const uint64_t bal = __ballot(in);
        const uint32_t pos = __builtin_amdgcn_mbcnt_hi((uint32_t)(bal >> 32), __builtin_amdgcn_mbcnt_lo((uint32_t)bal, 0u));
        if (in) sm.ukeys[call][wave * 64u + pos] = best[0];
        if (lane == 0u) sm.ucount[call][wave] = (uint32_t)__popcll(bal);
        lds_sync();
        if (wave == 0u) {
            uint32_t uk[kWaves];
#pragma unroll
            for (int w = 0; w < kWaves; ++w) uk[w] = lane < sm.ucount[call][w] ? sm.ukeys[call][w * 64 + lane] : 0u;
            const uint32_t t = wave_kth<kWaves, kBits>(uk, k);
            if (lane == 0u) sm.uthr[call] = t < 1u ? 1u : t;
        }
        lds_sync();
        return sm.uthr[call];
    };
    uint32_t thr = 1u;
    bool fast = false, skip_dead = true;
    // Masked lane-vectors are skipped unless a masked token could still
    // qualify (greedy rows treat masked tokens as -inf); a positive thr is
    // tested on the raw signed-integer maximum.
    auto set_thr = [&](uint32_t t) __attribute__((always_inline)) {
        thr = t;
        fast = thr > kZeroKey;
        skip_dead = sampled || thr > kNegInfKey;
    };
    uint32_t has_nan = 0u;  // greedy rows: any NaN selects the reference's lane-structure replay
    // Pass 2 for lane-vector j with the threshold test fixed at compile time:
    // FAST for thr above +0 (raw signed-integer maximum), else the order-key
    // upper bound.
    auto pass2 = [&](auto fast_tag, int j) __attribute__((always_inline)) {
        constexpr bool FAST = decltype(fast_tag)::value;
        if (!sampled) has_nan |= ((uint32_t)j < nval && VT::has_nan(data[j])) ? 1u : 0u;
        bool go;
        if constexpr (FAST) {
            // thr > +0: a slot past the run (loaded as zero) never passes, so
            // without a mask the live flag adds nothing
            const bool lv = !MASK || ((live[j >> 5] >> (j & 31)) & 1u);
            go = lv && VT::ge_pos(vmx[j], thr);
        } else {
            const bool lv = skip_dead ? ((live[j >> 5] >> (j & 31)) & 1u) : ((uint32_t)j < nval);
            go = lv && VT::upper(data[j]) >= thr;
        }
        if (go) {
            const uint32_t pos = atomicAdd(&sm.flag[2], 1u);
            if (pos < kStageCap) {
                s_svec[pos] = data[j];
                s_sslot[pos] = v0 + wbase + (uint32_t)j * 64u;
            }
        }
    };
    constexpr int NA = NV / 2;
    static_assert(NV % 8 == 0, "lane-vector count must be a multiple of 8");
    auto step_in = [&](auto J) __attribute__((always_inline)) {
        constexpr int j = J;
        if constexpr (j + D < NV) load(j + D);
        if constexpr ((j & 7) == 0) flags_at(std::integral_constant<int, j>{});
        pass1(j);
        // without a mask, keep each load in its step: hoisting the first
        // half's loads (the compiler's choice) puts too many in flight and
        // slows the stream (measured; with a mask the hoisting pays)
        if constexpr (!MASK) __builtin_amdgcn_sched_barrier(0);
    };
    // history ids: one per step from step 2 of the first half, where a step
    // has the least other work (measured 0.15 us faster than in the second)
    constexpr int kInsertFrom = 2;
    static_for<0, NA>([&](auto J) __attribute__((always_inline)) {
        step_in(J);
        if constexpr (J >= kInsertFrom && J - kInsertFrom < HPT) insert_history(J - kInsertFrom);
    });
    set_thr(report_threshold(0));
    build_penalty_state();
    auto second_half = [&](auto fast_tag) __attribute__((always_inline)) {
        static_for<NA, NV>([&](auto J) __attribute__((always_inline)) {
            step_in(J);
            pass2(fast_tag, J - NA);
            pass2(fast_tag, J);
        });
    };
    if (fast) second_half(std::true_type{});
    else second_half(std::false_type{});
    if constexpr (history && NA - kInsertFrom < HPT) {
        // history ids left over when the first half has fewer steps
        static_for<NA - kInsertFrom, HPT>([&](auto H) __attribute__((always_inline)) { insert_history(H); });
    }
    // the V % EPV tail of the last slice, one element per lane (loaded late:
    // it is rare and holding it across the stream costs a VGPR)
    const uint32_t tail_bits = has_tail ? f2u(load_elem<Elem>(lrow, tail_id)) : 0u;
    if (!sampled) {
        if (has_tail) has_nan |= ((tail_bits & 0x7fffffffu) > 0x7f800000u) ? 1u : 0u;
        const float pq = P.repetition_penalty + P.frequency_penalty + P.presence_penalty;
        if (PEN != 0 && !(pq - pq == 0.0f)) has_nan = 1u;  // non-finite penalty parameters
    }
    lds_sync();
    uint32_t nstaged = sm.flag[2];
    uint32_t thr_stage = thr;  // the threshold the staged set was chosen with
    if (nstaged > kStageCap) {
        // The first half's threshold let too much through (a skewed row):
        // take the threshold of every report and stage again, reloading the
        // slice in chunks of 8 lane-vectors (the registers were released as
        // the stream went).
        set_thr(report_threshold(1));
        thr_stage = thr;
        if (tid == 0) sm.flag[2] = 0u;
        lds_sync();
        constexpr int CH = 8;
        auto restage = [&](auto fast_tag) __attribute__((always_inline)) {
            static_for<0, NV / CH>([&](auto C) __attribute__((always_inline)) {
                constexpr int j0 = C * CH, j1 = j0 + CH;
                static_for<j0, j1>([&](auto J) __attribute__((always_inline)) { load(J); });
                static_for<j0, j1>([&](auto J) __attribute__((always_inline)) {
                    vmx[J] = VT::vmax(data[J]);
                    pass2(fast_tag, J);
                });
            });
        };
        if (fast) restage(std::true_type{});
        else restage(std::false_type{});
        lds_sync();
        nstaged = sm.flag[2];
    }

    // 5. exact keys of the staged elements (one lane per element), the tail,
    // and (for penalties that may raise a logit) every penalised token from
    // the history state
    auto push = [&](uint32_t key, uint32_t id) __attribute__((always_inline)) {
        const uint32_t pos = atomicAdd(&sm.flag[1], 1u);
        if (pos < kStreamCandCap) s_cand[pos] = cand_pack(key, id);
    };
    auto count_of = [&](uint32_t id) __attribute__((always_inline)) -> uint32_t {
        return history ? 1u + hash_lookup(s_hash, a.log2_slots, id) : 1u;
    };
    auto pen_key = [&](uint32_t bits, bool allowed, uint32_t count) __attribute__((always_inline)) -> uint32_t {
        if (!allowed) return masked_key;
        const float v = configured_logit(u2f(bits), true, count, P.repetition_penalty, P.frequency_penalty,
                                         P.presence_penalty);
        const uint32_t key = order_key(v);
        return key < valid_min ? 0u : key;
    };
    // configured key of a token from the vector passes (0: not a candidate;
    // penalised tokens under raising penalties are left to the history pass)
    auto elem_key = [&](uint32_t bits, uint32_t id) __attribute__((always_inline)) -> uint32_t {
        const uint32_t off = id - bm_base;
        const bool allowed = !mask || ((s_allow[off >> 5] >> (off & 31u)) & 1u);
        bool pen = false;
        if constexpr (PEN != 0) pen = (s_pen[off >> 5] >> (off & 31u)) & 1u;
        if (pen) return lowering ? pen_key(bits, allowed, count_of(id)) : 0u;
        const uint32_t key = allowed ? raw_order_key(bits) : masked_key;
        return key < valid_min ? 0u : key;
    };
    constexpr uint32_t kLog2Epv = EPV == 8 ? 3u : (EPV == 4 ? 2u : 0u);
    auto staged_key = [&](uint32_t q) __attribute__((always_inline)) -> uint32_t {
        const uint32_t i = q >> kLog2Epv, e = q & (uint32_t)(EPV - 1);
        return elem_key(VT::staged_bits(s_svec, i, e), s_sslot[i] * EPV + e);
    };
    auto push_staged = [&]() __attribute__((always_inline)) {
        if (has_tail) {
            const uint32_t key = elem_key(tail_bits, tail_id);
            if (key >= thr && key != 0u) push(key, tail_id);
        }
        // Staged lane-vectors are spread over the waves (vector i to wave
        // i % 8), kLPV lanes per vector, kEPL elements per lane. A raw key
        // below thr cannot qualify (the configured value of a token in the
        // vector passes never exceeds its raw value), so only raw keys >= thr
        // are examined further. Masked tokens of greedy rows count as -inf,
        // which only a threshold at or below -inf admits: then every element
        // is examined. The ids of a lane-vector share one word of each
        // bitmap; penalised ones (rare) take the table lookup. Appends are
        // counted per wave: one LDS atomic per wave and round.
        constexpr uint32_t kLPV = EPV >= 4 ? 4u : 1u, kEPL = (uint32_t)EPV / kLPV;
        static_assert(kEPL <= 2u, "at most two elements per lane");
        constexpr uint32_t kElemMask = (1u << kEPL) - 1u;
        const uint32_t thr_raw = thr > kNegInfKey ? thr : 0u;  // the raw-key prefilter
        const uint32_t sub = lane % kLPV;
        for (uint32_t base = 0; base < nstaged; base += (uint32_t)kBlock / kLPV) {
            const uint32_t i = base + (lane / kLPV) * (uint32_t)kWaves + wave;
            const bool valid = i < nstaged;
            const uint32_t ic = valid ? i : 0u;
            const uint32_t e0 = sub * kEPL;  // first element of this lane
            uint32_t bits[kEPL];
            static_for<0, (int)kEPL>([&](auto E) __attribute__((always_inline)) { bits[E] = VT::staged_bits(s_svec, ic, e0 + (uint32_t)E); });
            const uint32_t id0 = s_sslot[ic] * EPV + e0;
            const uint32_t off = id0 - bm_base;
            const uint32_t allow_bits = mask ? (s_allow[off >> 5] >> (off & 31u)) & kElemMask : kElemMask;
            uint32_t pen_bits = 0u;
            if constexpr (PEN != 0) pen_bits = (s_pen[off >> 5] >> (off & 31u)) & kElemMask;
            // branch-free: the key of every element, zero where it cannot qualify
            uint32_t keys[kEPL];
            uint32_t cand = 0u;
            static_for<0, (int)kEPL>([&](auto E) __attribute__((always_inline)) {
                constexpr uint32_t bit = 1u << (int)E;
                const uint32_t raw = raw_order_key(bits[E]);
                const bool c = valid && raw >= thr_raw;
                cand |= c ? bit : 0u;
                uint32_t key = (allow_bits & bit) ? raw : masked_key;
                key = (c && !(pen_bits & bit)) ? key : 0u;
                keys[E] = (key < valid_min || key < thr) ? 0u : key;
            });
            uint32_t pb = pen_bits & cand;
            while (pb) {
                // penalised candidates (rare): configured value from the count
                const uint32_t e = (uint32_t)__builtin_ctz(pb);
                pb &= pb - 1u;
                uint32_t key = 0u;
                if (lowering) {
                    const uint32_t be = e == 0u ? bits[0] : bits[kEPL - 1u];  // kEPL <= 2
                    key = pen_key(be, ((allow_bits >> e) & 1u) != 0u, count_of(id0 + e));
                    if (key < valid_min || key < thr) key = 0u;
                }
                static_for<0, (int)kEPL>([&](auto E) __attribute__((always_inline)) { keys[E] = e == (uint32_t)E ? key : keys[E]; });
            }
            uint32_t nq = 0u;
            static_for<0, (int)kEPL>([&](auto E) __attribute__((always_inline)) { nq += keys[E] != 0u ? 1u : 0u; });
            // exclusive prefix and total of nq over the wave, bit by bit
            uint32_t excl = 0u, tot = 0u;
            static_for<0, (kEPL > 1u ? 2 : 1)>([&](auto B) __attribute__((always_inline)) {
                const uint64_t m = __ballot((nq >> (int)B) & 1u);
                excl += __builtin_amdgcn_mbcnt_hi((uint32_t)(m >> 32), __builtin_amdgcn_mbcnt_lo((uint32_t)m, 0u)) << (int)B;
                tot += (uint32_t)__builtin_popcountll(m) << (int)B;
            });
            if (tot) {
                uint32_t pos0 = 0u;
                if (lane == 0u) pos0 = atomicAdd(&sm.flag[1], tot);
                uint32_t pos = (uint32_t)__builtin_amdgcn_readlane((int)pos0, 0) + excl;
                static_for<0, (int)kEPL>([&](auto E) __attribute__((always_inline)) {
                    if (keys[E] != 0u) {
                        if (pos < kStreamCandCap) s_cand[pos] = cand_pack(keys[E], id0 + (uint32_t)E);
                        ++pos;
                    }
                });
            }
        }
    };
    if (nstaged > kStageCap) {
        if (has_tail) {
            const uint32_t key = elem_key(tail_bits, tail_id);
            if (key >= thr && key != 0u) push(key, tail_id);
        }
    } else {
        push_staged();
        if (PEN != 0 && !lowering) {
            for (uint32_t w = tid; w < bm_n; w += kBlock) {
                uint32_t bits = s_pen[w];
                while (bits) {
                    const uint32_t b = (uint32_t)__builtin_ctz(bits);
                    bits &= bits - 1u;
                    const uint32_t id = bm_base + w * 32u + b;
                    const uint32_t off = id - bm_base;
                    const bool allowed = !mask || ((s_allow[off >> 5] >> (off & 31u)) & 1u);
                    const uint32_t key = pen_key(f2u(load_elem<Elem>(lrow, id)), allowed, count_of(id));
                    if (key >= thr && key != 0u) push(key, id);
                }
            }
        }
    }
    {
        // slice flags: bit 0 = some token allowed, bit 1 = greedy row holds a NaN
        const uint32_t f = (__ballot(any_allowed != 0u) ? 1u : 0u) | (__ballot(has_nan != 0u) ? 2u : 0u);
        if (lane == 0u && f) atomicOr(&sm.flag[3], f);
    }
    lds_sync();
    const uint32_t flags_slice = sm.flag[3];
    bool repad = false;  // the candidate list was rewritten: its padding is stale
    if constexpr (PEN != 0) {
        if (lowering && nstaged <= kStageCap && sm.flag[1] < k && thr_stage > kZeroKey) {
            // Second chance, from registers: penalties pushed more than C - k
            // of the raw reports below thr (typically a row whose top tokens
            // are in its own history). Lane reports over the clean
            // lane-vectors only (fully allowed, nothing penalised: there the
            // configured key is the raw key) give a threshold t that at
            // least k configured keys reach. The lane-vectors whose raw
            // maximum lies in [t, thr_stage) join the staged set (their slots
            // appended, the vectors gathered from memory by the whole
            // workgroup, one load each), and the exact pass runs again over
            // the whole set at t.
            acc0 = VT::kAccInit;
            acc1 = VT::kAccInit;
            static_for<0, NV>([&](auto J) __attribute__((always_inline)) {
                constexpr int j = J;
                const uint32_t pw = (s_pen[(tok_base >> 5) + (uint32_t)j * kWordsPerJ] >> wsh) & kFull;
                const bool clean = ((okm[j >> 5] >> (j & 31)) & 1u) && pw == 0u;
                const uint32_t vm = clean ? vmx[j] : VT::kAccInit;
                if (j & 1) acc1 = VT::merge(acc1, vm);
                else acc0 = VT::merge(acc0, vm);
            });
            const uint32_t t = report_threshold(1);
            if (t > kZeroKey) {
                // lane-vectors to append, counted per lane, then one LDS
                // atomic per wave
                uint32_t am[LW];
#pragma unroll
                for (int i = 0; i < LW; ++i) am[i] = 0u;
                static_for<0, NV>([&](auto J) __attribute__((always_inline)) {
                    constexpr int j = J;
                    const bool lv = ((live[j >> 5] >> (j & 31)) & 1u) != 0u;
                    if (lv && VT::ge_pos(vmx[j], t) && !VT::ge_pos(vmx[j], thr_stage)) am[j >> 5] |= 1u << (j & 31);
                });
                uint32_t cnt = 0u;
#pragma unroll
                for (int i = 0; i < LW; ++i) cnt += (uint32_t)__builtin_popcount(am[i]);
                const uint32_t incl = wave_inclusive_scan(cnt);
                const uint32_t total = (uint32_t)__builtin_amdgcn_readlane((int)incl, 63);
                uint32_t pos0 = 0u;
                if (lane == 63u && total) pos0 = atomicAdd(&sm.flag[2], total);
                uint32_t pos = (uint32_t)__builtin_amdgcn_readlane((int)pos0, 63) + incl - cnt;
#pragma unroll
                for (int i = 0; i < LW; ++i) {
                    uint32_t m = am[i];
                    while (m) {
                        const uint32_t j = (uint32_t)i * 32u + (uint32_t)__builtin_ctz(m);
                        m &= m - 1u;
                        if (pos < kStageCap) s_sslot[pos] = v0 + wbase + j * 64u;
                        ++pos;
                    }
                }
                lds_sync();
                const uint32_t n2 = sm.flag[2];
                const uint32_t n1 = nstaged;
                nstaged = n2;  // past kStageCap: the exact selection from memory below
                if (n2 <= kStageCap) {
                    const vec_t *lvec = (const vec_t *)lrow;
                    for (uint32_t i = n1 + tid; i < n2; i += kBlock) s_svec[i] = lvec[s_sslot[i]];
                    if (tid == 0) sm.flag[1] = 0u;
                    set_thr(t);
                    lds_sync();
                    push_staged();  // over all n2 staged lane-vectors
                    lds_sync();
                    repad = true;
                }
            }
        }
    }
    if (nstaged <= kStageCap && sm.flag[1] > kStreamCandCap && (PEN == 0 || lowering)) {
        repad = true;
        // Too many candidates for a weak threshold: the exact k-th key of the
        // staged elements (plus the tail) is a threshold that keeps at least k.
        lds_sync();
        const uint32_t n_el = (nstaged << kLog2Epv) + (last_slice ? (uint32_t)(a.vocab - nfull * EPV) : 0u);
        auto any_key = [&](uint32_t q) __attribute__((always_inline)) -> uint32_t {
            if (q < (nstaged << kLog2Epv)) return staged_key(q);
            const uint32_t t = nfull * EPV + (q - (nstaged << kLog2Epv));
            return elem_key(f2u(load_elem<Elem>(lrow, t)), t);
        };
        uint32_t unused_count;
        const uint32_t t = radix_threshold_fn(0u, n_el, k, sm.hist, sm.sel, unused_count, any_key);
        set_thr(t > thr ? t : thr);
        if (tid == 0) sm.flag[1] = 0u;
        lds_sync();
        push_staged();
        lds_sync();
    }

    RowCtx ctx;
    ctx.logits_row = lrow;
    ctx.allowed_row = arow;
    ctx.seen_row = srow;
    ctx.hash = s_hash;
    ctx.bitmap = PEN != 0 ? s_pen : nullptr;
    ctx.log2_slots = a.log2_slots;
    ctx.tok0 = bm_base;
    ctx.rep = P.repetition_penalty;
    ctx.freq = P.frequency_penalty;
    ctx.pres = P.presence_penalty;
    ctx.history = history;
    ctx.prefix = PEN == 1 && a.prefix_ids ? a.prefix_ids + (uint64_t)row * a.prefix_stride : nullptr;
    ctx.prefix_n = PEN == 1 ? prefix_count(a, row) : 0u;
    ctx.whole_row = a.slices == 1u && PEN != 0;  // one slice: its bitmap (from token 0) and table are the row's

    // 7. selection -> s_sorted[0 .. n_out)
    uint32_t C = sm.flag[1];
    if (nstaged > kStageCap || C > kStreamCandCap || (C < k && thr > 1u)) {
        // Skewed slice (for example a constant row), or penalties that pushed
        // more than C - k of the reported values below thr: exact selection
        // recomputed from memory. The k-th largest key kv, then the `need`
        // smallest ids among keys == kv.
        // Every (key, id) of the slice, read back like the stream: chunks of 8
        // lane-vectors through the wave's buffer resource, one bitmap word per
        // lane-vector, and the configured key of each element (penalised ones
        // from their counts); then the V % EPV tail.
        auto each_key = [&](auto &&fn) __attribute__((always_inline)) {
            for (uint32_t j = 0; j < nval; j += 4u) {
                vec_t v[4];
#pragma unroll
                for (int u = 0; u < 4; ++u) {
                    const uint32_t off = (lane + (j + (uint32_t)u) * 64u) * kVecBytes;
                    if constexpr (kVecBytes == 16) v[u] = __builtin_amdgcn_raw_buffer_load_b128(rsrc, off, 0, 0);
                    else if constexpr (kVecBytes == 4) v[u] = u2f(__builtin_amdgcn_raw_buffer_load_b32(rsrc, off, 0, 0));
                    else v[u] = __builtin_amdgcn_raw_buffer_load_b16(rsrc, off, 0, 0);
                }
#pragma unroll
                for (int u = 0; u < 4; ++u) {
                    const bool valid = j + (uint32_t)u < nval;
                    const uint32_t id0 = (v0 + wbase + (j + (uint32_t)u) * 64u) * EPV;
                    const uint32_t off = valid ? id0 - bm_base : 0u;
                    const uint32_t aw = mask ? (s_allow[off >> 5] >> (off & 31u)) : 0xffffffffu;
                    uint32_t pw = 0u;
                    if constexpr (PEN != 0) pw = s_pen[off >> 5] >> (off & 31u);
                    static_for<0, EPV>([&](auto E) __attribute__((always_inline)) {
                        const uint32_t bits = VT::bits(v[u], E);
                        const bool allowed = ((aw >> (int)E) & 1u) != 0u;
                        uint32_t key;
                        if ((pw >> (int)E) & 1u) {
                            key = pen_key(bits, allowed, count_of(id0 + (uint32_t)E));
                        } else {
                            key = allowed ? raw_order_key(bits) : masked_key;
                            key = key < valid_min ? 0u : key;
                        }
                        fn(valid ? key : 0u, id0 + (uint32_t)E);
                    });
                }
            }
            if (has_tail) {
                const uint32_t off = tail_id - bm_base;
                const bool allowed = !mask || ((s_allow[off >> 5] >> (off & 31u)) & 1u);
                bool pen = false;
                if constexpr (PEN != 0) pen = (s_pen[off >> 5] >> (off & 31u)) & 1u;
                uint32_t key;
                if (pen) {
                    key = pen_key(tail_bits, allowed, count_of(tail_id));
                } else {
                    key = allowed ? raw_order_key(tail_bits) : masked_key;
                    key = key < valid_min ? 0u : key;
                }
                fn(key, tail_id);
            }
        };
        repad = true;
        uint32_t count_ge, G;
        auto visit_keys = [&](auto &&fn) __attribute__((always_inline)) {
            each_key([&](uint32_t key, uint32_t) __attribute__((always_inline)) { fn(key); });
        };
        const uint32_t kv = radix_threshold_visit(k, sm.hist, sm.sel, count_ge, visit_keys, &G);
        // G keys above kv; `need` of the count_ge - G ties at kv qualify: all
        // of them when they fit, else the `need` smallest ids
        const uint32_t need = k > G ? k - G : 0u;
        auto visit_ties = [&](auto &&fn) __attribute__((always_inline)) {
            each_key([&](uint32_t key, uint32_t id) __attribute__((always_inline)) { fn(key == kv && key != 0u ? ~id : 0u); });
        };
        // When every key >= kv fits the candidate list, all of them are
        // collected and the rank sort orders the ties by id; otherwise the
        // `need` smallest tie ids are found first (4 more passes).
        uint32_t ties_ge;
        uint32_t id_cut = 0xffffffffu;
        if (need && count_ge - G > need && count_ge > kStreamCandCap)
            id_cut = ~radix_threshold_visit(need, sm.hist, sm.sel, ties_ge, visit_ties);
        if (tid == 0) sm.flag[1] = 0u;
        lds_sync();
        each_key([&](uint32_t key, uint32_t id) __attribute__((always_inline)) {
            if (key != 0u && (key > kv || (key == kv && need && id <= id_cut))) {
                const uint32_t q = atomicAdd(&sm.flag[1], 1u);
                if (q < kStreamCandCap) s_cand[q] = cand_pack(key, id);
            }
        });
        lds_sync();
        C = min(sm.flag[1], kStreamCandCap);
    }
    // Many candidates (a weak threshold): keep the entries at or above the
    // k-th largest key (LDS radix select) in the staging area, which is free
    // by now, so the rank sort below stays small.
    uint64_t *list = s_cand;
    constexpr uint32_t kTrimCap = kStageCap * (uint32_t)sizeof(vec_t) / 8u;
    if (C > 256u && C > 4u * k) {
        auto cand_key = [&](uint32_t i) __attribute__((always_inline)) -> uint32_t { return (uint32_t)(s_cand[i] >> 32); };
        uint32_t unused_count;
        const uint32_t kth = radix_threshold_fn(0u, C, k, sm.hist, sm.sel, unused_count, cand_key);
        uint64_t *s_trim = (uint64_t *)s_svec;
        if (tid == 0) sm.flag[0] = 0u;
        lds_sync();
        for (uint32_t i = tid; i < C; i += kBlock) {
            const uint64_t e = s_cand[i];
            if ((uint32_t)(e >> 32) >= kth) {
                const uint32_t q = atomicAdd(&sm.flag[0], 1u);
                if (q < kTrimCap) s_trim[q] = e;
            }
        }
        lds_sync();
        if (sm.flag[0] <= kTrimCap) {
            list = s_trim;
            C = sm.flag[0];
            repad = true;
        }
    }
    // The writer of rank r also settles the sign of a zero survivor (from its
    // own configured value).
    auto emit = [&](uint32_t r, uint2 e) __attribute__((always_inline)) {
        if (e.x == kZeroKey && f2u(configured_at<Elem>(ctx, e.y)) == 0x80000000u) e.y |= kNegZeroFlag;
        s_sorted[r] = e;
    };
    // rank sort (ids are distinct, so ranks are a permutation): G adjacent
    // lanes share a candidate, each counting the better entries in every G-th
    // position, and the partial ranks are summed across the group
    if (C <= kRankPad) {
        // The common case, unrolled: 8 adjacent lanes share a candidate (two,
        // i and i + 64, past 64 candidates), each comparing it with every 8th
        // list entry, and the group's first lane sums the counts. (key, ~id) as one unsigned 64-bit value orders like
        // entry_better; the list reads as (0, 0) past C, which ranks below
        // every candidate (keys are nonzero).
        if (repad) {
            for (uint32_t i = C + tid; i < kRankPad; i += kBlock) list[i] = 0u;
            lds_sync();
        }
        const uint32_t i = tid >> 3, part = tid & 7u;
        const uint64_t p0 = list[i];
        if (C <= 64u) {
            uint64_t o[8];
            static_for<0, 8>([&](auto J) __attribute__((always_inline)) { o[J] = list[part + 8u * (uint32_t)J]; });
            uint32_t r = 0;
            static_for<0, 8>([&](auto J) __attribute__((always_inline)) { r += o[J] > p0 ? 1u : 0u; });
            r = group8_sum(r);
            if (i < C && part == 0u && r < k) emit(r, cand_entry(p0));
        } else {
            const uint64_t p1 = list[i + 64u];
            uint64_t o[16];
            static_for<0, 16>([&](auto J) __attribute__((always_inline)) { o[J] = list[part + 8u * (uint32_t)J]; });
            uint32_t r0 = 0, r1 = 0;
            static_for<0, 16>([&](auto J) __attribute__((always_inline)) {
                r0 += o[J] > p0 ? 1u : 0u;
                r1 += o[J] > p1 ? 1u : 0u;
            });
            r0 = group8_sum(r0);
            r1 = group8_sum(r1);
            if (part == 0u) {
                if (i < C && r0 < k) emit(r0, cand_entry(p0));
                if (i + 64u < C && r1 < k) emit(r1, cand_entry(p1));
            }
        }
    } else {
    uint32_t G = 1u;
    while (G < 8u && C * G * 2u <= (uint32_t)kBlock) G <<= 1;
    for (uint32_t base = 0; base < C * G; base += kBlock) {
        const uint32_t q = base + tid, i = q / G, part = q % G;
        uint32_t r = 0;
        uint64_t e = 0u;
        if (i < C) {
            e = list[i];
            uint32_t r1 = 0;
            uint32_t j = part;
            for (; j + G < C; j += 2u * G) {
                r += list[j] > e ? 1u : 0u;
                r1 += list[j + G] > e ? 1u : 0u;
            }
            if (j < C) r += list[j] > e ? 1u : 0u;
            r += r1;
        }
        for (uint32_t o = 1u; o < G; o <<= 1) r += __shfl_xor(r, (int)o, 64);
        if (i < C && part == 0u && r < k) emit(r, cand_entry(e));
    }
    }
    const uint32_t n_out = C < k ? C : k;
    lds_sync();


    // 8. publish: with several slices the sorted list goes to scratch; the
    // last slice of the row to arrive merges the row's lists and finishes it
    // (or, when the lists exceed its merge area, the finish kernel does). A
    // single slice finishes here.
    if (a.slices > 1) {
        uint2 *lists = a.scratch_lists + (uint64_t)(row * a.slices + slice) * a.kcap;
        uint32_t *meta = a.scratch_meta + row * a.slices;
        if (!a.merge_in_kernel) {
            for (uint32_t i = tid; i < n_out; i += kBlock) lists[i] = s_sorted[i];
            if (tid == 0) meta[slice] = n_out | (flags_slice << 16);
            return;
        }
        // Written through to memory (system-scope stores) and completed before
        // the arrival count, so the last slice, on whichever XCD it runs,
        // reads them with loads that bypass the caches.
        for (uint32_t i = tid; i < n_out; i += kBlock) {
            const uint2 e = s_sorted[i];
            __hip_atomic_store((uint64_t *)&lists[i], ((uint64_t)e.y << 32) | e.x, __ATOMIC_RELAXED,
                               __HIP_MEMORY_SCOPE_SYSTEM);
        }
        if (tid == 0)
            __hip_atomic_store(&meta[slice], n_out | (flags_slice << 16), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_SYSTEM);
        __builtin_amdgcn_s_waitcnt(0x0f70);  // vmcnt(0): this lane's stores are complete
        __syncthreads();
        if (tid == 0) sm.flag[0] = __hip_atomic_fetch_add(&a.scratch_counts[row], 1u, __ATOMIC_RELAXED,
                                                         __HIP_MEMORY_SCOPE_SYSTEM);
        __syncthreads();
        if (sm.flag[0] != a.slices - 1u) return;
        // the last slice: the count is reset for the next step (every slice
        // of this one has arrived), then the merge and the finish
        if (tid == 0) __hip_atomic_store(&a.scratch_counts[row], 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_SYSTEM);
        const uint2 *all = a.scratch_lists + (uint64_t)row * a.slices * a.kcap;
        uint32_t row_flags;
        const uint32_t n = merge_slices<kBlock>(
            a, k, s_big, s_sorted, sm.hist, row_flags,
            [&](uint32_t i) {
                const uint64_t v = __hip_atomic_load((const uint64_t *)&all[i], __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_SYSTEM);
                return make_uint2((uint32_t)v, (uint32_t)(v >> 32));
            },
            [&](uint32_t s) { return __hip_atomic_load(&meta[s], __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_SYSTEM); });
        const RowIo io_m = {sm.io[0], sm.io[1], sm.io[2], sm.io[3]};
        const RowCtx ctx_row = row_ctx<Elem, PEN>(a, row, P, s_hash);
        finish_row<Elem, PEN, kBlock>(a, row, io_m, P, k, sampled, n, row_flags, s_sorted, s_big, (float *)s_sslot,
                                      (float *)s_big + 64, s_hash, ctx_row, sm.u);
        return;
    }
    const RowIo io_l = {sm.io[0], sm.io[1], sm.io[2], sm.io[3]};
    finish_row<Elem, PEN, kBlock>(a, row, io_l, P, k, sampled, n_out, flags_slice, s_sorted, s_big, (float *)s_sslot,
                                  (float *)s_big + 64, s_hash, ctx, sm.u);
}

// Merges the S sorted slice lists of a row into s_sorted[0 .. n) (n = min(k,
// total)): the lists go to s_big through load_entry(i) (entry i of the row's
// S * kcap), the counts and flags to s_meta through load_meta(s); an entry's
// rank is its position in its own list plus the number of better entries in
// every other list (binary search; ids are distinct). row_flags gets the OR
// of the slices' flags. Ends with a block barrier.
template <int NT, typename LoadEntry, typename LoadMeta>
__device__ __forceinline__ uint32_t merge_slices(const StepArgs &a, uint32_t k, uint2 *s_big, uint2 *s_sorted,
                                                 uint32_t *s_meta, uint32_t &row_flags, LoadEntry load_entry,
                                                 LoadMeta load_meta) {
    const uint32_t tid = threadIdx.x;
    // every list entry is copied, whatever the counts (entries past a count
    // are ignored below), so the list loads do not wait for the counts
    const uint32_t ne = a.slices * a.kcap;
    for (uint32_t i = tid; i < ne; i += NT) s_big[i] = load_entry(i);
    if (tid < a.slices) s_meta[tid] = load_meta(tid);
    __syncthreads();
    uint32_t total = 0;
    row_flags = 0;
    for (uint32_t s = 0; s < a.slices; ++s) {
        const uint32_t m = s_meta[s];
        total += m & 0xffffu;
        row_flags |= m >> 16;
    }
    for (uint32_t i = tid; i < ne; i += NT) {
        const uint32_t s = i / a.kcap, pos = i % a.kcap;
        if (pos >= (s_meta[s] & 0xffffu)) continue;
        const uint2 e = s_big[i];
        uint32_t r = pos;
        for (uint32_t o = 0; o < a.slices && r < k; ++o) {
            if (o == s) continue;
            const uint2 *lo = s_big + o * a.kcap;
            uint32_t lo_i = 0, hi_i = s_meta[o] & 0xffffu;
            while (lo_i < hi_i) {
                const uint32_t mid = (lo_i + hi_i) >> 1;
                if (entry_better(lo[mid], e)) lo_i = mid + 1; else hi_i = mid;
            }
            r += lo_i;
        }
        if (r < k) s_sorted[r] = e;
    }
    __syncthreads();
    return total < k ? total : k;
}

// The row's context for recomputing configured values over the whole row
// (no slice-local LDS bitmap).
template <typename Elem, int PEN>
__device__ __forceinline__ RowCtx row_ctx(const StepArgs &a, uint32_t row, const nerve_sampler_row_params &P,
                                          uint32_t *s_hash) {
    RowCtx ctx;
    ctx.logits_row = (const Elem *)a.logits + (uint64_t)row * a.ld;
    ctx.allowed_row = a.allowed ? a.allowed + (uint64_t)row * a.allowed_stride : nullptr;
    ctx.seen_row = PEN == 1 ? a.seen + (uint64_t)row * a.seen_stride : nullptr;
    ctx.hash = s_hash;
    ctx.bitmap = nullptr;
    ctx.log2_slots = a.log2_slots;
    ctx.tok0 = 0;
    ctx.rep = P.repetition_penalty;
    ctx.freq = P.frequency_penalty;
    ctx.pres = P.presence_penalty;
    ctx.history = PEN == 2;
    ctx.prefix = PEN == 1 && a.prefix_ids ? a.prefix_ids + (uint64_t)row * a.prefix_stride : nullptr;
    ctx.prefix_n = PEN == 1 ? prefix_count(a, row) : 0u;
    ctx.whole_row = false;
    return ctx;
}

// Merges the S sorted slice lists of each row (one workgroup per row) and
// finishes the row, when the slice kernel does not (slices * kcap larger
// than its merge area). Launched after sample_rows_kernel on the same
// stream, so the slice lists are visible without any cross-workgroup fence.
template <typename Elem, int PEN>
__global__ __launch_bounds__(kFinishBlock) void finish_rows_kernel(StepArgs a) {
    extern __shared__ uint32_t s_dyn[];
    __shared__ uint32_t s_meta[64];
    uint32_t *s_hash = s_dyn;
    uint2 *s_big = (uint2 *)(s_dyn + a.hash_slots);
    uint2 *s_sorted = s_big + a.big_entries;
    float *s_wt = (float *)(s_sorted + a.kcap);  // [kcap] weights
    const uint32_t row = blockIdx.x;
    const nerve_sampler_row_params P = a.params[row];
    const RowIo io = load_row_io(a, row);
    const bool sampled = P.method != NERVE_METHOD_GREEDY;
    uint32_t k = sampled ? P.top_k : 1u;
    k = k < 1u ? 1u : (k > a.kcap ? a.kcap : k);
    const float u = sampled ? random_unit(a.rng, io.seed, (uint64_t)io.tick_lo | ((uint64_t)io.tick_hi << 32), row) : 0.0f;
    const uint2 *all = a.scratch_lists + (uint64_t)row * a.slices * a.kcap;
    const uint32_t *meta = a.scratch_meta + row * a.slices;
    uint32_t row_flags;
    const uint32_t n = merge_slices<kFinishBlock>(a, k, s_big, s_sorted, s_meta, row_flags,
                                                  [&](uint32_t i) { return all[i]; }, [&](uint32_t s) { return meta[s]; });
    const RowCtx ctx = row_ctx<Elem, PEN>(a, row, P, s_hash);
    finish_row<Elem, PEN, kFinishBlock>(a, row, io, P, k, sampled, n, row_flags, s_sorted, s_big, s_wt, (float *)s_big,
                                        s_hash, ctx, u);
}

// ---- launch ------------------------------------------------------------------


// hipFuncSetAttribute(MaxDynamicSharedMemorySize) once per kernel, device and
// size: the largest size set so far is remembered, so the hot launch makes no
// attribute call.
template <typename Kern>
static hipError_t ensure_dyn_lds(Kern kern, int device, uint32_t bytes, std::atomic<uint32_t> (&done)[kMaxDevices]) {
    if (device < 0 || device >= kMaxDevices) return hipErrorInvalidDevice;
    if (done[device].load(std::memory_order_relaxed) >= bytes) return hipSuccess;
    const hipError_t e = hipFuncSetAttribute((const void *)kern, hipFuncAttributeMaxDynamicSharedMemorySize, (int)bytes);
    if (e != hipSuccess) return e;
    uint32_t prev = done[device].load(std::memory_order_relaxed);
    while (prev < bytes && !done[device].compare_exchange_weak(prev, bytes)) {
    }
    return hipSuccess;
}

template <typename Elem, int EPV, int NV, int PEN, bool MASK, int AUX>
static hipError_t launch_one(const StepArgs &a, hipStream_t stream) {
    static std::atomic<uint32_t> rows_set[kMaxDevices];
    static std::atomic<uint32_t> fin_set[kMaxDevices];
    auto kern = sample_rows_kernel<Elem, EPV, NV, PEN, MASK, AUX>;
    hipError_t e = ensure_dyn_lds(kern, a.device, a.dyn_lds_bytes, rows_set);
    if (e != hipSuccess) return e;
    hipLaunchKernelGGL(kern, dim3(a.batch * a.slices), dim3(kBlock), a.dyn_lds_bytes, stream, a);
    e = hipGetLastError();
    if (e != hipSuccess || a.slices == 1u || a.merge_in_kernel) return e;
    auto fin = finish_rows_kernel<Elem, PEN>;
    e = ensure_dyn_lds(fin, a.device, a.finish_lds_bytes, fin_set);
    if (e != hipSuccess) return e;
    hipLaunchKernelGGL(fin, dim3(a.batch), dim3(kFinishBlock), a.finish_lds_bytes, stream, a);
    return hipGetLastError();
}

template <typename Elem, int EPV, int NV, bool MASK, int AUX = 0>
static hipError_t launch_pen_mask(const StepArgs &a, hipStream_t stream) {
    if (a.history) return launch_one<Elem, EPV, NV, 2, MASK, AUX>(a, stream);
    if (a.seen) return launch_one<Elem, EPV, NV, 1, MASK, AUX>(a, stream);
    return launch_one<Elem, EPV, NV, 0, MASK, AUX>(a, stream);
}

// Non-temporal (NT, bit 1) cache policy for the logits stream: each logit is
// read once. It pays when the grid fills the chip (B=256 x V=151936 bf16:
// 20.65 -> 19.7 us per step) and costs latency when it does not (B=64, same
// V: 17.2 -> 18.2 us), so the long-row kernels are built both ways and the
// launch picks by grid size. sc0 or sc1 added to NT changed nothing measurable.
constexpr int kLoadNT = 2;
constexpr uint32_t kNtMinGroups = 256;  // one workgroup per CU

template <typename Elem, int EPV, int NV, bool MASK>
static hipError_t launch_pen_mask_policy(const StepArgs &a, hipStream_t stream) {
    if (a.batch * a.slices >= kNtMinGroups) return launch_pen_mask<Elem, EPV, NV, MASK, kLoadNT>(a, stream);
    return launch_pen_mask<Elem, EPV, NV, MASK, 0>(a, stream);
}


// Lane-vectors per lane (NV) of the compiled slice kernels, per variant: the
// largest keep the whole kernel within 256 VGPRs without spills.
constexpr uint32_t kBf16NV[] = {8, 16, 24, 32, 40};
constexpr uint32_t kF32NV[] = {8, 16, 24, 32};
constexpr uint32_t kScalarNV[] = {16, 32};

template <typename Elem, int EPV, bool MASK>
static hipError_t launch_vec(const StepArgs &a, hipStream_t stream) {
    switch (a.nv) {
        case 8: return launch_pen_mask<Elem, EPV, 8, MASK>(a, stream);
        case 16: return launch_pen_mask<Elem, EPV, 16, MASK>(a, stream);
        case 24: return launch_pen_mask<Elem, EPV, 24, MASK>(a, stream);
        case 32: return launch_pen_mask_policy<Elem, EPV, 32, MASK>(a, stream);
        case 40:
            if constexpr (sizeof(Elem) == 2) return launch_pen_mask_policy<Elem, EPV, 40, MASK>(a, stream);
            return hipErrorInvalidValue;
        default: return hipErrorInvalidValue;
    }
}

template <typename Elem, bool MASK>
static hipError_t launch_scalar(const StepArgs &a, hipStream_t stream) {
    switch (a.nv) {
        case 16: return launch_pen_mask<Elem, 1, 16, MASK>(a, stream);
        case 32: return launch_pen_mask<Elem, 1, 32, MASK>(a, stream);
        default: return hipErrorInvalidValue;
    }
}

}  // namespace nerve
