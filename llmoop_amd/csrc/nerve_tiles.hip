// nerve_tiles.hip -- sampling from per-tile maxima: the step that follows an
// LM-head projection whose epilogue recorded, for every row and every 64
// columns, the largest order key and the count of NaNs (a "tile record").
//
// The projection writes the logits anyway; the dense step then reads all of
// them again. With the records, a step reads the records (8 bytes per 64
// logits) and only the tiles that can hold a survivor:
//   threshold  each lane takes the largest record key among its *clean*
//              tiles (every token valid, allowed and unpenalised, so the
//              record's element has its raw value as configured value); the
//              k-th largest of those lane maxima is a value t that at least k
//              configured values reach (the same ballot search as the dense
//              kernel's lane reports);
//   gather     every tile whose record key reaches t is read (one load per
//              element, a wave per 64 elements), and each element whose
//              configured key reaches t is a candidate; penalties that may
//              raise a logit take the penalised tokens out of the tiles and
//              evaluate each one from the penalty state instead;
//   select     rank sort of the candidates (trimmed to the k-th key first
//              when many), then the shared finish (finish_row).
// A row that cannot use the records (fewer than k clean tiles, a threshold at
// or below -inf, too many candidate tiles or candidates) takes the exact
// selection over the whole row from memory. Results equal the dense step's on
// the same logits bit for bit.
//
// Reference: the projection is tied_output_projection_batch_bf16.comp.template
// (dispatched in batched_output_projection.rs:162-206); the semantics are the
// sampler's (temperature_top_k_candidates_f32.comp.template:59-126,
// temperature_top_k_top_p_sampler_f32.comp.template:90-216).
#include "nerve_sampler_device.h"

namespace nerve {

constexpr uint32_t kTileCols = 64;
constexpr uint32_t kTileCandCap = 1024;  // candidate tiles per row
constexpr uint32_t kMaxTiles = 4096;     // tiles per row (vocab <= 262144)

// Tile records of existing logits: one wave per (row, tile); block of 4 waves.
template <typename Elem>
__global__ __launch_bounds__(256) void tile_records_kernel(const Elem *logits, uint64_t ld, uint32_t batch, uint32_t vocab,
                                                           uint2 *records, uint32_t rec_stride) {
    const uint32_t ntiles = (vocab + kTileCols - 1u) / kTileCols;
    const uint32_t row = blockIdx.y;
    const uint32_t tile = blockIdx.x * 4u + (threadIdx.x >> 6);
    if (row >= batch || tile >= ntiles) return;
    const uint32_t id = tile * kTileCols + lane_id();
    uint32_t key = 0u;
    bool nan = false;
    if (id < vocab) {
        const uint32_t bits = f2u(load_elem<Elem>(logits + (uint64_t)row * ld, id));
        key = raw_order_key(bits);
        nan = (bits & 0x7fffffffu) > 0x7f800000u;
    }
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) key = max(key, (uint32_t)__shfl_xor((int)key, o, 64));
    const uint32_t nn = (uint32_t)__popcll(__ballot(nan));
    if (lane_id() == 0u) records[(uint64_t)row * rec_stride + tile] = make_uint2(key, nn);
}

// LDS of sample_tiles_kernel, in layout order.
__host__ __device__ constexpr uint32_t tiles_lds_bytes(uint32_t hash_slots, uint32_t pen_words, uint32_t ntiles,
                                                       uint32_t kcap) {
    return hash_slots * 4u + pen_words * 4u + ntiles * 8u + kTileCandCap * 4u + kStreamCandCap * 8u + kcap * 8u +
           kcap * 8u;
}

template <typename Elem, int PEN, bool MASK>
__global__ __launch_bounds__(kBlock) void sample_tiles_kernel(StepArgs a) {
    __shared__ SharedSmall sm;
    extern __shared__ __align__(16) uint32_t s_dyn[];
    const uint32_t V = a.vocab;
    const uint32_t ntiles = (V + kTileCols - 1u) / kTileCols;
    const uint32_t words = (V + 31u) / 32u;
    const uint32_t pen_words = PEN != 0 ? words : 0u;
    uint32_t *s_hash = s_dyn;                                   // [hash_slots] id -> repeats (occurrences past the first)
    uint32_t *s_pen = s_hash + a.hash_slots;                    // [pen_words] penalised ids of the row
    uint32_t *s_ck = s_pen + pen_words;                         // [ntiles] record key of clean tiles, else 0
    uint32_t *s_rk = s_ck + ntiles;                             // [ntiles] record key of every tile
    uint32_t *s_ct = s_rk + ntiles;                             // [kTileCandCap] candidate tiles
    // 8-byte aligned by index arithmetic on s_dyn (a cast through an integer
    // would lose the LDS address space and turn every access into a flat one)
    const uint32_t cand_off = (a.hash_slots + pen_words + 2u * ntiles + kTileCandCap + 1u) & ~1u;
    uint64_t *s_cand = (uint64_t *)(s_dyn + cand_off);          // [kStreamCandCap]
    uint2 *s_sorted = (uint2 *)(s_cand + kStreamCandCap);       // [kcap]
    float *s_w = (float *)(s_sorted + a.kcap);                  // [kcap]
    float *s_p = s_w + a.kcap;                                  // [kcap]
    uint2 *s_big = (uint2 *)s_cand;                             // finish scratch (after the selection)

    const uint32_t tid = threadIdx.x, lane = lane_id(), wave = tid >> 6;
    const uint32_t row = blockIdx.x;
    const Elem *lrow = (const Elem *)a.logits + (uint64_t)row * a.ld;
    const uint32_t *arow = MASK ? a.allowed + (uint64_t)row * a.allowed_stride : nullptr;
    const uint2 *rec = a.tile_records + (uint64_t)row * a.tile_stride;
    // every load that depends on nothing is issued first: the tile records
    // and mask word pairs of this lane (tile t = tid + 512 u, u < 8; ntiles
    // <= 4096) and its history ids (up to the stride; the length masks them
    // later), so their latencies overlap
    uint2 r[8];
    uint2 mw[MASK ? 8 : 1];
#pragma unroll
    for (int u = 0; u < 8; ++u) {
        const uint32_t t = tid + (uint32_t)u * kBlock;
        r[u] = t < ntiles ? rec[t] : make_uint2(0u, 0u);
        if constexpr (MASK) {
            const uint32_t w0 = 2u * t, w1 = w0 + 1u;
            mw[u] = make_uint2(t < ntiles ? arow[w0] : 0u, w1 < words && t < ntiles ? arow[w1] : 0u);
        }
    }
    uint32_t hid[PEN == 2 ? 8 : 1];
    if constexpr (PEN == 2) {
        const uint32_t *hrow = a.history + (uint64_t)row * a.history_stride;
#pragma unroll
        for (int h = 0; h < 8; ++h) {
            const uint32_t i = tid + (uint32_t)h * kBlock;
            hid[h] = i < a.history_stride ? hrow[i] : 0xffffffffu;
        }
    }
    const nerve_sampler_row_params P = a.params[row];
    const RowIo io = load_row_io(a, row);
    const bool sampled = P.method != NERVE_METHOD_GREEDY;
    uint32_t k = sampled ? P.top_k : 1u;
    k = k < 1u ? 1u : (k > a.kcap ? a.kcap : k);
    const uint32_t valid_min = sampled ? kMinFiniteKey : kNegInfKey;
    const uint32_t masked_key = sampled ? 0u : kNegInfKey;
    const bool lowering = P.repetition_penalty >= 1.0f && P.frequency_penalty >= 0.0f && P.presence_penalty >= 0.0f;

    // 1. penalty state: the row's penalised ids as an LDS bitmap, and (history)
    // the repeats of each id in the table
    if (tid == 0) {
        sm.flag[0] = 0u;  // candidate tiles
        sm.flag[1] = 0u;  // candidates
        sm.flag[3] = 0u;  // row flags
    }
    if constexpr (PEN == 2) {
        for (uint32_t i = tid; i < a.hash_slots; i += kBlock) s_hash[i] = kHashEmpty;
        for (uint32_t i = tid; i < words; i += kBlock) s_pen[i] = 0u;
        lds_sync();
        uint32_t len = a.history_len[row];
        len = len > a.history_stride ? a.history_stride : len;
#pragma unroll
        for (int h = 0; h < 8; ++h) {
            const uint32_t id = hid[h];
            if (tid + (uint32_t)h * kBlock < len && id < V) {
                // the bitmap holds first occurrences; the table only repeats
                // (short probe chains: a wave waits for its longest one)
                const uint32_t bit = 1u << (id & 31u);
                if (atomicOr(&s_pen[id >> 5], bit) & bit) hash_insert(s_hash, a.log2_slots, id);
            }
        }
    } else if constexpr (PEN == 1) {
        const uint32_t *srow = a.seen + (uint64_t)row * a.seen_stride;
        for (uint32_t i0 = tid; i0 < words; i0 += 8u * kBlock) {
            uint32_t sw[8];
#pragma unroll
            for (int u = 0; u < 8; ++u) {
                const uint32_t i = i0 + (uint32_t)u * kBlock;
                sw[u] = i < words ? srow[i] : 0u;
            }
#pragma unroll
            for (int u = 0; u < 8; ++u) {
                const uint32_t i = i0 + (uint32_t)u * kBlock;
                uint32_t w = sw[u];
                if (i == words - 1u && (V & 31u)) w &= (1u << (V & 31u)) - 1u;
                if (i < words) s_pen[i] = w;
            }
        }
        const uint32_t np = prefix_count(a, row);
        lds_sync();
        if (tid < np) {
            const uint32_t id = a.prefix_ids[(uint64_t)row * a.prefix_stride + tid];
            if (id < V) atomicOr(&s_pen[id >> 5], 1u << (id & 31u));
        }
    }
    lds_sync();

    // configured order key of token id with logit bits `bits` (0: never a
    // candidate); penalised tokens take their count
    auto key_of = [&](uint32_t id, uint32_t bits) __attribute__((always_inline)) -> uint32_t {
        if constexpr (MASK) {
            if (!((arow[id >> 5] >> (id & 31u)) & 1u)) return masked_key;
        }
        uint32_t key = raw_order_key(bits);
        if constexpr (PEN != 0) {
            if ((s_pen[id >> 5] >> (id & 31u)) & 1u) {
                const uint32_t count = PEN == 2 ? 1u + hash_lookup(s_hash, a.log2_slots, id) : 1u;
                key = order_key(configured_logit(u2f(bits), true, count, P.repetition_penalty, P.frequency_penalty,
                                                 P.presence_penalty));
            }
        }
        return key < valid_min ? 0u : key;
    };

    // 2. records: clean keys to LDS, the lane's largest clean key, the row's
    // NaN and allowed flags
    // every record (and mask pair) of this lane loaded before any is used:
    // tile t = tid + 512 u, u < 8 (ntiles <= 4096)
    uint32_t best = 0u, any_allowed = MASK ? 0u : 1u, nan_count = 0u;
    {
#pragma unroll
        for (int u = 0; u < 8; ++u) {
            const uint32_t t = tid + (uint32_t)u * kBlock;
            if (t >= ntiles) continue;
            nan_count += r[u].y;
            const uint32_t w0 = 2u * t, w1 = w0 + 1u;
            bool clean = (t + 1u) * kTileCols <= V;  // a partial last tile is never clean
            if constexpr (PEN != 0) clean = clean && s_pen[w0] == 0u && (w1 >= words || s_pen[w1] == 0u);
            if constexpr (MASK) {
                uint32_t m0 = mw[u].x, m1 = mw[u].y;
                if (w0 == words - 1u && (V & 31u)) m0 &= (1u << (V & 31u)) - 1u;
                if (w1 == words - 1u && (V & 31u)) m1 &= (1u << (V & 31u)) - 1u;
                any_allowed |= (m0 | m1) ? 1u : 0u;
                clean = clean && m0 == 0xffffffffu && m1 == 0xffffffffu;
            }
            const uint32_t key = r[u].x < valid_min ? 0u : r[u].x;
            s_rk[t] = r[u].x;
            const uint32_t ck = clean ? key : 0u;
            s_ck[t] = ck;
            best = max(best, ck);
        }
    }
    {
        const uint32_t f = (__ballot(any_allowed != 0u) ? 1u : 0u) | (__ballot(nan_count != 0u) ? 4u : 0u);
        if (lane == 0u && f) atomicOr(&sm.flag[3], f);
    }
    // 3. threshold: the k-th largest lane maximum (ballot search per wave, the
    // waves' top 64 in an LDS union, wave 0 takes the k-th), or for k > 64 the
    // k-th largest clean key by radix selection
    uint32_t thr;
    if (k <= 64u) {
        const uint32_t b1[1] = {best};
        const uint32_t tw = wave_kth<1, 16>(b1, k);
        const bool in = best != 0u && best >= tw;
        const uint64_t bal = __ballot(in);
        const uint32_t pos = __builtin_amdgcn_mbcnt_hi((uint32_t)(bal >> 32), __builtin_amdgcn_mbcnt_lo((uint32_t)bal, 0u));
        if (in) sm.ukeys[0][wave * 64u + pos] = best;
        if (lane == 0u) sm.ucount[0][wave] = (uint32_t)__popcll(bal);
        lds_sync();
        if (wave == 0u) {
            uint32_t uk[kWaves];
#pragma unroll
            for (int w = 0; w < kWaves; ++w) uk[w] = lane < sm.ucount[0][w] ? sm.ukeys[0][w * 64 + lane] : 0u;
            const uint32_t t = wave_kth<kWaves, 16>(uk, k);
            if (lane == 0u) sm.uthr[0] = t;
        }
        lds_sync();
        thr = sm.uthr[0];
    } else {
        uint32_t unused;
        thr = radix_threshold_fn(0u, ntiles, k, sm.hist, sm.sel, unused, [&](uint32_t t) { return s_ck[t]; });
        if (thr <= 1u) thr = 0u;
    }
    const uint32_t row_flags_in = sm.flag[3];
    // a usable threshold: positive-definite (above the masked keys of greedy rows)
    bool exact = !(thr > kNegInfKey && thr >= valid_min);

    // 4. candidate tiles, then their elements
    if (!exact) {
        for (uint32_t t = tid; t < ntiles; t += kBlock) {
            const uint32_t key = s_rk[t];
            if (key >= thr) {
                const uint32_t q = atomicAdd(&sm.flag[0], 1u);
                if (q < kTileCandCap) s_ct[q] = t;
            }
        }
        lds_sync();
        const uint32_t nct = sm.flag[0];
        if (nct > kTileCandCap) {
            exact = true;
        } else {
            const uint32_t nel = nct * kTileCols;
            auto push = [&](uint32_t key, uint32_t id) __attribute__((always_inline)) {
                const uint32_t q = atomicAdd(&sm.flag[1], 1u);
                if (q < kStreamCandCap) s_cand[q] = cand_pack(key, id);
            };
            // 16 elements per lane and round, every load issued before any key
            for (uint32_t e0 = tid; e0 < nel; e0 += 16u * kBlock) {
                uint32_t bits[16], ids[16];
#pragma unroll
                for (int u = 0; u < 16; ++u) {
                    const uint32_t e = e0 + (uint32_t)u * kBlock;
                    ids[u] = e < nel ? s_ct[e / kTileCols] * kTileCols + (e % kTileCols) : 0xffffffffu;
                    bits[u] = ids[u] < V ? f2u(load_elem<Elem>(lrow, ids[u])) : 0u;
                }
                // The raw test first (configured <= raw for lowering
                // penalties and masks); a lane's first two passing elements
                // go to two register slots, so the configured key (penalty
                // lookup, division) runs twice per lane, not 16 times; a lane
                // with more in the round (rare) computes the rest in place.
                uint32_t cm = 0u;
#pragma unroll
                for (int u = 0; u < 16; ++u) {
                    const uint32_t id = ids[u];
                    bool c = id < V && raw_order_key(bits[u]) >= thr;
                    if constexpr (PEN != 0) c = c && !(!lowering && ((s_pen[id >> 5] >> (id & 31u)) & 1u));  // the penalised pass below
                    cm |= c ? (1u << u) : 0u;
                }
                uint32_t id0 = 0u, b0 = 0u, id1 = 0u, b1 = 0u;
#pragma unroll
                for (int u = 0; u < 16; ++u) {
                    const uint32_t before = (uint32_t)__builtin_popcount(cm & ((1u << u) - 1u));
                    const bool c = (cm >> u) & 1u;
                    id0 = c && before == 0u ? ids[u] : id0;
                    b0 = c && before == 0u ? bits[u] : b0;
                    id1 = c && before == 1u ? ids[u] : id1;
                    b1 = c && before == 1u ? bits[u] : b1;
                }
                const uint32_t nc = (uint32_t)__builtin_popcount(cm);
                uint32_t k0 = nc > 0u ? key_of(id0, b0) : 0u;
                uint32_t k1 = nc > 1u ? key_of(id1, b1) : 0u;
                k0 = k0 >= thr ? k0 : 0u;
                k1 = k1 >= thr ? k1 : 0u;
                if (nc > 2u) {
#pragma unroll
                    for (int u = 0; u < 16; ++u) {
                        if (((cm >> u) & 1u) && __builtin_popcount(cm & ((1u << u) - 1u)) >= 2) {
                            const uint32_t key = key_of(ids[u], bits[u]);
                            if (key >= thr && key != 0u) push(key, ids[u]);
                        }
                    }
                }
                // one LDS atomic per wave for the slots' appends
                const uint32_t cnt = (k0 != 0u ? 1u : 0u) + (k1 != 0u ? 1u : 0u);
                const uint32_t incl = wave_inclusive_scan(cnt);
                const uint32_t total = (uint32_t)__builtin_amdgcn_readlane((int)incl, 63);
                if (total) {
                    uint32_t pos0 = 0u;
                    if (lane == 63u) pos0 = atomicAdd(&sm.flag[1], total);
                    uint32_t q = (uint32_t)__builtin_amdgcn_readlane((int)pos0, 63) + incl - cnt;
                    if (k0 != 0u) {
                        if (q < kStreamCandCap) s_cand[q] = cand_pack(k0, id0);
                        ++q;
                    }
                    if (k1 != 0u && q < kStreamCandCap) s_cand[q] = cand_pack(k1, id1);
                }
            }
            if constexpr (PEN != 0) {
                if (!lowering) {
                    // penalties that may raise a logit: every penalised token
                    for (uint32_t w = tid; w < words; w += kBlock) {
                        uint32_t b = s_pen[w];
                        while (b) {
                            const uint32_t id = w * 32u + (uint32_t)__builtin_ctz(b);
                            b &= b - 1u;
                            const uint32_t key = key_of(id, f2u(load_elem<Elem>(lrow, id)));
                            if (key >= thr && key != 0u) push(key, id);
                        }
                    }
                }
            }
            lds_sync();
            if (sm.flag[1] > kStreamCandCap || sm.flag[1] < k) exact = true;
        }
    }
    uint32_t C;
    if (exact) {
        // The exact selection over the whole row from memory: the k-th largest
        // key kv, then the `need` smallest ids among keys == kv.
        lds_sync();
        auto key_at = [&](uint32_t t) __attribute__((always_inline)) -> uint32_t {
            return key_of(t, f2u(load_elem<Elem>(lrow, t)));
        };
        uint32_t count_ge, G;
        const uint32_t kv = radix_threshold_fn(0u, V, k, sm.hist, sm.sel, count_ge, key_at, &G);
        const uint32_t need = k > G ? k - G : 0u;
        uint32_t id_cut = 0xffffffffu;
        if (need && count_ge - G > need && count_ge > kStreamCandCap) {
            uint32_t ties_ge;
            id_cut = ~radix_threshold_fn(0u, V, need, sm.hist, sm.sel, ties_ge, [&](uint32_t t) {
                const uint32_t key = key_at(t);
                return key == kv && key != 0u ? ~t : 0u;
            });
        }
        if (tid == 0) sm.flag[1] = 0u;
        lds_sync();
        for (uint32_t t = tid; t < V; t += kBlock) {
            const uint32_t key = key_at(t);
            if (key != 0u && (key > kv || (key == kv && need && t <= id_cut))) {
                const uint32_t q = atomicAdd(&sm.flag[1], 1u);
                if (q < kStreamCandCap) s_cand[q] = cand_pack(key, t);
            }
        }
        lds_sync();
    }
    C = min(sm.flag[1], kStreamCandCap);

    // 5. selection: trim many candidates to the k-th key, then a rank sort
    uint64_t *list = s_cand;
    if (C > 256u && C > 2u * k) {
        uint32_t unused;
        const uint32_t kth = radix_threshold_fn(0u, C, k, sm.hist, sm.sel, unused,
                                                [&](uint32_t i) { return (uint32_t)(s_cand[i] >> 32); });
        if (tid == 0) sm.flag[2] = 0u;
        lds_sync();
        // compact in place: entries >= kth move to the front (read all first)
        uint64_t keep[4];
        uint32_t nk = 0;
        for (uint32_t i = tid; i < C; i += kBlock) {
            const uint64_t e = s_cand[i];
            if ((uint32_t)(e >> 32) >= kth && nk < 4u) keep[nk++] = e;
        }
        lds_sync();
        for (uint32_t j = 0; j < nk; ++j) {
            const uint32_t q = atomicAdd(&sm.flag[2], 1u);
            s_cand[q] = keep[j];
        }
        lds_sync();
        C = sm.flag[2];
    }
    RowCtx ctx;
    ctx.logits_row = lrow;
    ctx.allowed_row = arow;
    ctx.seen_row = PEN == 1 ? a.seen + (uint64_t)row * a.seen_stride : nullptr;
    ctx.hash = s_hash;
    ctx.bitmap = PEN != 0 ? s_pen : nullptr;  // history: bitmap + the table of repeats
    ctx.log2_slots = a.log2_slots;
    ctx.tok0 = 0u;
    ctx.rep = P.repetition_penalty;
    ctx.freq = P.frequency_penalty;
    ctx.pres = P.presence_penalty;
    ctx.history = PEN == 2;
    ctx.prefix = nullptr;
    ctx.prefix_n = 0u;
    ctx.whole_row = PEN != 0;  // the bitmap covers the row (prefix included), the table holds its repeats
    // rank sort: 4 adjacent lanes per candidate, each counting the better
    // entries among every 4th one (8 reads in flight), the counts summed
    // across the 4 lanes (ids are distinct, so ranks are a permutation)
    for (uint32_t base = 0; base < C; base += kBlock / 4u) {
        const uint32_t i = base + (tid >> 2), part = tid & 3u;
        const uint64_t e = i < C ? list[i] : 0u;
        uint32_t rk = 0;
        for (uint32_t j0 = part; j0 < C; j0 += 32u) {
            uint64_t o[8];
#pragma unroll
            for (int q = 0; q < 8; ++q) {
                const uint32_t j = j0 + 4u * (uint32_t)q;
                o[q] = j < C ? list[j] : 0u;
            }
#pragma unroll
            for (int q = 0; q < 8; ++q) rk += o[q] > e ? 1u : 0u;
        }
        rk += (uint32_t)__shfl_xor((int)rk, 1, 64);
        rk += (uint32_t)__shfl_xor((int)rk, 2, 64);
        if (part == 0u && i < C && rk < k) {
            uint2 en = cand_entry(e);
            if (en.x == kZeroKey && f2u(configured_at<Elem>(ctx, en.y)) == 0x80000000u) en.y |= kNegZeroFlag;
            s_sorted[rk] = en;
        }
    }
    lds_sync();
    const uint32_t n = C < k ? C : k;
    uint32_t row_flags = row_flags_in & 1u;
    if (!sampled) {
        const float pq = P.repetition_penalty + P.frequency_penalty + P.presence_penalty;
        if ((row_flags_in & 4u) || (PEN != 0 && !(pq - pq == 0.0f))) row_flags |= 2u;
    }
    const float u = sampled ? random_unit(a.rng, io.seed, (uint64_t)io.tick_lo | ((uint64_t)io.tick_hi << 32), row) : 0.0f;
    finish_row<Elem, PEN, kBlock>(a, row, io, P, k, sampled, n, row_flags, s_sorted, s_big, s_w, s_p, s_hash, ctx, u);
}

template <typename Elem, int PEN, bool MASK>
static hipError_t launch_tiles_one(const StepArgs &a, hipStream_t stream) {
    static std::atomic<uint32_t> set[kMaxDevices];
    auto kern = sample_tiles_kernel<Elem, PEN, MASK>;
    const hipError_t e = ensure_dyn_lds(kern, a.device, a.dyn_lds_bytes, set);
    if (e != hipSuccess) return e;
    hipLaunchKernelGGL(kern, dim3(a.batch), dim3(kBlock), a.dyn_lds_bytes, stream, a);
    return hipGetLastError();
}

template <typename Elem>
static hipError_t launch_tiles_elem(const StepArgs &a, hipStream_t stream) {
    const bool mask = a.allowed != nullptr;
    const int pen = a.history ? 2 : (a.seen ? 1 : 0);
    if (mask) {
        if (pen == 2) return launch_tiles_one<Elem, 2, true>(a, stream);
        if (pen == 1) return launch_tiles_one<Elem, 1, true>(a, stream);
        return launch_tiles_one<Elem, 0, true>(a, stream);
    }
    if (pen == 2) return launch_tiles_one<Elem, 2, false>(a, stream);
    if (pen == 1) return launch_tiles_one<Elem, 1, false>(a, stream);
    return launch_tiles_one<Elem, 0, false>(a, stream);
}

hipError_t launch_sample_tiles(bool bf16, const StepArgs &a, hipStream_t stream) {
    return bf16 ? launch_tiles_elem<uint16_t>(a, stream) : launch_tiles_elem<float>(a, stream);
}

uint32_t sample_tiles_lds_bytes(uint32_t hash_slots, uint32_t vocab, bool pen, uint32_t kcap) {
    const uint32_t ntiles = (vocab + kTileCols - 1u) / kTileCols;
    return tiles_lds_bytes(hash_slots, pen ? (vocab + 31u) / 32u : 0u, ntiles, kcap) + 8u;
}

uint32_t tile_columns() { return kTileCols; }
uint32_t max_tiles() { return kMaxTiles; }

hipError_t launch_tile_records(bool bf16, const void *logits, uint64_t ld, uint32_t batch, uint32_t vocab, uint2 *records,
                               uint32_t rec_stride, hipStream_t stream) {
    const uint32_t ntiles = (vocab + kTileCols - 1u) / kTileCols;
    const dim3 grid((ntiles + 3u) / 4u, batch);
    if (bf16)
        hipLaunchKernelGGL(tile_records_kernel<uint16_t>, grid, dim3(256), 0, stream, (const uint16_t *)logits, ld, batch,
                           vocab, records, rec_stride);
    else
        hipLaunchKernelGGL(tile_records_kernel<float>, grid, dim3(256), 0, stream, (const float *)logits, ld, batch, vocab,
                           records, rec_stride);
    return hipGetLastError();
}

}  // namespace nerve
