// nerve_device_math.h -- binary32 primitives of the gfx950 sampler.
//
// Each function performs the same sequence of IEEE-754 binary32 operations,
// one rounding each, as the sampler's written definition (the file is built
// with -ffp-contract=off, so no multiply-add is fused):
//   nerve_expf: Cody-Waite reduction k = rint(x*log2e), r = (x - k*LN2_HI) - k*LN2_LO,
//               degree-7 Taylor polynomial in Horner form, scale by 2^k from exponent
//               bits (two steps below 2^-126 so only the last step rounds).
//   nerve_logf: x = m*2^e, m in [sqrt(1/2), sqrt(2)), ln m = 2*atanh((m-1)/(m+1)) by its
//               odd series to s^15, ln x = e*LN2_HI + (e*LN2_LO + ln m).
//   Philox4x32-10 of Salmon et al. (SC'11) and the reference shader hash
//   (temperature_top_k_top_p_sampler_f32.comp.template:56-72).
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace nerve {

constexpr uint32_t kLowestBits = 0xff7fffffu;  // -FLT_MAX, the reference's LOWEST_FLOAT
constexpr uint32_t kPadId = 0xffffffffu;
constexpr uint32_t kNegZeroFlag = 0x80000000u;  // marks a -0.0 survivor in the id word
constexpr uint32_t kIdMask = 0x7fffffffu;
constexpr uint32_t kZeroKey = 0x80000000u;      // order key of +0.0 and -0.0
constexpr uint32_t kNegInfKey = 0x007fffffu;    // order key of -inf
constexpr uint32_t kMinFiniteKey = 0x00800000u; // order key of -FLT_MAX

__device__ __forceinline__ float u2f(uint32_t u) { return __uint_as_float(u); }
__device__ __forceinline__ uint32_t f2u(float f) { return __float_as_uint(f); }

// Larger float -> larger key; -0.0 and +0.0 share a key (the reference
// compares with ==); NaN -> 0 (never a survivor).
__device__ __forceinline__ uint32_t order_key(float v) {
    if (v != v) return 0u;
    uint32_t bits = v == 0.0f ? 0u : f2u(v);
    return (bits & 0x80000000u) ? ~bits : (bits | 0x80000000u);
}

__device__ __forceinline__ float key_to_float(uint32_t key) {
    return u2f((key & 0x80000000u) ? (key & 0x7fffffffu) : ~key);
}

__device__ __forceinline__ float nerve_expf(float x) {
    if (x != x) return x;
    if (x > 88.72283935546875f) return __builtin_huge_valf();
    if (x < -103.972084045410156f) return 0.0f;
    const float log2e = 1.44269502162933349609375f;
    const float ln2_hi = 0.693145751953125f;
    const float ln2_lo = 1.428606765330187045e-06f;
    float t = x * log2e;
    float kf = __builtin_rintf(t);
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
    if (k >= -126) return p * u2f((uint32_t)(k + 127) << 23);
    p = p * u2f((uint32_t)(k + 64 + 127) << 23);
    return p * u2f((uint32_t)(-64 + 127) << 23);
}

__device__ __forceinline__ float nerve_logf(float x) {
    if (x != x || x < 0.0f) return __builtin_nanf("");
    if (x == 0.0f) return -__builtin_huge_valf();
    if (x == __builtin_huge_valf()) return x;
    uint32_t bits = f2u(x);
    int e = 0;
    if ((bits >> 23) == 0u) {
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

__device__ __forceinline__ uint32_t hash_u32(uint32_t v) {
    v ^= v >> 16;
    v *= 0x7feb352du;
    v ^= v >> 15;
    v *= 0x846ca68bu;
    v ^= v >> 16;
    return v;
}

__device__ __forceinline__ uint32_t philox4x32_10_word0(uint32_t c0, uint32_t c1, uint32_t c2, uint32_t c3,
                                                        uint32_t k0, uint32_t k1) {
#pragma unroll
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
    return c0;
}

// Uniform in [0, 1) with 24 bits. Reference hash: seed ^ tick_lo ^ tick_hi*0x9e3779b9.
// Philox: key (seed, row), counter (tick_lo, tick_hi, 0, 0), first output word.
__device__ __forceinline__ float random_unit(uint32_t rng, uint32_t seed, uint64_t tick, uint32_t row) {
    uint32_t lo = (uint32_t)tick, hi = (uint32_t)(tick >> 32);
    uint32_t bits = rng == 1u ? philox4x32_10_word0(lo, hi, 0u, 0u, seed, row)
                              : hash_u32(seed ^ lo ^ (hi * 0x9e3779b9u));
    return (float)(bits >> 8) * (1.0f / 16777216.0f);
}

// Mask, then repetition / frequency / presence in that order
// (greedy_sampler_repetition_f32.comp.template:42-50 plus the count term).
__device__ __forceinline__ float configured_logit(float x, bool allowed, uint32_t count, float rep, float freq,
                                                  float pres) {
    if (!allowed) return -__builtin_huge_valf();
    if (count == 0u) return x;
    float v = x < 0.0f ? x * rep : x / rep;
    float f = freq * (float)count;
    v = v - f;
    return v - pres;
}

}  // namespace nerve
