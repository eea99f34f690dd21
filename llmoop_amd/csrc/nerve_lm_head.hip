// nerve_lm_head.hip -- the LM-head projection with the sampler's epilogue:
// logits[b][v] = scale * sum_d frames[b][d] * weight[v][d] (bf16 inputs, f32
// accumulation and output), as tied_output_projection_batch_bf16.comp.template
// computes it (one output per (batch row, vocabulary row), OUTPUT_SCALE
// applied to the sum), plus, for every batch row and every 64 vocabulary
// columns, the tile record the sampling step reads: the largest order key of
// the 64 logits and the count of NaNs among them.
//
// A workgroup of 8 waves computes a 256 x 128 (batch x vocabulary) block with
// v_mfma_f32_32x32x16_bf16: wave w owns the 64 x 64 sub-block (w % 4, w / 4),
// 2 x 2 MFMA tiles of 32 x 32 (64 accumulators per lane). The reduction
// dimension goes through LDS 64 columns at a time, double-buffered, with the
// global loads of a stage issued several stages ahead (16-byte buffer loads; rows
// past the batch or the vocabulary read zero and cost no traffic). LDS rows
// are padded to 72 bf16 (144 bytes) so the 16-byte fragment reads of 32 rows
// spread over the banks.
//
// MFMA operand layout (v_mfma_f32_32x32x16_bf16, checked on the GPU): lane l
// supplies A[l % 32][8 (l / 32) .. + 8] and B[8 (l / 32) .. + 8][l % 32];
// accumulator r of lane l is C[8 (r / 4) + 4 (l / 32) + r % 4][l % 32].
#include <atomic>

#include "nerve_sampler_device.h"

namespace nerve {

namespace {

constexpr int kLmThreads = 512;
#ifndef NERVE_LM_KT
#define NERVE_LM_KT 64
#endif
#ifndef NERVE_LM_WG_PER_CU
#define NERVE_LM_WG_PER_CU 1
#endif
constexpr uint32_t kMt = 256, kNt = 128, kKt = NERVE_LM_KT, kRow = kKt + 8;  // LDS row: kKt + 8 bf16
constexpr uint32_t kStageA = kMt * kRow, kStageW = kNt * kRow;      // bf16 per stage buffer
constexpr uint32_t kLmLds = 2u * (kStageA + kStageW) * 2u;          // bytes (110,592 with 64-column stages)

typedef __attribute__((ext_vector_type(8))) __bf16 bf16x8;
typedef __attribute__((ext_vector_type(16))) float f32x16;
typedef __attribute__((ext_vector_type(4))) uint32_t u32x4v;

constexpr int kChunkA = (int)(kMt * kKt / 8u / kLmThreads);  // 16-byte chunks per thread and stage
constexpr int kChunkW = (int)(kNt * kKt / 8u / kLmThreads);
constexpr uint32_t kChunksPerRow = kKt / 8u;
struct StageRegs {
    u32x4v a[kChunkA];
    u32x4v w[kChunkW];
};

template <int NS>
__global__ __launch_bounds__(kLmThreads, NERVE_LM_WG_PER_CU) void lm_head_kernel(const uint16_t *frames, uint64_t lda, const uint16_t *weight,
                                                             uint64_t ldw, uint32_t B, uint32_t D, uint32_t V, float scale,
                                                             float *logits, uint64_t ldc, uint2 *records, uint32_t rec_stride) {
    extern __shared__ __align__(16) uint16_t s_lm[];
    const uint32_t tid = threadIdx.x, lane = tid & 63u, wave = tid >> 6;
    const uint32_t n0 = blockIdx.x * kNt, m0 = blockIdx.y * kMt;
    const uint32_t mrows = B - m0 < kMt ? B - m0 : kMt;
    const uint32_t nrows = V - n0 < kNt ? V - n0 : kNt;
    const __amdgpu_buffer_rsrc_t ra = __builtin_amdgcn_make_buffer_rsrc(
        (void *)(frames + (uint64_t)m0 * lda), (short)0, (int)((uint64_t)(mrows - 1u) * lda * 2u + (uint64_t)D * 2u), 0x00020000);
    const __amdgpu_buffer_rsrc_t rw = __builtin_amdgcn_make_buffer_rsrc(
        (void *)(weight + (uint64_t)n0 * ldw), (short)0, (int)((uint64_t)(nrows - 1u) * ldw * 2u + (uint64_t)D * 2u), 0x00020000);
    // chunk c of a stage: row c / 8, 16 bytes at column 8 (c % 8); rows past the
    // valid ones are out of the resource's range (they read zero)
    auto issue = [&](StageRegs &r, uint32_t k0) __attribute__((always_inline)) {
#pragma unroll
        for (int i = 0; i < kChunkA; ++i) {
            const uint32_t c = tid + (uint32_t)i * kLmThreads, row = c / kChunksPerRow, col = k0 + (c % kChunksPerRow) * 8u;
            const uint32_t off = row < mrows ? (uint32_t)(((uint64_t)row * lda + col) * 2u) : 0x7fffffffu;
            r.a[i] = __builtin_amdgcn_raw_buffer_load_b128(ra, off, 0, 0);
        }
#pragma unroll
        for (int i = 0; i < kChunkW; ++i) {
            const uint32_t c = tid + (uint32_t)i * kLmThreads, row = c / kChunksPerRow, col = k0 + (c % kChunksPerRow) * 8u;
            const uint32_t off = row < nrows ? (uint32_t)(((uint64_t)row * ldw + col) * 2u) : 0x7fffffffu;
            r.w[i] = __builtin_amdgcn_raw_buffer_load_b128(rw, off, 0, 0);
        }
    };
    auto store = [&](const StageRegs &r, uint32_t buf) __attribute__((always_inline)) {
        uint16_t *sa = s_lm + buf * (kStageA + kStageW);
        uint16_t *sw = sa + kStageA;
#pragma unroll
        for (int i = 0; i < kChunkA; ++i) {
            const uint32_t c = tid + (uint32_t)i * kLmThreads;
            *(u32x4v *)(sa + (c / kChunksPerRow) * kRow + (c % kChunksPerRow) * 8u) = r.a[i];
        }
#pragma unroll
        for (int i = 0; i < kChunkW; ++i) {
            const uint32_t c = tid + (uint32_t)i * kLmThreads;
            *(u32x4v *)(sw + (c / kChunksPerRow) * kRow + (c % kChunksPerRow) * 8u) = r.w[i];
        }
    };
    const uint32_t wm = wave & 3u, wn = wave >> 2;
    const bool active = wm * 64u < mrows;  // waves past the batch only load and sync
    f32x16 acc[2][2];
#pragma unroll
    for (int i = 0; i < 2; ++i)
#pragma unroll
        for (int j = 0; j < 2; ++j) acc[i][j] = (f32x16){};
    auto compute = [&](uint32_t buf) __attribute__((always_inline)) {
        if (!active) return;
        const uint16_t *sa = s_lm + buf * (kStageA + kStageW);
        const uint16_t *sw = sa + kStageA;
#pragma unroll
        for (int ks = 0; ks < (int)(kKt / 16u); ++ks) {
            const uint32_t kk = (uint32_t)ks * 16u + 8u * (lane >> 5);
            bf16x8 af[2], bf[2];
#pragma unroll
            for (int i = 0; i < 2; ++i)
                af[i] = __builtin_bit_cast(bf16x8, *(const u32x4v *)(sa + (wm * 64u + (uint32_t)i * 32u + (lane & 31u)) * kRow + kk));
#pragma unroll
            for (int j = 0; j < 2; ++j)
                bf[j] = __builtin_bit_cast(bf16x8, *(const u32x4v *)(sw + (wn * 64u + (uint32_t)j * 32u + (lane & 31u)) * kRow + kk));
#pragma unroll
            for (int i = 0; i < 2; ++i)
#pragma unroll
                for (int j = 0; j < 2; ++j) acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(af[i], bf[j], acc[i][j], 0, 0, 0);
        }
    };

    const uint32_t S = D / kKt;  // D is a multiple of 64 (checked by the host), so of kKt
    // A ring of NS register sets: stage s + 1 .. s + NS are in flight while
    // stage s is computed from LDS buffer s & 1; set s % NS is free once
    // stage s is in LDS, and takes stage s + NS.
    auto kofs = [&](uint32_t st) __attribute__((always_inline)) -> uint32_t { return st * kKt; };
    StageRegs R[NS];
    static_for<0, NS>([&](auto Q) __attribute__((always_inline)) {
        if ((uint32_t)Q < S) issue(R[Q], kofs((uint32_t)Q));
    });
    store(R[0], 0u);
    __syncthreads();
    // Steady state, free of conditionals (so the compiler's wait counts
    // follow each set exactly instead of waiting for every load in flight):
    // NS steps per trip, each issuing stage s + NS.
    uint32_t s0 = 0;
    for (; s0 + 2u * NS <= S; s0 += NS) {
        static_for<0, NS>([&](auto Q) __attribute__((always_inline)) {
            constexpr int q = Q;
            const uint32_t s = s0 + (uint32_t)q;
            issue(R[q], kofs(s + NS));
            compute(s & 1u);
            store(R[(q + 1) % NS], (s + 1u) & 1u);
            __syncthreads();
        });
    }
    // the last stages (fewer than 2 NS)
    static_for<0, 2 * NS>([&](auto Q) __attribute__((always_inline)) {
        constexpr int q = Q;
        const uint32_t s = s0 + (uint32_t)q;
        if (s < S) {
            if (s + NS < S) issue(R[q % NS], kofs(s + NS));
            compute(s & 1u);
            if (s + 1u < S) store(R[(q + 1) % NS], (s + 1u) & 1u);
            __syncthreads();
        }
    });

    // epilogue: scaled logits, and the tile record of each row's 64 columns
    if (!active) return;
    const uint32_t tile = n0 / 64u + wn;
    const uint64_t half = lane < 32u ? 0x00000000ffffffffull : 0xffffffff00000000ull;
#pragma unroll
    for (int i = 0; i < 2; ++i) {
#pragma unroll
        for (int r = 0; r < 16; ++r) {
            const uint32_t m = m0 + wm * 64u + (uint32_t)i * 32u + 8u * (uint32_t)(r / 4) + 4u * (lane >> 5) + (uint32_t)(r % 4);
            uint32_t key = 0u, nan = 0u;
            uint64_t nb = 0u;
#pragma unroll
            for (int j = 0; j < 2; ++j) {
                const uint32_t n = n0 + wn * 64u + (uint32_t)j * 32u + (lane & 31u);
                const float v = acc[i][j][r] * scale;
                const bool ok = m < B && n < V;
                if (ok) logits[(uint64_t)m * ldc + n] = v;
                const uint32_t bits = f2u(v);
                key = max(key, ok ? raw_order_key(bits) : 0u);
                nb = __ballot(ok && (bits & 0x7fffffffu) > 0x7f800000u);
                nan += (uint32_t)__popcll(nb & half);
            }
#pragma unroll
            for (int o = 1; o < 32; o <<= 1) key = max(key, (uint32_t)__shfl_xor((int)key, o, 64));
            if ((lane & 31u) == 0u && m < B && records && n0 + wn * 64u < V)
                records[(uint64_t)m * rec_stride + tile] = make_uint2(key, nan);
        }
    }
}

#ifndef NERVE_LM_STAGES
#define NERVE_LM_STAGES 3
#endif
constexpr int kLmStages = NERVE_LM_STAGES;  // register sets in the prefetch ring
std::atomic<uint32_t> g_lds_set[kMaxDevices];

}  // namespace

hipError_t launch_lm_head(const uint16_t *frames, uint64_t frames_ld, const uint16_t *weight, uint64_t weight_ld,
                          uint32_t batch, uint32_t input_size, uint32_t vocab, float scale, float *logits, uint64_t logits_ld,
                          uint2 *records, uint32_t rec_stride, hipStream_t stream) {
    int dev = 0;
    hipError_t e = hipGetDevice(&dev);
    if (e != hipSuccess) return e;
    e = ensure_dyn_lds(lm_head_kernel<kLmStages>, dev, kLmLds, g_lds_set);
    if (e != hipSuccess) return e;
    const dim3 grid((vocab + kNt - 1u) / kNt, (batch + kMt - 1u) / kMt);
    hipLaunchKernelGGL(lm_head_kernel<kLmStages>, grid, dim3(kLmThreads), kLmLds, stream, frames, frames_ld, weight, weight_ld, batch,
                       input_size, vocab, scale, logits, logits_ld, records, rec_stride);
    return hipGetLastError();
}

}  // namespace nerve
