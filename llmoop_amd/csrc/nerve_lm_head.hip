// nerve_lm_head.hip -- the LM-head projection with the sampler's epilogue:
// logits[b][v] = scale * sum_d frames[b][d] * weight[v][d] (bf16 inputs, f32
// accumulation and output), as tied_output_projection_batch_bf16.comp.template
// computes it (one output per (batch row, vocabulary row), OUTPUT_SCALE
// applied to the sum), plus, for every batch row and every 64 vocabulary
// columns, the tile record the sampling step reads: the largest order key of
// the 64 logits and the count of NaNs among them.
//
// A workgroup of 16 waves computes a 256 x 256 (batch x vocabulary) block
// with v_mfma_f32_32x32x16_bf16: wave w owns the 64 x 64 sub-block
// (w % 4, w / 4), 2 x 2 MFMA tiles of 32 x 32 (64 accumulators per lane). The
// reduction dimension goes through LDS 64 columns at a time, double-buffered,
// with the global loads of the next stage issued before the current one is
// computed (16-byte buffer loads; rows past the batch or the vocabulary read
// zero and cost no traffic). LDS rows are padded to 72 bf16 (144 bytes) so
// the 16-byte fragment reads of 32 rows spread over the banks. The block
// shape is a template parameter (LmCfg); the alternatives measured are listed
// where the shape is chosen.
//
// MFMA operand layout (v_mfma_f32_32x32x16_bf16, checked on the GPU): lane l
// supplies A[l % 32][8 (l / 32) .. + 8] and B[8 (l / 32) .. + 8][l % 32];
// accumulator r of lane l is C[8 (r / 4) + 4 (l / 32) + r % 4][l % 32].
#include <atomic>

#include "nerve_sampler_device.h"

namespace nerve {

namespace {

typedef __attribute__((ext_vector_type(8))) __bf16 bf16x8;
typedef __attribute__((ext_vector_type(16))) float f32x16;
typedef __attribute__((ext_vector_type(4))) uint32_t u32x4v;

// Block shape: WM x WN waves, each owning TI x TJ MFMA tiles of 32 x 32, the
// reduction staged KT columns at a time through double-buffered LDS, NS
// register sets of loads in flight.
template <int WM_, int WN_, int TI_, int TJ_, int KT_, int NS_, int WG_PER_CU_>
struct LmCfg {
    static constexpr int WM = WM_, WN = WN_, TI = TI_, TJ = TJ_, NS = NS_, WG_PER_CU = WG_PER_CU_;
    static constexpr int kThreads = 64 * WM * WN;
    static constexpr uint32_t kKt = KT_, kRow = KT_ + 8;  // LDS row: KT + 8 bf16 (spreads the 32 rows of a fragment read)
    static constexpr uint32_t kMt = 32u * WM * TI, kNt = 32u * WN * TJ;
    static constexpr uint32_t kStageA = kMt * kRow, kStageW = kNt * kRow;  // bf16 per stage buffer
    static constexpr uint32_t kLds = 2u * (kStageA + kStageW) * 2u;        // bytes
    static constexpr uint32_t kChunksPerRow = KT_ / 8u;
    static constexpr int kChunkA = (int)(kMt * KT_ / 8u / kThreads);  // 16-byte chunks per thread and stage
    static constexpr int kChunkW = (int)(kNt * KT_ / 8u / kThreads);
    static_assert(kChunkA * kThreads * 8 == (int)(kMt * KT_) && kChunkW * kThreads * 8 == (int)(kNt * KT_), "chunks");
    static_assert(TJ % 2 == 0, "a wave covers whole 64-column tiles");
};

// Float maximum over each aligned group of 32 lanes, NaN ignored (fmaxf
// returns the other operand): rotations by 1, 2, 4, 8 within each row of 16
// lanes (DPP row_ror, dpp_ctrl 0x121..0x128), then one swap of the two rows
// of the group.
__device__ __forceinline__ float fmax32(float v) {
    v = fmaxf(v, u2f((uint32_t)__builtin_amdgcn_update_dpp(0, (int)f2u(v), 0x121, 0xf, 0xf, false)));
    v = fmaxf(v, u2f((uint32_t)__builtin_amdgcn_update_dpp(0, (int)f2u(v), 0x122, 0xf, 0xf, false)));
    v = fmaxf(v, u2f((uint32_t)__builtin_amdgcn_update_dpp(0, (int)f2u(v), 0x124, 0xf, 0xf, false)));
    v = fmaxf(v, u2f((uint32_t)__builtin_amdgcn_update_dpp(0, (int)f2u(v), 0x128, 0xf, 0xf, false)));
    return fmaxf(v, u2f((uint32_t)__shfl_xor((int)f2u(v), 16, 64)));
}

template <typename Cfg>
__global__ __launch_bounds__(Cfg::kThreads, Cfg::WG_PER_CU) void lm_head_kernel(
    const uint16_t *frames, uint64_t lda, const uint16_t *weight, uint64_t ldw, uint32_t B, uint32_t D, uint32_t V,
    float scale, float *logits, uint64_t ldc, uint2 *records, uint32_t rec_stride, uint32_t full_blocks,
    uint32_t tail_width) {
    constexpr int NS = Cfg::NS, TI = Cfg::TI, TJ = Cfg::TJ;
    constexpr int NT = Cfg::kThreads;
    constexpr uint32_t kKt = Cfg::kKt, kRow = Cfg::kRow, kMt = Cfg::kMt, kNt = Cfg::kNt;
    constexpr uint32_t kStageA = Cfg::kStageA, kStageW = Cfg::kStageW, kCpr = Cfg::kChunksPerRow;
    struct StageRegs {
        u32x4v a[Cfg::kChunkA];
        u32x4v w[Cfg::kChunkW];
    };
    extern __shared__ __align__(16) uint16_t s_lm[];
    const uint32_t tid = threadIdx.x, lane = tid & 63u, wave = tid >> 6;
    // the first full_blocks blocks are kNt columns wide; the rest (the last,
    // partial round of the grid) tail_width, so that round spreads over more CUs
    const uint32_t bx = blockIdx.x;
    const uint32_t n0 = bx < full_blocks ? bx * kNt : full_blocks * kNt + (bx - full_blocks) * tail_width;
    const uint32_t width = bx < full_blocks ? kNt : tail_width;
    const uint32_t m0 = blockIdx.y * kMt;
    const uint32_t mrows = B - m0 < kMt ? B - m0 : kMt;
    const uint32_t nrows = V - n0 < width ? V - n0 : width;
    const uint32_t nend = n0 + nrows;  // columns of this block: [n0, nend)
    const __amdgpu_buffer_rsrc_t ra = __builtin_amdgcn_make_buffer_rsrc(
        (void *)(frames + (uint64_t)m0 * lda), (short)0, (int)((uint64_t)(mrows - 1u) * lda * 2u + (uint64_t)D * 2u), 0x00020000);
    const __amdgpu_buffer_rsrc_t rw = __builtin_amdgcn_make_buffer_rsrc(
        (void *)(weight + (uint64_t)n0 * ldw), (short)0, (int)((uint64_t)(nrows - 1u) * ldw * 2u + (uint64_t)D * 2u), 0x00020000);
    // chunk c of a stage: row c / kCpr, 16 bytes at column 8 (c % kCpr); rows
    // past the valid ones are out of the resource's range (they read zero)
    auto issue = [&](StageRegs &r, uint32_t k0) __attribute__((always_inline)) {
#pragma unroll
        for (int i = 0; i < Cfg::kChunkA; ++i) {
            const uint32_t c = tid + (uint32_t)i * NT, row = c / kCpr, col = k0 + (c % kCpr) * 8u;
            const uint32_t off = row < mrows ? (uint32_t)(((uint64_t)row * lda + col) * 2u) : 0x7fffffffu;
            r.a[i] = __builtin_amdgcn_raw_buffer_load_b128(ra, off, 0, 0);
        }
#pragma unroll
        for (int i = 0; i < Cfg::kChunkW; ++i) {
            const uint32_t c = tid + (uint32_t)i * NT, row = c / kCpr, col = k0 + (c % kCpr) * 8u;
            const uint32_t off = row < nrows ? (uint32_t)(((uint64_t)row * ldw + col) * 2u) : 0x7fffffffu;
            r.w[i] = __builtin_amdgcn_raw_buffer_load_b128(rw, off, 0, 0);
        }
    };
    auto store = [&](const StageRegs &r, uint32_t buf) __attribute__((always_inline)) {
        uint16_t *sa = s_lm + buf * (kStageA + kStageW);
        uint16_t *sw = sa + kStageA;
#pragma unroll
        for (int i = 0; i < Cfg::kChunkA; ++i) {
            const uint32_t c = tid + (uint32_t)i * NT;
            *(u32x4v *)(sa + (c / kCpr) * kRow + (c % kCpr) * 8u) = r.a[i];
        }
#pragma unroll
        for (int i = 0; i < Cfg::kChunkW; ++i) {
            const uint32_t c = tid + (uint32_t)i * NT;
            *(u32x4v *)(sw + (c / kCpr) * kRow + (c % kCpr) * 8u) = r.w[i];
        }
    };
    const uint32_t wm = wave % (uint32_t)Cfg::WM, wn = wave / (uint32_t)Cfg::WM;
    const bool active = wm * 32u * TI < mrows && wn * 32u * TJ < nrows;  // others only load and sync
    f32x16 acc[TI][TJ];
#pragma unroll
    for (int i = 0; i < TI; ++i)
#pragma unroll
        for (int j = 0; j < TJ; ++j) acc[i][j] = (f32x16){};
    auto compute = [&](uint32_t buf) __attribute__((always_inline)) {
        if (!active) return;
        const uint16_t *sa = s_lm + buf * (kStageA + kStageW);
        const uint16_t *sw = sa + kStageA;
#pragma unroll
        for (int ks = 0; ks < (int)(kKt / 16u); ++ks) {
            const uint32_t kk = (uint32_t)ks * 16u + 8u * (lane >> 5);
            bf16x8 af[TI], bf[TJ];
#pragma unroll
            for (int i = 0; i < TI; ++i)
                af[i] = __builtin_bit_cast(bf16x8, *(const u32x4v *)(sa + (wm * 32u * TI + (uint32_t)i * 32u + (lane & 31u)) * kRow + kk));
#pragma unroll
            for (int j = 0; j < TJ; ++j)
                bf[j] = __builtin_bit_cast(bf16x8, *(const u32x4v *)(sw + (wn * 32u * TJ + (uint32_t)j * 32u + (lane & 31u)) * kRow + kk));
#pragma unroll
            for (int i = 0; i < TI; ++i)
#pragma unroll
                for (int j = 0; j < TJ; ++j) acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(af[i], bf[j], acc[i][j], 0, 0, 0);
        }
    };

    const uint32_t S = D / kKt;  // D is a multiple of 64 (checked by the host), so of kKt
    // A ring of NS register sets: stages s + 1 .. s + NS are in flight while
    // stage s is computed from LDS buffer s & 1; set s % NS is free once
    // stage s is in LDS, and takes stage s + NS.
    StageRegs R[NS];
    static_for<0, NS>([&](auto Q) __attribute__((always_inline)) {
        if ((uint32_t)Q < S) issue(R[Q], (uint32_t)Q * kKt);
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
            issue(R[q], (s + NS) * kKt);
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
            if (s + NS < S) issue(R[q % NS], (s + NS) * kKt);
            compute(s & 1u);
            if (s + 1u < S) store(R[(q + 1) % NS], (s + 1u) & 1u);
            __syncthreads();
        }
    });

    // epilogue: scaled logits, and the tile record of each row's 64 columns
    // (columns 64 p .. 64 p + 63 of the wave are its MFMA tiles 2 p, 2 p + 1)
    if (!active) return;
    const uint64_t half = lane < 32u ? 0x00000000ffffffffull : 0xffffffff00000000ull;
#pragma unroll
    for (int i = 0; i < TI; ++i) {
#pragma unroll
        for (int r = 0; r < 16; ++r) {
            const uint32_t m = m0 + wm * 32u * TI + (uint32_t)i * 32u + 8u * (uint32_t)(r / 4) + 4u * (lane >> 5) + (uint32_t)(r % 4);
#pragma unroll
            for (int p = 0; p < TJ / 2; ++p) {
                // the largest value as a float (NaN and columns past the
                // vocabulary do not count), turned into its order key once;
                // +0 and -0 share a key, so fmaxf's choice between them is moot
                float mx = __builtin_nanf("");
                uint32_t nan = 0u;
#pragma unroll
                for (int jj = 0; jj < 2; ++jj) {
                    const int j = 2 * p + jj;
                    const uint32_t n = n0 + wn * 32u * TJ + (uint32_t)j * 32u + (lane & 31u);
                    const float v = acc[i][j][r] * scale;
                    const bool ok = m < B && n < nend;
                    if (ok) logits[(uint64_t)m * ldc + n] = v;
                    mx = fmaxf(mx, ok ? v : __builtin_nanf(""));
                    nan += (uint32_t)__popcll(__ballot(ok && v != v) & half);
                }
                const uint32_t key = raw_order_key(f2u(fmax32(mx)));
                const uint32_t c0 = n0 + wn * 32u * TJ + 64u * (uint32_t)p;
                if ((lane & 31u) == 0u && m < B && records && c0 < nend)
                    records[(uint64_t)m * rec_stride + c0 / 64u] = make_uint2(key, nan);
            }
        }
    }
}

// 1024 threads (16 waves), 256 x 256 blocks, 64 x 64 per wave, 64-column
// stages, one set of loads in flight (128 VGPRs: four waves per SIMD). The
// frames are read once per 256 vocabulary rows instead of once per 128.
// Measured on MI355X at B=256, D=4096, V=151936 (gemm + records, us, same
// session): this shape 491 against 527 for 8 waves in 256 x 128 blocks with
// 3 sets in flight. Also measured with 8 waves: 256 x 256 blocks with
// 128 x 128 per wave (4 waves, accumulators in AGPRs) 623; 256 x 256 with
// 64 x 128 per wave 515-518; 2 / 4 / 5 sets in flight 518-544; two
// workgroups per CU with 32-column stages 525; non-temporal weight loads,
// padded row strides and rotated stage order within noise. Loading the
// stages straight into LDS (buffer loads with the LDS bit, 32-column stages,
// 3 or 4 stages in flight in 4 or 5 LDS buffers, swizzled rows): 527-535
// against 472-485 for this shape in the same session.
using Lm = LmCfg<4, 4, 2, 2, 64, 1, 1>;

std::atomic<uint32_t> g_lds_set[kMaxDevices];

}  // namespace

hipError_t launch_lm_head(const uint16_t *frames, uint64_t frames_ld, const uint16_t *weight, uint64_t weight_ld,
                          uint32_t batch, uint32_t input_size, uint32_t vocab, float scale, float *logits, uint64_t logits_ld,
                          uint2 *records, uint32_t rec_stride, hipStream_t stream) {
    int dev = 0;
    hipError_t e = hipGetDevice(&dev);
    if (e != hipSuccess) return e;
    e = ensure_dyn_lds(lm_head_kernel<Lm>, dev, Lm::kLds, g_lds_set);
    if (e != hipSuccess) return e;
    // Blocks of kNt columns fill whole rounds of the CUs (one block per CU);
    // the columns left for a last, partial round go to blocks of kNt / 2, so
    // that round takes about half as long.
    static std::atomic<int> cu_count[kMaxDevices];
    if (dev < 0 || dev >= kMaxDevices) return hipErrorInvalidDevice;
    int cus = cu_count[dev].load(std::memory_order_relaxed);
    if (cus == 0) {
        e = hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev);
        if (e != hipSuccess) return e;
        cu_count[dev].store(cus, std::memory_order_relaxed);
    }
    const uint32_t blocks = (vocab + Lm::kNt - 1u) / Lm::kNt;
    uint32_t full = blocks, tail_width = Lm::kNt, tail = 0u;
    const uint32_t rounds = blocks / (uint32_t)cus;
    if (rounds > 0u && blocks % (uint32_t)cus != 0u) {
        full = rounds * (uint32_t)cus;
        tail_width = Lm::kNt / 2u;
        tail = (vocab - full * Lm::kNt + tail_width - 1u) / tail_width;
    }
    const dim3 grid(full + tail, (batch + Lm::kMt - 1u) / Lm::kMt);
    hipLaunchKernelGGL(lm_head_kernel<Lm>, grid, dim3(Lm::kThreads), Lm::kLds, stream, frames, frames_ld, weight, weight_ld, batch,
                       input_size, vocab, scale, logits, logits_ld, records, rec_stride, full, tail_width);
    return hipGetLastError();
}

}  // namespace nerve
