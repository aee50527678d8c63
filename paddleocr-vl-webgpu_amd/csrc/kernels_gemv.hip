// Decoder GEMV with fp16 weights for gfx950: out[r] = sum_c W[r][c] * x[c],
// W fp16 output-major [rows][columns], x and out f32, f32 accumulation.
// Replaces gemv_tiled_f16_weights (crates/pvlc-wgsl/src/lib.rs:1770-1835);
// arithmetic reference linear_f32 with a zero bias (crates/pvlc-cpu-ref/src/
// lib.rs:131-140, 1294-1303).  The LM-head variant also selects the top-1
// logit in the same launch (decoder_logits_top1_f32, pvlc-runtime-web
// decoder_stack_session.rs:308-366), and a standalone top-1 scans a logit row.
//
// A batch-1 GEMV streams the weights once, so it is HBM-bound: each wave owns
// RPW rows and reads them in 16-byte lanes (a wave-wide load is one 1 KiB
// contiguous run of a row); the vector, loaded once per workgroup through
// LDS, stays in registers (lane l holds the 8 columns of each of its 16-byte
// chunks); every row load of the wave is
// issued before the first dot product; one cross-lane reduction per row.
//
// Top-1 candidates are packed into one u64 whose unsigned order is the
// reference comparator: high word = total-order key with the sign bit flipped
// (signed order -> unsigned order), low word = ~index (equal keys: the lower
// index wins).  The waves of a workgroup combine their candidates in LDS and
// the last of them folds the result into slot blockIdx % 64 with an atomic max
// it does not wait for; a one-wave finish kernel, next on the stream, reads and
// clears the 64 slots and writes {index, f32 bits}.  No workgroup waits on a
// global round trip (a counted last-arrival hand-off kept a wave of every
// workgroup resident for two of them, which cost the LM head 6 us), and the
// slots sit one per 256-byte line so the atomics spread over 64 lines.  Slots
// are zero before a launch and zero after it, so stream-ordered launches reuse
// one zeroed workspace; launches that overlap on one workspace race.

#include <hip/hip_runtime.h>

#include <cstdint>

#include "pvlc_device.hpp"
#include "pvlc_internal.hpp"

namespace pvlc {
namespace {

constexpr int kGemvWaves = 4;
constexpr int kTopThreads = 256;
constexpr int kTopPerThread = 16;  // logits per thread per grid pass (4 x float4)
constexpr uint32_t kTopMaxWorkgroups = 1024;

// decoder_stack_session.rs:318-321, then the sign bit flipped so that the
// unsigned order of the high word is the signed order of the key.
__device__ inline uint64_t top1_pack(float value, uint32_t index) {
    const int32_t bits = __float_as_int(value);
    const uint32_t key = static_cast<uint32_t>(bits ^ static_cast<int32_t>(static_cast<uint32_t>(bits >> 31) >> 1));
    return (static_cast<uint64_t>(key ^ 0x80000000u) << 32) | static_cast<uint32_t>(~index);
}

__device__ inline uint64_t wave_max_u64(uint64_t v) {
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) {
        const uint64_t w = __shfl_xor(v, o);
        v = w > v ? w : v;
    }
    return v;
}

// LDS state of the top-1 fold; every wave runs top1_lds_init before any
// wave reaches top1_fold.
struct Top1Lds {
    uint64_t best;
    uint32_t waves_done;
};

// Zeroes the LDS state and synchronises the workgroup with fences limited to
// LDS, so the global loads in flight are not waited for here.
__device__ inline void top1_lds_init(Top1Lds &lds) {
    if (threadIdx.x == 0) {
        lds.best = 0;
        lds.waves_done = 0;
    }
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup", "local");
    __builtin_amdgcn_s_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "workgroup", "local");
}

// Folds a wave's candidate (wave-uniform) into the workgroup's in LDS; the
// last wave of the workgroup folds that into the workgroup's slot.
template <int WAVES>
__device__ void top1_fold(uint64_t wave_best, Top1Lds &lds, Top1Slot *slots) {
    if ((threadIdx.x & 63) != 0) return;
    __hip_atomic_fetch_max(&lds.best, wave_best, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
    const uint32_t rank = __hip_atomic_fetch_add(&lds.waves_done, 1u, __ATOMIC_ACQ_REL, __HIP_MEMORY_SCOPE_WORKGROUP);
    if (rank != WAVES - 1) return;
    const uint64_t b = __hip_atomic_load(&lds.best, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
    __hip_atomic_fetch_max(&slots[blockIdx.x % kTop1Slots].best, b, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// One wave: the best of the 64 slots (clearing them) as {index, f32 bits}.
__global__ __launch_bounds__(64) void top1_finish_kernel(Top1Slot *slots, uint32_t *result) {
    const int lane = threadIdx.x;
    uint64_t v = __hip_atomic_exchange(&slots[lane].best, uint64_t{0}, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    v = wave_max_u64(v);
    if (lane == 0) {
        const uint32_t key = static_cast<uint32_t>(v >> 32) ^ 0x80000000u;
        // the key transform is an involution: it recovers the f32 bits
        const uint32_t bits = key ^ (static_cast<uint32_t>(static_cast<int32_t>(key) >> 31) >> 1);
        result[0] = ~static_cast<uint32_t>(v);
        result[1] = bits;
    }
}

// CHUNKS = columns / 512: 16-byte chunks of a row per lane.

// The vector, loaded once per workgroup: thread t loads float4 chunks t,
// t + 256, ... into LDS, and after one barrier every lane reads the 8
// columns (c * 64 + lane) * 8 .. +8 of each chunk c it multiplies.  Each
// wave loading the whole vector itself put four times its bytes through the
// compute unit's load path next to the weights (decoder GEMV step replayed:
// 262.4 -> 253.8 us).  The 2048-column shape (o) measured 0.1 us slower this
// way and keeps the per-wave loads.
template <int CHUNKS>
__device__ inline void load_vector_lds(const float *__restrict__ vector, float4_t (&x)[CHUNKS][2]) {
    const int lane = threadIdx.x & 63;
    if constexpr (CHUNKS == 4) {
#pragma unroll
        for (int c = 0; c < CHUNKS; ++c) {
            x[c][0] = *reinterpret_cast<const float4_t *>(vector + (c * 64 + lane) * 8);
            x[c][1] = *reinterpret_cast<const float4_t *>(vector + (c * 64 + lane) * 8 + 4);
        }
    } else {
        constexpr int kQuads = CHUNKS * 512 / 4;  // float4 chunks of the vector
        static_assert(kQuads % (kGemvWaves * 64) == 0, "every thread loads the same number of chunks");
        __shared__ float4_t sv[kQuads];
        const int t = threadIdx.x;
#pragma unroll
        for (int i = 0; i < kQuads / (kGemvWaves * 64); ++i)
            sv[t + i * kGemvWaves * 64] = reinterpret_cast<const float4_t *>(vector)[t + i * kGemvWaves * 64];
        __syncthreads();
#pragma unroll
        for (int c = 0; c < CHUNKS; ++c) {
            x[c][0] = sv[(c * 64 + lane) * 2];
            x[c][1] = sv[(c * 64 + lane) * 2 + 1];
        }
    }
}

template <int CHUNKS, int RPW, bool TOP1>
__global__ __launch_bounds__(kGemvWaves * 64) void gemv_f16_kernel(const uint16_t *__restrict__ weights,
                                                                     const float *__restrict__ vector,
                                                                     float *__restrict__ out, uint32_t rows,
                                                                     Top1Slot *slots) {
    constexpr int kColumns = CHUNKS * 512;
    const int lane = threadIdx.x & 63;
    const int wave = threadIdx.x >> 6;
    const uint32_t row0 = (blockIdx.x * kGemvWaves + wave) * RPW;

    half8_t w[RPW][CHUNKS];
#pragma unroll
    for (int r = 0; r < RPW; ++r) {
        const uint32_t row = min(row0 + r, rows - 1);  // rows past the end re-read the last row, unstored
        const uint16_t *wr = weights + static_cast<size_t>(row) * kColumns;
#pragma unroll
        for (int c = 0; c < CHUNKS; ++c)  // streamed once: non-temporal, kept out of the caches' working set
            w[r][c] = __builtin_nontemporal_load(reinterpret_cast<const half8_t *>(wr + (c * 64 + lane) * 8));
    }
    float4_t x[CHUNKS][2];
    load_vector_lds<CHUNKS>(vector, x);
    __shared__ Top1Lds lds;
    if constexpr (TOP1) top1_lds_init(lds);  // while the loads are in flight
    uint64_t best = 0;  // below every candidate (the low word ~index is nonzero)
#pragma unroll
    for (int r = 0; r < RPW; ++r) {
        float acc = 0.f;
#pragma unroll
        for (int c = 0; c < CHUNKS; ++c)
#pragma unroll
            for (int j = 0; j < 8; ++j)
                acc = __builtin_fmaf(static_cast<float>(w[r][c][j]), x[c][j >> 2][j & 3], acc);
        acc = wave_sum(acc);
        if (row0 + r < rows) {
            if (out != nullptr && lane == 0) out[row0 + r] = acc;
            if constexpr (TOP1) {
                const uint64_t cand = top1_pack(acc, row0 + r);
                best = cand > best ? cand : best;
            }
        }
    }
    if constexpr (TOP1) top1_fold<kGemvWaves>(best, lds, slots);
}

// Global-memory access through an address picked as an integer: the cast to
// the global address space keeps global_load (not flat_load, which also
// drops the non-temporal hint).  Plain functions, not templates.
typedef const __attribute__((address_space(1))) half8_t *global_half8_ptr;
typedef __attribute__((address_space(1))) float *global_f32_ptr;
__device__ inline half8_t load_half8_nt(uint64_t base, size_t element) {
    return __builtin_nontemporal_load(reinterpret_cast<global_half8_ptr>(base + element * sizeof(uint16_t)));
}
__device__ inline void store_f32(uint64_t base, uint32_t index, float value) {
    *reinterpret_cast<global_f32_ptr>(base + static_cast<uint64_t>(index) * sizeof(float)) = value;
}

// Grouped GEMV: up to kGemvGroupMax matrices of one width that read the same
// vector (q, k and v of a layer; gate and up) in one launch, one row per wave
// with the arithmetic of gemv_f16_kernel (results bit-identical to separate
// launches).  Wave row i belongs to member m = the number of members that end
// at or before it.  Every argument is used unconditionally (pointers picked
// by masks, not branches), so they arrive in one batch of scalar loads rather
// than a chain of dependent ones (a chain cost about 1 us per launch).  The
// members come as separate arguments, weights, row ends, total and vector
// first: those 14 dwords are preloaded into SGPRs at wave launch
// (-amdgpu-kernarg-preload-count=16; a struct argument is not preloaded), so
// the weight loads issue without a scalar-load round trip.
template <int CHUNKS>
__global__ __launch_bounds__(kGemvWaves * 64) void gemv_group_f16_kernel(
    const uint16_t *w0, const uint16_t *w1, const uint16_t *w2, const uint16_t *w3, uint32_t end0, uint32_t end1,
    uint32_t end2, uint32_t total, const float *__restrict__ vector, float *o0, float *o1, float *o2, float *o3) {
    constexpr int kColumns = CHUNKS * 512;
    const int lane = threadIdx.x & 63;
    const uint32_t grow =
        static_cast<uint32_t>(__builtin_amdgcn_readfirstlane(static_cast<int>(blockIdx.x * kGemvWaves + (threadIdx.x >> 6))));
    const uint32_t rr = min(grow, total - 1);  // rows past the end re-read the last row, unstored
    const uint32_t m = (rr >= end0 ? 1u : 0u) + (rr >= end1 ? 1u : 0u) + (rr >= end2 ? 1u : 0u);
    auto pick = [m](uint64_t a0, uint64_t a1, uint64_t a2, uint64_t a3) {
        return (m == 0 ? a0 : 0ull) | (m == 1 ? a1 : 0ull) | (m == 2 ? a2 : 0ull) | (m == 3 ? a3 : 0ull);
    };
    const uint64_t wbase = pick(reinterpret_cast<uint64_t>(w0), reinterpret_cast<uint64_t>(w1),
                                reinterpret_cast<uint64_t>(w2), reinterpret_cast<uint64_t>(w3));
    const uint64_t obase = pick(reinterpret_cast<uint64_t>(o0), reinterpret_cast<uint64_t>(o1),
                                reinterpret_cast<uint64_t>(o2), reinterpret_cast<uint64_t>(o3));
    const uint32_t begin = static_cast<uint32_t>(pick(0, end0, end1, end2));
    const uint32_t row = rr - begin;
    half8_t w[CHUNKS];
#pragma unroll
    for (int c = 0; c < CHUNKS; ++c) w[c] = load_half8_nt(wbase, static_cast<size_t>(row) * kColumns + (c * 64 + lane) * 8);
    // The output pointers (not preloaded) are read only by the storing lane at
    // the end; named here, behind the weight loads, their scalar load returns
    // while the weights stream instead of in a round trip of its own after
    // the reduction.
    asm volatile("" ::"s"(o0), "s"(o1), "s"(o2), "s"(o3));
    float4_t x[CHUNKS][2];
    load_vector_lds<CHUNKS>(vector, x);
    float acc = 0.f;
#pragma unroll
    for (int c = 0; c < CHUNKS; ++c)
#pragma unroll
        for (int j = 0; j < 8; ++j) acc = __builtin_fmaf(static_cast<float>(w[c][j]), x[c][j >> 2][j & 3], acc);
    acc = wave_sum(acc);
    if (grow < total && lane == 0) store_f32(obase, row, acc);
}

// Standalone top-1 over a logit row: a grid-stride scan in float4 lanes
// (VEC: 16-byte aligned row) or scalars, then the same fold into the slots.
template <bool VEC>
__global__ __launch_bounds__(kTopThreads) void logits_top1_kernel(const float *__restrict__ logits, uint32_t vocab,
                                                                  Top1Slot *slots) {
    __shared__ Top1Lds lds;
    top1_lds_init(lds);
    uint64_t best = 0;
    const uint32_t stride = gridDim.x * (kTopThreads * kTopPerThread);
    for (uint32_t base = blockIdx.x * (kTopThreads * kTopPerThread); base < vocab; base += stride) {
#pragma unroll
        for (int k = 0; k < kTopPerThread / 4; ++k) {
            const uint32_t i = base + (k * kTopThreads + threadIdx.x) * 4;
            if (VEC && i + 3 < vocab) {
                const float4_t v = *reinterpret_cast<const float4_t *>(logits + i);
#pragma unroll
                for (int j = 0; j < 4; ++j) {
                    const uint64_t c = top1_pack(v[j], i + j);
                    best = c > best ? c : best;
                }
            } else {
#pragma unroll
                for (int j = 0; j < 4; ++j) {
                    if (i + j < vocab) {
                        const uint64_t c = top1_pack(logits[i + j], i + j);
                        best = c > best ? c : best;
                    }
                }
            }
        }
    }
    top1_fold<kTopThreads / 64>(wave_max_u64(best), lds, slots);
}

template <int CHUNKS, bool TOP1>
int launch_gemv_rows(const uint16_t *weights, const float *vector, float *out, uint32_t rows, Top1Slot *slots,
                     hipStream_t st) {
    // One row per wave for the per-layer projections (the launch is one
    // memory round trip), two rows per wave for the LM head (measured best:
    // 6.9 TB/s at 103424 x 1024, against 6.1 TB/s at four rows per wave).
    if (rows <= 8192) {
        const unsigned wgs = (rows + kGemvWaves - 1) / kGemvWaves;
        hipLaunchKernelGGL((gemv_f16_kernel<CHUNKS, 1, TOP1>), dim3(wgs), dim3(kGemvWaves * 64), 0, st, weights,
                           vector, out, rows, slots);
    } else {
        const unsigned wgs = (rows + kGemvWaves * 2 - 1) / (kGemvWaves * 2);
        hipLaunchKernelGGL((gemv_f16_kernel<CHUNKS, 2, TOP1>), dim3(wgs), dim3(kGemvWaves * 64), 0, st, weights,
                           vector, out, rows, slots);
    }
    return static_cast<int>(hipGetLastError());
}

template <bool TOP1>
int launch_gemv(const uint16_t *weights, const float *vector, float *out, uint32_t rows, uint32_t columns,
                Top1Slot *slots, void *stream) {
    hipStream_t st = static_cast<hipStream_t>(stream);
    switch (columns) {
        case 1024: return launch_gemv_rows<2, TOP1>(weights, vector, out, rows, slots, st);
        case 2048: return launch_gemv_rows<4, TOP1>(weights, vector, out, rows, slots, st);
        case 3072: return launch_gemv_rows<6, TOP1>(weights, vector, out, rows, slots, st);
        default: return static_cast<int>(hipErrorInvalidValue);
    }
}

int launch_top1_finish(Top1Slot *slots, uint32_t *result, hipStream_t st) {
    hipLaunchKernelGGL(top1_finish_kernel, dim3(1), dim3(64), 0, st, slots, result);
    return static_cast<int>(hipGetLastError());
}

}  // namespace

int launch_gemv_group_f16(const GemvGroup &group, const float *vector, uint32_t columns, void *stream) {
    hipStream_t st = static_cast<hipStream_t>(stream);
    const unsigned wgs = (group.total + kGemvWaves - 1) / kGemvWaves;
    static_assert(kGemvGroupMax == 4, "four member slots");
#define PVLC_GEMV_GROUP_LAUNCH(C)                                                                                   \
    hipLaunchKernelGGL(gemv_group_f16_kernel<C>, dim3(wgs), dim3(kGemvWaves * 64), 0, st, group.weights[0],        \
                       group.weights[1], group.weights[2], group.weights[3], group.end[0], group.end[1], group.end[2], \
                       group.total, vector, group.out[0], group.out[1], group.out[2], group.out[3])
    switch (columns) {
        case 1024: PVLC_GEMV_GROUP_LAUNCH(2); break;
        case 2048: PVLC_GEMV_GROUP_LAUNCH(4); break;
        case 3072: PVLC_GEMV_GROUP_LAUNCH(6); break;
        default: return static_cast<int>(hipErrorInvalidValue);
    }
#undef PVLC_GEMV_GROUP_LAUNCH
    return static_cast<int>(hipGetLastError());
}

int launch_gemv_f16(const uint16_t *weights, const float *vector, float *out, uint32_t rows, uint32_t columns,
                    void *stream) {
    return launch_gemv<false>(weights, vector, out, rows, columns, nullptr, stream);
}

int launch_gemv_top1_f16(const uint16_t *weights, const float *vector, float *logits, uint32_t rows,
                         uint32_t columns, Top1Slot *slots, uint32_t *result, void *stream) {
    if (const int e = launch_gemv<true>(weights, vector, logits, rows, columns, slots, stream)) return e;
    return launch_top1_finish(slots, result, static_cast<hipStream_t>(stream));
}

int launch_logits_top1_f32(const float *logits, uint32_t vocab, Top1Slot *slots, uint32_t *result, void *stream) {
    hipStream_t st = static_cast<hipStream_t>(stream);
    const uint32_t per_wg = kTopThreads * kTopPerThread;
    const uint32_t wgs = std::min<uint32_t>((vocab + per_wg - 1) / per_wg, kTopMaxWorkgroups);
    if (reinterpret_cast<uintptr_t>(logits) % 16 == 0)
        hipLaunchKernelGGL(logits_top1_kernel<true>, dim3(wgs), dim3(kTopThreads), 0, st, logits, vocab, slots);
    else
        hipLaunchKernelGGL(logits_top1_kernel<false>, dim3(wgs), dim3(kTopThreads), 0, st, logits, vocab, slots);
    if (const int e = static_cast<int>(hipGetLastError())) return e;
    return launch_top1_finish(slots, result, st);
}

}  // namespace pvlc
