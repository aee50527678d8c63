// Decoder GEMV with fp16 weights for gfx950: out[r] = sum_c W[r][c] * x[c],
// W fp16 output-major [rows][columns], x and out f32, f32 accumulation.
// Replaces gemv_tiled_f16_weights (crates/pvlc-wgsl/src/lib.rs:1770-1835);
// arithmetic reference linear_f32 with a zero bias (crates/pvlc-cpu-ref/src/
// lib.rs:131-140, 1294-1303).
//
// A batch-1 GEMV streams the weights once, so it is HBM-bound: each wave owns
// RPW rows and reads them in 16-byte lanes (a wave-wide load is one 1 KiB
// contiguous run of a row); the vector stays in registers (lane l holds the 8
// columns of each of its 16-byte chunks); every row load of the wave is
// issued before the first dot product; one cross-lane reduction per row.

#include <hip/hip_runtime.h>

#include <cstdint>

#include "pvlc_device.hpp"
#include "pvlc_internal.hpp"

namespace pvlc {
namespace {

constexpr int kGemvWaves = 4;

// CHUNKS = columns / 512: 16-byte chunks of a row per lane.
template <int CHUNKS, int RPW>
__global__ __launch_bounds__(kGemvWaves * 64) void gemv_f16_kernel(const uint16_t *__restrict__ weights,
                                                                     const float *__restrict__ vector,
                                                                     float *__restrict__ out, uint32_t rows) {
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
        for (int c = 0; c < CHUNKS; ++c) w[r][c] = *reinterpret_cast<const half8_t *>(wr + (c * 64 + lane) * 8);
    }
    float4_t x[CHUNKS][2];
#pragma unroll
    for (int c = 0; c < CHUNKS; ++c) {
        x[c][0] = *reinterpret_cast<const float4_t *>(vector + (c * 64 + lane) * 8);
        x[c][1] = *reinterpret_cast<const float4_t *>(vector + (c * 64 + lane) * 8 + 4);
    }
#pragma unroll
    for (int r = 0; r < RPW; ++r) {
        float acc = 0.f;
#pragma unroll
        for (int c = 0; c < CHUNKS; ++c)
#pragma unroll
            for (int j = 0; j < 8; ++j)
                acc = __builtin_fmaf(static_cast<float>(w[r][c][j]), x[c][j >> 2][j & 3], acc);
#pragma unroll
        for (int o = 32; o > 0; o >>= 1) acc += __shfl_xor(acc, o);
        if (lane == 0 && row0 + r < rows) out[row0 + r] = acc;
    }
}

template <int CHUNKS>
int launch_gemv_rows(const uint16_t *weights, const float *vector, float *out, uint32_t rows, hipStream_t st) {
    // One row per wave while that still leaves under ~4 waves per SIMD of the
    // chip, four rows per wave (more bytes in flight per wave) beyond.
    if (rows <= 4096) {
        const unsigned wgs = (rows + kGemvWaves - 1) / kGemvWaves;
        hipLaunchKernelGGL((gemv_f16_kernel<CHUNKS, 1>), dim3(wgs), dim3(kGemvWaves * 64), 0, st, weights, vector,
                           out, rows);
    } else {
        const unsigned wgs = (rows + kGemvWaves * 4 - 1) / (kGemvWaves * 4);
        hipLaunchKernelGGL((gemv_f16_kernel<CHUNKS, 4>), dim3(wgs), dim3(kGemvWaves * 64), 0, st, weights, vector,
                           out, rows);
    }
    return static_cast<int>(hipGetLastError());
}

}  // namespace

int launch_gemv_f16(const uint16_t *weights, const float *vector, float *out, uint32_t rows, uint32_t columns,
                    void *stream) {
    hipStream_t st = static_cast<hipStream_t>(stream);
    switch (columns) {
        case 1024: return launch_gemv_rows<2>(weights, vector, out, rows, st);
        case 2048: return launch_gemv_rows<4>(weights, vector, out, rows, st);
        case 3072: return launch_gemv_rows<6>(weights, vector, out, rows, st);
        default: return static_cast<int>(hipErrorInvalidValue);
    }
}

}  // namespace pvlc
