// Prefill projection with fp16 weights for gfx950: out[r][n] = sum_k in[r][k]
// * W[n][k] + bias[n], f32 activations, fp16 weights output-major, f32 bias
// and output.  Replaces linear_projection_f16_weights (crates/pvlc-wgsl/src/
// lib.rs:1836-1964), which widens the weights and accumulates in f32
// (arithmetic reference: linear_f32, crates/pvlc-cpu-ref/src/lib.rs:88-140).
//
// The products run on MFMA without giving up f32 activations: each input row
// is scaled by a power of two 2^-e (so its largest element lies in
// [2^13, 2^14)) and split exactly into fp16 hi + fp16 lo (lo = the f32
// remainder, rounded), so hi + lo carries about 22 bits of every element.
// Two fp16 MFMAs per product (W.hi + W.lo, exact products, f32 accumulation)
// then give f32-grade sums at half the fp16 MFMA rate; the epilogue multiplies
// by 2^e (exact) and adds the bias.
//
// Kernel 1 (split): one workgroup per row: the row maximum, the exponent, the
// hi/lo planes [rows][K] in the workspace.
// Kernel 2 (GEMM): 128 x 128 output tiles, K in steps of 32, 4 waves of
// 64 x 64 (4 x 4 MFMA tiles of v_mfma_f32_16x16x32_f16 each, hi and lo);
// hi, lo and weight tiles move by direct global-to-LDS loads into
// [k-chunk][row][8] layouts (every operand read of 16 lanes is one 256-byte
// run), through a three-stage ring with one barrier per step.

#include <hip/hip_runtime.h>

#include <cstdint>

#include "pvlc_device.hpp"
#include "pvlc_internal.hpp"

namespace pvlc {
namespace {

constexpr int kSplitThreads = 256;
constexpr int kTileM = 128, kTileN = 128, kTileK = 32;
constexpr int kGemmThreads = 256;
constexpr uint32_t kXcds = 8;  // MI355X: 8 XCDs, each with its own L2
constexpr int kTileElems = kTileM * kTileK;  // fp16 elements of one 128 x 32 operand tile
// s_waitcnt immediates (gfx9 encoding: vmcnt bits 3:0, expcnt 6:4, lgkmcnt
// 11:8, the last two left at their maximum) -- as builtins, so the compiler's
// own wait insertion knows which loads they retire.
constexpr int kWaitVm6 = 0x0F76, kWaitVm0 = 0x0F70;  // vmcnt(6) / vmcnt(0)

// Exponent e of a row whose largest magnitude is m: m * 2^-e in [2^13, 2^14)
// (0 for an all-zero row).
__device__ inline int split_exponent(float m) {
    if (!(m > 0.f)) return 0;
    int x;
    (void)__builtin_frexpf(m, &x);  // m = f * 2^x, f in [0.5, 1)
    return x - 14;
}

__global__ __launch_bounds__(kSplitThreads) void projection_split_kernel(const float *__restrict__ input,
                                                                        uint32_t k_width, uint16_t *__restrict__ hi,
                                                                        uint16_t *__restrict__ lo,
                                                                        int32_t *__restrict__ exponents) {
    const size_t row = blockIdx.x;
    const float *in = input + row * k_width;
    float m = 0.f;
    for (uint32_t k = threadIdx.x * 4; k < k_width; k += kSplitThreads * 4) {
        const float4_t v = *reinterpret_cast<const float4_t *>(in + k);
        m = fmaxf(m, fmaxf(fmaxf(fabsf(v[0]), fabsf(v[1])), fmaxf(fabsf(v[2]), fabsf(v[3]))));
    }
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) m = fmaxf(m, __shfl_xor(m, o));
    __shared__ float sm_max[kSplitThreads / 64];
    if ((threadIdx.x & 63) == 0) sm_max[threadIdx.x >> 6] = m;
    __syncthreads();
    m = fmaxf(fmaxf(sm_max[0], sm_max[1]), fmaxf(sm_max[2], sm_max[3]));
    const int e = split_exponent(m);
    if (threadIdx.x == 0) exponents[row] = e;
    for (uint32_t k = threadIdx.x * 4; k < k_width; k += kSplitThreads * 4) {
        const float4_t v = *reinterpret_cast<const float4_t *>(in + k);
        u16x4_t h, l;
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            const float s = __builtin_ldexpf(v[j], -e);  // exact: a power of two
            const _Float16 sh = to_h(s);
            h[j] = __builtin_bit_cast(uint16_t, sh);
            l[j] = __builtin_bit_cast(uint16_t, to_h(s - static_cast<float>(sh)));  // the remainder is exact in f32
        }
        *reinterpret_cast<u16x4_t *>(hi + row * k_width + k) = h;
        *reinterpret_cast<u16x4_t *>(lo + row * k_width + k) = l;
    }
}

// LDS tile layout [k-chunk (4)][row (128)][8]: the fragment a 16-lane group
// reads (16 rows, one 8-element chunk) is one contiguous 256-byte run.
__device__ inline int tile_offset(int kchunk, int row) { return (kchunk * kTileM + row) * 8; }

__global__ __launch_bounds__(kGemmThreads, 2) void projection_gemm_kernel(
    const uint16_t *__restrict__ hi, const uint16_t *__restrict__ lo, const int32_t *__restrict__ exponents,
    const uint16_t *__restrict__ weight, const float *__restrict__ bias, float *__restrict__ out, uint32_t rows,
    uint32_t k_width, uint32_t n_width) {
    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane(static_cast<int>(threadIdx.x >> 6));
    const int row16 = lane & 15, kg = lane >> 4;
    // XCD-aware tile order: workgroups are dispatched round-robin over the 8
    // XCDs, so workgroup b runs on XCD b % 8; the permutation below gives XCD
    // x a contiguous range of tiles in row-major order (whole bands of output
    // rows), and the L2 of that XCD serves every column tile of its rows.
    const uint32_t n_tiles = (n_width + kTileN - 1) / kTileN;
    const uint32_t total = gridDim.x, xcd = blockIdx.x % kXcds, idx = blockIdx.x / kXcds;
    const uint32_t q = total / kXcds, r = total % kXcds;
    const uint32_t tile = xcd < r ? xcd * (q + 1) + idx : r * (q + 1) + (xcd - r) * q + idx;
    const uint32_t m0 = (tile / n_tiles) * kTileM, n0 = (tile % n_tiles) * kTileN;
    const int wm = wave >> 1, wn = wave & 1;  // the wave's 64 x 64 quadrant

    // Three-stage ring of distinct LDS arrays (picked at compile time in the
    // loop unrolled by three): step s computes stage s while the loads of
    // stage s+1 and s+2 are in flight, and its closing barrier waits only for
    // stage s+1 (vmcnt(6): the 6 loads per thread of stage s+2 may still be
    // outstanding).  Loads of stage 1 and of stage s+2 beyond the last clamp
    // to the last stage, so a single-step K is also exact.  The compiler sees that loads into one array and reads of
    // another do not alias, so it adds no wait of its own before the reads.
    __shared__ uint16_t sh0[kTileElems], sl0[kTileElems], sw0[kTileElems];
    __shared__ uint16_t sh1[kTileElems], sl1[kTileElems], sw1[kTileElems];
    __shared__ uint16_t sh2[kTileElems], sl2[kTileElems], sw2[kTileElems];
    typedef __attribute__((address_space(3))) void *lds_ptr;

    // Direct global-to-LDS loads: LDS chunk q = 64 j + lane of a tile holds
    // k-chunk q / 128 of tile row q % 128.  Each wave moves 2 of the 8
    // instructions per tile (6 loads per thread per stage).  Rows past the
    // end re-read the last row (never stored).
    const uint32_t last_row = rows - 1, last_col = n_width - 1;
    auto stage = [&](uint32_t k0, uint16_t *dh, uint16_t *dl, uint16_t *dw) {
#pragma unroll
        for (int r = 0; r < 2; ++r) {
            const int j = wave * 2 + r;
            const int q = 64 * j + lane;
            const uint32_t trow = static_cast<uint32_t>(q & 127), kc = static_cast<uint32_t>(q >> 7);
            const size_t a_off = static_cast<size_t>(min(m0 + trow, last_row)) * k_width + k0 + kc * 8;
            const size_t w_off = static_cast<size_t>(min(n0 + trow, last_col)) * k_width + k0 + kc * 8;
            __builtin_amdgcn_global_load_lds(hi + a_off, (lds_ptr)(dh + 64 * j * 8), 16, 0, 0);
            __builtin_amdgcn_global_load_lds(lo + a_off, (lds_ptr)(dl + 64 * j * 8), 16, 0, 0);
            __builtin_amdgcn_global_load_lds(weight + w_off, (lds_ptr)(dw + 64 * j * 8), 16, 0, 0);
        }
    };

    float4_t acc[4][4];
#pragma unroll
    for (int a = 0; a < 4; ++a)
#pragma unroll
        for (int b = 0; b < 4; ++b) acc[a][b] = float4_t{0.f, 0.f, 0.f, 0.f};

    // 16 x 16 x 32 tiles: A = activations (lane row = l % 16, k = (l / 16) * 8 ..),
    // B = W^T (lane column = l % 16, same k), C: column l % 16, rows (l / 16) * 4 + i.
    auto compute = [&](const uint16_t *sh, const uint16_t *sl, const uint16_t *sw) {
        half8_t bf[4];
#pragma unroll
        for (int cb = 0; cb < 4; ++cb)
            bf[cb] = *reinterpret_cast<const half8_t *>(sw + tile_offset(kg, wn * 64 + cb * 16 + row16));
#pragma unroll
        for (int rb = 0; rb < 4; ++rb) {
            const int trow = wm * 64 + rb * 16 + row16;
            const half8_t ah = *reinterpret_cast<const half8_t *>(sh + tile_offset(kg, trow));
            const half8_t al = *reinterpret_cast<const half8_t *>(sl + tile_offset(kg, trow));
#pragma unroll
            for (int cb = 0; cb < 4; ++cb) {
                acc[rb][cb] = __builtin_amdgcn_mfma_f32_16x16x32_f16(ah, bf[cb], acc[rb][cb], 0, 0, 0);
                acc[rb][cb] = __builtin_amdgcn_mfma_f32_16x16x32_f16(al, bf[cb], acc[rb][cb], 0, 0, 0);
            }
        }
    };
    // Step s: load stage s+2 (past the end: the last stage again, into the
    // buffer step s-1 freed, never read), compute stage s, wait for stage s+1,
    // barrier.  Unconditional loads keep the waits exact.
    const uint32_t steps = k_width / kTileK;
    auto step = [&](uint32_t s, uint16_t *ch, uint16_t *cl, uint16_t *cw, uint16_t *nh, uint16_t *nl, uint16_t *nw) {
        stage(min(s + 2, steps - 1) * kTileK, nh, nl, nw);
        compute(ch, cl, cw);
        __builtin_amdgcn_s_waitcnt(kWaitVm6);
        __builtin_amdgcn_s_barrier();
    };

    stage(0, sh0, sl0, sw0);
    stage(min(1u, steps - 1) * kTileK, sh1, sl1, sw1);
    __builtin_amdgcn_s_waitcnt(kWaitVm6);
    __builtin_amdgcn_s_barrier();
    uint32_t s = 0;
    for (; s + 3 <= steps; s += 3) {
        step(s, sh0, sl0, sw0, sh2, sl2, sw2);
        step(s + 1, sh1, sl1, sw1, sh0, sl0, sw0);
        step(s + 2, sh2, sl2, sw2, sh1, sl1, sw1);
    }
    if (s < steps) step(s, sh0, sl0, sw0, sh2, sl2, sw2);
    if (s + 1 < steps) step(s + 1, sh1, sl1, sw1, sh0, sl0, sw0);
    __builtin_amdgcn_s_waitcnt(kWaitVm0);  // no load into LDS outlives the loop

    // Epilogue: x 2^e of the row (exact), + bias, f32 stores.
#pragma unroll
    for (int rb = 0; rb < 4; ++rb) {
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const uint32_t r = m0 + wm * 64 + rb * 16 + kg * 4 + i;
            if (r >= rows) continue;
            const int e = exponents[r];
#pragma unroll
            for (int cb = 0; cb < 4; ++cb) {
                const uint32_t n = n0 + wn * 64 + cb * 16 + row16;
                if (n < n_width) out[static_cast<size_t>(r) * n_width + n] = __builtin_ldexpf(acc[rb][cb][i], e) + bias[n];
            }
        }
    }
}

}  // namespace

int launch_linear_projection_f16(const float *input, const uint16_t *weight, const float *bias, float *out,
                                 uint32_t rows, uint32_t k_width, uint32_t n_width, const ProjectionWorkspace &ws,
                                 void *stream) {
    hipStream_t st = static_cast<hipStream_t>(stream);
    hipLaunchKernelGGL(projection_split_kernel, dim3(rows), dim3(kSplitThreads), 0, st, input, k_width, ws.hi, ws.lo,
                       ws.exponents);
    if (hipError_t e = hipGetLastError()) return static_cast<int>(e);
    const uint32_t tiles = ((n_width + kTileN - 1) / kTileN) * ((rows + kTileM - 1) / kTileM);
    hipLaunchKernelGGL(projection_gemm_kernel, dim3(tiles), dim3(kGemmThreads), 0, st, ws.hi, ws.lo, ws.exponents, weight,
                       bias, out, rows, k_width, n_width);
    return static_cast<int>(hipGetLastError());
}

}  // namespace pvlc
