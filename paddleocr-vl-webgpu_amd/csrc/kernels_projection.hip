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
// Kernel 1 (split): one workgroup per 8 rows: the row maxima, the exponents,
// and the hi/lo planes written in the GEMM's tile order (per 128-row tile and
// 32-wide k step one 16 KiB block [plane][k-chunk (4)][row (128)][8]), so a
// GEMM stage of the activations is one contiguous 16 KiB run.
// Kernel 2 (GEMM): 128 x 128 output tiles, K in steps of 32, 4 waves of
// 64 x 64 (4 x 4 MFMA tiles of v_mfma_f32_16x16x32_f16 each, hi and lo);
// operand tiles move by direct global-to-LDS loads through a three-stage
// ring with one barrier per step.  Every load instruction reads long runs:
// 1 KiB of the activation block, or 16 weight rows x 64 bytes.  Projections
// with at least 512 tiles of 128 x 256 (gate|up at N=4096) run the wide
// variant instead (kernel 2b below): 128 x 256 or 128 x 192 tiles, 4 waves,
// and the tiles of each XCD in one block of the output, so both operands are
// reused from the XCD's L2.

#include <hip/hip_runtime.h>

#include <cstdint>
#include <type_traits>

#include "pvlc_device.hpp"
#include "pvlc_internal.hpp"

namespace pvlc {
namespace {

constexpr int kSplitThreads = 256;
constexpr int kSplitRows = 8;  // rows per split workgroup: 8 x 16 bytes = one 128-byte line per chunk
constexpr int kTileM = kProjectionTileRows, kTileN = 128, kTileK = kProjectionStepK;
constexpr int kGemmThreads = 256;
constexpr uint32_t kXcds = 8;  // MI355X: 8 XCDs, each with its own L2
constexpr int kTileElems = kTileM * kTileK;  // fp16 elements of one 128 x 32 operand tile
constexpr int kBlockElems = 2 * kTileElems;  // one activation block: hi and lo planes
// s_waitcnt immediates (gfx9 encoding: vmcnt bits 3:0, expcnt 6:4, lgkmcnt
// 11:8, the last two left at their maximum) -- as builtins, so the compiler's
// own wait insertion knows which loads they retire.
constexpr int kWaitVm4 = 0x0F74, kWaitVm0 = 0x0F70;  // vmcnt(4) / vmcnt(0)

// Exponent e of a row whose largest magnitude is m: m * 2^-e in [2^13, 2^14)
// (0 for an all-zero row).
__device__ inline int split_exponent(float m) {
    if (!(m > 0.f)) return 0;
    int x;
    (void)__builtin_frexpf(m, &x);  // m = f * 2^x, f in [0.5, 1)
    return x - 14;
}

// Offset (fp16 elements) of row r, k-chunk c (8 elements) in the tile-ordered
// planes: block (r / 128, c / 4), plane hi; lo is kTileElems further.
__device__ inline size_t plane_offset(uint32_t r, uint32_t c, uint32_t steps) {
    const size_t block = static_cast<size_t>(r / kTileM) * steps + c / 4;
    return block * kBlockElems + ((c % 4) * kTileM + r % kTileM) * 8;
}

// Thread t of the workgroup serves row 8 g + t % 8 and the k-chunks t / 8 +
// 32 i; the 8 threads of one chunk write one whole 128-byte line of each
// plane.  Rows past the end (padding of the last tile) are written as zeros.
// CPT > 0: K = 256 CPT, the thread's CPT chunks stay in registers between the
// row maximum and the split (one pass over the input); CPT = 0: any K that is
// a multiple of 32, the chunks are read again for the split.
template <int CPT>
__global__ __launch_bounds__(kSplitThreads) void projection_split_kernel(const float *__restrict__ input,
                                                                        uint32_t rows, uint32_t k_width,
                                                                        uint16_t *__restrict__ tiles,
                                                                        int32_t *__restrict__ exponents) {
    const uint32_t rr = threadIdx.x % kSplitRows, c0 = threadIdx.x / kSplitRows;
    constexpr uint32_t kChunkStride = kSplitThreads / kSplitRows;
    const uint32_t row = blockIdx.x * kSplitRows + rr, chunks = k_width / 8, steps = k_width / kTileK;
    const bool live = row < rows;
    const float *in = input + static_cast<size_t>(live ? row : 0) * k_width;
    auto load = [&](uint32_t c, float4_t &a, float4_t &b) {
        a = *reinterpret_cast<const float4_t *>(in + c * 8);
        b = *reinterpret_cast<const float4_t *>(in + c * 8 + 4);
    };
    auto chunk_max = [](float m, const float4_t &a, const float4_t &b) {
#pragma unroll
        for (int j = 0; j < 4; ++j) m = fmaxf(m, fmaxf(fabsf(a[j]), fabsf(b[j])));
        return m;
    };
    float m = 0.f;
    float4_t va[CPT > 0 ? CPT : 1], vb[CPT > 0 ? CPT : 1];
    if constexpr (CPT > 0) {
        // Padding rows read row 0 (every load unconditional) and are zeroed below.
#pragma unroll
        for (int i = 0; i < CPT; ++i) load(c0 + i * kChunkStride, va[i], vb[i]);
#pragma unroll
        for (int i = 0; i < CPT; ++i) m = chunk_max(m, va[i], vb[i]);
        if (!live) m = 0.f;
    } else if (live) {
        for (uint32_t c = c0; c < chunks; c += kChunkStride) {
            float4_t a, b;
            load(c, a, b);
            m = chunk_max(m, a, b);
        }
    }
    // Lanes of one row differ in lane bits 3..5; then the 4 waves.
#pragma unroll
    for (int o = 8; o < 64; o <<= 1) m = fmaxf(m, __shfl_xor(m, o));
    __shared__ float sm_max[kSplitThreads / 64][kSplitRows];
    if ((threadIdx.x & 63) < kSplitRows) sm_max[threadIdx.x >> 6][rr] = m;
    __syncthreads();
    m = fmaxf(fmaxf(sm_max[0][rr], sm_max[1][rr]), fmaxf(sm_max[2][rr], sm_max[3][rr]));
    const int e = split_exponent(m);
    if (threadIdx.x < kSplitRows) exponents[row] = e;
    auto split_store = [&](uint32_t c, const float4_t &a, const float4_t &b) {
        half8_t h, l;
#pragma unroll
        for (int j = 0; j < 8; ++j) {
            const float s = live ? __builtin_ldexpf(j < 4 ? a[j] : b[j - 4], -e) : 0.f;  // exact: a power of two
            h[j] = to_h(s);
            l[j] = to_h(s - static_cast<float>(h[j]));  // the remainder is exact in f32
        }
        const size_t off = plane_offset(row, c, steps);
        *reinterpret_cast<half8_t *>(tiles + off) = h;
        *reinterpret_cast<half8_t *>(tiles + off + kTileElems) = l;
    };
    if constexpr (CPT > 0) {
#pragma unroll
        for (int i = 0; i < CPT; ++i) split_store(c0 + i * kChunkStride, va[i], vb[i]);
    } else {
        for (uint32_t c = c0; c < chunks; c += kChunkStride) {
            float4_t a = {0.f, 0.f, 0.f, 0.f}, b = a;
            if (live) load(c, a, b);
            split_store(c, a, b);
        }
    }
}

// LDS layouts.  Activations: the block as stored, [plane][k-chunk (4)][row
// (128)][8], so the fragment a 16-lane group reads (16 rows, one chunk) is one
// 256-byte run.  Weights: [row (128)][slot (4)][8] with k-chunk c of row r in
// slot c ^ ((r / 2) % 4): the 4 slots of a row are one 64-byte run of the
// weight row (one load of 4 lanes), and the fragment reads (16 rows, one chunk
// each) have no bank conflicts (measured: SQ_LDS_BANK_CONFLICT 0, against a
// quarter of the LDS cycles with the swizzle c ^ ((r / 4) % 4)).
__device__ inline int a_offset(int kchunk, int row) { return (kchunk * kTileM + row) * 8; }
__device__ inline int w_offset(int kchunk, int row) { return (row * 4 + (kchunk ^ ((row >> 1) & 3))) * 8; }

// Ring stage u of the narrow GEMM: distinct LDS arrays per stage (one
// function-scope array per instantiation), so the compiler sees that loads
// into one stage and fragment reads of another do not alias and adds no wait
// of its own before the reads.
template <int U> __device__ __forceinline__ uint16_t *ring_a() {
    __shared__ __align__(16) uint16_t buf[kBlockElems];
    return buf;
}
template <int U, int NT> __device__ __forceinline__ uint16_t *ring_w() {
    __shared__ __align__(16) uint16_t buf[NT * kTileK];
    return buf;
}
// Calls f(integral_constant<U>) for U = B .. E-1 (compile-time ring indices).
template <int B, int E> struct StageUnroll {
    template <class F> __device__ __forceinline__ static void run(F &&f) {
        f(std::integral_constant<int, B>{});
        StageUnroll<B + 1, E>::run(f);
    }
};
template <int E> struct StageUnroll<E, E> {
    template <class F> __device__ __forceinline__ static void run(F &&) {}
};

// 128 x NT output tiles (NT = 128 or 160 columns), 4 waves of 64 x NT/2.
// STAGES-deep ring of (activation block 16 KiB, weight tile NT x 32) stages:
// step s computes stage s while the loads of stages s+1 .. s+STAGES-1 are in
// flight.  Three stages (72 or 78 KiB) leave room for two workgroups per
// compute unit; six (144 KiB, NT = 128) are for launches of at most one
// workgroup per compute unit, where nothing else on the unit covers the load
// latency.  NT = 160 serves widths that are multiples of 160 with as many
// tiles as two workgroups per compute unit hold (q|k|v at N=4096: 512 tiles in
// one round, against 640 tiles of 128 that leave a second round a quarter
// full).
template <int STAGES, int MIN_WGS, int NT>
__global__ __launch_bounds__(kGemmThreads, MIN_WGS) void projection_gemm_kernel(
    const uint16_t *__restrict__ tiles, const int32_t *__restrict__ exponents, const uint16_t *__restrict__ weight,
    const float *__restrict__ bias, float *__restrict__ out, uint32_t rows, uint32_t k_width, uint32_t n_width) {
    static_assert(NT == 128 || NT == 160, "column tile of 128 or 160");
    constexpr int CB = NT / 32;                 // 16-column MFMA tiles per wave
    constexpr int kWLoads = NT == 128 ? 2 : 3;  // weight loads per thread and stage
    constexpr int kLoads = 4 + kWLoads;         // loads per thread and stage
    static_assert(STAGES >= 3 && kLoads * (STAGES - 1) <= 63, "vmcnt holds at most 63 outstanding loads");
    constexpr int kWaitRing = 0x0F70 | (kLoads * (STAGES - 2) & 15) | ((kLoads * (STAGES - 2) >> 4) << 14);
    constexpr int kWaitRingPrologue = 0x0F70 | (kLoads * (STAGES - 1) & 15) | ((kLoads * (STAGES - 1) >> 4) << 14);
    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane(static_cast<int>(threadIdx.x >> 6));
    const int row16 = lane & 15, kg = lane >> 4;
    // XCD-aware tile order: workgroups are dispatched round-robin over the 8
    // XCDs, so workgroup b runs on XCD b % 8; the permutation below gives XCD
    // x a contiguous range of tiles in row-major order (whole bands of output
    // rows), and the L2 of that XCD serves every column tile of its rows.
    const uint32_t n_tiles = n_width / NT + (n_width % NT != 0);
    const uint32_t total = gridDim.x, xcd = blockIdx.x % kXcds, idx = blockIdx.x / kXcds;
    const uint32_t q = total / kXcds, r = total % kXcds;
    const uint32_t tile = xcd < r ? xcd * (q + 1) + idx : r * (q + 1) + (xcd - r) * q + idx;
    const uint32_t mt = tile / n_tiles, m0 = mt * kTileM, n0 = (tile % n_tiles) * NT;
    const int wm = wave >> 1, wn = wave & 1;  // the wave's 64 x NT/2 part
    const uint32_t steps = k_width / kTileK;
    typedef __attribute__((address_space(3))) void *lds_ptr;

    // Direct global-to-LDS loads, 64 lanes x 16 bytes per instruction, lane l
    // landing at 16 l of the instruction's 1 KiB.  Activations: the 16 KiB
    // block (tile mt, step s) as 16 instructions of 1 KiB, 4 per wave.
    // Weights: NT / 16 instructions of 16 rows each; lane l of instruction j
    // fills LDS slot p = 64 j + l, i.e. row p / 4, slot p % 4.  Wave w issues
    // instructions 2w and 2w+1 and, for NT = 160, instruction 8 + (w & 1) (so
    // waves 2 and 3 repeat waves 0 and 1's: the same bytes into the same
    // place, and every wave counts the same loads).  Weight rows past the end
    // re-read the last row (never stored).
    const uint16_t *a_tiles = tiles + static_cast<size_t>(mt) * steps * kBlockElems + (wave * 4) * 512 + lane * 8;
    const uint32_t last_col = n_width - 1;
    // (Fixed-size arrays: hipcc's host pass drops the kernel's launch stub,
    // without a diagnostic, when a lambda called from the generic step lambda
    // captures a local array whose size depends on the template arguments.)
    int w_inst[3];
    size_t w_row_off[3];
#pragma unroll
    for (int rw = 0; rw < kWLoads; ++rw) {
        w_inst[rw] = rw < 2 ? wave * 2 + rw : 8 + (wave & 1);
        const int p = 64 * w_inst[rw] + lane, wrow = p >> 2;
        const int kc = (p & 3) ^ ((wrow >> 1) & 3);
        w_row_off[rw] = static_cast<size_t>(min(n0 + wrow, last_col)) * k_width + kc * 8;
    }
    auto stage = [&](uint32_t s, uint16_t *da, uint16_t *dw) {
        const uint16_t *a = a_tiles + static_cast<size_t>(s) * kBlockElems;
#pragma unroll
        for (int j = 0; j < 4; ++j)
            __builtin_amdgcn_global_load_lds(a + j * 512, (lds_ptr)(da + (wave * 4 + j) * 512), 16, 0, 0);
#pragma unroll
        for (int rw = 0; rw < kWLoads; ++rw)
            __builtin_amdgcn_global_load_lds(weight + w_row_off[rw] + s * kTileK,
                                             (lds_ptr)(dw + w_inst[rw] * 512), 16, 0, 0);
    };

    float4_t acc[4][CB];
#pragma unroll
    for (int a = 0; a < 4; ++a)
#pragma unroll
        for (int b = 0; b < CB; ++b) acc[a][b] = float4_t{0.f, 0.f, 0.f, 0.f};

    // 16 x 16 x 32 tiles: A = activations (lane row = l % 16, k = (l / 16) * 8 ..),
    // B = W^T (lane column = l % 16, same k), C: column l % 16, rows (l / 16) * 4 + i.
    // A step's 8 + CB fragments (CB weight, 4 hi, 4 lo) are read from LDS
    // during the previous step's MFMAs (two register sets).
    struct Frags {
        half8_t b[CB], h[4], l[4];
    };
    auto read_frags = [&](Frags &f, const uint16_t *sa, const uint16_t *sw) {
#pragma unroll
        for (int cb = 0; cb < CB; ++cb)
            f.b[cb] = *reinterpret_cast<const half8_t *>(sw + w_offset(kg, wn * (NT / 2) + cb * 16 + row16));
#pragma unroll
        for (int rb = 0; rb < 4; ++rb) {
            const int trow = wm * 64 + rb * 16 + row16;
            f.h[rb] = *reinterpret_cast<const half8_t *>(sa + a_offset(kg, trow));
            f.l[rb] = *reinterpret_cast<const half8_t *>(sa + kTileElems + a_offset(kg, trow));
        }
    };
    auto mfmas = [&](const Frags &f) {
#pragma unroll
        for (int rb = 0; rb < 4; ++rb) {
#pragma unroll
            for (int cb = 0; cb < CB; ++cb)
                acc[rb][cb] = __builtin_amdgcn_mfma_f32_16x16x32_f16(f.h[rb], f.b[cb], acc[rb][cb], 0, 0, 0);
#pragma unroll
            for (int cb = 0; cb < CB; ++cb)
                acc[rb][cb] = __builtin_amdgcn_mfma_f32_16x16x32_f16(f.l[rb], f.b[cb], acc[rb][cb], 0, 0, 0);
        }
    };
    // Step s (ring slot U = s % STAGES), entered with stage s's fragments in
    // registers: wait for this thread's loads of stage s+1, finish its
    // fragment reads of stage s, barrier (every wave's stage s+1 has landed
    // and nobody reads slot U any more); load stage s+STAGES into slot U
    // (past the end: the last stage again, never read); then stage s's 8 CB
    // MFMAs with stage s+1's 8 + CB fragment reads and the kLoads loads
    // spread among them (sched_group_barrier masks: 0x008 MFMA, 0x100 LDS
    // read, 0x020 global load).  Unconditional loads keep the waits exact.
    Frags fa, fb;
    uint32_t s = 0;
    auto step = [&](auto uc, Frags &cur, Frags &nxt) {
        constexpr int U = decltype(uc)::value, N = (U + 1) % STAGES;
        __builtin_amdgcn_s_waitcnt(kWaitRing & ~0x0F00);  // ... and lgkmcnt(0)
        __builtin_amdgcn_s_barrier();
        stage(min(s + U + STAGES, steps - 1), ring_a<U>(), ring_w<U, NT>());
        read_frags(nxt, ring_a<N>(), ring_w<N, NT>());
        mfmas(cur);
        if constexpr (NT == 128) {
#pragma unroll
            for (int i = 0; i < 6; ++i) {
                __builtin_amdgcn_sched_group_barrier(0x008, 2, 0);
                __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);
                __builtin_amdgcn_sched_group_barrier(0x008, 2, 0);
                __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);
                __builtin_amdgcn_sched_group_barrier(0x020, 1, 0);
            }
            __builtin_amdgcn_sched_group_barrier(0x008, 8, 0);
        } else {
#pragma unroll
            for (int i = 0; i < 6; ++i) {
                __builtin_amdgcn_sched_group_barrier(0x008, 3, 0);
                __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);
                __builtin_amdgcn_sched_group_barrier(0x008, 2, 0);
                __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);
                __builtin_amdgcn_sched_group_barrier(0x020, 1, 0);
            }
            __builtin_amdgcn_sched_group_barrier(0x008, 3, 0);
            __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);
            __builtin_amdgcn_sched_group_barrier(0x020, 1, 0);
            __builtin_amdgcn_sched_group_barrier(0x008, 7, 0);
        }
    };
    // Prologue: stages 0 .. STAGES-1 into every slot, wait for stage 0 (the
    // other STAGES-1 stages' loads may be outstanding), read its fragments.
    StageUnroll<0, STAGES>::run([&](auto uc) {
        constexpr int U = decltype(uc)::value;
        stage(min(static_cast<uint32_t>(U), steps - 1), ring_a<U>(), ring_w<U, NT>());
    });
    __builtin_amdgcn_s_waitcnt(kWaitRingPrologue);
    __builtin_amdgcn_s_barrier();
    read_frags(fa, ring_a<0>(), ring_w<0, NT>());
    // Unrolled by 2 STAGES: the ring slot and the register set are both
    // compile-time in every step.
    for (; s + 2 * STAGES <= steps; s += 2 * STAGES) {
        StageUnroll<0, STAGES>::run([&](auto uc) {
            if constexpr (decltype(uc)::value % 2 == 0) step(uc, fa, fb); else step(uc, fb, fa);
        });
        s += STAGES;
        StageUnroll<0, STAGES>::run([&](auto uc) {
            if constexpr ((decltype(uc)::value + STAGES) % 2 == 0) step(uc, fa, fb); else step(uc, fb, fa);
        });
        s -= STAGES;
    }
    // The remaining < 2 STAGES steps (the fragments of stage s are in fa).
    StageUnroll<0, STAGES>::run([&](auto uc) {
        if (s + decltype(uc)::value < steps) {
            if constexpr (decltype(uc)::value % 2 == 0) step(uc, fa, fb); else step(uc, fb, fa);
        }
    });
    if (s + STAGES < steps) {
        s += STAGES;
        StageUnroll<0, STAGES - 1>::run([&](auto uc) {
            if (s + decltype(uc)::value < steps) {
                if constexpr ((decltype(uc)::value + STAGES) % 2 == 0) step(uc, fa, fb); else step(uc, fb, fa);
            }
        });
    }
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
            for (int cb = 0; cb < CB; ++cb) {
                const uint32_t n = n0 + wn * (NT / 2) + cb * 16 + row16;
                if (n < n_width) out[static_cast<size_t>(r) * n_width + n] = __builtin_ldexpf(acc[rb][cb][i], e) + bias[n];
            }
        }
    }
}

// Kernel 2b (wide projections: enough 128 x 256 output tiles to give every
// compute unit two): projection_gemm_wide_kernel<NW>, 128 x NW output tiles
// (NW = 256, or 192 where 192-column tiles fill their rounds of two
// workgroups per compute unit with fewer columns: gate|up at N=4096), 4 waves
// of 64 x NW/2 (4 x NW/32 MFMA tiles, hi and lo), K in steps of 32.  The
// activation stages (16 KiB) move through a three-stage ring, loaded two
// steps ahead, the weight stages (NW x 64 bytes) through a two-stage ring,
// loaded one step ahead: 80 (72) KiB, two workgroups per compute unit.  Per
// 32-wide k step a wave reads 8 activation and NW/32 weight fragments for
// NW/2 MFMAs, at NW = 256 two thirds of the 128 x 128 kernel's LDS reads per
// MFMA (12 for 32), and a workgroup stores 32 KiB into LDS for twice the
// products of the 24 KiB the narrow kernel stores.
constexpr uint32_t kWideResident = 64;          // workgroups one XCD runs at once (32 compute units x 2)

// Tile order of the wide GEMM.  Workgroup b runs on XCD b % 8, so XCD x
// takes the workgroups b = 8 i + x and, with them, one block of the output:
// the row tiles split into 8 / col_groups bands and the column tiles into
// col_groups bands, col_groups chosen by the host to minimise the operand
// bytes one XCD reads (a row tile's activations and a column tile's weights
// are the same size).  Inside the block, generations of `gen` columns: all
// row tiles of the block for columns [g gen, g gen + gen), row-major, so the
// workgroups resident at once share both operands in the XCD's L2.
struct WideOrder {
    uint32_t row_tiles, col_tiles, col_groups, gen;
};

__device__ inline bool wide_tile(const WideOrder &o, uint32_t b, uint32_t *mt, uint32_t *nt) {
    const uint32_t x = b % kXcds, idx = b / kXcds;
    const uint32_t row_groups = kXcds / o.col_groups;
    const uint32_t xr = x / o.col_groups, xc = x % o.col_groups;
    const uint32_t r0 = xr * o.row_tiles / row_groups, r1 = (xr + 1) * o.row_tiles / row_groups;
    const uint32_t c0 = xc * o.col_tiles / o.col_groups, c1 = (xc + 1) * o.col_tiles / o.col_groups;
    const uint32_t rb = r1 - r0, cb = c1 - c0;
    if (idx >= rb * cb) return false;
    const uint32_t gen = o.gen < cb ? o.gen : cb;
    const uint32_t span = rb * gen, full = cb / gen;
    uint32_t g, rem, w;
    if (idx < full * span) {
        g = idx / span;
        rem = idx % span;
        w = gen;
    } else {
        g = full;
        rem = idx - full * span;
        w = cb - full * gen;
    }
    *mt = r0 + rem / w;
    *nt = c0 + g * gen + rem % w;
    return true;
}

template <int NW>
__global__ __launch_bounds__(kGemmThreads, 2) void projection_gemm_wide_kernel(
    const uint16_t *__restrict__ tiles, const int32_t *__restrict__ exponents, const uint16_t *__restrict__ weight,
    const float *__restrict__ bias, float *__restrict__ out, uint32_t rows, uint32_t k_width, uint32_t n_width,
    WideOrder order) {
    static_assert(NW == 256 || NW == 192, "wide column tile of 256 or 192");
    constexpr int CB = NW / 32;    // 16-column MFMA tiles per wave
    constexpr int kWL = NW / 64;   // weight loads (16 rows each) per wave and stage
    constexpr int kWideElems = NW * kTileK;  // one weight stage: NW rows x 32 k
    uint32_t mt, nt;
    if (!wide_tile(order, blockIdx.x, &mt, &nt)) return;  // uniform: a smaller block of this XCD
    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane(static_cast<int>(threadIdx.x >> 6));
    const int row16 = lane & 15, kg = lane >> 4;
    const uint32_t m0 = mt * kTileM, n0 = nt * NW;
    const int wm = wave >> 1, wn = wave & 1;  // the wave's 64 x NW/2 part: rows wm * 64, columns wn * NW/2
    const uint32_t steps = k_width / kTileK;

    // The stages as distinct arrays, picked at compile time by the loop
    // unrolled by six (the period of the two rings).
    __shared__ uint16_t sa0[kBlockElems], sa1[kBlockElems], sa2[kBlockElems];
    __shared__ uint16_t sw0[kWideElems], sw1[kWideElems];
    typedef __attribute__((address_space(3))) void *lds_ptr;

    // Direct global-to-LDS loads, 1 KiB per instruction: activations as in
    // the narrow kernel (4 per wave); weights NW / 16 instructions of 16 rows,
    // NW / 64 per wave, lane l of instruction j filling LDS slot p = 64 j + l
    // (row p / 4, slot p % 4, the row's k-chunk slot ^ ((row / 2) % 4)).
    // Weight rows past the end re-read the last row (never stored).
    const uint16_t *a_tiles = tiles + static_cast<size_t>(mt) * steps * kBlockElems + (wave * 4) * 512 + lane * 8;
    const uint32_t last_col = n_width - 1;
    // (The per-thread arrays here have fixed sizes, the largest width's, and
    // only their first kWL / CB entries are used: arrays whose size depends on
    // the template argument make hipcc's host pass drop the launch stub.)
    size_t w_row_off[4];
#pragma unroll
    for (int rw = 0; rw < kWL; ++rw) {
        const int p = 64 * (wave * kWL + rw) + lane, wrow = p >> 2;
        const int kc = (p & 3) ^ ((wrow >> 1) & 3);
        w_row_off[rw] = static_cast<size_t>(min(n0 + wrow, last_col)) * k_width + kc * 8;
    }
    auto load_a = [&](uint32_t s, uint16_t *da) {
        const uint16_t *a = a_tiles + static_cast<size_t>(s) * kBlockElems;
#pragma unroll
        for (int j = 0; j < 4; ++j)
            __builtin_amdgcn_global_load_lds(a + j * 512, (lds_ptr)(da + (wave * 4 + j) * 512), 16, 0, 0);
    };
    auto load_w = [&](uint32_t s, uint16_t *dw) {
#pragma unroll
        for (int rw = 0; rw < kWL; ++rw)
            __builtin_amdgcn_global_load_lds(weight + w_row_off[rw] + s * kTileK,
                                             (lds_ptr)(dw + (wave * kWL + rw) * 512), 16, 0, 0);
    };

    float4_t acc[4][8];
#pragma unroll
    for (int a = 0; a < 4; ++a)
#pragma unroll
        for (int b = 0; b < CB; ++b) acc[a][b] = float4_t{0.f, 0.f, 0.f, 0.f};

    // The fragment layouts of the narrow kernel: A = activations (lane row
    // l % 16, k (l / 16) * 8 ..), B = W^T (lane column l % 16, same k).
    auto compute = [&](const uint16_t *sa, const uint16_t *sw) {
        half8_t bf[8];
#pragma unroll
        for (int cb = 0; cb < CB; ++cb)
            bf[cb] = *reinterpret_cast<const half8_t *>(sw + w_offset(kg, wn * (NW / 2) + cb * 16 + row16));
#pragma unroll
        for (int rb = 0; rb < 4; ++rb) {
            const int trow = wm * 64 + rb * 16 + row16;
            const half8_t ah = *reinterpret_cast<const half8_t *>(sa + a_offset(kg, trow));
            const half8_t al = *reinterpret_cast<const half8_t *>(sa + kTileElems + a_offset(kg, trow));
#pragma unroll
            for (int cb = 0; cb < CB; ++cb)
                acc[rb][cb] = __builtin_amdgcn_mfma_f32_16x16x32_f16(ah, bf[cb], acc[rb][cb], 0, 0, 0);
#pragma unroll
            for (int cb = 0; cb < CB; ++cb)
                acc[rb][cb] = __builtin_amdgcn_mfma_f32_16x16x32_f16(al, bf[cb], acc[rb][cb], 0, 0, 0);
        }
        // Schedule: the weight fragments and the first row block's first,
        // then each row block's 2 CB MFMAs with the next row block's two
        // fragment reads issued after its first MFMA and the step's 4 + NW / 64
        // global-to-LDS loads spread among them (masks: 0x100 LDS read,
        // 0x008 MFMA, 0x020 global load).  Measured against the compiler's own
        // order (a wait for each row block's reads): gate|up 138 -> 127 us.
        __builtin_amdgcn_sched_group_barrier(0x100, CB + 2, 0);
#pragma unroll
        for (int rb = 0; rb < 4; ++rb) {
            __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
            if (rb < 3) __builtin_amdgcn_sched_group_barrier(0x100, 2, 0);
#pragma unroll
            for (int q = 0; q < 3; ++q) {
                __builtin_amdgcn_sched_group_barrier(0x008, (2 * CB - 1) / 3, 0);
                __builtin_amdgcn_sched_group_barrier(0x020, 1, 0);
            }
            if constexpr ((2 * CB - 1) % 3 != 0) __builtin_amdgcn_sched_group_barrier(0x008, (2 * CB - 1) % 3, 0);
        }
    };
    // Step s: wait until at most the 4 activation loads of stage s + 1 are
    // outstanding (this wave's loads of the activations and weights of stage
    // s have landed), barrier (every wave's have, and every wave has finished
    // reading the buffers of stage s - 1), load the weights of stage s + 1
    // and then the activations of stage s + 2 into those buffers (past the
    // end: the last stage again, never read), compute stage s.  Unconditional
    // loads keep the waits exact.
    auto step = [&](uint32_t s, uint16_t *ca, uint16_t *cw, uint16_t *na2, uint16_t *nw1) {
        __builtin_amdgcn_s_waitcnt(kWaitVm4);
        __builtin_amdgcn_s_barrier();
        load_w(min(s + 1, steps - 1), nw1);
        load_a(min(s + 2, steps - 1), na2);
        compute(ca, cw);
    };

    load_a(0, sa0);
    load_w(0, sw0);
    load_a(min(1u, steps - 1), sa1);
    uint32_t s = 0;
    for (; s + 6 <= steps; s += 6) {
        step(s, sa0, sw0, sa2, sw1);
        step(s + 1, sa1, sw1, sa0, sw0);
        step(s + 2, sa2, sw0, sa1, sw1);
        step(s + 3, sa0, sw1, sa2, sw0);
        step(s + 4, sa1, sw0, sa0, sw1);
        step(s + 5, sa2, sw1, sa1, sw0);
    }
    if (s < steps) step(s, sa0, sw0, sa2, sw1);
    if (s + 1 < steps) step(s + 1, sa1, sw1, sa0, sw0);
    if (s + 2 < steps) step(s + 2, sa2, sw0, sa1, sw1);
    if (s + 3 < steps) step(s + 3, sa0, sw1, sa2, sw0);
    if (s + 4 < steps) step(s + 4, sa1, sw0, sa0, sw1);
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
            for (int cb = 0; cb < CB; ++cb) {
                const uint32_t n = n0 + wn * (NW / 2) + cb * 16 + row16;
                if (n < n_width) out[static_cast<size_t>(r) * n_width + n] = __builtin_ldexpf(acc[rb][cb][i], e) + bias[n];
            }
        }
    }
}

// Order of the wide GEMM's tiles for rows x n_width: the column grouping that
// minimises the operand bytes of the largest XCD block, and generations of
// columns sized so that one generation is what an XCD runs at once.
WideOrder wide_order(uint32_t row_tiles, uint32_t col_tiles) {
    WideOrder best{row_tiles, col_tiles, 1, 1};
    uint32_t best_cost = UINT32_MAX;
    for (uint32_t gc = 1; gc <= kXcds; gc *= 2) {
        const uint32_t gr = kXcds / gc;
        const uint32_t rb = (row_tiles + gr - 1) / gr, cb = (col_tiles + gc - 1) / gc;
        if (rb + cb < best_cost) {
            best_cost = rb + cb;
            best.col_groups = gc;
        }
    }
    const uint32_t rb = (row_tiles + kXcds / best.col_groups - 1) / (kXcds / best.col_groups);
    best.gen = kWideResident / rb > 0 ? kWideResident / rb : 1;
    return best;
}

}  // namespace

int launch_linear_projection_f16(const float *input, const uint16_t *weight, const float *bias, float *out,
                                 uint32_t rows, uint32_t k_width, uint32_t n_width, const ProjectionWorkspace &ws,
                                 void *stream) {
    hipStream_t st = static_cast<hipStream_t>(stream);
    const uint32_t m_tiles = (rows + kTileM - 1) / kTileM;
    const dim3 split_grid(m_tiles * (kTileM / kSplitRows));
    switch (k_width) {
    case 1024: hipLaunchKernelGGL(projection_split_kernel<4>, split_grid, dim3(kSplitThreads), 0, st, input, rows, k_width, ws.tiles, ws.exponents); break;
    case 2048: hipLaunchKernelGGL(projection_split_kernel<8>, split_grid, dim3(kSplitThreads), 0, st, input, rows, k_width, ws.tiles, ws.exponents); break;
    case 3072: hipLaunchKernelGGL(projection_split_kernel<12>, split_grid, dim3(kSplitThreads), 0, st, input, rows, k_width, ws.tiles, ws.exponents); break;
    case 4096: hipLaunchKernelGGL(projection_split_kernel<16>, split_grid, dim3(kSplitThreads), 0, st, input, rows, k_width, ws.tiles, ws.exponents); break;
    default: hipLaunchKernelGGL(projection_split_kernel<0>, split_grid, dim3(kSplitThreads), 0, st, input, rows, k_width, ws.tiles, ws.exponents); break;
    }
    if (hipError_t e = hipGetLastError()) return static_cast<int>(e);
    const uint32_t cols256 = n_width / 256 + (n_width % 256 != 0), cols192 = n_width / 192 + (n_width % 192 != 0);
    const uint64_t slots = 2 * kTargetWorkgroups;
    if (static_cast<uint64_t>(cols256) * m_tiles >= slots) {
        // Enough wide tiles for two workgroups on every compute unit: the
        // wide kernel (with fewer, its second slot on most compute units
        // stays empty, and the narrow kernel's twice as many tiles finish
        // sooner: q|k|v at N=4096, 320 wide tiles, 80 us against 72).
        // 192-column tiles where their rounds of two workgroups per compute
        // unit hold fewer columns than the 256-column tiles' (gate|up at
        // N=4096: 1024 tiles in two full rounds, against 768 tiles that leave
        // the second round half empty).
        const uint64_t rounds256 = (cols256 * m_tiles + slots - 1) / slots, rounds192 = (cols192 * m_tiles + slots - 1) / slots;
        const bool narrow192 = rounds192 * 192 < rounds256 * 256;
        const uint32_t wide_cols = narrow192 ? cols192 : cols256;
        const WideOrder order = wide_order(m_tiles, wide_cols);
        const uint32_t row_groups = kXcds / order.col_groups;
        const uint32_t block = ((m_tiles + row_groups - 1) / row_groups) * ((wide_cols + order.col_groups - 1) / order.col_groups);
        if (narrow192)
            hipLaunchKernelGGL(projection_gemm_wide_kernel<192>, dim3(kXcds * block), dim3(kGemmThreads), 0, st,
                               ws.tiles, ws.exponents, weight, bias, out, rows, k_width, n_width, order);
        else
            hipLaunchKernelGGL(projection_gemm_wide_kernel<256>, dim3(kXcds * block), dim3(kGemmThreads), 0, st,
                               ws.tiles, ws.exponents, weight, bias, out, rows, k_width, n_width, order);
        return static_cast<int>(hipGetLastError());
    }
    const uint32_t tiles = (n_width / kTileN + (n_width % kTileN != 0)) * m_tiles;  // < 2^24 (checked by the caller)
    const uint32_t tiles160 = (n_width / 160 + (n_width % 160 != 0)) * m_tiles;
    if (tiles <= kTargetWorkgroups) {
        // One workgroup per compute unit at most: the six-stage ring.
        hipLaunchKernelGGL((projection_gemm_kernel<6, 1, 128>), dim3(tiles), dim3(kGemmThreads), 0, st, ws.tiles,
                           ws.exponents, weight, bias, out, rows, k_width, n_width);
    } else if (n_width % 160 == 0 && tiles160 <= 2 * kTargetWorkgroups && tiles > 2 * kTargetWorkgroups) {
        // 160-column tiles fit one round of two workgroups per compute unit
        // where 128-column tiles need a second.
        hipLaunchKernelGGL((projection_gemm_kernel<3, 2, 160>), dim3(tiles160), dim3(kGemmThreads), 0, st, ws.tiles,
                           ws.exponents, weight, bias, out, rows, k_width, n_width);
    } else {
        hipLaunchKernelGGL((projection_gemm_kernel<3, 2, 128>), dim3(tiles), dim3(kGemmThreads), 0, st, ws.tiles,
                           ws.exponents, weight, bias, out, rows, k_width, n_width);
    }
    return static_cast<int>(hipGetLastError());
}

}  // namespace pvlc
