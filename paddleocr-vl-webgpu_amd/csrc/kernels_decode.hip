// Paged GQA decode for gfx950: fused rotary + KV append + split-K attention
// with an in-kernel LSE merge.
//
// Work unit: one workgroup per (partition, kv head, sequence).  Each wave of
// the workgroup streams 64-token chunks (4 blocks of 16 tokens) of its kv
// head's keys and values straight from HBM into registers in MFMA operand
// order -- the blocked cache layout makes every wave-wide load one contiguous
// 1 KiB (keys) or 512 B (values) run -- and serves all 8 query heads of the
// group with matrix instructions:
//   scores  S[token][head] = K[token][:] . Q[head][:]   v_mfma_f32_16x16x32_f16
//   output  O[head][dim]  += P[head][token] V[token][dim] v_mfma_f32_16x16x16_f16
// The QK accumulator layout (lane holds 4 consecutive tokens of one head) is
// exactly the PV A-operand layout, so probabilities never leave the lane.
// Softmax statistics use cross-lane shuffles; waves combine through LDS; the
// last partition to finish (device-scope counter) merges all partitions.
//
// Latency discipline (the whole step is a few microseconds): every wave
// issues its first chunk's loads before anything else; block ids come from
// scalar loads; the appended row is rotated with vector loads while those
// loads are in flight; the merge loads partials in batches.
//
// Reference behaviour replaced: decoder_kv_append_f32, decoder_mrope_f32 (k
// and optionally q), decoder_gqa_split_partial_f32 and
// decoder_gqa_split_merge_f32 (crates/pvlc-wgsl/src/lib.rs:927-952,
// 1024-1234); arithmetic reference decode_gqa_f32 (crates/pvlc-cpu-ref/src/
// lib.rs:858-927).

#include <hip/hip_runtime.h>

#include <cstdint>

#include "pvlc_device.hpp"
#include "pvlc_internal.hpp"

namespace pvlc {
namespace {

constexpr int kMaxParts = static_cast<int>(kMaxMergeParts);
constexpr float kLog2e = 1.4426950408889634f;

struct DecodeParams {
    uint32_t num_blocks;
    uint32_t max_blocks_per_seq;
    const int32_t *block_tables;
    const int32_t *cache_lens;
    uint32_t uniform_cache_len;
    uint16_t *key_cache;
    uint16_t *value_cache;
    const uint16_t *query;
    const uint16_t *new_key;
    const uint16_t *new_value;
    uint16_t *out;
    const float *rope_cos;
    const float *rope_sin;
    uint32_t rope_rows;
    const int32_t *positions;
    uint32_t rotate_query;
    uint32_t partition_tokens;
    uint32_t max_parts;
    float *part_o;      // [seq][kv head][part][8 heads][128]
    float *part_ml;     // [seq][kv head][part][2][8]: max (log2 units) then sum
    uint32_t *counters; // [seq][kv head]
    uint32_t *error_word;
    float scale_log2;   // log2(e)/sqrt(128)
};

// Physical block of (sequence, tile); `tile` is wave-uniform so the table
// read is a scalar load.
__device__ inline uint32_t block_id(const DecodeParams &p, uint32_t seq, uint32_t tile) {
    if (p.block_tables == nullptr) return seq * p.max_blocks_per_seq + tile;
    const int32_t b = load_const(p.block_tables, static_cast<size_t>(seq) * p.max_blocks_per_seq + tile);
    if (b < 0 || static_cast<uint32_t>(b) >= p.num_blocks) {
        atomicOr(p.error_word, 2u);
        return 0;  // clamp: never address outside the planes
    }
    return static_cast<uint32_t>(b);
}

// Issue the loads of one chunk (TILES blocks of 16 tokens) starting at ws.  Tiles at or
// past part_end re-read the last valid tile (never outside the planes) and
// are masked by the caller; loading unconditionally keeps the loads of all
// four tiles back to back.
template <int TILES>
__device__ inline void load_chunk(const DecodeParams &p, uint32_t s, uint32_t g, int ws, int part_end, int row,
                                  int kg, half8_t (&kr)[TILES][4], half4_t (&vr)[TILES][8]) {
    const int last_tile = (part_end - 1) >> 4;
    uint32_t blk[TILES];
#pragma unroll
    for (int i = 0; i < TILES; ++i) blk[i] = block_id(p, s, static_cast<uint32_t>(min((ws >> 4) + i, last_tile)));
#pragma unroll
    for (int i = 0; i < TILES; ++i) {
        const size_t slab = (static_cast<size_t>(blk[i]) * kKvHeads + g) * kBlockHeadElems;
        const uint16_t *kbase = p.key_cache + slab;
        const uint16_t *vbase = p.value_cache + slab;
#pragma unroll
        for (int kb = 0; kb < 4; ++kb)
            kr[i][kb] = *reinterpret_cast<const half8_t *>(kbase + (kb * 4 + kg) * 128 + row * 8);
#pragma unroll
        for (int c = 0; c < 8; ++c)
            vr[i][c] = *reinterpret_cast<const half4_t *>(vbase + (c * 16 + row) * 16 + kg * 4);
    }
}

template <int WAVES, int TILES>
__global__ __launch_bounds__(WAVES * 64, 2) void paged_decode_kernel(DecodeParams p) {
    constexpr int kChunkTokens = TILES * 16;  // tokens a wave holds in registers at once
    const uint32_t part = blockIdx.x;
    const uint32_t g = blockIdx.y;  // kv head
    const uint32_t s = blockIdx.z;  // sequence (or layer)
    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane(static_cast<int>(threadIdx.x >> 6));
    const int row = lane & 15;  // MFMA row/column index of this lane
    const int kg = lane >> 4;   // MFMA k-group of this lane
    constexpr int kThreads = WAVES * 64;

    const int64_t len_raw = p.cache_lens ? load_const(p.cache_lens, s) : static_cast<int64_t>(p.uniform_cache_len);
    const int64_t capacity = static_cast<int64_t>(p.max_blocks_per_seq) * 16;
    const int64_t span = static_cast<int64_t>(p.max_parts) * p.partition_tokens;
    if (len_raw < 0 || len_raw + 1 > capacity || len_raw + 1 > span) {
        if (part == 0 && g == 0 && threadIdx.x == 0) atomicOr(p.error_word, 1u);
        return;
    }
    const int cache_len = static_cast<int>(len_raw);
    const int T = cache_len + 1;  // rows attended after the append
    const int P = static_cast<int>(p.partition_tokens);
    const int part_start = static_cast<int>(part) * P;
    if (part_start >= T) return;
    const int part_end = min(part_start + P, T);
    const int num_parts = (T + P - 1) / P;

    // First chunk's keys and values: issued before anything else.
    half8_t kr[TILES][4];
    half4_t vr[TILES][8];
    int ws = part_start + wave * kChunkTokens;
    load_chunk(p, s, g, ws, part_end, row, kg, kr, vr);

    // Rotary position of the appended row (and of the query).
    bool rope = p.rope_cos != nullptr;
    const int pos = p.positions ? load_const(p.positions, s) : cache_len;
    if (rope && (pos < 0 || static_cast<uint32_t>(pos) >= p.rope_rows)) {
        if (threadIdx.x == 0) atomicOr(p.error_word, 4u);
        rope = false;
    }
    const float *cos_row = rope ? p.rope_cos + static_cast<size_t>(pos) * 64 : nullptr;
    const float *sin_row = rope ? p.rope_sin + static_cast<size_t>(pos) * 64 : nullptr;

    // Query as the B operand of the score MFMA: column = query head of the
    // group (8 real, 8 zero), k = dims kb*32 + kg*8 .. +8.
    half8_t qb[4];
    {
        const uint16_t *qrow = p.query + (static_cast<size_t>(s) * kQueryHeads + g * kGroup + row) * kHeadDim;
#pragma unroll
        for (int kb = 0; kb < 4; ++kb) {
            const int d0 = kb * 32 + kg * 8;
            if (row < static_cast<int>(kGroup)) {
                qb[kb] = (rope && p.rotate_query) ? rotate_chunk(qrow, d0, cos_row, sin_row)
                                                  : *reinterpret_cast<const half8_t *>(qrow + d0);
            } else {
                qb[kb] = half8_t{};
            }
        }
    }

    // The workgroup whose partition holds the appended row rotates the new
    // key once, writes the new K/V row into the cache, and keeps it in LDS to
    // stand in for that row of its tile loads (which may see the old row).
    const int append_tile = cache_len >> 4;
    const int append_row = cache_len & 15;
    __shared__ uint16_t sm_new_k[kHeadDim];
    __shared__ uint16_t sm_new_v[kHeadDim];
    const bool owns_append = (append_tile << 4) >= part_start && (append_tile << 4) < part_end;
    if (owns_append) {
        if (threadIdx.x < 32) {
            const uint32_t blk = block_id(p, s, static_cast<uint32_t>(append_tile));
            const size_t slab = (static_cast<size_t>(blk) * kKvHeads + g) * kBlockHeadElems;
            if (threadIdx.x < 16) {
                const uint16_t *new_k = p.new_key + (static_cast<size_t>(s) * kKvHeads + g) * kHeadDim;
                const int d0 = threadIdx.x * 8;
                const half8_t nk = rope ? rotate_chunk(new_k, d0, cos_row, sin_row)
                                        : *reinterpret_cast<const half8_t *>(new_k + d0);
                *reinterpret_cast<half8_t *>(sm_new_k + d0) = nk;
                *reinterpret_cast<half8_t *>(p.key_cache + slab + threadIdx.x * 128 + append_row * 8) = nk;
            } else {
                const uint16_t *new_v = p.new_value + (static_cast<size_t>(s) * kKvHeads + g) * kHeadDim;
                const int d0 = (threadIdx.x - 16) * 8;
                // A uint16 vector: scattering elements of a _Float16 vector
                // with 16-bit stores stored element 0 eight times on gfx950.
                const u16x8_t nv = *reinterpret_cast<const u16x8_t *>(new_v + d0);
                *reinterpret_cast<u16x8_t *>(sm_new_v + d0) = nv;
#pragma unroll
                for (int j = 0; j < 8; ++j) p.value_cache[slab + (d0 + j) * 16 + append_row] = nv[j];
            }
        }
        __syncthreads();  // uniform: owns_append depends on the workgroup only
    }

    float m_run = -INFINITY;  // running max (log2 units) of head `row`
    float l_run = 0.0f;       // this lane's share of the running sum
    float4_t o[8];
#pragma unroll
    for (int c = 0; c < 8; ++c) o[c] = float4_t{0.f, 0.f, 0.f, 0.f};

    for (int chunk = 0; ws < part_end; ++chunk, ws += WAVES * kChunkTokens) {
        if (chunk > 0) load_chunk(p, s, g, ws, part_end, row, kg, kr, vr);

        // Zero the values of tiles past the partition (their scores are
        // masked to -inf, but a re-read tile may hold poison rows, and
        // NaN * 0 would reach P.V).
#pragma unroll
        for (int i = 0; i < TILES; ++i) {
            if (ws + i * 16 >= part_end) {
#pragma unroll
                for (int c = 0; c < 8; ++c) vr[i][c] = half4_t{};
            }
        }
        // Patch the appended row; zero rows past it (they may hold poison).
        const int ti = append_tile - (ws >> 4);
        if (ti >= 0 && ti < TILES) {
#pragma unroll
            for (int i = 0; i < TILES; ++i) {
                if (i != ti) continue;
                if (row == append_row) {
#pragma unroll
                    for (int kb = 0; kb < 4; ++kb)
                        kr[i][kb] = *reinterpret_cast<const half8_t *>(sm_new_k + (kb * 4 + kg) * 8);
                }
#pragma unroll
                for (int j = 0; j < 4; ++j) {
                    const int r = kg * 4 + j;
#pragma unroll
                    for (int c = 0; c < 8; ++c) {
                        if (r == append_row)
                            vr[i][c][j] = __builtin_bit_cast(_Float16, sm_new_v[c * 16 + row]);
                        else if (r > append_row)
                            vr[i][c][j] = static_cast<_Float16>(0.0f);
                    }
                }
            }
        }

        // Scores: lane holds tokens ws + i*16 + kg*4 + r (r = 0..3) of head `row`.
        float x[TILES][4];
        float cmax = -INFINITY;
#pragma unroll
        for (int i = 0; i < TILES; ++i) {
            float4_t acc = float4_t{0.f, 0.f, 0.f, 0.f};
#pragma unroll
            for (int kb = 0; kb < 4; ++kb)
                acc = __builtin_amdgcn_mfma_f32_16x16x32_f16(kr[i][kb], qb[kb], acc, 0, 0, 0);
            const int tbase = ws + i * 16 + kg * 4;
#pragma unroll
            for (int r = 0; r < 4; ++r) {
                x[i][r] = (tbase + r < part_end) ? acc[r] * p.scale_log2 : -INFINITY;
                cmax = fmaxf(cmax, x[i][r]);
            }
        }
        cmax = fmaxf(cmax, __shfl_xor(cmax, 16));
        cmax = fmaxf(cmax, __shfl_xor(cmax, 32));
        const float m_new = fmaxf(m_run, cmax);  // finite: token ws is valid
        const float alpha = __builtin_amdgcn_exp2f(m_run - m_new);
        l_run *= alpha;
        m_run = m_new;
        if (chunk > 0) {
            // Output rows are heads kg*4 + r; their rescale factors live in
            // the lanes whose column index is that head.
#pragma unroll
            for (int r = 0; r < 4; ++r) {
                const float a = __shfl(alpha, kg * 4 + r);
#pragma unroll
                for (int c = 0; c < 8; ++c) o[c][r] *= a;
            }
        }

#pragma unroll
        for (int i = 0; i < TILES; ++i) {
            half4_t pa;
#pragma unroll
            for (int r = 0; r < 4; ++r) {
                const _Float16 ph = to_h(__builtin_amdgcn_exp2f(x[i][r] - m_new));
                pa[r] = ph;
                l_run += static_cast<float>(ph);  // the weights P.V actually uses
            }
#pragma unroll
            for (int c = 0; c < 8; ++c) o[c] = __builtin_amdgcn_mfma_f32_16x16x16f16(pa, vr[i][c], o[c], 0, 0, 0);
        }
    }
    l_run += __shfl_xor(l_run, 16);
    l_run += __shfl_xor(l_run, 32);

    // Combine the waves of this partition in LDS.
    __shared__ float sm_m[WAVES][kGroup];
    __shared__ float sm_l[WAVES][kGroup];
    __shared__ float sm_o[WAVES][kGroup][kHeadDim + 4];
    __shared__ int sm_last;
    if (lane < static_cast<int>(kGroup)) {
        sm_m[wave][lane] = m_run;
        sm_l[wave][lane] = l_run;
    }
    if (kg < 2) {
#pragma unroll
        for (int c = 0; c < 8; ++c)
#pragma unroll
            for (int r = 0; r < 4; ++r) sm_o[wave][kg * 4 + r][c * 16 + row] = o[c][r];
    }
    __syncthreads();

    constexpr int kPerThread = (kGroup * kHeadDim) / kThreads;
    float po[kPerThread], pm[kPerThread], pl[kPerThread];
#pragma unroll
    for (int e = 0; e < kPerThread; ++e) {
        const int idx = threadIdx.x + e * kThreads;
        const int h = idx >> 7, d = idx & 127;
        float M = -INFINITY;
#pragma unroll
        for (int w = 0; w < WAVES; ++w) M = fmaxf(M, sm_m[w][h]);
        float L = 0.f, O = 0.f;
#pragma unroll
        for (int w = 0; w < WAVES; ++w) {
            const float f = __builtin_amdgcn_exp2f(sm_m[w][h] - M);
            L += sm_l[w][h] * f;
            O += sm_o[w][h][d] * f;
        }
        po[e] = O;
        pm[e] = M;
        pl[e] = L;
    }

    uint16_t *out = p.out + (static_cast<size_t>(s) * kQueryHeads + g * kGroup) * kHeadDim;
    if (num_parts == 1) {
#pragma unroll
        for (int e = 0; e < kPerThread; ++e) {
            const int idx = threadIdx.x + e * kThreads;
            out[idx] = __builtin_bit_cast(uint16_t, to_h(po[e] / pl[e]));
        }
        return;
    }

    // Cross-workgroup hand-off without L2 maintenance: partials, the arrival
    // counter and the merge reads are relaxed agent-scope atomics (sc1), which
    // are coherent across the XCDs' L2s by themselves.  Every store of the
    // workgroup completes (s_waitcnt vmcnt(0), then the barrier) before thread
    // 0 counts the arrival, which orders the partials before the count.
    // (A C++ release/acquire fence at agent scope would instead write back and
    // invalidate the whole L2 of the XCD in every workgroup.)
    const size_t unit = (static_cast<size_t>(s) * kKvHeads + g) * p.max_parts;
    float *part_o = p.part_o + (unit + part) * (kGroup * kHeadDim);
    float *part_ml = p.part_ml + (unit + part) * (2 * kGroup);
#pragma unroll
    for (int e = 0; e < kPerThread; ++e) {
        const int idx = threadIdx.x + e * kThreads;
        __hip_atomic_store(part_o + idx, po[e], __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        if ((idx & 127) == 0) {
            __hip_atomic_store(part_ml + (idx >> 7), pm[e], __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            __hip_atomic_store(part_ml + kGroup + (idx >> 7), pl[e], __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        }
    }
    // Wait for this wave's partial stores to complete (a single-wave
    // workgroup's __syncthreads() emits no wait), then for every wave.
    asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
    __syncthreads();
    if (threadIdx.x == 0) {
        const uint32_t prev = __hip_atomic_fetch_add(p.counters + s * kKvHeads + g, 1u, __ATOMIC_RELAXED,
                                                     __HIP_MEMORY_SCOPE_AGENT);
        sm_last = (prev == static_cast<uint32_t>(num_parts - 1));
    }
    __syncthreads();
    if (!sm_last) return;

    // Merge: the (max, sum) of every partition is staged in LDS (one load
    // per thread) while the first batch of partial outputs is already in
    // flight; one weight per (partition, head) then scales the partials.
    const float *all_o = p.part_o + unit * (kGroup * kHeadDim);
    const float *all_ml = p.part_ml + unit * (2 * kGroup);
    __shared__ float sm_ml[kMaxParts * 2 * kGroup];
    __shared__ float sm_w[kMaxParts * kGroup];
    auto ld = [](const float *q) { return __hip_atomic_load(q, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT); };
    constexpr int kBatch = 8;
    float acc[kPerThread];
    float v[kBatch][kPerThread];
#pragma unroll
    for (int e = 0; e < kPerThread; ++e) acc[e] = 0.f;
    auto load_batch = [&](int q0) {
#pragma unroll
        for (int b = 0; b < kBatch; ++b) {
            const int q = min(q0 + b, num_parts - 1);  // clamped re-reads get weight 0 below
#pragma unroll
            for (int e = 0; e < kPerThread; ++e)
                v[b][e] = ld(all_o + static_cast<size_t>(q) * (kGroup * kHeadDim) + threadIdx.x + e * kThreads);
        }
    };
    load_batch(0);
    for (int i = threadIdx.x; i < num_parts * 2 * static_cast<int>(kGroup); i += kThreads) sm_ml[i] = ld(all_ml + i);
    __syncthreads();
    if (threadIdx.x < static_cast<int>(kGroup)) {
        const int h = threadIdx.x;
        float M = -INFINITY;
        for (int q = 0; q < num_parts; ++q) M = fmaxf(M, sm_ml[q * 2 * kGroup + h]);
        float L = 0.f;
        for (int q = 0; q < num_parts; ++q) {
            const float f = __builtin_amdgcn_exp2f(sm_ml[q * 2 * kGroup + h] - M);
            sm_w[q * kGroup + h] = f;
            L += sm_ml[q * 2 * kGroup + kGroup + h] * f;
        }
        const float inv = 1.0f / L;
        for (int q = 0; q < num_parts; ++q) sm_w[q * kGroup + h] *= inv;
    }
    __syncthreads();
    for (int q0 = 0; q0 < num_parts; q0 += kBatch) {
        if (q0 > 0) load_batch(q0);
#pragma unroll
        for (int b = 0; b < kBatch; ++b)
#pragma unroll
            for (int e = 0; e < kPerThread; ++e) {
                const int h = (threadIdx.x + e * kThreads) >> 7;
                acc[e] += (q0 + b < num_parts) ? v[b][e] * sm_w[(q0 + b) * kGroup + h] : 0.f;
            }
    }
#pragma unroll
    for (int e = 0; e < kPerThread; ++e) {
        const int idx = threadIdx.x + e * kThreads;
        out[idx] = __builtin_bit_cast(uint16_t, to_h(acc[e]));
    }
    if (threadIdx.x == 0)
        __hip_atomic_store(p.counters + s * kKvHeads + g, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

__global__ void fill_u32_kernel(uint32_t *dst, size_t words, uint32_t value) {
    const size_t i = static_cast<size_t>(blockIdx.x) * blockDim.x + threadIdx.x;
    if (i < words) dst[i] = value;
}

}  // namespace

int launch_paged_decode(const DecodeLaunch &launch, void *stream) {
    const pvlc_hip_paged_decode_args &a = *launch.args;
    DecodeParams p{};
    p.num_blocks = a.num_blocks;
    p.max_blocks_per_seq = a.max_blocks_per_seq;
    p.block_tables = a.block_tables;
    p.cache_lens = a.cache_lens;
    p.uniform_cache_len = a.uniform_cache_len;
    p.key_cache = a.key_cache;
    p.value_cache = a.value_cache;
    p.query = a.query;
    p.new_key = a.new_key;
    p.new_value = a.new_value;
    p.out = a.out;
    p.rope_cos = a.rope_cos;
    p.rope_sin = a.rope_sin;
    p.rope_rows = a.rope_rows;
    p.positions = a.positions;
    p.rotate_query = a.rotate_query;
    p.partition_tokens = launch.partition_tokens;
    p.max_parts = launch.max_parts;
    p.part_o = launch.part_o;
    p.part_ml = launch.part_ml;
    p.counters = launch.counters;
    p.error_word = launch.error_word;
    p.scale_log2 = kLog2e / sqrtf(static_cast<float>(kHeadDim));

    const dim3 grid(launch.max_parts, kKvHeads, a.num_seqs);
    hipStream_t st = static_cast<hipStream_t>(stream);
    // Workgroup shape from the partition: TILES blocks of 16 tokens per wave
    // and chunk, WAVES waves; partitions longer than WAVES*TILES*16 loop.
    const uint32_t P = launch.partition_tokens;
    const uint32_t tiles = launch.tiles_per_wave;
#define PVLC_DECODE_LAUNCH(W, TL) hipLaunchKernelGGL((paged_decode_kernel<W, TL>), grid, dim3((W) * 64), 0, st, p)
    if (tiles == 1) {
        if (P >= 128) PVLC_DECODE_LAUNCH(8, 1); else PVLC_DECODE_LAUNCH(4, 1);
    } else if (tiles == 2) {
        if (P >= 256) PVLC_DECODE_LAUNCH(8, 2); else PVLC_DECODE_LAUNCH(4, 2);
    } else {
        if (P >= 512) PVLC_DECODE_LAUNCH(8, 4); else if (P >= 256) PVLC_DECODE_LAUNCH(4, 4); else PVLC_DECODE_LAUNCH(2, 4);
    }
#undef PVLC_DECODE_LAUNCH
    return static_cast<int>(hipGetLastError());
}

int launch_fill_u32(uint32_t *dst, size_t words, uint32_t value, void *stream) {
    if (words == 0) return 0;
    const unsigned blocks = static_cast<unsigned>((words + 255) / 256);
    hipLaunchKernelGGL(fill_u32_kernel, dim3(blocks), dim3(256), 0, static_cast<hipStream_t>(stream), dst, words,
                       value);
    return static_cast<int>(hipGetLastError());
}

}  // namespace pvlc
