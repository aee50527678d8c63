// Causal prefill for gfx950: rotary + range append into the paged cache, then
// MFMA flash attention over the cache.
//
// Kernel 1 (one 16-token cache block per workgroup): rotates the 2 key heads
// and writes them with the values into the blocked cache (the same rounding as the decode
// append, so prefill and decode leave bit-identical rows), and, when the
// caller passes a query scratch, writes the rotated queries there.  Replaces
// decoder_prefill_mrope_f32 and decoder_kv_append_range_f32
// (crates/pvlc-wgsl/src/lib.rs:1334-1416).
//
// Kernel 2: one workgroup per (16-token query block, kv head) serves the 8
// query heads of the group; each of its 4 waves owns 2 heads, i.e. two
// 16-column MFMA tiles of query rows.  Keys and values stream through
// double-buffered LDS in steps of 64 keys (2 pairs of cache blocks), laid out
// so every operand read is conflict-free, with the next step loaded into
// registers while the current one is computed:
//   S^T[key][row] = K . Q^T           v_mfma_f32_16x16x32_f16
//   O[row][dim]  += P[row][key] V      v_mfma_f32_16x16x32_f16
//   l[row]       += P[row][key] 1      (same MFMA, ones operand)
// The key slot order of the cache (key_slot) makes the score MFMA leave each
// lane 8 consecutive keys of one tile, which is the P operand of the P.V MFMA.
// Online softmax in log2 units (scale folded into one FMA per score), the
// causal mask only on steps that reach the diagonal, and the rescale skipped
// while the running max is unchanged.  Heavy and light query blocks are
// paired over the grid for balance.  Replaces
// decoder_prefill_gqa_f32 (crates/pvlc-wgsl/src/lib.rs:1262-1332); arithmetic
// reference causal_gqa_f32 (crates/pvlc-cpu-ref/src/lib.rs:782-853).

#include <hip/hip_runtime.h>

#include <cstdint>
#include <type_traits>

#include "pvlc_device.hpp"
#include "pvlc_internal.hpp"

namespace pvlc {
namespace {

constexpr float kLog2e = 1.4426950408889634f;
constexpr int kQueryBlock = 16;  // query tokens per workgroup
constexpr int kKeyStep = 64;     // keys per softmax step (4 cache blocks)
constexpr int kStepTiles = kKeyStep / 16;
constexpr int kWaves = 4;        // each wave: 2 of the 8 heads of the group
constexpr float kLazyRescaleLog2 = 8.0f;  // softmax reference moves only past 2^8

struct PrefillParams {
    uint32_t tokens;
    uint32_t num_blocks;
    const int32_t *block_table;
    uint16_t *key_cache;
    uint16_t *value_cache;
    const uint16_t *query;
    const uint16_t *key;
    const uint16_t *value;
    uint16_t *out;
    const float *rope_cos;
    const float *rope_sin;
    uint32_t rope_rows;
    const int32_t *positions;
    uint16_t *qrot;
    uint32_t *error_word;
    float scale_log2;
    // split-K pair schedule (a workspace was given and the blocks are long)
    bool split;
    uint32_t *counters;  // [pair][kv head]
    float *partials;     // [pair][kv head][2 parts][kPrefillPartialFloats]
    // f32 operands (pvlc_hip_paged_prefill_f32io): query, key, value, output;
    // null for the fp16 entry point.
    const float *query32;
    const float *key32;
    const float *value32;
    float *out32;
};

__device__ inline uint32_t cache_block(const PrefillParams &p, uint32_t tile, bool *ok) {
    if (p.block_table == nullptr) {
        *ok = tile < p.num_blocks;
        return *ok ? tile : 0u;
    }
    const int32_t b = load_const(p.block_table, tile);
    *ok = b >= 0 && static_cast<uint32_t>(b) < p.num_blocks;
    return *ok ? static_cast<uint32_t>(b) : 0u;
}

// Kernel 1: one workgroup per 16-token cache block, both key heads.  Every
// thread rotates two 8-dim key chunks (item = head, chunk, token; 16
// consecutive threads fill one 256-byte run of the key slab) and writes one
// 32-byte value row of the slab (head, dim: 16 tokens) after a transpose of
// the block's value rows through LDS, so every cache store is a full 16-byte
// vector and each 32-byte sector is written once.  With a query scratch the
// workgroup also writes the rotated queries of its tokens (the attention
// kernel rotates its own query fragments, so the scratch is only an output for
// callers that want it).
constexpr int kAppendThreads = 256;

// Rotary position of token t and whether its tables hold it (bit 4 of the
// error word otherwise, reported once per token by the caller's choice).
__device__ inline int rope_position(const PrefillParams &p, uint32_t t, bool *rope) {
    const int pos = p.positions ? p.positions[t] : static_cast<int>(t);
    *rope = p.rope_cos != nullptr && pos >= 0 && static_cast<uint32_t>(pos) < p.rope_rows;
    return pos;
}

template <bool F32IO>
__global__ __launch_bounds__(kAppendThreads) void prefill_rope_append_kernel(PrefillParams p) {
    const int i = threadIdx.x;
    const uint32_t b = blockIdx.x;  // cache block (16 tokens) of the sequence
    const uint32_t t0 = b * kBlockTokens;
    const uint32_t ntok = min(p.tokens - t0, kBlockTokens);
    __shared__ uint16_t sv[kBlockTokens][kRowElems + 8];  // value rows, padded against bank conflicts

    // value rows of the block: 16 tokens x 256 fp16, two 16-byte pieces per
    // thread, loaded now and staged into LDS after the key loads are issued
    u16x8_t vrow[2];
#pragma unroll
    for (int r = 0; r < 2; ++r) {
        const int k = i + r * kAppendThreads;
        const uint32_t t = t0 + min(static_cast<uint32_t>(k >> 5), ntok - 1);
        if constexpr (F32IO)
            vrow[r] = __builtin_bit_cast(u16x8_t, round_chunk(p.value32 + static_cast<size_t>(t) * kRowElems + (k & 31) * 8));
        else
            vrow[r] = *reinterpret_cast<const u16x8_t *>(p.value + static_cast<size_t>(t) * kRowElems + (k & 31) * 8);
    }

    bool ok;
    const uint32_t blk = cache_block(p, b, &ok);
    if (!ok && i == 0 && p.error_word) atomicOr(p.error_word, 2u);
    // keys: item (head, chunk, token), 16 consecutive threads per 256-byte run
#pragma unroll
    for (int r = 0; r < 2; ++r) {
        const int k = i + r * kAppendThreads;
        const int tt = k & 15, c = (k >> 4) & 15, hh = k >> 8;
        if (static_cast<uint32_t>(tt) < ntok) {
            const uint32_t t = t0 + tt;
            bool rope;
            const int pos = rope_position(p, t, &rope);
            if (!rope && p.rope_cos != nullptr && c == 0 && hh == 0 && p.error_word) atomicOr(p.error_word, 4u);
            const size_t koff = (static_cast<size_t>(t) * kKvHeads + hh) * kHeadDim;
            half8_t kv;
            if constexpr (F32IO) {
                kv = rope ? rotate_chunk(p.key32 + koff, c * 8, p.rope_cos + static_cast<size_t>(pos) * 64,
                                         p.rope_sin + static_cast<size_t>(pos) * 64)
                          : round_chunk(p.key32 + koff + c * 8);
            } else {
                const uint16_t *krow = p.key + koff;
                kv = rope ? rotate_chunk(krow, c * 8, p.rope_cos + static_cast<size_t>(pos) * 64,
                                         p.rope_sin + static_cast<size_t>(pos) * 64)
                          : *reinterpret_cast<const half8_t *>(krow + c * 8);
            }
            const size_t slab = (static_cast<size_t>(blk) * kKvHeads + hh) * kBlockHeadElems;
            if (ok) *reinterpret_cast<half8_t *>(p.key_cache + slab + c * 128 + key_slot(tt) * 8) = kv;
        }
    }
#pragma unroll
    for (int r = 0; r < 2; ++r) {
        const int k = i + r * kAppendThreads;
        *reinterpret_cast<u16x8_t *>(&sv[k >> 5][(k & 31) * 8]) = vrow[r];
    }
    __syncthreads();
    if (ok) {
        // value slab row (head, dim): the block's 16 tokens; a partial last
        // block keeps the slab's other tokens as they were
        const int hh = i >> 7, d = i & 127;
        const size_t slab = (static_cast<size_t>(blk) * kKvHeads + hh) * kBlockHeadElems;
        uint16_t *dst = p.value_cache + slab + d * kBlockTokens;
        if (ntok == kBlockTokens) {
            u16x8_t lo, hi;
#pragma unroll
            for (int tt = 0; tt < 8; ++tt) {
                lo[tt] = sv[tt][hh * kHeadDim + d];
                hi[tt] = sv[tt + 8][hh * kHeadDim + d];
            }
            *reinterpret_cast<u16x8_t *>(dst) = lo;
            *reinterpret_cast<u16x8_t *>(dst + 8) = hi;
        } else {
            for (uint32_t tt = 0; tt < ntok; ++tt) dst[tt] = sv[tt][hh * kHeadDim + d];
        }
    }
    if (p.qrot) {
        // (token, head, 8-dim chunk) items of the block's tokens
        for (int k = i; k < static_cast<int>(kBlockTokens * kQueryHeads * 16); k += kAppendThreads) {
            const int tt = k / (kQueryHeads * 16);
            if (static_cast<uint32_t>(tt) >= ntok) break;
            const uint32_t tq = t0 + tt;
            const int h = (k >> 4) % kQueryHeads, d0 = (k & 15) * 8;
            bool rope;
            const int pos = rope_position(p, tq, &rope);
            const size_t qoff = (static_cast<size_t>(tq) * kQueryHeads + h) * kHeadDim;
            half8_t q;
            if constexpr (F32IO) {
                q = rope ? rotate_chunk(p.query32 + qoff, d0, p.rope_cos + static_cast<size_t>(pos) * 64,
                                        p.rope_sin + static_cast<size_t>(pos) * 64)
                         : round_chunk(p.query32 + qoff + d0);
            } else {
                const uint16_t *qrow = p.query + qoff;
                q = rope ? rotate_chunk(qrow, d0, p.rope_cos + static_cast<size_t>(pos) * 64,
                                        p.rope_sin + static_cast<size_t>(pos) * 64)
                         : *reinterpret_cast<const half8_t *>(qrow + d0);
            }
            *reinterpret_cast<half8_t *>(p.qrot + (static_cast<size_t>(tq) * kQueryHeads + h) * kHeadDim + d0) = q;
        }
    }
}

// LDS layouts of one 64-key step (2 pairs of 16-token tiles), chosen so every
// 16-lane group of an MFMA operand read is one contiguous 256-byte run (no
// bank conflicts):
//   keys   [pair][16 dim-chunks][score MFMA h][tile of pair][8 slots][8 dims]
//   values [pair][tile of pair][token half][128 dims][8 tokens]
constexpr int kStepElems = kStepTiles * kBlockHeadElems;  // fp16 elements per plane and step

__device__ inline int lds_key_offset(int j, int chunk, int h, int tile, int slot8) {
    return ((((j * 16 + chunk) * 2 + h) * 2 + tile) * 8 + slot8) * 8;
}
__device__ inline int lds_value_offset(int j, int tile, int half, int dim) {
    return (((j * 2 + tile) * 2 + half) * kHeadDim + dim) * 8;
}

// Work item b of the grid: query blocks are paired heaviest with lightest,
// so that the two items a compute unit runs (b and b + qblocks, dispatched
// in order) sum to about the same number of key steps everywhere.
__device__ inline void prefill_item(int b, int qblocks, int *qb, uint32_t *g) {
    if (b < qblocks) {
        *qb = qblocks - 1 - b;
        *g = 0;
    } else {
        *qb = b - qblocks;
        *g = 1;
    }
}

template <bool F32IO>
__global__ __launch_bounds__(kWaves * 64, 2) void prefill_attention_kernel(PrefillParams p) {
    const int n = static_cast<int>(p.tokens);
    const int qblocks = (n + kQueryBlock - 1) / kQueryBlock;
    uint32_t g, pair = 0;
    PrefillSegment seg0{}, seg1{};
    int nseg = 1;
    if (p.split) {
        nseg = static_cast<int>(prefill_pair_segments(blockIdx.x, static_cast<uint32_t>(qblocks), &g, &pair, &seg0, &seg1));
    } else {
        int qb0;
        prefill_item(static_cast<int>(blockIdx.x), qblocks, &qb0, &g);
        seg0 = {static_cast<uint32_t>(qb0), 0u, 1u, 0u, prefill_block_steps(static_cast<uint32_t>(qb0))};
    }
    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane(static_cast<int>(threadIdx.x >> 6));
    const int row = lane & 15, kg = lane >> 4;
    // Four distinct arrays (not one indexed by parity): the main loop picks
    // them at compile time, so the compiler sees that a step's loads into LDS
    // and its LDS reads touch different buffers and does not wait for the
    // loads before the reads.
    __shared__ __align__(16) uint16_t sk0[kStepElems], sk1[kStepElems];
    __shared__ __align__(16) uint16_t sv0[kStepElems], sv1[kStepElems];
    __shared__ bool sm_last;

  // One segment: a whole query block, or one part of a split one.
  auto run_segment = [&](const PrefillSegment sg) {
    const int qb = static_cast<int>(sg.qb);
    const uint32_t part = sg.part, nparts = sg.nparts;
    const int s_begin = static_cast<int>(sg.step_begin), steps = static_cast<int>(sg.steps);
    const int t0 = qb * kQueryBlock;
    const int my_token = t0 + row;  // query token of this lane's column

    // Query fragments (B operand): column = token t0 + row of head h, dims
    // kb*32 + kg*8 .. +8, rotated here (rotate-half: the partner of chunk kb
    // is chunk kb^2 of the same lane) exactly as rotate_chunk does.
    const int tq = min(my_token, n - 1);
    const int qpos = p.positions ? p.positions[tq] : tq;
    const bool qrope = p.rope_cos != nullptr && qpos >= 0 && static_cast<uint32_t>(qpos) < p.rope_rows;
    float4_t qc[2][2], qs[2][2];  // cos/sin of pairs hk*32 + kg*8 .. +8 (hk = kb & 1)
    {
        const float *cr = qrope ? p.rope_cos + static_cast<size_t>(qpos) * 64 : reinterpret_cast<const float *>(p.query);
        const float *sr = qrope ? p.rope_sin + static_cast<size_t>(qpos) * 64 : reinterpret_cast<const float *>(p.query);
#pragma unroll
        for (int hk = 0; hk < 2; ++hk)
#pragma unroll
            for (int f = 0; f < 2; ++f) {
                qc[hk][f] = *reinterpret_cast<const float4_t *>(cr + hk * 32 + kg * 8 + f * 4);
                qs[hk][f] = *reinterpret_cast<const float4_t *>(sr + hk * 32 + kg * 8 + f * 4);
            }
    }
    half8_t qf[2][4];
#pragma unroll
    for (int ct = 0; ct < 2; ++ct) {
        const int h = static_cast<int>(g) * kGroup + wave * 2 + ct;
        const size_t qoff = (static_cast<size_t>(tq) * kQueryHeads + h) * kHeadDim;
        if constexpr (F32IO) {
            // f32 query: rotated from its f32 values and rounded once.
            float raw[4][8];
#pragma unroll
            for (int kb = 0; kb < 4; ++kb) {
                const float4_t lo = *reinterpret_cast<const float4_t *>(p.query32 + qoff + kb * 32 + kg * 8);
                const float4_t hi = *reinterpret_cast<const float4_t *>(p.query32 + qoff + kb * 32 + kg * 8 + 4);
#pragma unroll
                for (int jj = 0; jj < 4; ++jj) {
                    raw[kb][jj] = lo[jj];
                    raw[kb][jj + 4] = hi[jj];
                }
            }
#pragma unroll
            for (int kb = 0; kb < 4; ++kb) {
                half8_t q;
#pragma unroll
                for (int jj = 0; jj < 8; ++jj) {
                    if (qrope) {
                        const float c = qc[kb & 1][jj >> 2][jj & 3];
                        const float sn = qs[kb & 1][jj >> 2][jj & 3];
                        const float x = raw[kb][jj];
                        const float y = raw[kb ^ 2][jj];
                        q[jj] = kb < 2 ? to_h(x * c + (-y) * sn) : to_h(x * c + y * sn);
                    } else {
                        q[jj] = to_h(raw[kb][jj]);
                    }
                }
                qf[ct][kb] = my_token < n ? q : half8_t{};
            }
        } else {
            const uint16_t *qrow = p.query + qoff;
            half8_t raw[4];
#pragma unroll
            for (int kb = 0; kb < 4; ++kb) raw[kb] = *reinterpret_cast<const half8_t *>(qrow + kb * 32 + kg * 8);
#pragma unroll
            for (int kb = 0; kb < 4; ++kb) {
                half8_t q = raw[kb];
                if (qrope) {
#pragma unroll
                    for (int jj = 0; jj < 8; ++jj) {
                        const float c = qc[kb & 1][jj >> 2][jj & 3];
                        const float sn = qs[kb & 1][jj >> 2][jj & 3];
                        const float x = static_cast<float>(raw[kb][jj]);
                        const float y = static_cast<float>(raw[kb ^ 2][jj]);
                        q[jj] = kb < 2 ? to_h(x * c + (-y) * sn) : to_h(x * c + y * sn);
                    }
                }
                qf[ct][kb] = my_token < n ? q : half8_t{};
            }
        }
    }

    const int nkeys = min(t0 + kQueryBlock, n);
    const int last_tile = (nkeys - 1) >> 4;
    const bool last_part = part + 1 == nparts;

    // Double-buffered LDS, filled by direct global-to-LDS loads (16 bytes a
    // lane: lane l of a wave's load lands at the wave's LDS base + 16 l).
    // Each wave issues 4 key and 4 value loads per step; lane and load index
    // pick the global chunk that belongs at that LDS position of the layouts
    // above.  Steps past the end re-read the last tile (never used).
    typedef __attribute__((address_space(3))) void *lds_ptr;
    // ln: the lane id (passed in, so the last steps can use a separately
    // computed copy; see the tail loop below).
    auto dma_k = [&](int step, uint16_t *dst, int ln) {
        // LDS chunk q = 64 k + ln (k = 4 wave + r): slot8 = ln & 7,
        // tile = ln bit 3, h = ln bit 4, dim-chunk = 2 (k & 7) + ln bit 5, pair j = k >> 3
        const int j = wave >> 1;
        bool ok;
        const uint32_t b0 = cache_block(p, static_cast<uint32_t>(min(step * kStepTiles + 2 * j, last_tile)), &ok);
        const uint32_t b1 = cache_block(p, static_cast<uint32_t>(min(step * kStepTiles + 2 * j + 1, last_tile)), &ok);
        const uint32_t blk = (ln & 8) ? b1 : b0;
        const uint16_t *src = p.key_cache + (static_cast<size_t>(blk) * kKvHeads + g) * kBlockHeadElems +
                              (((ln >> 4) & 1) * 8 + (ln & 7)) * 8 + (ln >> 5) * 128;
#pragma unroll
        for (int r = 0; r < 4; ++r) {
            const int k = 4 * wave + r;
            __builtin_amdgcn_global_load_lds(src + (2 * (k & 7)) * 128, (lds_ptr)(dst + 64 * k * 8), 16, 0, 0);
        }
    };
    auto dma_v = [&](int step, uint16_t *dst, int ln) {
        // LDS chunk q = 64 k + ln: dim = (k & 1) 64 + ln, half = (k >> 1) & 1,
        // tile = (k >> 2) & 1 = wave & 1, pair j = k >> 3 = wave >> 1
        bool ok;
        const uint32_t blk = cache_block(p, static_cast<uint32_t>(min(step * kStepTiles + wave, last_tile)), &ok);
        const uint16_t *src = p.value_cache + (static_cast<size_t>(blk) * kKvHeads + g) * kBlockHeadElems + ln * 16;
#pragma unroll
        for (int r = 0; r < 4; ++r) {
            const int k = 4 * wave + r;
            __builtin_amdgcn_global_load_lds(src + (r & 1) * 64 * 16 + (r >> 1) * 8, (lds_ptr)(dst + 64 * k * 8), 16,
                                             0, 0);
        }
    };

    float4_t o[2][9];  // 8 column tiles of the output, then the row sums
#pragma unroll
    for (int ct = 0; ct < 2; ++ct)
#pragma unroll
        for (int c = 0; c < 9; ++c) o[ct][c] = float4_t{0.f, 0.f, 0.f, 0.f};
    half8_t ones;
#pragma unroll
    for (int e = 0; e < 8; ++e) ones[e] = static_cast<_Float16>(1.0f);
    const float scale = p.scale_log2;

    // Scores of one step: MFMA h of pair j leaves lane (column = query token,
    // kg) the keys (kg & 1)*8 + h*4 + r of the pair's tile kg >> 1.
    typedef float Scores[2][2][8];
    auto scores = [&](const uint16_t *kl, Scores &x) {
        // 8 independent accumulator chains (pair j, slot half h, head ct), the
        // 32-dim chunk kb outermost, so no MFMA waits on the previous one
        float4_t acc[2][2][2];
#pragma unroll
        for (int j = 0; j < 2; ++j)
#pragma unroll
            for (int h = 0; h < 2; ++h)
#pragma unroll
                for (int ct = 0; ct < 2; ++ct) acc[j][h][ct] = float4_t{0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int kb = 0; kb < 4; ++kb) {
            half8_t kf[2][2];
#pragma unroll
            for (int j = 0; j < 2; ++j)
#pragma unroll
                for (int h = 0; h < 2; ++h)
                    kf[j][h] = *reinterpret_cast<const half8_t *>(kl + lds_key_offset(j, kb * 4 + kg, h, row >> 3, row & 7));
#pragma unroll
            for (int j = 0; j < 2; ++j)
#pragma unroll
                for (int h = 0; h < 2; ++h)
#pragma unroll
                    for (int ct = 0; ct < 2; ++ct)
                        acc[j][h][ct] = __builtin_amdgcn_mfma_f32_16x16x32_f16(kf[j][h], qf[ct][kb], acc[j][h][ct], 0, 0, 0);
        }
#pragma unroll
        for (int ct = 0; ct < 2; ++ct)
#pragma unroll
            for (int j = 0; j < 2; ++j)
#pragma unroll
                for (int h = 0; h < 2; ++h)
#pragma unroll
                    for (int r = 0; r < 4; ++r) x[ct][j][h * 4 + r] = acc[j][h][ct][r];
    };
    // The causal mask and the end of the sequence only touch steps that
    // reach past the first query token of the block.
    auto needs_mask = [&](int step) { return step * kKeyStep + kKeyStep - 1 > t0 || step * kKeyStep + kKeyStep > n; };
    auto apply_mask = [&](int step, Scores &x) {
#pragma unroll
        for (int j = 0; j < 2; ++j)
#pragma unroll
            for (int e = 0; e < 8; ++e) {
                const int key = step * kKeyStep + (2 * j + (kg >> 1)) * 16 + (kg & 1) * 8 + e;
                const bool keep = key <= my_token && key < n;
#pragma unroll
                for (int ct = 0; ct < 2; ++ct) x[ct][j][e] = keep ? x[ct][j][e] : -INFINITY;
            }
    };
    // Running max of the column (the 4 lanes of a column hold its 64 keys).
    auto column_max = [&](const Scores &x, const float (&m)[2], float (&m_new)[2]) {
#pragma unroll
        for (int ct = 0; ct < 2; ++ct) {
            float c = m[ct];
#pragma unroll
            for (int j = 0; j < 2; ++j)
#pragma unroll
                for (int e = 0; e < 8; ++e) c = fmaxf(c, x[ct][j][e]);
            c = fmaxf(c, __shfl_xor(c, 16));
            m_new[ct] = fmaxf(c, __shfl_xor(c, 32));
        }
    };
    // P of pair j in fp16 (the A operand of P.V), log2 units, scale folded in.
    auto probs = [&](const Scores &x, const float (&ms)[2], int j, half8_t (&pa)[2][2]) {
#pragma unroll
        for (int ct = 0; ct < 2; ++ct)
#pragma unroll
            for (int e = 0; e < 8; ++e) pa[ct][j][e] = to_h(__builtin_amdgcn_exp2f(__builtin_fmaf(x[ct][j][e], scale, -ms[ct])));
    };
    // O += P.V over pair j, and the row sums += P.1 (exactly the rounded weights).
    // The pair's 8 value fragments are read from LDS before its MFMAs.
    auto pv_mfma = [&](const uint16_t *vl, int j, const half8_t (&pa)[2][2]) {
        half8_t vf[8];
#pragma unroll
        for (int c = 0; c < 8; ++c)
            vf[c] = *reinterpret_cast<const half8_t *>(vl + lds_value_offset(j, kg >> 1, kg & 1, c * 16 + row));
#pragma unroll
        for (int c = 0; c < 8; ++c) {
#pragma unroll
            for (int ct = 0; ct < 2; ++ct) o[ct][c] = __builtin_amdgcn_mfma_f32_16x16x32_f16(pa[ct][j], vf[c], o[ct][c], 0, 0, 0);
        }
#pragma unroll
        for (int ct = 0; ct < 2; ++ct) o[ct][8] = __builtin_amdgcn_mfma_f32_16x16x32_f16(pa[ct][j], ones, o[ct][8], 0, 0, 0);
    };

    // The f32 entry point's weights and P.V for pair j: each weight p as the
    // pair hi = fp16(p), lo = fp16(p - hi) (p - hi is exact in f32), so the
    // weights keep ~22 bits instead of 11; P.V and the row sums take hi, then
    // lo, over one read of the value fragments.
    auto pv_mfma_hi_lo = [&](const uint16_t *vl, int j, const Scores &x, const float (&ms)[2]) {
        half8_t hi[2], lo[2];
#pragma unroll
        for (int ct = 0; ct < 2; ++ct)
#pragma unroll
            for (int e = 0; e < 8; ++e) {
                const float pf = __builtin_amdgcn_exp2f(__builtin_fmaf(x[ct][j][e], scale, -ms[ct]));
                hi[ct][e] = to_h(pf);
                lo[ct][e] = to_h(pf - static_cast<float>(hi[ct][e]));
            }
        half8_t vf[8];
#pragma unroll
        for (int c = 0; c < 8; ++c)
            vf[c] = *reinterpret_cast<const half8_t *>(vl + lds_value_offset(j, kg >> 1, kg & 1, c * 16 + row));
#pragma unroll
        for (int pass = 0; pass < 2; ++pass) {
#pragma unroll
            for (int c = 0; c < 8; ++c) {
#pragma unroll
                for (int ct = 0; ct < 2; ++ct)
                    o[ct][c] = __builtin_amdgcn_mfma_f32_16x16x32_f16(pass ? lo[ct] : hi[ct], vf[c], o[ct][c], 0, 0, 0);
            }
#pragma unroll
            for (int ct = 0; ct < 2; ++ct)
                o[ct][8] = __builtin_amdgcn_mfma_f32_16x16x32_f16(pass ? lo[ct] : hi[ct], ones, o[ct][8], 0, 0, 0);
        }
    };

    // Software pipeline: while the score MFMAs of step i+1 run, the VALU
    // exponentiates step i (and rescales O when the reference moved); while
    // P.V of step i runs, it masks step i+1 and takes its max.
    // K stays one step ahead of V through LDS: step i (parity i & 1) reads
    // K(i+1) from sk[(i+1)&1] and V(i) from sv[i&1], and at its start loads
    // K(i+2) into sk[i&1] and V(i+1) into sv[(i+1)&1] (both freed by step
    // i-1), waited for at its closing barrier.
    dma_k(s_begin, sk0, lane);
    dma_v(s_begin, sv0, lane);
    dma_k(s_begin + 1, sk1, lane);
    __syncthreads();
    Scores xa, xb;
    float m_run[2], ms[2], alpha[2] = {1.f, 1.f};
    bool rescale = false;
    {
        scores(sk0, xa);
        if (needs_mask(s_begin)) apply_mask(s_begin, xa);  // uniform: only the block's last step
        const float minus_inf[2] = {-INFINITY, -INFINITY};
        column_max(xa, minus_inf, m_run);  // finite: key 0 <= every query token
    }
    __syncthreads();  // every wave has read sk[0] before step 0 stores K(2) there

    // Step i of the unit (block step s_begin + i).  more: a step i+1 exists
    // (its scores are computed here); mask_next: step i+1 is the block's last
    // step, the only one that reaches the diagonal or the end of the sequence
    // (query blocks are 16-aligned inside 64-key steps), so the mask stays out
    // of the main loop.  K(i+2) is loaded when more && !mask_next (a unit that
    // is not the block's last part loads one step past its end, never read).  The main loop passes compile-time
    // flags (one straight-line region, buffers known at compile time); the
    // last steps pass runtime flags.
    auto step_body = [&](auto more, auto mask_next, auto odd, int i, Scores &xc, Scores &xn, int ln) {
        uint16_t *k_read = odd ? sk0 : sk1;  // K(i+1)
        uint16_t *k_load = odd ? sk1 : sk0;  // K(i+2)
        uint16_t *v_read = odd ? sv1 : sv0;  // V(i)
        uint16_t *v_load = odd ? sv0 : sv1;  // V(i+1)
        if (rescale) {  // uniform: some column's max moved in step i
#pragma unroll
            for (int ct = 0; ct < 2; ++ct)
#pragma unroll
                for (int r = 0; r < 4; ++r) {
                    const float a = __shfl(alpha[ct], kg * 4 + r);
#pragma unroll
                    for (int c = 0; c < 9; ++c) o[ct][c][r] *= a;
                }
        }
        if (more && !mask_next) dma_k(s_begin + i + 2, k_load, ln);
        if (more) dma_v(s_begin + i + 1, v_load, ln);
#pragma unroll
        for (int ct = 0; ct < 2; ++ct) ms[ct] = m_run[ct] * scale;
        half8_t pa[2][2];
        if constexpr (F32IO) {
            // The f32 entry point: weights as hi + lo fp16 pairs, one tile
            // pair at a time (pv_mfma_hi_lo), before the scores of step i+1
            // (with both steps' scores live the registers run out).
            __builtin_amdgcn_s_setprio(1);
            pv_mfma_hi_lo(v_read, 0, xc, ms);
            pv_mfma_hi_lo(v_read, 1, xc, ms);
            __builtin_amdgcn_s_setprio(0);
            if (more) scores(k_read, xn);
        } else {
            // scores of step i+1 | P of step i, pair 0
            if (more) scores(k_read, xn);
            probs(xc, ms, 0, pa);
            probs(xc, ms, 1, pa);
            // P.V of both pairs | mask and max of step i+1.  The P.V MFMAs run at
            // raised wave priority, so the SIMD's other wave fills the gaps with
            // its VALU work.
            __builtin_amdgcn_s_setprio(1);
            pv_mfma(v_read, 0, pa);
            pv_mfma(v_read, 1, pa);
            __builtin_amdgcn_s_setprio(0);
        }
        if (more) {
            if (mask_next) apply_mask(s_begin + i + 1, xn);
            // Lazy rescale: m_run is the exponent reference of the column,
            // and it moves (with O and the row sums rescaled) only when the
            // column's maximum exceeds it by more than kLazyRescaleLog2;
            // until then every weight 2^(s - m_run) stays below 2^8, exact
            // in fp16 and far from f32 overflow in the sums.  O / l is the
            // same quotient whatever the reference, and the split merge
            // takes m_run as the reference its part used.
            float m_new[2];
            column_max(xn, m_run, m_new);
            bool far = false;
#pragma unroll
            for (int ct = 0; ct < 2; ++ct) far |= (m_new[ct] - m_run[ct]) * scale > kLazyRescaleLog2;
            rescale = __any(far);
            if (rescale) {  // uniform
#pragma unroll
                for (int ct = 0; ct < 2; ++ct) {
                    alpha[ct] = __builtin_amdgcn_exp2f((m_run[ct] - m_new[ct]) * scale);
                    m_run[ct] = m_new[ct];
                }
            }
        }
        __syncthreads();  // waits for this wave's loads into LDS, then for every wave
    };
    const std::integral_constant<bool, true> yes;
    const std::integral_constant<bool, false> no;
    int i = 0;
    for (; i + 3 < steps; i += 2) {
        step_body(yes, no, no, i, xa, xb, lane);
        step_body(yes, no, yes, i + 1, xb, xa, lane);
    }
    // The last steps and the epilogue take their lane coordinates from a lane
    // id computed here (mbcnt), a value the compiler cannot merge with the one
    // computed before the main loop.  Otherwise it computes their per-lane
    // addresses before the main loop, where they share the loop's registers
    // and are spilled around it.
    const int tail_lane = static_cast<int>(__builtin_amdgcn_mbcnt_hi(~0u, __builtin_amdgcn_mbcnt_lo(~0u, 0u)));
    for (; i < steps; ++i) {  // the last one to three steps
        step_body(i + 1 < steps, i + 2 == steps && last_part, (i & 1) != 0, i, xa, xb, tail_lane);
#pragma unroll
        for (int ct = 0; ct < 2; ++ct)
#pragma unroll
            for (int j = 0; j < 2; ++j)
#pragma unroll
                for (int e = 0; e < 8; ++e) xa[ct][j][e] = xb[ct][j][e];
    }

    const int lane_e = tail_lane, row_e = tail_lane & 15, kg_e = tail_lane >> 4;
    if (nparts > 1) {
        // Split block: store this part's (m, O, l), count it, and let the part
        // that arrives last merge the other one.  Partials move as 8-byte
        // relaxed agent-scope atomics (coherent across the XCDs' L2s); every
        // store of the workgroup completes before thread 0 counts the arrival.
        // The second part first reads the count: when the first part has
        // arrived (its workgroup runs it before its light block, so it
        // usually has), its stores are complete, and the second part merges
        // it without storing its own (the first part's count is then the
        // last it touches).  Slab of a part: O/l tiles [wave][ct][tile][half]
        // [lane] as float pairs, then m [wave][ct][lane].
        const uint32_t item = pair * kKvHeads + g;  // the heavy block of the pair
        auto slab = [&](uint32_t q) {
            return reinterpret_cast<uint64_t *>(p.partials + (static_cast<size_t>(item) * 2 + q) * kPrefillPartialFloats);
        };
        auto pair_idx = [&](int ct, int c, int hf) { return (((wave * 2 + ct) * 9 + c) * 2 + hf) * 64 + lane_e; };
        auto m_ptr = [&](uint32_t q, int ct) {
            return p.partials + (static_cast<size_t>(item) * 2 + q) * kPrefillPartialFloats + 4 * 2 * 9 * 4 * 64 +
                   (wave * 2 + ct) * 64 + lane_e;
        };
        bool merge_now = false;
        if (part == 1) {
            if (wave == 0 && lane_e == 0)
                sm_last = __hip_atomic_load(p.counters + item, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) == 1u;
            __syncthreads();
            merge_now = sm_last;  // uniform
            __syncthreads();      // every wave has read it before it is written again below
        }
        if (!merge_now) {
            uint64_t *own = slab(part);
#pragma unroll
            for (int ct = 0; ct < 2; ++ct) {
#pragma unroll
                for (int c = 0; c < 9; ++c)
#pragma unroll
                    for (int hf = 0; hf < 2; ++hf) {
                        const uint64_t bits = static_cast<uint64_t>(__float_as_uint(o[ct][c][2 * hf])) |
                                              (static_cast<uint64_t>(__float_as_uint(o[ct][c][2 * hf + 1])) << 32);
                        __hip_atomic_store(own + pair_idx(ct, c, hf), bits, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
                    }
                __hip_atomic_store(m_ptr(part, ct), m_run[ct], __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            }
            asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
            __syncthreads();
            if (wave == 0 && lane_e == 0) {
                const uint32_t prev =
                    __hip_atomic_fetch_add(p.counters + item, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
                sm_last = prev == nparts - 1;
            }
            __syncthreads();
            if (!sm_last) return;  // uniform: the other part merges and writes the block
        }
        const uint32_t q = part ^ 1u;  // two parts
        const uint64_t *other = slab(q);
#pragma unroll
        for (int ct = 0; ct < 2; ++ct) {
            const float mo = __hip_atomic_load(m_ptr(q, ct), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            float4_t ov[9];
#pragma unroll
            for (int c = 0; c < 9; ++c)
#pragma unroll
                for (int hf = 0; hf < 2; ++hf) {
                    const uint64_t bits = __hip_atomic_load(other + pair_idx(ct, c, hf), __ATOMIC_RELAXED,
                                                            __HIP_MEMORY_SCOPE_AGENT);
                    ov[c][2 * hf] = __uint_as_float(static_cast<uint32_t>(bits));
                    ov[c][2 * hf + 1] = __uint_as_float(static_cast<uint32_t>(bits >> 32));
                }
            const float m_new = fmaxf(m_run[ct], mo);
            const float a_self = __builtin_amdgcn_exp2f((m_run[ct] - m_new) * scale);
            const float a_other = __builtin_amdgcn_exp2f((mo - m_new) * scale);
            m_run[ct] = m_new;
#pragma unroll
            for (int r = 0; r < 4; ++r) {
                const float as = __shfl(a_self, kg_e * 4 + r);
                const float ao = __shfl(a_other, kg_e * 4 + r);
#pragma unroll
                for (int c = 0; c < 9; ++c) o[ct][c][r] = o[ct][c][r] * as + ov[c][r] * ao;
            }
        }
        if (wave == 0 && lane_e == 0)
            __hip_atomic_store(p.counters + item, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    }

    // Normalise: output row kg*4 + r of tile ct is query token t0 + kg*4 + r;
    // its row sum is element r of the sums tile in the same lane.  Each wave
    // stages its two heads' 16 x 128 outputs in its own K/V buffer (free after
    // the last step: no load into LDS is in flight) as [head][token][dim],
    // then stores whole 16-byte chunks (8 fp16 or 4 f32 outputs) instead of
    // one 2- or 4-byte element per lane and store.
    using OutT = std::conditional_t<F32IO, float, uint16_t>;
    constexpr int kChunk = 16 / static_cast<int>(sizeof(OutT));  // outputs per 16-byte chunk
    static_assert(2 * kQueryBlock * kHeadDim * sizeof(OutT) <= sizeof(sk0),
                  "a wave's two staged 16 x 128 output tiles fit its own K/V buffer");
    OutT *stage =reinterpret_cast<OutT *>(wave == 0 ? sk0 : wave == 1 ? sk1 : wave == 2 ? sv0 : sv1);
#pragma unroll
    for (int ct = 0; ct < 2; ++ct) {
#pragma unroll
        for (int r = 0; r < 4; ++r) {
            const float inv = 1.0f / o[ct][8][r];
            OutT *srow = stage + (ct * kQueryBlock + kg_e * 4 + r) * kHeadDim + row_e;
#pragma unroll
            for (int c = 0; c < 8; ++c) {
                if constexpr (F32IO) srow[c * 16] = o[ct][c][r] * inv;
                else srow[c * 16] = __builtin_bit_cast(uint16_t, to_h(o[ct][c][r] * inv));
            }
        }
    }
    __builtin_amdgcn_wave_barrier();  // the wave reads what its other lanes wrote (LDS is in order per wave)
    constexpr int kChunks = 2 * kQueryBlock * kHeadDim / kChunk;  // of the wave: 512 (fp16) or 1024 (f32)
#pragma unroll
    for (int j = 0; j < kChunks / 64; ++j) {
        const int q = j * 64 + lane_e;                   // chunk: [head][token][chunk of the row]
        const int ct = q / (kQueryBlock * kHeadDim / kChunk);
        const int tt = (q / (kHeadDim / kChunk)) % kQueryBlock, d0 = (q % (kHeadDim / kChunk)) * kChunk;
        const int t = t0 + tt, h = static_cast<int>(g) * kGroup + wave * 2 + ct;
        if (t < n) {
            const float4_t v = *reinterpret_cast<const float4_t *>(stage + (ct * kQueryBlock + tt) * kHeadDim + d0);
            OutT *dst = (F32IO ? reinterpret_cast<OutT *>(p.out32) : reinterpret_cast<OutT *>(p.out)) +
                        (static_cast<size_t>(t) * kQueryHeads + h) * kHeadDim + d0;
            *reinterpret_cast<float4_t *>(dst) = v;
        }
    }
    // Every wave has read its staged outputs before the next segment loads
    // its first stages into these buffers.
    __syncthreads();
  };
  // the first part of a heavy block, then a light block (two inlined
  // copies: each is register-allocated like a single segment)
  if (nseg > 0) run_segment(seg0);
  if (nseg > 1) run_segment(seg1);
}

}  // namespace

int launch_prefill(const pvlc_hip_paged_prefill_args *a, void *stream, const PrefillOperands32 *f32) {
    PrefillParams p{};
    p.tokens = a->tokens;
    p.num_blocks = a->num_blocks;
    p.block_table = a->block_table;
    p.key_cache = a->key_cache;
    p.value_cache = a->value_cache;
    p.query = a->query;
    p.key = a->key;
    p.value = a->value;
    p.out = a->out;
    p.rope_cos = a->rope_cos;
    p.rope_sin = a->rope_sin;
    p.rope_rows = a->rope_rows;
    p.positions = a->positions;
    p.qrot = a->query_scratch;
    p.error_word = a->error_word;
    p.scale_log2 = kLog2e / sqrtf(static_cast<float>(kHeadDim));
    if (f32) {
        p.query32 = f32->query;
        p.key32 = f32->key;
        p.value32 = f32->value;
        p.out32 = f32->out;
    }
    hipStream_t st = static_cast<hipStream_t>(stream);
    const dim3 append_grid((a->tokens + kBlockTokens - 1) / kBlockTokens);
    if (f32) hipLaunchKernelGGL(prefill_rope_append_kernel<true>, append_grid, dim3(kAppendThreads), 0, st, p);
    else hipLaunchKernelGGL(prefill_rope_append_kernel<false>, append_grid, dim3(kAppendThreads), 0, st, p);
    hipError_t e = hipGetLastError();
    if (e != hipSuccess) return static_cast<int>(e);
    const unsigned qblocks = (a->tokens + kQueryBlock - 1) / kQueryBlock;
    const PrefillWorkspace ws = prefill_workspace_layout(a->tokens);
    p.split = a->workspace != nullptr && ws.total > 0;
    if (p.split) {
        p.counters = static_cast<uint32_t *>(a->workspace);
        p.partials = reinterpret_cast<float *>(static_cast<unsigned char *>(a->workspace) + ws.partial_offset);
    }
    const unsigned grid = p.split ? prefill_pair_workgroups(qblocks) : qblocks * kKvHeads;
    if (f32) hipLaunchKernelGGL(prefill_attention_kernel<true>, dim3(grid), dim3(kWaves * 64), 0, st, p);
    else hipLaunchKernelGGL(prefill_attention_kernel<false>, dim3(grid), dim3(kWaves * 64), 0, st, p);
    return static_cast<int>(hipGetLastError());
}

}  // namespace pvlc
