// Causal prefill for gfx950: rotary + range append into the paged cache, then
// MFMA flash attention over the cache.
//
// Kernel 1 (4 tokens per workgroup): rotates the 2 key heads and writes them
// with the values into the blocked cache (the same rounding as the decode
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

#include "pvlc_device.hpp"
#include "pvlc_internal.hpp"

namespace pvlc {
namespace {

constexpr float kLog2e = 1.4426950408889634f;
constexpr int kQueryBlock = 16;  // query tokens per workgroup
constexpr int kKeyStep = 64;     // keys per softmax step (4 cache blocks)
constexpr int kStepTiles = kKeyStep / 16;
constexpr int kWaves = 4;        // each wave: 2 of the 8 heads of the group

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

// Kernel 1: 4 tokens per workgroup, 64 threads per token: threads 0-31
// rotate the token's 2 key heads (8 dims each) and write them into the
// cache, threads 32-63 scatter its values.  With a query scratch the
// workgroup also writes the rotated queries of its tokens (the attention
// kernel rotates its own query fragments, so the scratch is only an output
// for callers that want it).
constexpr int kAppendTokens = 4;

__global__ __launch_bounds__(256) void prefill_rope_append_kernel(PrefillParams p) {
    const int i = threadIdx.x;
    const uint32_t t = blockIdx.x * kAppendTokens + (i >> 6);
    const int sub = i & 63;
    if (t < p.tokens) {
        bool rope = p.rope_cos != nullptr;
        const int pos = p.positions ? p.positions[t] : static_cast<int>(t);
        if (rope && (pos < 0 || static_cast<uint32_t>(pos) >= p.rope_rows)) {
            if (sub == 0 && p.error_word) atomicOr(p.error_word, 4u);
            rope = false;
        }
        const float *cos_row = rope ? p.rope_cos + static_cast<size_t>(pos) * 64 : nullptr;
        const float *sin_row = rope ? p.rope_sin + static_cast<size_t>(pos) * 64 : nullptr;
        bool ok;
        const uint32_t blk = cache_block(p, t / kBlockTokens, &ok);
        if (!ok) {
            if (sub == 0 && p.error_word) atomicOr(p.error_word, 2u);
        } else {
            const int hh = (sub >> 4) & 1, c = sub & 15, d0 = c * 8;
            const size_t slab = (static_cast<size_t>(blk) * kKvHeads + hh) * kBlockHeadElems;
            const uint32_t tt = t % kBlockTokens;
            if (sub < 32) {
                const uint16_t *krow = p.key + (static_cast<size_t>(t) * kKvHeads + hh) * kHeadDim;
                const half8_t k = rope ? rotate_chunk(krow, d0, cos_row, sin_row)
                                       : *reinterpret_cast<const half8_t *>(krow + d0);
                *reinterpret_cast<half8_t *>(p.key_cache + slab + c * 128 + key_slot(static_cast<int>(tt)) * 8) = k;
            } else {
                const u16x8_t v = *reinterpret_cast<const u16x8_t *>(
                    p.value + (static_cast<size_t>(t) * kKvHeads + hh) * kHeadDim + d0);
#pragma unroll
                for (int j = 0; j < 8; ++j) p.value_cache[slab + (d0 + j) * kBlockTokens + tt] = v[j];
            }
        }
    }
    if (p.qrot) {
        // (token, head, 8-dim chunk) items of the workgroup's tokens.
        for (int k = i; k < kAppendTokens * kQueryHeads * 16; k += 256) {
            const uint32_t tq = blockIdx.x * kAppendTokens + k / (kQueryHeads * 16);
            if (tq >= p.tokens) break;
            const int h = (k >> 4) % kQueryHeads, d0 = (k & 15) * 8;
            const int pos = p.positions ? p.positions[tq] : static_cast<int>(tq);
            const bool rope = p.rope_cos != nullptr && pos >= 0 && static_cast<uint32_t>(pos) < p.rope_rows;
            const uint16_t *qrow = p.query + (static_cast<size_t>(tq) * kQueryHeads + h) * kHeadDim;
            const half8_t q = rope ? rotate_chunk(qrow, d0, p.rope_cos + static_cast<size_t>(pos) * 64,
                                                  p.rope_sin + static_cast<size_t>(pos) * 64)
                                   : *reinterpret_cast<const half8_t *>(qrow + d0);
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

__global__ __launch_bounds__(kWaves * 64, 2) void prefill_attention_kernel(PrefillParams p) {
    const int n = static_cast<int>(p.tokens);
    const int qblocks = (n + kQueryBlock - 1) / kQueryBlock;
    int qb;
    uint32_t g;
    prefill_item(static_cast<int>(blockIdx.x), qblocks, &qb, &g);
    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane(static_cast<int>(threadIdx.x >> 6));
    const int row = lane & 15, kg = lane >> 4;
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
        const uint16_t *qrow = p.query + (static_cast<size_t>(tq) * kQueryHeads + h) * kHeadDim;
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

    const int nkeys = min(t0 + kQueryBlock, n);
    const int steps = (nkeys + kKeyStep - 1) / kKeyStep;
    const int last_tile = (nkeys - 1) >> 4;

    // Double-buffered LDS; each thread moves 4 key and 4 value chunks of 16
    // bytes per step through registers (loaded one step ahead).
    __shared__ uint16_t sk[2][kStepElems];
    __shared__ uint16_t sv[2][kStepElems];
    u16x8_t pk[4], pv[4];
    int koff[4], voff[4];
    {
        const int c = static_cast<int>(threadIdx.x);  // chunk of a tile: keys chunk*16 + slot, values dim*2 + half
        const int kchunk = c >> 4, kslot = c & 15;
        const int vdim = c >> 1, vhalf = c & 1;
#pragma unroll
        for (int i = 0; i < 4; ++i) {  // tile i of the step
            koff[i] = lds_key_offset(i >> 1, kchunk, kslot >> 3, i & 1, kslot & 7);
            voff[i] = lds_value_offset(i >> 1, i & 1, vhalf, vdim);
        }
    }
    // Thread t moves 16-byte chunk t of each of the step's 4 tiles (the
    // tile index is uniform, so the block-table read is a scalar load).
    auto gload = [&](int step) {
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            bool ok;
            const uint32_t blk = cache_block(p, static_cast<uint32_t>(min(step * kStepTiles + i, last_tile)), &ok);
            const size_t slab = (static_cast<size_t>(blk) * kKvHeads + g) * kBlockHeadElems;
            pk[i] = *reinterpret_cast<const u16x8_t *>(p.key_cache + slab + threadIdx.x * 8);
            pv[i] = *reinterpret_cast<const u16x8_t *>(p.value_cache + slab + threadIdx.x * 8);
        }
    };
    auto lstore = [&](int buf) {
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            *reinterpret_cast<u16x8_t *>(&sk[buf][koff[i]]) = pk[i];
            *reinterpret_cast<u16x8_t *>(&sv[buf][voff[i]]) = pv[i];
        }
    };

    float m_run[2] = {-INFINITY, -INFINITY};  // raw (unscaled) running max of this lane's column
    float4_t o[2][9];                          // 8 column tiles of the output, then the row sums
#pragma unroll
    for (int ct = 0; ct < 2; ++ct)
#pragma unroll
        for (int c = 0; c < 9; ++c) o[ct][c] = float4_t{0.f, 0.f, 0.f, 0.f};
    half8_t ones;
#pragma unroll
    for (int e = 0; e < 8; ++e) ones[e] = static_cast<_Float16>(1.0f);
    const float scale = p.scale_log2;

    gload(0);
    lstore(0);
    if (steps > 1) gload(1);
    __syncthreads();
    for (int step = 0; step < steps; ++step) {
        const int buf = step & 1;
        const uint16_t *kl = sk[buf];
        const uint16_t *vl = sv[buf];
        const int kbase = step * kKeyStep;
        // Scores: MFMA h of pair j leaves lane (column = query token, kg) the
        // keys (kg & 1)*8 + h*4 + r of the pair's tile kg >> 1.
        float x[2][2][8];
#pragma unroll
        for (int j = 0; j < 2; ++j)
#pragma unroll
            for (int h = 0; h < 2; ++h) {
                float4_t acc[2] = {float4_t{0.f, 0.f, 0.f, 0.f}, float4_t{0.f, 0.f, 0.f, 0.f}};
#pragma unroll
                for (int kb = 0; kb < 4; ++kb) {
                    const half8_t kf = *reinterpret_cast<const half8_t *>(
                        kl + lds_key_offset(j, kb * 4 + kg, h, row >> 3, row & 7));
#pragma unroll
                    for (int ct = 0; ct < 2; ++ct)
                        acc[ct] = __builtin_amdgcn_mfma_f32_16x16x32_f16(kf, qf[ct][kb], acc[ct], 0, 0, 0);
                }
#pragma unroll
                for (int ct = 0; ct < 2; ++ct)
#pragma unroll
                    for (int r = 0; r < 4; ++r) x[ct][j][h * 4 + r] = acc[ct][r];
            }
        // The causal mask and the end of the sequence only touch steps that
        // reach past the first query token of the block.
        if (kbase + kKeyStep - 1 > t0 || kbase + kKeyStep > n) {  // uniform
#pragma unroll
            for (int j = 0; j < 2; ++j)
#pragma unroll
                for (int e = 0; e < 8; ++e) {
                    const int key = kbase + (2 * j + (kg >> 1)) * 16 + (kg & 1) * 8 + e;
                    const bool keep = key <= my_token && key < n;
#pragma unroll
                    for (int ct = 0; ct < 2; ++ct) x[ct][j][e] = keep ? x[ct][j][e] : -INFINITY;
                }
        }
        half8_t pa[2][2];
#pragma unroll
        for (int ct = 0; ct < 2; ++ct) {
            float cmax = -INFINITY;
#pragma unroll
            for (int j = 0; j < 2; ++j)
#pragma unroll
                for (int e = 0; e < 8; ++e) cmax = fmaxf(cmax, x[ct][j][e]);
            cmax = fmaxf(cmax, __shfl_xor(cmax, 16));
            cmax = fmaxf(cmax, __shfl_xor(cmax, 32));
            // Step 0 always holds key 0 <= every query token, so m_new is finite.
            const float m_new = fmaxf(m_run[ct], cmax);
            const float ms = m_new * scale;
            if (__any(m_new != m_run[ct]) && step > 0) {
                const float alpha = __builtin_amdgcn_exp2f(m_run[ct] * scale - ms);
#pragma unroll
                for (int r = 0; r < 4; ++r) {
                    const float a = __shfl(alpha, kg * 4 + r);
#pragma unroll
                    for (int c = 0; c < 9; ++c) o[ct][c][r] *= a;
                }
            }
            m_run[ct] = m_new;
#pragma unroll
            for (int j = 0; j < 2; ++j)
#pragma unroll
                for (int e = 0; e < 8; ++e)
                    pa[ct][j][e] = to_h(__builtin_amdgcn_exp2f(__builtin_fmaf(x[ct][j][e], scale, -ms)));
        }
        // P.V, and P.1 for the row sums (exactly the rounded weights P.V uses).
#pragma unroll
        for (int j = 0; j < 2; ++j) {
#pragma unroll
            for (int c = 0; c < 8; ++c) {
                const half8_t vf = *reinterpret_cast<const half8_t *>(
                    vl + lds_value_offset(j, kg >> 1, kg & 1, c * 16 + row));
#pragma unroll
                for (int ct = 0; ct < 2; ++ct)
                    o[ct][c] = __builtin_amdgcn_mfma_f32_16x16x32_f16(pa[ct][j], vf, o[ct][c], 0, 0, 0);
            }
#pragma unroll
            for (int ct = 0; ct < 2; ++ct)
                o[ct][8] = __builtin_amdgcn_mfma_f32_16x16x32_f16(pa[ct][j], ones, o[ct][8], 0, 0, 0);
        }
        if (step + 1 < steps) {
            lstore(buf ^ 1);  // its last readers finished before the previous barrier
            if (step + 2 < steps) gload(step + 2);
        }
        __syncthreads();
    }

    // Normalise: output row kg*4 + r of tile ct is query token t0 + kg*4 + r;
    // its row sum is element r of the sums tile in the same lane.
#pragma unroll
    for (int ct = 0; ct < 2; ++ct) {
        const int h = static_cast<int>(g) * kGroup + wave * 2 + ct;
#pragma unroll
        for (int r = 0; r < 4; ++r) {
            const float inv = 1.0f / o[ct][8][r];
            const int t = t0 + kg * 4 + r;
            if (t < n) {
                uint16_t *orow = p.out + (static_cast<size_t>(t) * kQueryHeads + h) * kHeadDim;
#pragma unroll
                for (int c = 0; c < 8; ++c) orow[c * 16 + row] = __builtin_bit_cast(uint16_t, to_h(o[ct][c][r] * inv));
            }
        }
    }
}

}  // namespace

int launch_prefill(const pvlc_hip_paged_prefill_args *a, void *stream) {
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
    hipStream_t st = static_cast<hipStream_t>(stream);
    hipLaunchKernelGGL(prefill_rope_append_kernel, dim3((a->tokens + kAppendTokens - 1) / kAppendTokens), dim3(256), 0,
                       st, p);
    hipError_t e = hipGetLastError();
    if (e != hipSuccess) return static_cast<int>(e);
    const unsigned qblocks = (a->tokens + kQueryBlock - 1) / kQueryBlock;
    hipLaunchKernelGGL(prefill_attention_kernel, dim3(qblocks * kKvHeads), dim3(kWaves * 64), 0, st, p);
    return static_cast<int>(hipGetLastError());
}

}  // namespace pvlc
