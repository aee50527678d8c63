// Causal prefill for gfx950: rotary + range append into the paged cache, then
// MFMA flash attention over the cache.
//
// Kernel 1 (one workgroup per token): rotates the 16 query heads into a
// scratch row, rotates the 2 key heads and writes them with the values into
// the blocked cache (the same rounding as the decode append, so prefill and
// decode leave bit-identical rows).  Replaces decoder_prefill_mrope_f32 and
// decoder_kv_append_range_f32 (crates/pvlc-wgsl/src/lib.rs:1334-1416).
//
// Kernel 2: one workgroup per (16-token query block, kv head) serves the 8
// query heads of the group; each of its 4 waves owns 2 heads, i.e. two
// 16-column MFMA tiles of query rows.  Keys and values stream through LDS in
// steps of 64 keys (4 cache blocks), straight in MFMA operand order, with the
// next step prefetched into registers while the current one is computed:
//   S^T[key][row] = K . Q^T          v_mfma_f32_16x16x32_f16
//   O[row][dim]  += P[row][key] V     v_mfma_f32_16x16x16_f16
// with an online softmax in log2 units and the causal mask on the diagonal
// steps.  Query blocks are scheduled latest (heaviest) first.  Replaces
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

__global__ __launch_bounds__(256) void prefill_rope_append_kernel(PrefillParams p) {
    const uint32_t t = blockIdx.x;
    const int i = threadIdx.x;
    bool rope = p.rope_cos != nullptr;
    const int pos = p.positions ? load_const(p.positions, t) : static_cast<int>(t);
    if (rope && (pos < 0 || static_cast<uint32_t>(pos) >= p.rope_rows)) {
        if (i == 0 && p.error_word) atomicOr(p.error_word, 4u);
        rope = false;
    }
    const float *cos_row = rope ? p.rope_cos + static_cast<size_t>(pos) * 64 : nullptr;
    const float *sin_row = rope ? p.rope_sin + static_cast<size_t>(pos) * 64 : nullptr;
    // Query: thread = (head, 8-dim chunk).
    {
        const int h = i >> 4, d0 = (i & 15) * 8;
        const uint16_t *qrow = p.query + (static_cast<size_t>(t) * kQueryHeads + h) * kHeadDim;
        const half8_t q = rope ? rotate_chunk(qrow, d0, cos_row, sin_row) : *reinterpret_cast<const half8_t *>(qrow + d0);
        *reinterpret_cast<half8_t *>(p.qrot + (static_cast<size_t>(t) * kQueryHeads + h) * kHeadDim + d0) = q;
    }
    if (i < 64) {
        bool ok;
        const uint32_t blk = cache_block(p, t / kBlockTokens, &ok);
        if (!ok) {
            if (i == 0 && p.error_word) atomicOr(p.error_word, 2u);
            return;
        }
        const int hh = (i >> 4) & 1, c = i & 15, d0 = c * 8;
        const size_t slab = (static_cast<size_t>(blk) * kKvHeads + hh) * kBlockHeadElems;
        const uint32_t tt = t % kBlockTokens;
        if (i < 32) {
            const uint16_t *krow = p.key + (static_cast<size_t>(t) * kKvHeads + hh) * kHeadDim;
            const half8_t k = rope ? rotate_chunk(krow, d0, cos_row, sin_row)
                                   : *reinterpret_cast<const half8_t *>(krow + d0);
            *reinterpret_cast<half8_t *>(p.key_cache + slab + c * 128 + key_slot(tt) * 8) = k;
        } else {
            const u16x8_t v = *reinterpret_cast<const u16x8_t *>(p.value + (static_cast<size_t>(t) * kKvHeads + hh) *
                                                                                    kHeadDim + d0);
#pragma unroll
            for (int j = 0; j < 8; ++j) p.value_cache[slab + (d0 + j) * kBlockTokens + tt] = v[j];
        }
    }
}

__global__ __launch_bounds__(kWaves * 64, 2) void prefill_attention_kernel(PrefillParams p) {
    const int n = static_cast<int>(p.tokens);
    const int qblocks = (n + kQueryBlock - 1) / kQueryBlock;
    const int qb = qblocks - 1 - static_cast<int>(blockIdx.x);  // heaviest first
    const uint32_t g = blockIdx.y;
    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane(static_cast<int>(threadIdx.x >> 6));
    const int row = lane & 15, kg = lane >> 4;
    const int t0 = qb * kQueryBlock;
    const int my_token = t0 + row;  // query token of this lane's column

    // Query fragments (B operand): column = token t0 + row of head h.
    half8_t qf[2][4];
#pragma unroll
    for (int ct = 0; ct < 2; ++ct) {
        const int h = static_cast<int>(g) * kGroup + wave * 2 + ct;
        const uint16_t *qrow = p.qrot + (static_cast<size_t>(min(my_token, n - 1)) * kQueryHeads + h) * kHeadDim;
#pragma unroll
        for (int kb = 0; kb < 4; ++kb) {
            const half8_t q = *reinterpret_cast<const half8_t *>(qrow + kb * 32 + kg * 8);
            qf[ct][kb] = my_token < n ? q : half8_t{};
        }
    }

    const int nkeys = min(t0 + kQueryBlock, n);
    const int steps = (nkeys + kKeyStep - 1) / kKeyStep;
    const int last_tile = (nkeys - 1) >> 4;

    __shared__ uint16_t sk[kStepTiles][kBlockHeadElems];
    __shared__ uint16_t sv[kStepTiles][kBlockHeadElems];
    u16x8_t pk[kStepTiles], pv[kStepTiles];
    auto gload = [&](int step) {
#pragma unroll
        for (int i = 0; i < kStepTiles; ++i) {
            bool ok;
            const uint32_t blk = cache_block(p, static_cast<uint32_t>(min(step * kStepTiles + i, last_tile)), &ok);
            const size_t slab = (static_cast<size_t>(blk) * kKvHeads + g) * kBlockHeadElems;
            pk[i] = *reinterpret_cast<const u16x8_t *>(p.key_cache + slab + threadIdx.x * 8);
            pv[i] = *reinterpret_cast<const u16x8_t *>(p.value_cache + slab + threadIdx.x * 8);
        }
    };

    float m_run[2] = {-INFINITY, -INFINITY};
    float l_run[2] = {0.f, 0.f};
    float4_t o[2][8];
#pragma unroll
    for (int ct = 0; ct < 2; ++ct)
#pragma unroll
        for (int c = 0; c < 8; ++c) o[ct][c] = float4_t{0.f, 0.f, 0.f, 0.f};

    gload(0);
    for (int step = 0; step < steps; ++step) {
        __syncthreads();  // every wave is done with the previous step's tiles
#pragma unroll
        for (int i = 0; i < kStepTiles; ++i) {
            *reinterpret_cast<u16x8_t *>(&sk[i][threadIdx.x * 8]) = pk[i];
            *reinterpret_cast<u16x8_t *>(&sv[i][threadIdx.x * 8]) = pv[i];
        }
        __syncthreads();
        if (step + 1 < steps) gload(step + 1);

        const int kbase = step * kKeyStep;
        float x[2][kStepTiles][4];
#pragma unroll
        for (int i = 0; i < kStepTiles; ++i) {
            half8_t kf[4];
#pragma unroll
            for (int kb = 0; kb < 4; ++kb)
                kf[kb] = *reinterpret_cast<const half8_t *>(&sk[i][(kb * 4 + kg) * 128 + key_slot(row) * 8]);
#pragma unroll
            for (int ct = 0; ct < 2; ++ct) {
                float4_t acc = float4_t{0.f, 0.f, 0.f, 0.f};
#pragma unroll
                for (int kb = 0; kb < 4; ++kb) acc = __builtin_amdgcn_mfma_f32_16x16x32_f16(kf[kb], qf[ct][kb], acc, 0, 0, 0);
#pragma unroll
                for (int r = 0; r < 4; ++r) {
                    const int key = kbase + i * 16 + kg * 4 + r;
                    x[ct][i][r] = (key <= my_token && key < n) ? acc[r] * p.scale_log2 : -INFINITY;
                }
            }
        }
        half4_t pa[2][kStepTiles];
#pragma unroll
        for (int ct = 0; ct < 2; ++ct) {
            float cmax = -INFINITY;
#pragma unroll
            for (int i = 0; i < kStepTiles; ++i)
#pragma unroll
                for (int r = 0; r < 4; ++r) cmax = fmaxf(cmax, x[ct][i][r]);
            cmax = fmaxf(cmax, __shfl_xor(cmax, 16));
            cmax = fmaxf(cmax, __shfl_xor(cmax, 32));
            // Step 0 always holds key 0 <= every query token, so m_new is finite.
            const float m_new = fmaxf(m_run[ct], cmax);
            const float alpha = __builtin_amdgcn_exp2f(m_run[ct] - m_new);
            l_run[ct] *= alpha;
            m_run[ct] = m_new;
            if (step > 0) {
#pragma unroll
                for (int r = 0; r < 4; ++r) {
                    const float a = __shfl(alpha, kg * 4 + r);
#pragma unroll
                    for (int c = 0; c < 8; ++c) o[ct][c][r] *= a;
                }
            }
#pragma unroll
            for (int i = 0; i < kStepTiles; ++i)
#pragma unroll
                for (int r = 0; r < 4; ++r) {
                    const _Float16 ph = to_h(__builtin_amdgcn_exp2f(x[ct][i][r] - m_new));
                    pa[ct][i][r] = ph;
                    l_run[ct] += static_cast<float>(ph);
                }
        }
#pragma unroll
        for (int i = 0; i < kStepTiles; ++i)
#pragma unroll
            for (int c = 0; c < 8; ++c) {
                const half4_t vf = *reinterpret_cast<const half4_t *>(&sv[i][(c * 16 + row) * 16 + kg * 4]);
#pragma unroll
                for (int ct = 0; ct < 2; ++ct)
                    o[ct][c] = __builtin_amdgcn_mfma_f32_16x16x16f16(pa[ct][i], vf, o[ct][c], 0, 0, 0);
            }
    }

    // Normalise: output row kg*4 + r of tile ct is query token t0 + kg*4 + r;
    // its sum lives in the lanes whose column index is that row.
#pragma unroll
    for (int ct = 0; ct < 2; ++ct) {
        float l = l_run[ct];
        l += __shfl_xor(l, 16);
        l += __shfl_xor(l, 32);
        const int h = static_cast<int>(g) * kGroup + wave * 2 + ct;
#pragma unroll
        for (int r = 0; r < 4; ++r) {
            const float inv = 1.0f / __shfl(l, kg * 4 + r);
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
    hipLaunchKernelGGL(prefill_rope_append_kernel, dim3(a->tokens), dim3(256), 0, st, p);
    hipError_t e = hipGetLastError();
    if (e != hipSuccess) return static_cast<int>(e);
    const unsigned qblocks = (a->tokens + kQueryBlock - 1) / kQueryBlock;
    hipLaunchKernelGGL(prefill_attention_kernel, dim3(qblocks, kKvHeads), dim3(kWaves * 64), 0, st, p);
    return static_cast<int>(hipGetLastError());
}

}  // namespace pvlc
