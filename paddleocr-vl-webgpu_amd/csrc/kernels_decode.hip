// Paged GQA decode for gfx950: fused rotary + KV append + split-K attention
// with an in-kernel LSE merge.
//
// Work unit: one workgroup per (partition, kv head, sequence).  A partition is
// a whole number of 16-token blocks.  Each wave of the workgroup streams
// chunks of 1-4 blocks of its kv head's keys and values straight from HBM
// into registers in MFMA operand order -- the blocked cache layout makes every wave-wide load one contiguous
// 1 KiB (keys) or 512 B (values) run -- and serves all 8 query heads of the
// group with matrix instructions:
//   scores  S[token][head] = K[token][:] . Q[head][:]   v_mfma_f32_16x16x32_f16
//   output  O[head][dim]  += P[head][token] V[token][dim] v_mfma_f32_16x16x32_f16
// The two score MFMAs of a tile pair leave each lane 8 consecutive tokens of
// one head: exactly the PV A-operand layout, so probabilities never leave the
// lane.  Softmax statistics use cross-lane shuffles; waves combine through
// LDS; the partitions of a (sequence, kv head) count their arrivals on a
// device-scope counter, and the last to arrive merges all partitions.
//
// Latency discipline (the whole step is a few microseconds): the arguments
// the first key loads need arrive preloaded in SGPRs, so every wave issues
// its first chunk's keys before anything else (unless it rotates the query,
// whose operands then go first); block ids come from one vector load per
// wave (or arithmetic); the appended row is rotated while the key and value
// loads are in flight; the merge loads partials in batches.
//
// Reference behaviour replaced: decoder_kv_append_f32, decoder_mrope_f32 (k
// and optionally q), decoder_gqa_split_partial_f32 and
// decoder_gqa_split_merge_f32 (crates/pvlc-wgsl/src/lib.rs:927-952,
// 1024-1234); arithmetic reference decode_gqa_f32 (crates/pvlc-cpu-ref/src/
// lib.rs:858-927).

#include <hip/hip_runtime.h>

#include <cstdint>
#include <mutex>

#include "pvlc_device.hpp"
#include "pvlc_internal.hpp"

namespace pvlc {
namespace {

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
    uint32_t part_stride;  // partial slots per (seq, kv head): max_parts rounded up to odd
    float *part_o;      // [seq][kv head][part_stride][8 heads][128]
    float *part_ml;     // [seq][kv head][part_stride][8 heads][2]: max (log2 units), sum
    uint32_t *counters; // [seq][kv head]
    uint32_t *error_word;
    uint32_t *partition_word;  // streaming, automatic partition: the one used (else null)
    uint32_t compute_units;    // streaming: compute units of the device
    float scale_log2;   // log2(e)/sqrt(128)
    // f32 operands (pvlc_hip_paged_decode_f32io): query, new key and value,
    // output; null for the fp16 entry points.
    const float *query32;
    const float *new_key32;
    const float *new_value32;
    float *out32;
};

// Block ids of every tile this wave loads in one partition, one per lane:
// lane c*TILES + i holds the block of tile i of the wave's chunk c.  Tiles
// past the partition take the partition's last tile (loaded and masked).
// An id outside the planes reads block 0 and sets *bad.  One vector load
// per wave and partition, so it can be issued ahead of the key/value loads
// (or a whole work item ahead).
template <int WAVES, int TILES>
__device__ inline uint32_t wave_tile_ids(const DecodeParams &p, uint32_t s, int part_start, int part_end, int wave,
                                         bool *bad) {
    const int lane = threadIdx.x & 63;
    const int tile = (part_start >> 4) + (lane / TILES) * (WAVES * TILES) + wave * TILES + lane % TILES;
    const int t = min(tile, (part_end - 1) >> 4);
    if (p.block_tables == nullptr) return s * p.max_blocks_per_seq + static_cast<uint32_t>(t);
    const int32_t b = p.block_tables[static_cast<size_t>(s) * p.max_blocks_per_seq + t];
    const bool out = b < 0 || static_cast<uint32_t>(b) >= p.num_blocks;
    *bad = *bad || out;
    return out ? 0u : static_cast<uint32_t>(b);
}

// Issue the loads of chunk c of this wave: PAIRS pairs of 16-token tiles.
// Keys: score MFMA h of pair j takes rows 0-7 from the pair's first tile and
// rows 8-15 from its second, key slots h*8 .. h*8+7 (see key_slot).  Values:
// k-groups 0-1 read the first tile, 2-3 the second, 8 consecutive tokens
// (16 bytes) each.  Every key load is issued before the value loads, so the
// scores can be computed while the values are still arriving.  The loads are
// non-temporal, since a step reads each cache row once: configs 3 and 5
// measured 11% and 8% faster with them, the 18-layer step 2% (a step whose
// cache already sits in the Infinity Cache is slower, 11.1 -> 11.8 us).
template <int PAIRS>
__device__ inline void load_chunk_keys(const DecodeParams &p, uint32_t g, uint32_t ids, int c, int row, int kg,
                                       half8_t (&kr)[PAIRS][2][4]) {
#pragma unroll
    for (int j = 0; j < PAIRS; ++j) {
        const int t0 = c * 2 * PAIRS + 2 * j;
        const size_t b0 = static_cast<uint32_t>(__builtin_amdgcn_readlane(static_cast<int>(ids), t0));
        const size_t b1 = static_cast<uint32_t>(__builtin_amdgcn_readlane(static_cast<int>(ids), t0 + 1));
        const uint16_t *kbase = p.key_cache + ((row < 8 ? b0 : b1) * kKvHeads + g) * kBlockHeadElems;
#pragma unroll
        for (int h = 0; h < 2; ++h)
#pragma unroll
            for (int kb = 0; kb < 4; ++kb)
                kr[j][h][kb] = __builtin_nontemporal_load(
                    reinterpret_cast<const half8_t *>(kbase + (kb * 4 + kg) * 128 + (h * 8 + (row & 7)) * 8));
    }
}
template <int PAIRS>
__device__ inline void load_chunk_values(const DecodeParams &p, uint32_t g, uint32_t ids, int c, int row, int kg,
                                         half8_t (&vr)[PAIRS][8]) {
#pragma unroll
    for (int j = 0; j < PAIRS; ++j) {
        const int t0 = c * 2 * PAIRS + 2 * j;
        const size_t b0 = static_cast<uint32_t>(__builtin_amdgcn_readlane(static_cast<int>(ids), t0));
        const size_t b1 = static_cast<uint32_t>(__builtin_amdgcn_readlane(static_cast<int>(ids), t0 + 1));
        const uint16_t *vbase = p.value_cache + ((kg < 2 ? b0 : b1) * kKvHeads + g) * kBlockHeadElems;
#pragma unroll
        for (int cc = 0; cc < 8; ++cc)
            vr[j][cc] = __builtin_nontemporal_load(
                reinterpret_cast<const half8_t *>(vbase + (cc * 16 + row) * 16 + (kg & 1) * 8));
    }
}
template <int PAIRS>
__device__ inline void load_chunk(const DecodeParams &p, uint32_t g, uint32_t ids, int c, int row, int kg,
                                  half8_t (&kr)[PAIRS][2][4], half8_t (&vr)[PAIRS][8]) {
    load_chunk_keys<PAIRS>(p, g, ids, c, row, kg, kr);
    __builtin_amdgcn_sched_barrier(0);  // keep every key load ahead of the value loads
    load_chunk_values<PAIRS>(p, g, ids, c, row, kg, vr);
}

typedef uint32_t u32x4_t __attribute__((ext_vector_type(4)));
constexpr int kSc1 = 16;  // cache-policy operand of the buffer intrinsics: sc1 (agent scope)

// An 8-byte agent-scope (sc1) load of two floats.
__device__ inline void load_pair_sc1(const float *q, float *lo, float *hi) {
    const uint64_t v =
        __hip_atomic_load(reinterpret_cast<const uint64_t *>(q), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    *lo = __uint_as_float(static_cast<uint32_t>(v));
    *hi = __uint_as_float(static_cast<uint32_t>(v >> 32));
}

// One work item: partition `part` of kv head g of sequence s, whose cache
// holds cache_len rows before the append (rotary position pos, or, with
// pos_from_params, p.positions[s] -- cache_len without positions -- read
// behind the first key loads); ids are the
// wave's tile block ids (wave_tile_ids) and ids_bad whether one of them was
// out of range.  With DEFER_MERGE the partial is only stored (plain stores)
// for paged_decode_merge_kernel, launched after this kernel; otherwise the
// last partition to arrive merges all partitions in-kernel.  Every return is
// uniform over the workgroup.  Errors are reported after the key/value loads
// are consumed, so no conditional memory operation sits among them.
template <int WAVES, int PAIRS, bool DEFER_MERGE, bool F32IO, bool KEYS_FIRST = true>
__device__ inline void decode_item(const DecodeParams &p, int P, uint32_t s, uint32_t g, uint32_t part, int cache_len,
                                   int pos, uint32_t ids, bool ids_bad, bool pos_from_params = false) {
    constexpr int kChunkTiles = 2 * PAIRS;         // 16-token tiles a wave holds in registers at once
    constexpr int kChunkTokens = kChunkTiles * 16;
    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane(static_cast<int>(threadIdx.x >> 6));
    const int row = lane & 15;  // MFMA row/column index of this lane
    const int kg = lane >> 4;   // MFMA k-group of this lane
    constexpr int kThreads = WAVES * 64;

    const int T = cache_len + 1;  // rows attended after the append (P: the partition length)
    const int part_start = static_cast<int>(part) * P;
    if (part_start >= T) return;
    const int part_end = min(part_start + P, T);
    const int num_parts = (T + P - 1) / P;

    // KEYS_FIRST: the first chunk's keys go out first -- their addresses need
    // only the arguments the single-shot kernel takes preloaded in SGPRs, so
    // the key stream starts without waiting for a scalar load -- then the
    // small operands (their pointers' scalar loads return while the keys
    // stream), then the values; the query and rotary rows are waited for with
    // the keys, which the scores need first anyway (config 2: 11.67-11.69 ->
    // 11.44-11.46 us).  Without it (a launch that rotates the query) the small
    // operands go first, so the rotation runs while the keys and values are
    // in flight instead of after the keys arrive (single-layer f32-operand
    // decode: 7.71-7.74 us, against 8.18-8.21 with the keys first).  (Waves
    // past the end of a short partition re-read the partition's last tile and
    // never use it.)
    half8_t kr[PAIRS][2][4];
    half8_t vr[PAIRS][8];
    int ws = part_start + wave * kChunkTokens;
    if constexpr (KEYS_FIRST) {
        load_chunk_keys<PAIRS>(p, g, ids, 0, row, kg, kr);
        __builtin_amdgcn_sched_barrier(0);
    }
    // Every pointer the small operands and the prologue need, named here so
    // they arrive in one round of scalar loads (left to itself the compiler
    // loads each where it is first needed, behind branches on the optional
    // ones: four dependent rounds).
    asm volatile("" ::"s"(p.positions), "s"(p.rope_cos), "s"(p.rope_sin), "s"(p.rope_rows));
    if constexpr (F32IO) asm volatile("" ::"s"(p.query32), "s"(p.new_key32), "s"(p.new_value32));
    else asm volatile("" ::"s"(p.query), "s"(p.new_key), "s"(p.new_value));

    // Rotary position of the appended row (and of the query).
    if (pos_from_params) pos = p.positions ? load_const(p.positions, s) : cache_len;
    bool rope = p.rope_cos != nullptr;
    const bool rope_bad = rope && (pos < 0 || static_cast<uint32_t>(pos) >= p.rope_rows);
    if (rope_bad) rope = false;
    const float *cos_row = rope ? p.rope_cos + static_cast<size_t>(pos) * 64 : nullptr;
    const float *sin_row = rope ? p.rope_sin + static_cast<size_t>(pos) * 64 : nullptr;

    const size_t qoff = (static_cast<size_t>(s) * kQueryHeads + g * kGroup + (row & 7)) * kHeadDim;
    const size_t new_base = (static_cast<size_t>(s) * kKvHeads + g) * kHeadDim;
    // (Without rotary the cos/sin loads read the new key row as a stand-in,
    // so they stay unconditional; the values are then replaced by cos 1,
    // sin 0.)
    const float *stand_in = F32IO ? p.new_key32 + new_base : reinterpret_cast<const float *>(p.new_key + new_base);
    const float *cos_src = rope ? cos_row : stand_in;
    const float *sin_src = rope ? sin_row : stand_in;
    // Raw loads first, every lane, then the first chunk's values, and only
    // then any arithmetic on the small operands: a conversion between them
    // made the compiler wait for the keys before issuing the values.  With f32
    // operands the zero columns' lanes read the rows of columns 0-7 again (the
    // same cache lines) and are selected away afterwards; loads on only some
    // lanes, behind the key loads, also forced that wait (single-layer decode
    // 7.80 -> 8.22 us).
    half8_t qb[4];
    float4_t q32[F32IO ? 4 : 1][2];
    float nkf_lo = 0.f, nkf_hi = 0.f, nvf_lo = 0.f, nvf_hi = 0.f;  // f32 operands: the new row as given
    uint16_t nk_lo = 0, nk_hi = 0, nv_lo = 0, nv_hi = 0;
    if constexpr (F32IO) {
#pragma unroll
        for (int kb = 0; kb < 4; ++kb) {
            q32[kb][0] = *reinterpret_cast<const float4_t *>(p.query32 + qoff + kb * 32 + kg * 8);
            q32[kb][1] = *reinterpret_cast<const float4_t *>(p.query32 + qoff + kb * 32 + kg * 8 + 4);
        }
        nkf_lo = p.new_key32[new_base + lane];
        nkf_hi = p.new_key32[new_base + lane + 64];
        nvf_lo = p.new_value32[new_base + lane];
        nvf_hi = p.new_value32[new_base + lane + 64];
    } else {
        const uint16_t *qrow = p.query + qoff;
#pragma unroll
        for (int kb = 0; kb < 4; ++kb) qb[kb] = *reinterpret_cast<const half8_t *>(qrow + kb * 32 + kg * 8);
        nk_lo = p.new_key[new_base + lane];
        nk_hi = p.new_key[new_base + lane + 64];
        nv_lo = p.new_value[new_base + lane];
        nv_hi = p.new_value[new_base + lane + 64];
    }
    const float rc_raw = cos_src[lane];
    const float rs_raw = sin_src[lane];

    // First chunk's keys (if not issued above) and values.
    __builtin_amdgcn_sched_barrier(0);
    if constexpr (!KEYS_FIRST) {
        load_chunk_keys<PAIRS>(p, g, ids, 0, row, kg, kr);
        __builtin_amdgcn_sched_barrier(0);
    }
    load_chunk_values<PAIRS>(p, g, ids, 0, row, kg, vr);
    __builtin_amdgcn_sched_barrier(0);

    // The query is the B operand of the score MFMA: column = query head of
    // the group (8 real, 8 zero), k = dims kb*32 + kg*8 .. +8 (with fp16
    // operands the lanes of the zero columns load a real row and discard it).
    // With f32 operands the query is kept as given until it is rotated, and
    // rounded to fp16 once (RNE), as the new key below.  The appended row:
    // lane t holds dims t and t+64 (the rotate-half pair) and cos/sin of pair
    // t.
    float qf[F32IO ? 4 : 1][8];
    if constexpr (F32IO) {
        const bool real = row < static_cast<int>(kGroup);
#pragma unroll
        for (int kb = 0; kb < 4; ++kb) {
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                qf[kb][j] = real ? q32[kb][0][j] : 0.f;
                qf[kb][j + 4] = real ? q32[kb][1][j] : 0.f;
            }
#pragma unroll
            for (int j = 0; j < 8; ++j) qb[kb][j] = to_h(qf[kb][j]);
        }
        nk_lo = __builtin_bit_cast(uint16_t, to_h(nkf_lo));
        nk_hi = __builtin_bit_cast(uint16_t, to_h(nkf_hi));
        nv_lo = __builtin_bit_cast(uint16_t, to_h(nvf_lo));
        nv_hi = __builtin_bit_cast(uint16_t, to_h(nvf_hi));
    }
    const float rc = rope ? rc_raw : 1.0f;
    const float rs = rope ? rs_raw : 0.0f;

    if (rope && p.rotate_query) {
        // Rotate-half of the query in place: the partner of chunk kb is
        // chunk kb^2 of the same lane, and cos/sin of pair i live in lane i.
        half8_t qr[4];
#pragma unroll
        for (int kb = 0; kb < 4; ++kb) {
#pragma unroll
            for (int j = 0; j < 8; ++j) {
                const int pair = (kb & 1) * 32 + kg * 8 + j;
                const float c = __shfl(rc, pair);
                const float sn = __shfl(rs, pair);
                const float x = F32IO ? qf[kb][j] : static_cast<float>(qb[kb][j]);
                const float y = F32IO ? qf[kb ^ 2][j] : static_cast<float>(qb[kb ^ 2][j]);
                qr[kb][j] = kb < 2 ? to_h(x * c + (-y) * sn) : to_h(x * c + y * sn);
            }
        }
#pragma unroll
        for (int kb = 0; kb < 4; ++kb) qb[kb] = qr[kb];
    }
#pragma unroll
    for (int kb = 0; kb < 4; ++kb)
        if (row >= static_cast<int>(kGroup)) qb[kb] = half8_t{};

    // Append: the wave whose chunks hold the appended row's tile rotates the
    // new key, writes the new K/V row into the cache, and keeps it in LDS to
    // stand in for that row of its own tile loads (which may see the old
    // row).  Only that wave reads the row back, so no barrier is needed: a
    // workgroup barrier here held every wave of the appending workgroup until
    // the slowest wave's first loads had returned (config 2: 12.66 -> 12.25
    // us).  Rotate-half in f32 exactly as apply_rope_neox (cpu-ref
    // lib.rs:459-463): x'[d] = x[d]*cos + (-x[d+64])*sin and
    // x'[d+64] = x[d+64]*cos + x[d]*sin, products rounded separately (no
    // contraction in this file), then RNE to fp16.
    const int append_tile = cache_len >> 4;
    const int append_row = cache_len & 15;
    const bool owns_append = (append_tile << 4) >= part_start && (append_tile << 4) < part_end;
    __shared__ uint16_t sm_new_k[kHeadDim];
    __shared__ uint16_t sm_new_v[kHeadDim];
    if (owns_append) {
        const int rel = append_tile - (part_start >> 4);  // tile of the partition holding the row
        if (wave == (rel / kChunkTiles) % WAVES) {
            uint16_t k_lo = nk_lo, k_hi = nk_hi;
            if (rope) {
                const float x = F32IO ? nkf_lo : static_cast<float>(__builtin_bit_cast(_Float16, nk_lo));
                const float y = F32IO ? nkf_hi : static_cast<float>(__builtin_bit_cast(_Float16, nk_hi));
                k_lo = __builtin_bit_cast(uint16_t, to_h(x * rc + (-y) * rs));
                k_hi = __builtin_bit_cast(uint16_t, to_h(y * rc + x * rs));
            }
            // The append block's id was checked with the partition's ids (a
            // bad one is reported there); the row is then not written.
            int64_t blk = static_cast<int64_t>(s) * p.max_blocks_per_seq + append_tile;
            if (p.block_tables) {
                const int32_t b = load_const(p.block_tables, static_cast<size_t>(s) * p.max_blocks_per_seq + append_tile);
                blk = (b < 0 || static_cast<uint32_t>(b) >= p.num_blocks) ? -1 : b;
            }
            sm_new_k[lane] = k_lo;
            sm_new_k[lane + 64] = k_hi;
            sm_new_v[lane] = nv_lo;
            sm_new_v[lane + 64] = nv_hi;
            if (blk >= 0) {
                const size_t slab = (static_cast<size_t>(blk) * kKvHeads + g) * kBlockHeadElems;
                // key (append_row, d) at (d/8)*128 + key_slot(append_row)*8 + d%8; value at d*16 + append_row
                const int kslot = key_slot(append_row);
                p.key_cache[slab + (lane >> 3) * 128 + kslot * 8 + (lane & 7)] = k_lo;
                p.key_cache[slab + ((lane + 64) >> 3) * 128 + kslot * 8 + (lane & 7)] = k_hi;
                p.value_cache[slab + lane * 16 + append_row] = nv_lo;
                p.value_cache[slab + (lane + 64) * 16 + append_row] = nv_hi;
            }
        }
    }

    float m_run = -INFINITY;  // running max (log2 units) of head `row`
    float l_run = 0.0f;       // this lane's share of the running sum
    float4_t o[8];
#pragma unroll
    for (int c = 0; c < 8; ++c) o[c] = float4_t{0.f, 0.f, 0.f, 0.f};

    for (int chunk = 0; ws < part_end; ++chunk, ws += WAVES * kChunkTokens) {
        if (chunk > 0) load_chunk<PAIRS>(p, g, ids, chunk, row, kg, kr, vr);

        // Patch the appended key (the tile loads may predate the append): its
        // slot is row (ti & 1)*8 + (slot & 7) of score MFMA slot >> 3 of pair
        // ti >> 1.
        const int ti = append_tile - (ws >> 4);  // chunk tile holding the appended row
        if (ti >= 0 && ti < kChunkTiles) {
            const int slot = key_slot(append_row);
            if (row == (ti & 1) * 8 + (slot & 7)) {
#pragma unroll
                for (int j = 0; j < PAIRS; ++j)
#pragma unroll
                    for (int h = 0; h < 2; ++h) {
                        if (j != (ti >> 1) || h != (slot >> 3)) continue;
#pragma unroll
                        for (int kb = 0; kb < 4; ++kb)
                            kr[j][h][kb] = *reinterpret_cast<const half8_t *>(sm_new_k + (kb * 4 + kg) * 8);
                    }
            }
        }

        // Scores: MFMA h of pair j leaves lane (head `row`, kg) the tokens
        // (kg & 1)*8 + h*4 + r (r = 0..3) of the pair's tile kg >> 1, so
        // x[j][0..7] are 8 consecutive tokens of one tile.
        float x[PAIRS][8];
        float cmax = -INFINITY;
#pragma unroll
        for (int j = 0; j < PAIRS; ++j) {
#pragma unroll
            for (int h = 0; h < 2; ++h) {
                float4_t acc = float4_t{0.f, 0.f, 0.f, 0.f};
#pragma unroll
                for (int kb = 0; kb < 4; ++kb)
                    acc = __builtin_amdgcn_mfma_f32_16x16x32_f16(kr[j][h][kb], qb[kb], acc, 0, 0, 0);
                const int tbase = ws + (2 * j + (kg >> 1)) * 16 + (kg & 1) * 8 + h * 4;
#pragma unroll
                for (int r = 0; r < 4; ++r) {
                    x[j][h * 4 + r] = (tbase + r < part_end) ? acc[r] * p.scale_log2 : -INFINITY;
                    cmax = fmaxf(cmax, x[j][h * 4 + r]);
                }
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

        // Values: lane (dim, kg) holds tokens (kg & 1)*8 + e of tile
        // 2j + (kg >> 1).  Zero the tiles past the partition and the tokens
        // after the appended one (their weights are 0, but they may hold
        // poison and NaN * 0 would reach P.V); patch the appended token.
        if (ws + kChunkTokens > part_end || (ti >= 0 && ti < kChunkTiles)) {  // uniform
            // The appended token's value at this lane's 8 dims, read from LDS
            // by every lane whether it patches or not: with the reads inside
            // the per-element condition the compiler branched around each of
            // the 64 elements and waited for each read in turn (~2 us).
            _Float16 nvv[8];
#pragma unroll
            for (int c = 0; c < 8; ++c) nvv[c] = __builtin_bit_cast(_Float16, sm_new_v[c * 16 + row]);
#pragma unroll
            for (int j = 0; j < PAIRS; ++j) {
                const int tile = 2 * j + (kg >> 1);
                const bool past = ws + tile * 16 >= part_end;
                const bool append_here = tile == ti;
#pragma unroll
                for (int e = 0; e < 8; ++e) {
                    const int tok = (kg & 1) * 8 + e;
                    const bool zero = past || (append_here && tok > append_row);
                    const bool patch = append_here && tok == append_row;
#pragma unroll
                    for (int c = 0; c < 8; ++c) {
                        const _Float16 v = patch ? nvv[c] : vr[j][c][e];
                        vr[j][c][e] = zero ? static_cast<_Float16>(0.0f) : v;
                    }
                }
            }
        }

        // P.V with P in fp16: the weights of the fp16 entry points.  The f32
        // entry points carry each weight as an exact-in-f32 pair hi + lo of
        // fp16 values (hi = fp16(p), lo = fp16(p - hi)), so P.V takes two
        // MFMAs and the weights keep ~22 bits instead of 11 (the fp16 P is the
        // dominant error of the output against the f32 reference: rel-L2
        // ~2e-4 with it, ~1e-6 with the pair).
#pragma unroll
        for (int j = 0; j < PAIRS; ++j) {
            half8_t pa, pl;
#pragma unroll
            for (int e = 0; e < 8; ++e) {
                const float pf = __builtin_amdgcn_exp2f(x[j][e] - m_new);
                const _Float16 ph = to_h(pf);
                pa[e] = ph;
                if constexpr (F32IO) {
                    const _Float16 plo = to_h(pf - static_cast<float>(ph));  // pf - ph is exact in f32
                    pl[e] = plo;
                    l_run += static_cast<float>(ph) + static_cast<float>(plo);  // the weights P.V uses
                } else {
                    l_run += static_cast<float>(ph);  // the weights P.V actually uses
                }
            }
#pragma unroll
            for (int c = 0; c < 8; ++c) {
                o[c] = __builtin_amdgcn_mfma_f32_16x16x32_f16(pa, vr[j][c], o[c], 0, 0, 0);
                if constexpr (F32IO) o[c] = __builtin_amdgcn_mfma_f32_16x16x32_f16(pl, vr[j][c], o[c], 0, 0, 0);
            }
        }
    }
    l_run += __shfl_xor(l_run, 16);
    l_run += __shfl_xor(l_run, 32);
    // Deferred error report: bit 1 = a block id outside the planes (that
    // block read block 0), bit 2 = rotary position outside the table (no
    // rotation applied).
    if (__any(ids_bad) && lane == 0) atomicOr(p.error_word, 2u);
    if (rope_bad && threadIdx.x == 0) atomicOr(p.error_word, 4u);

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

    // Each of the first kCT threads (a power of two) owns kPer consecutive
    // output elements of one head; the others shadow thread 0 and store
    // nothing.
    constexpr int kCT =
        kThreads >= 1024 ? 1024 : (kThreads >= 512 ? 512 : (kThreads >= 256 ? 256 : (kThreads >= 128 ? 128 : 64)));
    constexpr int kPer = (kGroup * kHeadDim) / kCT;
    const bool active = threadIdx.x < kCT;
    const int e0 = active ? static_cast<int>(threadIdx.x) * kPer : 0;
    const int h = e0 >> 7, d0 = e0 & 127;
    // Every wave's (m, l, o) read first, in one batch: folded as they were
    // read, the reads went out one or two at a time, each behind a wait.
    float mw[WAVES], lw[WAVES], ow[WAVES][kPer];
#pragma unroll
    for (int w = 0; w < WAVES; ++w) {
        mw[w] = sm_m[w][h];
        lw[w] = sm_l[w][h];
#pragma unroll
        for (int e = 0; e < kPer; ++e) ow[w][e] = sm_o[w][h][d0 + e];
    }
    __builtin_amdgcn_sched_barrier(0);
    float M = -INFINITY;
#pragma unroll
    for (int w = 0; w < WAVES; ++w) M = fmaxf(M, mw[w]);
    float L = 0.f;
    float po[kPer];
#pragma unroll
    for (int e = 0; e < kPer; ++e) po[e] = 0.f;
#pragma unroll
    for (int w = 0; w < WAVES; ++w) {
        const float f = __builtin_amdgcn_exp2f(mw[w] - M);  // 0 for a wave without tokens
        L += lw[w] * f;
#pragma unroll
        for (int e = 0; e < kPer; ++e) po[e] += ow[w][e] * f;
    }

    // Output element i of this (sequence, kv head): fp16 (RNE) or f32.
    const size_t out_off = (static_cast<size_t>(s) * kQueryHeads + g * kGroup) * kHeadDim;
    auto put = [&](int i, float v) {
        if constexpr (F32IO) p.out32[out_off + i] = v;
        else p.out[out_off + i] = __builtin_bit_cast(uint16_t, to_h(v));
    };
    if (num_parts == 1) {
        const float inv = 1.0f / L;
        if (active) {
#pragma unroll
            for (int e = 0; e < kPer; ++e) put(e0 + e, po[e] * inv);
        }
        return;
    }

    const size_t unit = (static_cast<size_t>(s) * kKvHeads + g) * p.part_stride;
    float *part_o = p.part_o + (unit + part) * (kGroup * kHeadDim);
    float *part_ml = p.part_ml + (unit + part) * (2 * kGroup);  // [head][max, sum]
    if constexpr (DEFER_MERGE) {
        // The kernel boundary orders these stores before the merge kernel.
        if (active) {
#pragma unroll
            for (int e = 0; e < kPer; ++e) part_o[e0 + e] = po[e];
            if (d0 == 0) {
                part_ml[2 * h] = M;
                part_ml[2 * h + 1] = L;
            }
        }
        return;
    }

    // Cross-workgroup hand-off without L2 maintenance: partials, the arrival
    // counter and the merge reads are relaxed agent-scope atomics (sc1), which
    // are coherent across the XCDs' L2s by themselves.  Every store of the
    // workgroup completes (s_waitcnt vmcnt(0), then the barrier) before thread
    // 0 counts the arrival, which orders the partials before the count.
    // (A C++ release/acquire fence at agent scope would instead write back and
    // invalidate the whole L2 of the XCD in every workgroup.)  Values move in
    // 8-byte pairs: half the transactions of single floats.  Shapes whose
    // threads own 4 or more elements (kWide: at most 256 combining threads,
    // the single-sequence decodes of 16 partitions) move them as 16-byte
    // buffer stores and loads with the same agent-scope (sc1) policy, issued
    // through the compiler's buffer intrinsics so that its waits cover them:
    // single-layer decode 8.48 -> 8.17 us.
    static_assert(kPer % 2 == 0, "partials move as float pairs");
    constexpr bool kWide = kPer % 4 == 0;
    // Raw buffer over this unit's partials: stride 0, 2^31 - 1 bytes, and the
    // fourth descriptor word of a raw 32-bit-element buffer on gfx9-family
    // parts (data format 32 in bits 15-18).
    const __amdgpu_buffer_rsrc_t o_rsrc =
        __builtin_amdgcn_make_buffer_rsrc(p.part_o + unit * (kGroup * kHeadDim), 0, 0x7fffffff, 0x00020000);
    auto pack = [](float lo, float hi) {
        return static_cast<uint64_t>(__float_as_uint(lo)) | (static_cast<uint64_t>(__float_as_uint(hi)) << 32);
    };
    if (active) {
        if constexpr (kWide) {
#pragma unroll
            for (int e = 0; e < kPer; e += 4) {
                const u32x4_t v = {__float_as_uint(po[e]), __float_as_uint(po[e + 1]), __float_as_uint(po[e + 2]),
                                   __float_as_uint(po[e + 3])};
                __builtin_amdgcn_raw_buffer_store_b128(
                    v, o_rsrc, static_cast<int>((part * (kGroup * kHeadDim) + e0 + e) * 4), 0, kSc1);
            }
        } else {
#pragma unroll
            for (int e = 0; e < kPer; e += 2)
                __hip_atomic_store(reinterpret_cast<uint64_t *>(part_o + e0 + e), pack(po[e], po[e + 1]),
                                   __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        }
        if (d0 == 0)
            __hip_atomic_store(reinterpret_cast<uint64_t *>(part_ml + 2 * h), pack(M, L), __ATOMIC_RELAXED,
                               __HIP_MEMORY_SCOPE_AGENT);
    }
    // Wait for this wave's partial stores to complete (a single-wave
    // workgroup's __syncthreads() emits no wait), then for every wave.
    asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
    __syncthreads();
    // Arrival, counted in generations (kArrivalSpan): the partition with the
    // highest index adds kArrivalSpan - (num_parts - 1), the others 1, so the
    // arrival that completes a multiple of kArrivalSpan is the last one, and
    // the counter is left ready for the next launch without a reset.
    if (threadIdx.x == 0) {
        const uint32_t inc =
            part == static_cast<uint32_t>(num_parts - 1) ? kArrivalSpan - static_cast<uint32_t>(num_parts - 1) : 1u;
        const uint32_t prev =
            __hip_atomic_fetch_add(p.counters + s * kKvHeads + g, inc, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        sm_last = ((prev + inc) & (kArrivalSpan - 1)) == 0;
    }
    __syncthreads();
    if (!sm_last) return;

    const float *all_ml = p.part_ml + unit * (2 * kGroup);

    // Merge, per thread and without barriers: each thread loads the (max,
    // sum) of its head and its elements of every other partition, a batch of
    // partitions at a time (its own are still in registers: reading them back
    // cost config 2 ~0.2 us), and folds them into a running LSE combination.
    const float *all_o = p.part_o + unit * (kGroup * kHeadDim);
    // The wide shapes take 16 partitions per batch (one round of loads for
    // the single-sequence decode's 16: 8.17 -> 7.87 us; 4 with the 16
    // elements a thread of the one-wave shape owns) and load only the
    // partitions that exist; the others keep batches of 8 with clamped
    // re-reads.
    constexpr int kBatch = kPer >= 16 ? 4 : (kWide ? 16 : 8);
    float Mg = -INFINITY, Lg = 0.f, og[kPer];
#pragma unroll
    for (int e = 0; e < kPer; ++e) og[e] = 0.f;
    for (int q0 = 0; q0 < num_parts; q0 += kBatch) {
        float mv[kBatch], lv[kBatch], ov[kBatch][kPer];
#pragma unroll
        for (int b = 0; b < kBatch; ++b) {
            const int q = min(q0 + b, num_parts - 1);  // clamped re-reads get weight 0 below
            if (q == static_cast<int>(part) || (kWide && q0 + b >= num_parts)) {  // uniform
                // this partition's own partial, still in registers (or, past
                // the last partition, a stand-in of weight 0)
                mv[b] = M;
                lv[b] = L;
#pragma unroll
                for (int e = 0; e < kPer; ++e) ov[b][e] = po[e];
            } else {
                load_pair_sc1(all_ml + q * (2 * kGroup) + 2 * h, &mv[b], &lv[b]);
                if constexpr (kWide) {
#pragma unroll
                    for (int e = 0; e < kPer; e += 4) {
                        const u32x4_t v = __builtin_amdgcn_raw_buffer_load_b128(
                            o_rsrc, static_cast<int>((q * (kGroup * kHeadDim) + e0 + e) * 4), 0, kSc1);
#pragma unroll
                        for (int k = 0; k < 4; ++k) ov[b][e + k] = __uint_as_float(v[k]);
                    }
                } else {
#pragma unroll
                    for (int e = 0; e < kPer; e += 2)
                        load_pair_sc1(all_o + static_cast<size_t>(q) * (kGroup * kHeadDim) + e0 + e, &ov[b][e],
                                      &ov[b][e + 1]);
                }
            }
        }
        float Mb = Mg;
#pragma unroll
        for (int b = 0; b < kBatch; ++b)
            if (q0 + b < num_parts) Mb = fmaxf(Mb, mv[b]);  // finite: every partition holds a token
        const float a = __builtin_amdgcn_exp2f(Mg - Mb);   // 0 on the first batch
        Lg *= a;
#pragma unroll
        for (int e = 0; e < kPer; ++e) og[e] *= a;
#pragma unroll
        for (int b = 0; b < kBatch; ++b) {
            const float w = (q0 + b < num_parts) ? __builtin_amdgcn_exp2f(mv[b] - Mb) : 0.f;
            Lg += lv[b] * w;
#pragma unroll
            for (int e = 0; e < kPer; ++e) og[e] += ov[b][e] * w;
        }
        Mg = Mb;
    }
    const float inv = 1.0f / Lg;
    if (active) {
#pragma unroll
        for (int e = 0; e < kPer; ++e) put(e0 + e, og[e] * inv);
    }
}

// Cache length of sequence s if it is valid for this launch (one row to
// append, inside the block table and the partitions of the workspace), else -1.
__device__ inline int64_t checked_cache_len(const DecodeParams &p, int64_t len) {
    const int64_t capacity = static_cast<int64_t>(p.max_blocks_per_seq) * 16;
    const int64_t span = static_cast<int64_t>(p.max_parts) * p.partition_tokens;
    return (len < 0 || len + 1 > capacity || len + 1 > span) ? -1 : len;
}

// Grid (partition, kv head, sequence): sequences of one uniform length, or
// ragged lengths when there are too many sequences for the ragged kernel.
// The arguments the first key loads' addresses depend on come ahead of the
// parameter block, as scalars: the first 14 dwords of kernel arguments are
// preloaded into SGPRs at wave launch (-amdgpu-kernarg-preload-count=16; a
// struct argument is not), so the key stream starts without a scalar-load
// round trip.  The copies in p are not read.
template <int WAVES, int PAIRS, bool F32IO, bool KEYS_FIRST>
__global__ __launch_bounds__(WAVES * 64, 2) void paged_decode_kernel(
    uint16_t *key_cache, uint16_t *value_cache, const int32_t *cache_lens, const int32_t *block_tables,
    uint32_t uniform_cache_len, uint32_t max_blocks_per_seq, uint32_t num_blocks, uint32_t partition_tokens,
    uint32_t max_parts, DecodeParams p) {
    p.key_cache = key_cache;
    p.value_cache = value_cache;
    p.cache_lens = cache_lens;
    p.block_tables = block_tables;
    p.uniform_cache_len = uniform_cache_len;
    p.max_blocks_per_seq = max_blocks_per_seq;
    p.num_blocks = num_blocks;
    p.partition_tokens = partition_tokens;
    p.max_parts = max_parts;
    const uint32_t part = blockIdx.x;
    const uint32_t g = blockIdx.y;  // kv head
    const uint32_t s = blockIdx.z;  // sequence (or layer)
    const int64_t len = checked_cache_len(
        p, p.cache_lens ? load_const(p.cache_lens, s) : static_cast<int64_t>(p.uniform_cache_len));
    if (len < 0) {
        if (part == 0 && g == 0 && threadIdx.x == 0) atomicOr(p.error_word, 1u);
        return;
    }
    const int cache_len = static_cast<int>(len);
    const int P = static_cast<int>(p.partition_tokens);
    const int part_start = static_cast<int>(part) * P;
    if (part_start > cache_len) return;
    const int wave = __builtin_amdgcn_readfirstlane(static_cast<int>(threadIdx.x >> 6));
    bool bad = false;
    const uint32_t ids =
        wave_tile_ids<WAVES, 2 * PAIRS>(p, s, part_start, min(part_start + P, cache_len + 1), wave, &bad);
    decode_item<WAVES, PAIRS, false, F32IO, KEYS_FIRST>(p, static_cast<int>(p.partition_tokens), s, g, part,
                                                        cache_len, 0, ids, bad, /*pos_from_params=*/true);
}

// Exclusive scan of one int per thread over the workgroup; *total receives
// the sum.
template <int kThreads>
__device__ inline int workgroup_exclusive_scan(int v, int *sm_wave_sums, int *total) {
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    int x = v;
#pragma unroll
    for (int o = 1; o < 64; o <<= 1) {
        const int y = __shfl_up(x, o);
        if (lane >= o) x += y;
    }
    if (lane == 63) sm_wave_sums[wave] = x;
    __syncthreads();
    int before = 0, sum = 0;
#pragma unroll
    for (int w = 0; w < kThreads / 64; ++w) {
        const int t = sm_wave_sums[w];
        before += w < wave ? t : 0;
        sum += t;
    }
    __syncthreads();
    *total = sum;
    return before + x - v;
}

// Persistent grid for ragged lengths and long contexts: every workgroup
// reads the cache lengths (and positions) once into LDS, numbers the (sequence, partition,
// kv head) items that hold rows, and walks items blockIdx.x,
// blockIdx.x + gridDim.x, ...  Sequences with fewer partitions launch no
// empty workgroups, so every compute unit stays on real work, and the block
// ids of the next item are loaded while the current one runs.
template <int WAVES, int PAIRS, bool F32IO>
__global__ __launch_bounds__(WAVES * 64, 2) void paged_decode_ragged_kernel(DecodeParams p, uint32_t num_seqs) {
    constexpr int kThreads = WAVES * 64;
    __shared__ int sm_first[kMaxRaggedSeqs + 1];  // first item (per kv head) of each sequence
    __shared__ int sm_len[kMaxRaggedSeqs];        // cache length, -1 if invalid
    __shared__ int sm_pos[kMaxRaggedSeqs];        // rotary position of the appended row
    __shared__ int sm_wave_sums[WAVES];
    __shared__ int sm_counts[kPartitionChoices][WAVES];
    const int n = static_cast<int>(num_seqs);
    const int per = (n + kThreads - 1) / kThreads;
    const int i0 = static_cast<int>(threadIdx.x) * per;
    // Validity is judged against the partition the host planned with.
    const int P0 = static_cast<int>(p.partition_tokens);
    static_assert(2 * PAIRS == 2, "wave_tile_ids holds 32 chunks of 2 tiles per wave");
    constexpr uint32_t kSpan = streaming_span(WAVES);
    int counts[kPartitionChoices] = {};
    for (int i = i0; i < min(i0 + per, n); ++i) {
        const int64_t len =
            checked_cache_len(p, p.cache_lens ? p.cache_lens[i] : static_cast<int64_t>(p.uniform_cache_len));
        if (len < 0 && blockIdx.x == 0) atomicOr(p.error_word, 1u);
        sm_len[i] = static_cast<int>(len);
        sm_pos[i] = p.positions ? p.positions[i] : static_cast<int>(len);
        if (p.partition_word) {
#pragma unroll
            for (int c = 0; c < kPartitionChoices; ++c) {
                const int pc = static_cast<int>(streaming_partition_candidate(static_cast<uint32_t>(P0), c, kSpan));
                counts[c] += (len < 0 || pc == 0) ? 0 : static_cast<int>((len + pc) / pc);
            }
        }
    }
    // Automatic partition (choose_streaming_partition): item k runs on
    // workgroup k mod grid, and the grid fills every compute unit before it
    // doubles up, so item k lands on unit k mod units and a unit streams
    // ceil(items / units) items one after the other at the per-unit HBM rate.
    // Every workgroup computes the same counts from the same lengths.  The
    // candidates stop at kSpan, the tokens covered by the block ids the
    // workgroup's waves hold (wave_tile_ids).
    int P = P0;
    if (p.partition_word) {
        const int wave = threadIdx.x >> 6;
#pragma unroll
        for (int c = 0; c < kPartitionChoices; ++c) {
            int v = counts[c];
#pragma unroll
            for (int o = 1; o < 64; o <<= 1) v += __shfl_xor(v, o);
            if ((threadIdx.x & 63) == 0) sm_counts[c][wave] = v;
        }
        __syncthreads();
        const uint32_t units = max(1u, p.compute_units);
        uint32_t items[kPartitionChoices] = {};
        for (int c = 0; c < kPartitionChoices; ++c) {
            for (int w = 0; w < WAVES; ++w) items[c] += static_cast<uint32_t>(sm_counts[c][w]);
            items[c] *= kKvHeads;  // at most 2048 sequences x 64 partitions x 2 heads
        }
        P = static_cast<int>(choose_streaming_partition(items, static_cast<uint32_t>(P0), units, kSpan));
        P = __builtin_amdgcn_readfirstlane(P);  // uniform: keep the item arithmetic scalar
        if (blockIdx.x == 0 && threadIdx.x == 0) {
            p.partition_word[0] = static_cast<uint32_t>(P);
            p.partition_word[1] = static_cast<uint32_t>(units);  // for inspection
        }
    }
    int local = 0;
    for (int i = i0; i < min(i0 + per, n); ++i) {
        const int len = sm_len[i];  // written by this thread above
        const int parts = len < 0 ? 0 : (len + P) / P;  // ceil((len + 1) / P)
        sm_first[i + 1] = parts;
        local += parts;
    }
    int total = 0;
    int run = workgroup_exclusive_scan<kThreads>(local, sm_wave_sums, &total);
    for (int i = i0; i < min(i0 + per, n); ++i) {
        run += sm_first[i + 1];
        sm_first[i + 1] = run;
    }
    if (threadIdx.x == 0) sm_first[0] = 0;
    __syncthreads();

    const int wave = __builtin_amdgcn_readfirstlane(static_cast<int>(threadIdx.x >> 6));
    // Item k (per kv head) lies in the last sequence s with sm_first[s] <= k
    // (sequences without partitions share their successor's start).
    auto locate = [&](int k, uint32_t *s_out, uint32_t *part_out) {
        int lo = 0, hi = n - 1;
        while (lo < hi) {
            const int mid = (lo + hi + 1) >> 1;
            if (sm_first[mid] <= k) lo = mid;
            else hi = mid - 1;
        }
        *s_out = static_cast<uint32_t>(__builtin_amdgcn_readfirstlane(lo));
        *part_out = static_cast<uint32_t>(__builtin_amdgcn_readfirstlane(k - sm_first[lo]));
    };
    const int items = total * static_cast<int>(kKvHeads);
    int item = blockIdx.x;
    if (item >= items) return;
    uint32_t s = 0, part = 0;
    locate(item >> 1, &s, &part);
    bool bad = false;
    uint32_t ids = wave_tile_ids<WAVES, 2 * PAIRS>(p, s, static_cast<int>(part) * P,
                                               min(static_cast<int>(part + 1) * P, sm_len[s] + 1), wave, &bad);
    for (;;) {
        const int next = item + static_cast<int>(gridDim.x);
        uint32_t s_next = 0, part_next = 0, ids_next = 0;
        bool bad_next = false;
        if (next < items) {
            locate(next >> 1, &s_next, &part_next);
            ids_next = wave_tile_ids<WAVES, 2 * PAIRS>(p, s_next, static_cast<int>(part_next) * P,
                                                   min(static_cast<int>(part_next + 1) * P, sm_len[s_next] + 1), wave,
                                                   &bad_next);
        }
        decode_item<WAVES, PAIRS, true, F32IO>(p, P, s, static_cast<uint32_t>(item & 1), part, sm_len[s], sm_pos[s],
                                               ids, bad);
        if (next >= items) break;
        __syncthreads();  // the next item reuses the workgroup's LDS
        item = next;
        s = s_next;
        part = part_next;
        ids = ids_next;
        bad = bad_next;
    }
}

// LSE merge of the partials the ragged kernel stored: one workgroup per
// (kv head, sequence); each thread folds 4 consecutive output elements of one
// head over every partition, 16 partitions per batch of loads.  Sequences of
// one partition were written directly by the ragged kernel.
template <bool F32IO>
__global__ __launch_bounds__(256) void paged_decode_merge_kernel(DecodeParams p) {
    const uint32_t g = blockIdx.x;
    const uint32_t s = blockIdx.y;
    const int64_t len = checked_cache_len(
        p, p.cache_lens ? load_const(p.cache_lens, s) : static_cast<int64_t>(p.uniform_cache_len));
    if (len < 0) return;
    // The ragged kernel wrote the partition it used before this launch began.
    const int P = static_cast<int>(p.partition_word ? load_const(reinterpret_cast<const int32_t *>(p.partition_word), 0)
                                                    : p.partition_tokens);
    const int num_parts = static_cast<int>((len + P) / P);
    if (num_parts <= 1) return;
    const int e0 = threadIdx.x * 4;
    const int h = e0 >> 7;
    const size_t unit = (static_cast<size_t>(s) * kKvHeads + g) * p.part_stride;
    const float *all_o = p.part_o + unit * (kGroup * kHeadDim);
    const float *all_ml = p.part_ml + unit * (2 * kGroup);
    constexpr int kBatch = 16;
    float Mg = -INFINITY, Lg = 0.f;
    float4_t og = float4_t{0.f, 0.f, 0.f, 0.f};
    for (int q0 = 0; q0 < num_parts; q0 += kBatch) {
        float mv[kBatch], lv[kBatch];
        float4_t ov[kBatch];
#pragma unroll
        for (int b = 0; b < kBatch; ++b) {
            const int q = min(q0 + b, num_parts - 1);  // clamped re-reads get weight 0 below
            mv[b] = all_ml[q * (2 * kGroup) + 2 * h];
            lv[b] = all_ml[q * (2 * kGroup) + 2 * h + 1];
            ov[b] = *reinterpret_cast<const float4_t *>(all_o + static_cast<size_t>(q) * (kGroup * kHeadDim) + e0);
        }
        float Mb = Mg;
#pragma unroll
        for (int b = 0; b < kBatch; ++b)
            if (q0 + b < num_parts) Mb = fmaxf(Mb, mv[b]);  // finite: every partition holds a token
        const float a = __builtin_amdgcn_exp2f(Mg - Mb);   // 0 on the first batch
        Lg *= a;
        og *= a;
#pragma unroll
        for (int b = 0; b < kBatch; ++b) {
            const float w = (q0 + b < num_parts) ? __builtin_amdgcn_exp2f(mv[b] - Mb) : 0.f;
            Lg += lv[b] * w;
            og += ov[b] * w;
        }
        Mg = Mb;
    }
    const float inv = 1.0f / Lg;
    const size_t out_off = (static_cast<size_t>(s) * kQueryHeads + g * kGroup) * kHeadDim + e0;
#pragma unroll
    for (int e = 0; e < 4; ++e) {
        if constexpr (F32IO) p.out32[out_off + e] = og[e] * inv;
        else p.out[out_off + e] = __builtin_bit_cast(uint16_t, to_h(og[e] * inv));
    }
}

__global__ void fill_u32_kernel(uint32_t *dst, size_t words, uint32_t value) {
    const size_t i = static_cast<size_t>(blockIdx.x) * blockDim.x + threadIdx.x;
    if (i < words) dst[i] = value;
}

}  // namespace

// Workgroups of `kernel` the current device keeps resident at once (compute
// units x workgroups per unit), at most max_items; cached per kernel and device
// in a fixed table (no allocation after the first launches; a full table only
// means the query is repeated).
uint32_t resident_workgroups(const void *kernel, int threads, uint64_t max_items, uint32_t *units, int *err) {
    struct Entry {
        const void *kernel;
        int device;
        uint32_t wgs;
        uint32_t cus;
    };
    constexpr int kEntries = 256;
    static std::mutex mu;
    static Entry cache[kEntries];
    static int cached = 0;
    int device = 0;
    if (hipError_t r = hipGetDevice(&device)) {
        *err = static_cast<int>(r);
        return 0;
    }
    uint32_t wgs = 0, cus_seen = 0;
    {
        std::lock_guard<std::mutex> lock(mu);
        for (int i = 0; i < cached; ++i)
            if (cache[i].kernel == kernel && cache[i].device == device) {
                wgs = cache[i].wgs;
                cus_seen = cache[i].cus;
            }
    }
    if (wgs == 0) {
        int cus = 0, per_cu = 0;
        if (hipError_t r = hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, device)) {
            *err = static_cast<int>(r);
            return 0;
        }
        if (hipError_t r = hipOccupancyMaxActiveBlocksPerMultiprocessor(&per_cu, kernel, threads, 0)) {
            *err = static_cast<int>(r);
            return 0;
        }
        wgs = static_cast<uint32_t>(cus * (per_cu > 0 ? per_cu : 1));
        cus_seen = static_cast<uint32_t>(cus > 0 ? cus : 1);
        std::lock_guard<std::mutex> lock(mu);
        if (cached < kEntries) cache[cached++] = {kernel, device, wgs, cus_seen};
    }
    *units = cus_seen;
    return static_cast<uint32_t>(max_items < wgs ? (max_items ? max_items : 1) : wgs);
}

// One regime's launches for operands of either width (F32IO: the f32 entry
// point's query, new key and value, output).
template <bool F32IO>
int launch_paged_decode_kernels(const DecodeLaunch &launch, DecodeParams &p, hipStream_t st) {
    const pvlc_hip_paged_decode_args &a = *launch.args;
    int e = 0;
    if (launch.streaming) {
        // Persistent kernel storing partials, then the merge kernel: no
        // workgroup waits on a cross-workgroup hand-off.
        const uint64_t max_items = static_cast<uint64_t>(launch.max_parts) * kKvHeads * a.num_seqs;
#define PVLC_RAGGED_LAUNCH(W, PR)                                                                                  \
    do {                                                                                                           \
        const uint32_t wgs = resident_workgroups(                                                                  \
            reinterpret_cast<const void *>(&paged_decode_ragged_kernel<W, PR, F32IO>), (W) * 64, max_items,        \
            &p.compute_units, &e);                                                                                 \
        if (e == 0) {                                                                                              \
            hipLaunchKernelGGL((paged_decode_ragged_kernel<W, PR, F32IO>), dim3(wgs), dim3((W) * 64), 0, st, p,    \
                               a.num_seqs);                                                                        \
            hipLaunchKernelGGL(paged_decode_merge_kernel<F32IO>, dim3(kKvHeads, a.num_seqs), dim3(256), 0, st, p); \
        }                                                                                                          \
    } while (0)
        if (launch.waves == 4) PVLC_RAGGED_LAUNCH(4, 1);
        else PVLC_RAGGED_LAUNCH(2, 1);
#undef PVLC_RAGGED_LAUNCH
        if (e != 0) return e;
        return static_cast<int>(hipGetLastError());
    }

    // Single-shot regime: one workgroup per (partition, kv head, sequence);
    // the last partition to arrive merges.
    const dim3 grid(launch.max_parts, kKvHeads, a.num_seqs);
#define PVLC_DECODE_LAUNCH(W, PR)                                                                               \
    do {                                                                                                        \
        if (p.rotate_query)                                                                                     \
            hipLaunchKernelGGL((paged_decode_kernel<W, PR, F32IO, false>), grid, dim3((W) * 64), 0, st,         \
                               p.key_cache, p.value_cache, p.cache_lens, p.block_tables, p.uniform_cache_len,   \
                               p.max_blocks_per_seq, p.num_blocks, p.partition_tokens, p.max_parts, p);         \
        else                                                                                                    \
            hipLaunchKernelGGL((paged_decode_kernel<W, PR, F32IO, true>), grid, dim3((W) * 64), 0, st,          \
                               p.key_cache, p.value_cache, p.cache_lens, p.block_tables, p.uniform_cache_len,   \
                               p.max_blocks_per_seq, p.num_blocks, p.partition_tokens, p.max_parts, p);         \
    } while (0)
    switch (launch.waves) {
        case 1: PVLC_DECODE_LAUNCH(1, 1); break;
        case 2: PVLC_DECODE_LAUNCH(2, 1); break;
        case 4: PVLC_DECODE_LAUNCH(4, 1); break;
        case 6: PVLC_DECODE_LAUNCH(6, 1); break;
        case 10: PVLC_DECODE_LAUNCH(10, 1); break;
        case 12: PVLC_DECODE_LAUNCH(12, 1); break;
        default: PVLC_DECODE_LAUNCH(8, 1); break;
    }
#undef PVLC_DECODE_LAUNCH
    return static_cast<int>(hipGetLastError());
}

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
    p.part_stride = launch.part_stride;
    p.part_o = launch.part_o;
    p.part_ml = launch.part_ml;
    p.counters = launch.counters;
    p.error_word = launch.error_word;
    p.partition_word = launch.partition_word;
    p.scale_log2 = kLog2e / sqrtf(static_cast<float>(kHeadDim));
    hipStream_t st = static_cast<hipStream_t>(stream);
    if (launch.f32) {
        p.query32 = launch.f32->query;
        p.new_key32 = launch.f32->new_key;
        p.new_value32 = launch.f32->new_value;
        p.out32 = launch.f32->out;
        return launch_paged_decode_kernels<true>(launch, p, st);
    }
    return launch_paged_decode_kernels<false>(launch, p, st);
}

int launch_fill_u32(uint32_t *dst, size_t words, uint32_t value, void *stream) {
    if (words == 0) return 0;
    const unsigned blocks = static_cast<unsigned>((words + 255) / 256);
    hipLaunchKernelGGL(fill_u32_kernel, dim3(blocks), dim3(256), 0, static_cast<hipStream_t>(stream), dst, words,
                       value);
    return static_cast<int>(hipGetLastError());
}

}  // namespace pvlc
