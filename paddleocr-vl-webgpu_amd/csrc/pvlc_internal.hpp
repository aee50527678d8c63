// Internal declarations shared by the pvlc_hip translation units.
#pragma once

#include <cstddef>
#include <cstdint>
#include <string>

#include "pvlc_hip.h"

namespace pvlc {

constexpr uint32_t kQueryHeads = PVLC_HIP_QUERY_HEADS;
constexpr uint32_t kKvHeads = PVLC_HIP_KV_HEADS;
constexpr uint32_t kHeadDim = PVLC_HIP_HEAD_DIM;
constexpr uint32_t kGroup = kQueryHeads / kKvHeads;
constexpr uint32_t kBlockTokens = PVLC_HIP_BLOCK_TOKENS;
constexpr uint32_t kRowElems = kKvHeads * kHeadDim;          // one cache row, both heads
constexpr uint32_t kBlockHeadElems = kBlockTokens * kHeadDim;  // one (block, head) slab

// Key slot of token t (0..15) inside a 16-token block of the key plane: bits
// 2 and 3 of t swapped, so that slots 0-7 hold tokens 0-3 and 8-11 and slots
// 8-15 tokens 4-7 and 12-15.  With this order one 16x16x32 score MFMA over
// rows "slots 0-7 of tile A, slots 0-7 of tile B" (and a second over slots
// 8-15) leaves each lane the scores of 8 consecutive tokens of one tile:
// exactly the probability operand of a 16x16x32 P.V MFMA whose values are
// 16-byte loads.  The map is its own inverse (constexpr: usable on host and
// device).
constexpr int key_slot(int t) { return (t & 3) | ((t & 4) << 1) | ((t & 8) >> 1); }
constexpr uint32_t kMaxDecoderHeadDim = 128;                   // runtime-core lib.rs:180
constexpr uint32_t kMaxWebgpuDispatch = 65535;                 // runtime-core lib.rs:187
constexpr uint32_t kMaxMergeParts = 64;  // split-K partitions one in-kernel merge combines
// Automatic partitioning: workgroups one launch aims to keep resident (one
// per MI355X compute unit), the most tiles one workgroup covers without
// looping (12 waves x one pair of tiles), and the most partitions of the
// balanced rule.
constexpr uint32_t kTargetWorkgroups = 256;
constexpr uint32_t kSingleShotTiles = 24;
constexpr uint32_t kMaxBalancedParts = 16;
// Arrival counters of the single-shot split-K hand-off count in generations:
// every partition adds 1 except the one with the highest index, which adds
// kArrivalSpan - (parts - 1), so a launch adds exactly kArrivalSpan to the
// counter of each (sequence, kv head) it merges.  The counter is never reset:
// the arrival that brings it to a multiple of kArrivalSpan is the last, and
// any value is ready for the next launch (a power of two above the 64
// partitions a merge combines, so the arithmetic holds modulo 2^32).
constexpr uint32_t kArrivalSpan = 1024;
static_assert((kArrivalSpan & (kArrivalSpan - 1)) == 0 && kArrivalSpan > 64, "arrival span");
// Sequences the ragged (persistent) decode kernel numbers in LDS; launches
// with more ragged sequences use one workgroup per (partition, head, sequence).
constexpr uint32_t kMaxRaggedSeqs = 2048;

// Automatic streaming partition.  The host plans p0; the streaming kernel may
// lengthen it to a candidate p0 + c*step (c < kPartitionChoices, step = p0/4
// rounded down to 16 tokens, at least 16), never beyond the span one
// workgroup of the streaming shape covers: a wave keeps the block ids of its
// tiles one per lane (64 lanes = 32 chunks of 2 tiles), and a chunk round of
// `waves` waves covers waves x 2 tiles, so a partition spans at most
// 32 x waves x 2 x 16 = 1024 x waves tokens (4096 for the 4-wave shape).
// Candidates beyond the span are skipped (0 below).
constexpr int kPartitionChoices = 5;
constexpr uint32_t streaming_span(uint32_t waves) { return 1024u * waves; }
constexpr uint32_t streaming_partition_candidate(uint32_t p0, int c, uint32_t span) {
    const uint32_t quarter = (p0 / 4) & ~15u;
    const uint32_t pc = p0 + static_cast<uint32_t>(c) * (quarter > 16 ? quarter : 16);
    return pc <= span ? pc : 0;
}
// The candidate with the least ceil(items / units) * P (the first on ties),
// where items[c] counts the (sequence, partition, kv head) items at candidate
// c: item k runs on compute unit k mod units, so a unit streams
// ceil(items / units) partitions one after the other.  p0 itself is a
// candidate whenever p0 <= span, which the host's shape choice guarantees.
constexpr uint32_t choose_streaming_partition(const uint32_t (&items)[kPartitionChoices], uint32_t p0,
                                              uint32_t units, uint32_t span) {
    const uint32_t u = units > 0 ? units : 1;
    uint32_t best_p = p0;
    uint64_t best = ~0ull;
    for (int c = 0; c < kPartitionChoices; ++c) {
        const uint32_t pc = streaming_partition_candidate(p0, c, span);
        if (pc == 0) continue;
        const uint64_t cost = static_cast<uint64_t>((items[c] + u - 1) / u) * pc;
        if (cost < best) {
            best = cost;
            best_p = pc;
        }
    }
    return best_p;
}

// Status of a failed call: RuntimeErrorCode in bits 8..15, InvocationErrorCode
// in bits 0..7; records the message for pvlc_hip_last_error_message().
pvlc_hip_status fail(int runtime_code, int invocation_code, const std::string &message);
inline pvlc_hip_status invalid(int invocation_code, const std::string &message) {
    return fail(PVLC_HIP_INVALID_INVOCATION, invocation_code, message);
}
pvlc_hip_status ok();

// Plan-layer error: an InvocationErrorCode plus message (runtime-core's
// InvocationError, lib.rs:5365-5395).
struct PlanError {
    int code = PVLC_HIP_INV_NONE;
    std::string message;
    explicit operator bool() const { return code != PVLC_HIP_INV_NONE; }
};

PlanError plan_session_geometry(uint32_t query_heads, uint32_t key_value_heads, uint32_t head_dim,
                                uint32_t prefix_tokens, uint32_t cache_capacity, pvlc_hip_kv_session_plan *out);
PlanError plan_split(uint32_t cache_tokens, uint32_t query_heads, uint32_t key_value_heads, uint32_t head_dim,
                     pvlc_hip_gqa_split_plan *out);
PlanError plan_descriptor(const pvlc_hip_kv_session_descriptor *d, pvlc_hip_kv_session_plan *out);
PlanError plan_step(const pvlc_hip_kv_session_plan *plan, uint32_t cache_tokens, const pvlc_hip_kv_step_operands *step,
                    pvlc_hip_kv_step_plan *out);
PlanError plan_cached_gqa(const pvlc_hip_cached_gqa_invocation *inv, pvlc_hip_kv_session_plan *session_out,
                          pvlc_hip_kv_step_plan *step_out);

// fp16 storage admits only values whose RNE rounding is finite (|x| < 65520).
bool fp16_representable(const float *values, size_t n);
uint16_t f32_to_f16_rne(float value);
float f16_to_f32(uint16_t bits);

// Host copies between the compact reference rows [tokens][2][128] and the
// blocked device layout (contiguous blocks 0..ceil(tokens/16)-1).
size_t key_blocked_index(uint32_t token, uint32_t head, uint32_t dim);
size_t value_blocked_index(uint32_t token, uint32_t head, uint32_t dim);

// Kernel launchers (kernels_*.hip).  Return hipError_t as int.
// The f32 operands of pvlc_hip_paged_decode_f32io (device pointers).
struct DecodeOperands32 {
    const float *query;      // [num_seqs][16][128]
    const float *new_key;    // [num_seqs][2][128]
    const float *new_value;  // [num_seqs][2][128]
    float *out;              // [num_seqs][16][128]
};
struct DecodeLaunch {
    const pvlc_hip_paged_decode_args *args;
    uint32_t partition_tokens;
    uint32_t waves;      // waves per workgroup
    uint32_t pairs;      // pairs of 16-token tiles a wave holds per chunk
    bool streaming;      // persistent kernel + merge kernel (else one workgroup per partition)
    uint32_t max_parts;
    uint32_t part_stride;
    float *part_o;
    float *part_ml;
    uint32_t *counters;
    uint32_t *error_word;
    // Streaming regime with an automatic partition: the persistent kernel may
    // lengthen the partition to fill its last round of items and writes the
    // partition it used here for the merge kernel, and the compute units it
    // assumed in the next word (null: partition_tokens as is).
    uint32_t *partition_word;
    // f32 operands instead of args' fp16 query, new key and value, output
    // (null: the fp16 ones).
    const DecodeOperands32 *f32 = nullptr;
};
int launch_paged_decode(const DecodeLaunch &launch, void *stream);
int launch_fill_u32(uint32_t *dst, size_t words, uint32_t value, void *stream);
int launch_kv_pack(const uint16_t *key_rows, const uint16_t *value_rows, uint32_t tokens, const int32_t *table,
                   uint32_t num_blocks, uint16_t *key_cache, uint16_t *value_cache, uint32_t *error_word,
                   void *stream);
int launch_kv_unpack(const uint16_t *key_cache, const uint16_t *value_cache, uint32_t tokens, const int32_t *table,
                     uint32_t num_blocks, uint16_t *key_rows, uint16_t *value_rows, void *stream);
// The f32 operands of pvlc_hip_paged_prefill_f32io (device pointers).
struct PrefillOperands32 {
    const float *query;  // [tokens][16][128]
    const float *key;    // [tokens][2][128]
    const float *value;  // [tokens][2][128]
    float *out;          // [tokens][16][128]
};
int launch_prefill(const pvlc_hip_paged_prefill_args *args, void *stream, const PrefillOperands32 *f32 = nullptr);

// Prefill projection with fp16 weights: workspace of the exact hi/lo split
// of the activations ([rows][K] fp16 each) and the per-row exponents.
// Workspace of the projection: the hi/lo planes of the split activations in
// the GEMM's tile order -- for each 128-row tile t and each 32-wide k step s
// one 16 KiB block [plane (hi, lo)][k-chunk (4)][row (128)][8 fp16] -- then
// one exponent per row; rows are padded to a multiple of 128 (zeros).
constexpr uint32_t kProjectionTileRows = 128, kProjectionStepK = 32;
struct ProjectionWorkspace {
    uint16_t *tiles;
    int32_t *exponents;
};
struct ProjectionWorkspaceLayout {
    size_t exponents_offset, total;
};
inline ProjectionWorkspaceLayout projection_workspace_layout(uint32_t rows, uint32_t k_width) {
    const size_t padded = (static_cast<size_t>(rows) + kProjectionTileRows - 1) / kProjectionTileRows * kProjectionTileRows;
    const size_t tiles = padded * k_width * 4;  // two fp16 planes
    return {tiles, tiles + (padded * 4 + 255) / 256 * 256};
}
int launch_linear_projection_f16(const float *input, const uint16_t *weight, const float *bias, float *out,
                                 uint32_t rows, uint32_t k_width, uint32_t n_width, const ProjectionWorkspace &ws,
                                 void *stream);

// Split-K pair schedule of the causal prefill.  Query block qb (16 tokens)
// of one kv head attends qb/4 + 1 steps of 64 keys, so a grid of one
// workgroup per block is as long as its last block while most compute units
// idle.  With a workspace, block l and block qblocks-1-l of a kv head (about
// qblocks/4 + 2 steps together) go to two workgroups of about equal time:
// the first runs the first k steps of the heavy block, hands that part over,
// then runs the light block; the second runs the rest of the heavy block
// (which holds the diagonal) and merges the first part, which has arrived by
// then (otherwise the part that arrives last merges).  Running the heavy part
// first lets the second workgroup find it complete and merge it without
// storing its own part: config 4 at N=4096, 99.8-100.8 -> 96.6-97.3 us mean
// per call.  Used when the longest block is longer than kPrefillSplitSteps.  A pair whose light workgroup
// would take fewer than kPrefillSplitMin heavy steps at an even split is not
// split (the light block and the heavy block run whole on the two
// workgroups): a second segment costs its workgroup a query load, a pipeline
// fill and the partial hand-off, about what 4 to 5 steps cost (measured at
// N=4096: 9-13 us for 1-2 steps).  Of that, the light workgroup's extra
// segment (the one the heavy workgroup does not run: query load, fill, last
// steps and output stores of the light block) costs about 4 steps, so a
// split pair moves kPrefillSplitShift heavy steps from the light workgroup to
// the heavy one (config 4 at N=4096, shifts 0-3 on one box with the light
// block first: 103.0-103.7, 102.3, 100.0, 100.6-100.7 us mean per call; with
// the heavy part first, shifts 1-4: 97.7-97.9, 96.6-97.3, 97.6-98.8,
// 99.2-99.9).
constexpr uint32_t kPrefillSplitSteps = 32;
constexpr uint32_t kPrefillSplitMin = 5;
constexpr uint32_t kPrefillSplitShift = 2;
static_assert(kPrefillSplitMin > kPrefillSplitShift, "a split pair leaves the light workgroup a heavy step");
constexpr uint32_t kPrefillPartialFloats = 4 * 64 * 74;  // 4 waves x 64 lanes x (2 x 9 x 4 O/l + 2 m)

constexpr uint32_t prefill_block_steps(uint32_t qb) { return qb / 4 + 1; }
constexpr uint32_t prefill_max_steps(uint32_t qblocks) { return (qblocks - 1) / 4 + 1; }
constexpr uint32_t prefill_pairs(uint32_t qblocks) { return (qblocks + 1) / 2; }
constexpr uint32_t prefill_pair_workgroups(uint32_t qblocks) { return 4u * prefill_pairs(qblocks); }

struct PrefillSegment {
    uint32_t qb, part, nparts, step_begin, steps;
};

// Segments of workgroup w of the pair grid (w = (pair * 2 + g) * 2 + role);
// returns their number (0..2).
constexpr uint32_t prefill_pair_segments(uint32_t w, uint32_t qblocks, uint32_t *g, uint32_t *pair,
                                         PrefillSegment *first, PrefillSegment *second) {
    const uint32_t role = w & 1u, pg = w >> 1;
    *g = pg & 1u;
    *pair = pg >> 1;
    const uint32_t heavy = qblocks - 1u - *pair, light = *pair;
    const uint32_t sh = prefill_block_steps(heavy), sl = light == heavy ? 0u : prefill_block_steps(light);
    const uint32_t half = (sh - sl + 1u) / 2u;
    // heavy steps the light block's workgroup takes (>= 3 when split)
    const uint32_t k = half < kPrefillSplitMin ? 0u : half - kPrefillSplitShift;
    // Straight-line assignments (no runtime-indexed pointer), so that on the
    // device both segments stay in registers.  sh >= 1, so k >= sh implies k > 0.
    PrefillSegment s0{}, s1{};
    uint32_t n = 0;
    if (role == 0) {
        const PrefillSegment hs = k >= sh ? PrefillSegment{heavy, 0u, 1u, 0u, sh} : PrefillSegment{heavy, 0u, 2u, 0u, k};
        if (sl) {
            const PrefillSegment ls{light, 0u, 1u, 0u, sl};
            s0 = k > 0 ? hs : ls;  // the heavy part first, then the light block
            s1 = ls;
            n = k > 0 ? 2u : 1u;
        } else if (k > 0) {
            s0 = hs;
            n = 1;
        }
    } else if (k == 0) {
        s0 = {heavy, 0u, 1u, 0u, sh};
        n = 1;
    } else if (k < sh) {
        s0 = {heavy, 1u, 2u, k, sh - k};
        n = 1;
    }
    *first = s0;
    *second = s1;
    return n;
}
// Workspace of the pair schedule: an arrival counter per (pair, kv head),
// then two partial slabs each; 0 when the blocks are short enough.
struct PrefillWorkspace {
    size_t partial_offset, total;
};
inline PrefillWorkspace prefill_workspace_layout(uint32_t tokens) {
    const uint32_t qblocks = (tokens + 15u) / 16u;
    if (tokens == 0 || prefill_max_steps(qblocks) <= kPrefillSplitSteps) return {0, 0};
    const uint32_t items = 2u * prefill_pairs(qblocks);
    const size_t counters = (static_cast<size_t>(items) * 4 + 255) / 256 * 256;
    return {counters, counters + static_cast<size_t>(items) * 2 * kPrefillPartialFloats * 4};
}
int launch_gemv_f16(const uint16_t *weights, const float *vector, float *out, uint32_t rows, uint32_t columns,
                    void *stream);
constexpr uint32_t kGemvGroupMax = 4;
struct GemvGroup {  // members of one grouped GEMV launch (by value: kernel argument)
    const uint16_t *weights[kGemvGroupMax];
    float *out[kGemvGroupMax];
    uint32_t end[kGemvGroupMax - 1];  // rows up to the end of members 0..2; UINT32_MAX from the last member on
    uint32_t total;                   // rows of all members
};
int launch_gemv_group_f16(const GemvGroup &group, const float *vector, uint32_t columns, void *stream);

// Top-1 workspace: kTop1Slots slots of 256 bytes, each a packed u64
// candidate; zero before the first launch, zero again after each launch.
constexpr uint32_t kTop1Slots = 64;
struct Top1Slot {
    uint64_t best;
    uint64_t pad[31];
};
static_assert(sizeof(Top1Slot) == 256, "one slot per 256-byte line");
constexpr size_t kTop1WorkspaceBytes = kTop1Slots * sizeof(Top1Slot);
int launch_gemv_top1_f16(const uint16_t *weights, const float *vector, float *logits, uint32_t rows,
                         uint32_t columns, Top1Slot *slots, uint32_t *result, void *stream);
int launch_logits_top1_f32(const float *logits, uint32_t vocab, Top1Slot *slots, uint32_t *result, void *stream);

// VisionPatchProjectionBytesDescriptor::plan (runtime-core lib.rs:1768-1840);
// returns a pvlc_hip_projection_error.
int32_t plan_projection(uint32_t patch_count, uint32_t input_width, uint32_t output_width, uint32_t weight_storage,
                        pvlc_hip_projection_plan *out);

// GemvTiledDescriptor::plan (runtime-core lib.rs:753-785); returns a status.
int plan_gemv_tiled(uint32_t rows, uint32_t columns, pvlc_hip_gemv_tiled_plan *out);

// Workspace layout of the paged decode.
struct DecodeWorkspace {
    size_t part_o_offset, part_ml_offset, counters_offset, error_offset, total;
    uint32_t part_stride;  // partials per (sequence, kv head) slot: max_parts rounded up to odd
};
DecodeWorkspace decode_workspace_layout(uint32_t num_seqs, uint32_t max_parts);
// Split-K state of one decode launch: partial outputs and (max, sum), merge
// counters (zero before the first launch; see kArrivalSpan), the error
// word and the two status words (automatic streaming partition, compute
// units).
struct DecodeState {
    float *part_o;
    float *part_ml;
    uint32_t *counters;
    uint32_t *error_word;
    uint32_t *status_words;
    uint32_t part_stride;  // partials per (sequence, kv head) slot: max_parts rounded up to odd
};
// Checks of pvlc_hip_paged_decode_f16's arguments, the workspace aside: the
// partition and the partitions per (sequence, kv head) of the launch.  With
// f32 operands (pvlc_hip_paged_decode_f32io) args' fp16 query, new key and
// value and output must be NULL and the f32 ones given.
pvlc_hip_status validate_decode_geometry(const pvlc_hip_paged_decode_args *a, uint32_t *partition_out,
                                         uint32_t *max_parts_out, const DecodeOperands32 *f32 = nullptr);
// Launch a validated decode with its split-K state at `state`; launches_out
// receives the kernels launched (1, or 2 for the persistent kernel and its
// merge kernel).
pvlc_hip_status launch_decode_state(const pvlc_hip_paged_decode_args *a, uint32_t partition, uint32_t max_parts,
                                    const DecodeState &state, void *stream, uint32_t *launches_out,
                                    const DecodeOperands32 *f32 = nullptr);
// Partition rules: balanced_parts is the partition count per (sequence, kv
// head) of the single-shot rule; single_shot_partition returns 0 when a
// partition would exceed kSingleShotTiles; auto_partition falls back to
// 512-token (or longer) streaming partitions; auto_workspace_parts bounds the
// partitions of every automatic launch up to max_context.
uint32_t balanced_parts(uint32_t num_seqs);
uint32_t single_shot_partition(uint32_t num_seqs, uint32_t context);
uint32_t auto_partition(uint32_t num_seqs, uint32_t context);
uint32_t auto_workspace_parts(uint32_t num_seqs, uint32_t max_context);
// Launch shape for a partition: (waves, pairs) of the single-shot kernel,
// or of the persistent kernel when `streaming`.
struct DecodeShape {
    uint32_t waves, pairs;
};
DecodeShape decode_shape(uint32_t partition_tokens, bool streaming);

}  // namespace pvlc
