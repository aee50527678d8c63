// Plan authority: the admission rules of crates/pvlc-runtime-core
// (glebkudr/paddleocr-vl-webgpu) for the decoder KV session, the cached GQA
// invocation, the split-K geometry and the prefill token bound.  Host only.
//
// Error precedence follows the Rust code line by line, so a caller switching
// backends sees the same InvocationErrorCode for the same bad input.

#include <cmath>
#include <cstring>
#include <limits>
#include <string>

#include "pvlc_internal.hpp"

namespace pvlc {
namespace {

thread_local std::string g_last_error;

PlanError err(int code, std::string message) { return PlanError{code, std::move(message)}; }
PlanError none() { return PlanError{}; }

// overflow(), runtime-core lib.rs:5311-5316
PlanError overflow() { return err(PVLC_HIP_INV_ARITHMETIC_OVERFLOW, "invocation size arithmetic overflowed"); }

// require_dimensions, lib.rs:5216-5224
PlanError require_dimensions(std::initializer_list<uint32_t> dims) {
    for (uint32_t d : dims) {
        if (d == 0) return err(PVLC_HIP_INV_ZERO_DIMENSION, "all invocation dimensions must be nonzero");
    }
    return none();
}

// require_len, lib.rs:5251-5259
PlanError require_len(size_t actual, uint64_t expected) {
    if (static_cast<uint64_t>(actual) != expected) {
        return err(PVLC_HIP_INV_LENGTH_MISMATCH, "buffer has " + std::to_string(actual) +
                                                     " elements but the invocation requires " +
                                                     std::to_string(expected));
    }
    return none();
}

// require_finite, lib.rs:5261-5269
PlanError require_finite(const float *values, size_t n) {
    for (size_t i = 0; i < n; ++i) {
        if (!std::isfinite(values[i]))
            return err(PVLC_HIP_INV_NON_FINITE_INPUT, "floating input contains NaN or infinity");
    }
    return none();
}

bool mul_u64(uint64_t a, uint64_t b, uint64_t *out) {
    if (a != 0 && b > std::numeric_limits<uint64_t>::max() / a) return false;
    *out = a * b;
    return true;
}

PlanError invalid_geometry(std::string message) {
    return err(PVLC_HIP_INV_INVALID_DECODER_GEOMETRY, std::move(message));
}

uint32_t ceil_div(uint32_t v, uint32_t d) { return v / d + (v % d != 0 ? 1u : 0u); }

}  // namespace

pvlc_hip_status fail(int runtime_code, int invocation_code, const std::string &message) {
    g_last_error = message;
    return static_cast<pvlc_hip_status>((runtime_code << 8) | invocation_code);
}

pvlc_hip_status ok() {
    g_last_error.clear();
    return PVLC_HIP_OK;
}

// DecoderGqaSplitDescriptor::plan, lib.rs:2889-2978
PlanError plan_split(uint32_t cache_tokens, uint32_t query_heads, uint32_t key_value_heads, uint32_t head_dim,
                     pvlc_hip_gqa_split_plan *out) {
    if (cache_tokens == 0 || query_heads == 0 || key_value_heads == 0 || head_dim == 0) {
        return invalid_geometry("decoder GQA split geometry T" + std::to_string(cache_tokens) + " / Q" +
                                std::to_string(query_heads) + " / KV" + std::to_string(key_value_heads) + " / D" +
                                std::to_string(head_dim) + " contains a zero dimension");
    }
    if (head_dim != kMaxDecoderHeadDim) {
        return invalid_geometry("decoder GQA split head dimension " + std::to_string(head_dim) +
                                " drifted from the pinned 128");
    }
    if (query_heads % key_value_heads != 0) {
        return invalid_geometry("decoder GQA split query heads are not contiguous groups of key-value heads");
    }
    if (query_heads != kQueryHeads || key_value_heads != kKvHeads) {
        return invalid_geometry("decoder GQA split head counts drifted from the pinned Q16 / KV2");
    }
    const uint32_t chunk_count = ceil_div(cache_tokens, PVLC_HIP_REFERENCE_SPLIT_CHUNK);
    const uint64_t partial_workgroups = static_cast<uint64_t>(query_heads) * chunk_count;
    if (partial_workgroups > kMaxWebgpuDispatch) {
        return invalid_geometry("decoder GQA split partial dispatch " + std::to_string(partial_workgroups) +
                                " exceeds the single-dispatch workgroup bound");
    }
    pvlc_hip_gqa_split_plan p{};
    p.chunk_size = PVLC_HIP_REFERENCE_SPLIT_CHUNK;
    p.chunk_count = chunk_count;
    p.partials_elements = partial_workgroups * PVLC_HIP_REFERENCE_PARTIAL_STRIDE_F32;
    p.partials_bytes = p.partials_elements * 4u;
    p.partial_stride_f32 = PVLC_HIP_REFERENCE_PARTIAL_STRIDE_F32;
    p.partial_workgroups = static_cast<uint32_t>(partial_workgroups);
    p.merge_workgroups = ceil_div(query_heads * head_dim, 64);
    p.uniform_words[0] = cache_tokens;
    p.uniform_words[1] = chunk_count;
    if (out) *out = p;
    return none();
}

// plan_decoder_kv_session_geometry, lib.rs:1057-1159
PlanError plan_session_geometry(uint32_t query_heads, uint32_t key_value_heads, uint32_t head_dim,
                                uint32_t prefix_tokens, uint32_t cache_capacity, pvlc_hip_kv_session_plan *out) {
    if (PlanError e = require_dimensions({query_heads, key_value_heads, head_dim, prefix_tokens, cache_capacity}))
        return e;
    if (head_dim > kMaxDecoderHeadDim) {
        return err(PVLC_HIP_INV_UNSUPPORTED_HEAD_DIMENSION, "decoder head dimension " + std::to_string(head_dim) +
                                                                " exceeds the supported maximum 128");
    }
    const uint64_t query_elements = static_cast<uint64_t>(query_heads) * head_dim;
    const uint64_t key_value_width = static_cast<uint64_t>(key_value_heads) * head_dim;
    uint64_t cache_elements;
    if (!mul_u64(cache_capacity, key_value_width, &cache_elements)) return overflow();
    if (prefix_tokens == std::numeric_limits<uint32_t>::max()) return overflow();
    const uint64_t cache_tokens_after = static_cast<uint64_t>(prefix_tokens) + 1;
    uint64_t valid_elements;
    if (!mul_u64(cache_tokens_after, key_value_width, &valid_elements)) return overflow();
    for (uint64_t elements : {query_elements, key_value_width, cache_elements, valid_elements}) {
        if (elements == 0 || elements - 1 > std::numeric_limits<uint32_t>::max()) return overflow();
    }
    if (query_heads % key_value_heads != 0 || query_heads != kQueryHeads || key_value_heads != kKvHeads ||
        head_dim != kMaxDecoderHeadDim) {
        return invalid_geometry(
            "cached decoder GQA is pinned to Q16/KV2/D128 with contiguous query-head groups");
    }
    if (prefix_tokens >= cache_capacity) {
        return invalid_geometry("cache capacity " + std::to_string(cache_capacity) +
                                " has no append slot after prefix length " + std::to_string(prefix_tokens));
    }
    pvlc_hip_gqa_split_plan split{};
    if (PlanError e = plan_split(cache_capacity, kQueryHeads, kKvHeads, kMaxDecoderHeadDim, &split)) return e;
    pvlc_hip_kv_session_plan p{};
    p.initial_cache_tokens = prefix_tokens;
    p.cache_capacity = cache_capacity;
    p.query_heads = query_heads;
    p.key_value_heads = key_value_heads;
    p.head_dim = head_dim;
    p.query_elements = query_elements;
    p.key_value_width = key_value_width;
    p.cache_elements = cache_elements;
    p.cache_bytes = cache_elements * 4u;
    p.attention_bytes = query_elements * 4u;
    p.split_partials_bytes = split.partials_bytes;
    if (out) *out = p;
    return none();
}

// DecoderKvSessionDescriptor::plan, lib.rs:952-968
PlanError plan_descriptor(const pvlc_hip_kv_session_descriptor *d, pvlc_hip_kv_session_plan *out) {
    pvlc_hip_kv_session_plan p{};
    if (PlanError e = plan_session_geometry(d->query_heads, d->key_value_heads, d->head_dim, d->prefix_tokens,
                                            d->cache_capacity, &p))
        return e;
    if (PlanError e = require_len(d->key_cache ? d->key_cache_len : 0, p.cache_elements)) return e;
    if (PlanError e = require_len(d->value_cache ? d->value_cache_len : 0, p.cache_elements)) return e;
    const size_t semantic = static_cast<size_t>(d->prefix_tokens) * p.key_value_width;
    if (PlanError e = require_finite(d->key_cache, semantic)) return e;
    if (PlanError e = require_finite(d->value_cache, semantic)) return e;
    if (out) *out = p;
    return none();
}

// DecoderKvSessionPlan::plan_cache_transition + plan_step, lib.rs:976-1054
PlanError plan_step(const pvlc_hip_kv_session_plan *plan, uint32_t cache_tokens, const pvlc_hip_kv_step_operands *step,
                    pvlc_hip_kv_step_plan *out) {
    if (cache_tokens < plan->initial_cache_tokens) {
        return invalid_geometry("persistent decoder cache length cannot move before its admitted prefix");
    }
    if (cache_tokens >= plan->cache_capacity) {
        return invalid_geometry("persistent decoder cache has no remaining append slot");
    }
    const uint64_t after = static_cast<uint64_t>(cache_tokens) + 1;
    uint64_t valid;
    if (!mul_u64(after, plan->key_value_width, &valid)) return overflow();
    if (valid == 0 || valid - 1 > std::numeric_limits<uint32_t>::max()) return overflow();
    pvlc_hip_kv_step_plan p{};
    p.cache_tokens_before = cache_tokens;
    p.cache_tokens_after = static_cast<uint32_t>(after);
    p.valid_cache_elements = valid;
    p.append_uniform_words[0] = cache_tokens;
    p.append_uniform_words[1] = plan->key_value_heads;
    p.append_uniform_words[2] = plan->head_dim;
    p.append_uniform_words[3] = plan->cache_capacity;
    p.attention_uniform_words[0] = p.cache_tokens_after;
    p.attention_uniform_words[1] = plan->query_heads;
    p.attention_uniform_words[2] = plan->key_value_heads;
    p.attention_uniform_words[3] = plan->head_dim;
    if (PlanError e = plan_split(p.cache_tokens_after, kQueryHeads, kKvHeads, kMaxDecoderHeadDim, &p.split_gqa))
        return e;
    if (step) {
        if (PlanError e = require_len(step->query ? step->query_len : 0, plan->query_elements)) return e;
        if (PlanError e = require_len(step->appended_key ? step->appended_key_len : 0, plan->key_value_width))
            return e;
        if (PlanError e = require_len(step->appended_value ? step->appended_value_len : 0, plan->key_value_width))
            return e;
        if (PlanError e = require_finite(step->query, step->query_len)) return e;
        if (PlanError e = require_finite(step->appended_key, step->appended_key_len)) return e;
        if (PlanError e = require_finite(step->appended_value, step->appended_value_len)) return e;
    }
    if (out) *out = p;
    return none();
}

// DecoderCachedGqaInvocation::plan, lib.rs:903-951
PlanError plan_cached_gqa(const pvlc_hip_cached_gqa_invocation *inv, pvlc_hip_kv_session_plan *session_out,
                          pvlc_hip_kv_step_plan *step_out) {
    pvlc_hip_kv_session_plan session{};
    if (PlanError e = plan_session_geometry(inv->query_heads, inv->key_value_heads, inv->head_dim, inv->prefix_tokens,
                                            inv->cache_capacity, &session))
        return e;
    const uint64_t prefix_elements = static_cast<uint64_t>(inv->prefix_tokens) * session.key_value_width;
    if (PlanError e = require_len(inv->query ? inv->query_len : 0, session.query_elements)) return e;
    if (PlanError e = require_len(inv->appended_key ? inv->appended_key_len : 0, session.key_value_width)) return e;
    if (PlanError e = require_len(inv->appended_value ? inv->appended_value_len : 0, session.key_value_width))
        return e;
    if (PlanError e = require_len(inv->key_cache ? inv->key_cache_len : 0, session.cache_elements)) return e;
    if (PlanError e = require_len(inv->value_cache ? inv->value_cache_len : 0, session.cache_elements)) return e;
    if (PlanError e = require_finite(inv->query, inv->query_len)) return e;
    if (PlanError e = require_finite(inv->appended_key, inv->appended_key_len)) return e;
    if (PlanError e = require_finite(inv->appended_value, inv->appended_value_len)) return e;
    if (PlanError e = require_finite(inv->key_cache, prefix_elements)) return e;
    if (PlanError e = require_finite(inv->value_cache, prefix_elements)) return e;
    pvlc_hip_kv_step_operands step{inv->query, inv->query_len, inv->appended_key, inv->appended_key_len,
                                  inv->appended_value, inv->appended_value_len};
    pvlc_hip_kv_step_plan sp{};
    if (PlanError e = plan_step(&session, inv->prefix_tokens, &step, &sp)) return e;
    if (session_out) *session_out = session;
    if (step_out) *step_out = sp;
    return none();
}

// IEEE binary16 round-to-nearest-even, written on the float bit pattern:
// add half an ulp of the target precision (plus the tie-to-even bit) and
// truncate; subnormal results are rounded by the hardware's f32 addition.
uint16_t f32_to_f16_rne(float value) {
    uint32_t x;
    std::memcpy(&x, &value, 4);
    const uint32_t sign = (x >> 16) & 0x8000u;
    uint32_t abs = x & 0x7fffffffu;
    if (abs > 0x7f800000u) return static_cast<uint16_t>(sign | 0x7e00u | ((abs >> 13) & 0x3ffu));  // NaN
    if (abs >= 0x477ff000u) return static_cast<uint16_t>(sign | 0x7c00u);  // >= 65520 rounds to inf
    if (abs < 0x38800000u) {
        // |x| < 2^-14: result is subnormal (or zero).  x + 0.5 aligns the binary
        // point so the f32 addition itself performs the RNE rounding at 2^-24.
        float a;
        std::memcpy(&a, &abs, 4);
        const float shifted = a + 0.5f;
        uint32_t s;
        std::memcpy(&s, &shifted, 4);
        return static_cast<uint16_t>(sign | (s - 0x3f000000u));
    }
    const uint32_t odd = (abs >> 13) & 1u;
    abs += 0xfffu + odd;  // round half to even at bit 13
    return static_cast<uint16_t>(sign | (((abs >> 13) - (112u << 10)) & 0x7fffu));
}

float f16_to_f32(uint16_t bits) {
    const uint32_t sign = static_cast<uint32_t>(bits & 0x8000u) << 16;
    const uint32_t exp = (bits >> 10) & 0x1fu;
    const uint32_t mant = bits & 0x3ffu;
    uint32_t out;
    if (exp == 0) {
        const float mag = static_cast<float>(mant) * 5.9604644775390625e-08f;  // 2^-24
        std::memcpy(&out, &mag, 4);
        out |= sign;
    } else if (exp == 31) {
        out = sign | 0x7f800000u | (mant << 13);
    } else {
        out = sign | ((exp + 112u) << 23) | (mant << 13);
    }
    float f;
    std::memcpy(&f, &out, 4);
    return f;
}

bool fp16_representable(const float *values, size_t n) {
    for (size_t i = 0; i < n; ++i) {
        if (!(std::fabs(values[i]) < 65520.0f)) return false;
    }
    return true;
}

size_t key_blocked_index(uint32_t token, uint32_t head, uint32_t dim) {
    const size_t block = token / kBlockTokens, t = token % kBlockTokens;
    return ((block * kKvHeads + head) * (kHeadDim / 8) + dim / 8) * (kBlockTokens * 8) +
           static_cast<size_t>(key_slot(static_cast<int>(t))) * 8 + dim % 8;
}

size_t value_blocked_index(uint32_t token, uint32_t head, uint32_t dim) {
    const size_t block = token / kBlockTokens, t = token % kBlockTokens;
    return ((block * kKvHeads + head) * kHeadDim + dim) * kBlockTokens + t;
}

DecodeWorkspace decode_workspace_layout(uint32_t num_seqs, uint32_t max_parts) {
    // [error word, padded to 256 B][counters][partial max/sum][partial outputs]
    DecodeWorkspace w{};
    auto align = [](size_t v) { return (v + 255) & ~static_cast<size_t>(255); };
    // An odd number of 4 KiB partial slots per (sequence, kv head): with 16
    // slots (a power-of-two stride) the automatic config-3 step took 52.2 us,
    // with 17 slots 51.5 us.
    w.part_stride = max_parts | 1u;
    const size_t units = static_cast<size_t>(num_seqs) * kKvHeads * w.part_stride;
    w.error_offset = 0;
    w.counters_offset = 256;
    w.part_ml_offset = align(w.counters_offset + static_cast<size_t>(num_seqs) * kKvHeads * sizeof(uint32_t));
    w.part_o_offset = align(w.part_ml_offset + units * 2 * kGroup * sizeof(float));
    w.total = align(w.part_o_offset + units * kGroup * kHeadDim * sizeof(float));
    return w;
}

int plan_gemv_tiled(uint32_t rows, uint32_t columns, pvlc_hip_gemv_tiled_plan *out) {
    // runtime-core lib.rs:746-785
    constexpr uint32_t kTileRows = 8, kThreadsPerRow = 32, kVectorWidth = 4;
    constexpr uint32_t kSharedCapacity = 3072, kStorageBytes = 13312, kMaxDispatch = 65535;
    if (rows == 0 || !(columns == 1024 || columns == 2048 || columns == 3072))
        return invalid(PVLC_HIP_INV_INVALID_DECODER_GEOMETRY,
                       "tiled decoder GEMV geometry " + std::to_string(rows) + "x" + std::to_string(columns) +
                           " is outside the admitted nonzero rows and 1024/2048/3072 input widths");
    const uint32_t dispatch_x = rows / kTileRows + (rows % kTileRows != 0);
    if (dispatch_x > kMaxDispatch)
        return invalid(PVLC_HIP_INV_INVALID_DECODER_GEOMETRY,
                       "tiled decoder GEMV rows " + std::to_string(rows) + " exceed the single-dispatch workgroup bound");
    pvlc_hip_gemv_tiled_plan p{};
    p.tile_rows = kTileRows;
    p.threads_per_row = kThreadsPerRow;
    p.vector_width = kVectorWidth;
    p.shared_capacity = kSharedCapacity;
    p.workgroup_storage_bytes = kStorageBytes;
    p.dispatch[0] = dispatch_x;
    p.dispatch[1] = p.dispatch[2] = 1;
    p.workgroup_size[0] = 256;
    p.workgroup_size[1] = p.workgroup_size[2] = 1;
    p.uniform_words[0] = rows;
    p.uniform_words[1] = columns;
    p.output_elements = rows;
    p.output_bytes = static_cast<uint64_t>(rows) * 4;
    if (out) *out = p;
    return ok();
}

// VisionPatchProjectionBytesDescriptor::plan, runtime-core lib.rs:1768-1840.
int32_t plan_projection(uint32_t patch_count, uint32_t input_width, uint32_t output_width, uint32_t weight_storage,
                        pvlc_hip_projection_plan *out) {
    if (patch_count == 0 || input_width == 0 || output_width == 0) return PVLC_HIP_PROJ_INVALID_GEOMETRY;
    const bool f16 = weight_storage == 1;
    if (f16 && (input_width % 4 != 0 || output_width % 4 != 0)) return PVLC_HIP_PROJ_INVALID_GEOMETRY;
    // u32 x u32 fits in u64; the byte counts are the checked multiplications
    const uint64_t input_elements = static_cast<uint64_t>(patch_count) * input_width;
    const uint64_t weight_elements = static_cast<uint64_t>(output_width) * input_width;
    const uint64_t output_elements = static_cast<uint64_t>(patch_count) * output_width;
    uint64_t input_bytes = 0, weight_bytes = 0, output_bytes = 0;
    if (__builtin_mul_overflow(input_elements, uint64_t{4}, &input_bytes) ||
        __builtin_mul_overflow(weight_elements, uint64_t{f16 ? 2u : 4u}, &weight_bytes) ||
        __builtin_mul_overflow(output_elements, uint64_t{4}, &output_bytes))
        return PVLC_HIP_PROJ_OVERFLOW;
    pvlc_hip_projection_plan p{};
    p.kernel = f16 ? 1u : 0u;
    p.weight_storage = f16 ? 1u : 0u;
    p.input_bytes = input_bytes;
    p.weight_bytes = weight_bytes;
    p.bias_bytes = static_cast<uint64_t>(output_width) * 4;
    p.output_bytes = output_bytes;
    auto ceil_div = [](uint32_t v, uint32_t d) { return v / d + (v % d != 0); };  // lib.rs:5295-5297
    p.dispatch[0] = ceil_div(output_width, 32);
    p.dispatch[1] = ceil_div(patch_count, 32);
    p.dispatch[2] = 1;
    if (out) *out = p;
    return PVLC_HIP_PROJ_OK;
}

DecodeShape decode_shape(uint32_t partition_tokens, bool streaming) {
    const uint32_t tiles = (partition_tokens + kBlockTokens - 1) / kBlockTokens;
    if (streaming) return tiles >= 8 ? DecodeShape{4, 1} : DecodeShape{2, 1};
    // Single shot: the smallest workgroup of 1, 2, 4, 6, 8, 10 or 12 waves
    // holding one pair of tiles each that covers the partition; longer
    // partitions loop over 8 waves.
    if (tiles <= 2) return {1, 1};
    if (tiles <= 4) return {2, 1};
    if (tiles <= 8) return {4, 1};
    if (tiles <= 12) return {6, 1};
    if (tiles <= 16) return {8, 1};
    if (tiles <= 20) return {10, 1};
    if (tiles <= 24) return {12, 1};
    return {8, 1};
}

uint32_t balanced_parts(uint32_t num_seqs) {
    const uint64_t units = static_cast<uint64_t>(num_seqs) * kKvHeads;
    const uint64_t parts = kTargetWorkgroups / units;
    return static_cast<uint32_t>(parts < 1 ? 1 : (parts > kMaxBalancedParts ? kMaxBalancedParts : parts));
}

uint32_t single_shot_partition(uint32_t num_seqs, uint32_t context) {
    // Split every (sequence, kv head) into the same number of partitions so
    // that about one workgroup per compute unit covers the whole step in one
    // round, each partition a whole number of 16-token tiles.
    // Partitions are rounded up to the tile capacity of a single-shot shape
    // (decode_shape), so no wave of a full partition idles; the last
    // partition of each sequence is then the short one.
    const uint32_t tiles = (context + kBlockTokens - 1) / kBlockTokens;
    const uint32_t parts = balanced_parts(num_seqs);
    uint32_t part_tiles = (tiles + parts - 1) / parts;
    static const uint32_t kCapacities[] = {4, 8, 12, 16, 20, 24};  // tiles of the single-shot shapes
    for (uint32_t c : kCapacities) {
        if (part_tiles <= c) return c * kBlockTokens;
    }
    return 0;
}

uint32_t auto_partition(uint32_t num_seqs, uint32_t context) {
    if (const uint32_t p = single_shot_partition(num_seqs, context)) return p;
    // Streaming regime: 512-token partitions, doubled while one merge would
    // combine more than 64 partitions.
    uint32_t p = 512;
    while ((context + p - 1) / p > kMaxMergeParts && p < 4096) p *= 2;
    return p;
}

uint32_t auto_workspace_parts(uint32_t num_seqs, uint32_t max_context) {
    // Any automatic launch with cache lengths up to max_context fits: a
    // single-shot launch uses at most balanced_parts partitions, a streaming
    // launch the partition of max_context.
    const uint32_t p = auto_partition(num_seqs, max_context);
    const uint32_t parts = (max_context + p - 1) / p;
    const uint32_t balanced = balanced_parts(num_seqs);
    return parts > balanced ? parts : balanced;
}

}  // namespace pvlc

using namespace pvlc;

extern "C" {

pvlc_hip_status pvlc_hip_gemv_tiled_plan_create(uint32_t rows, uint32_t columns, pvlc_hip_gemv_tiled_plan *plan_out) {
    if (!plan_out) return invalid(PVLC_HIP_INV_LENGTH_MISMATCH, "plan output is NULL");
    return plan_gemv_tiled(rows, columns, plan_out);
}

int32_t pvlc_hip_projection_plan_create(uint32_t patch_count, uint32_t input_width, uint32_t output_width,
                                        uint32_t weight_storage, pvlc_hip_projection_plan *plan_out) {
    if (weight_storage > 1) return PVLC_HIP_PROJ_INVALID_GEOMETRY;
    return pvlc::plan_projection(patch_count, input_width, output_width, weight_storage, plan_out);
}

int32_t pvlc_hip_projection_validate_capabilities(const pvlc_hip_projection_plan *plan, int32_t shader_f16_available,
                                                  uint32_t max_workgroups_per_dimension) {
    // VisionPatchProjectionBytesPlan::validate_capabilities, lib.rs:1863-1885
    if (!plan) return PVLC_HIP_PROJ_INVALID_GEOMETRY;
    if (plan->weight_storage == 1 && !shader_f16_available) return PVLC_HIP_PROJ_MISSING_SHADER_F16;
    if (max_workgroups_per_dimension == 0 || plan->dispatch[0] > max_workgroups_per_dimension ||
        plan->dispatch[1] > max_workgroups_per_dimension)
        return PVLC_HIP_PROJ_DISPATCH_LIMIT_EXCEEDED;
    return PVLC_HIP_PROJ_OK;
}

int32_t pvlc_hip_projection_validate_operands(const pvlc_hip_projection_plan *plan, const void *input,
                                              size_t input_bytes, const void *weight, size_t weight_bytes,
                                              const void *bias, size_t bias_bytes) {
    // VisionPatchProjectionBytesPlan::validate_operands, lib.rs:1887-1913:
    // every length first (input, weight, bias), then finiteness in the same order
    if (!plan) return PVLC_HIP_PROJ_INVALID_GEOMETRY;
    if (input_bytes != plan->input_bytes || weight_bytes != plan->weight_bytes || bias_bytes != plan->bias_bytes)
        return PVLC_HIP_PROJ_LENGTH_MISMATCH;
    if ((input_bytes && !input) || (weight_bytes && !weight) || (bias_bytes && !bias))
        return PVLC_HIP_PROJ_LENGTH_MISMATCH;
    auto finite_f32 = [](const void *bytes, size_t n) {
        const unsigned char *b = static_cast<const unsigned char *>(bytes);
        for (size_t i = 0; i + 4 <= n; i += 4) {
            uint32_t v;
            std::memcpy(&v, b + i, 4);
            if ((v & 0x7f800000u) == 0x7f800000u) return false;
        }
        return true;
    };
    auto finite_f16 = [](const void *bytes, size_t n) {
        const unsigned char *b = static_cast<const unsigned char *>(bytes);
        for (size_t i = 0; i + 2 <= n; i += 2) {
            uint16_t v;
            std::memcpy(&v, b + i, 2);
            if ((v & 0x7c00u) == 0x7c00u) return false;
        }
        return true;
    };
    if (!finite_f32(input, input_bytes)) return PVLC_HIP_PROJ_NON_FINITE;
    if (plan->weight_storage == 1 ? !finite_f16(weight, weight_bytes) : !finite_f32(weight, weight_bytes))
        return PVLC_HIP_PROJ_NON_FINITE;
    if (!finite_f32(bias, bias_bytes)) return PVLC_HIP_PROJ_NON_FINITE;
    return PVLC_HIP_PROJ_OK;
}

const char *pvlc_hip_last_error_message(void) { return g_last_error.c_str(); }

pvlc_hip_status pvlc_hip_kv_session_plan_create(const pvlc_hip_kv_session_descriptor *descriptor,
                                                pvlc_hip_kv_session_plan *plan_out) {
    if (!descriptor) return invalid(PVLC_HIP_INV_LENGTH_MISMATCH, "descriptor is NULL");
    if (PlanError e = plan_descriptor(descriptor, plan_out)) return invalid(e.code, e.message);
    return ok();
}

pvlc_hip_status pvlc_hip_kv_session_plan_step(const pvlc_hip_kv_session_plan *plan, uint32_t cache_tokens,
                                              const pvlc_hip_kv_step_operands *step,
                                              pvlc_hip_kv_step_plan *step_plan_out) {
    if (!plan) return invalid(PVLC_HIP_INV_LENGTH_MISMATCH, "plan is NULL");
    if (PlanError e = plan_step(plan, cache_tokens, step, step_plan_out)) return invalid(e.code, e.message);
    return ok();
}

pvlc_hip_status pvlc_hip_gqa_split_plan_create(uint32_t cache_tokens, uint32_t query_heads,
                                               uint32_t key_value_heads, uint32_t head_dim,
                                               pvlc_hip_gqa_split_plan *plan_out) {
    if (PlanError e = plan_split(cache_tokens, query_heads, key_value_heads, head_dim, plan_out))
        return invalid(e.code, e.message);
    return ok();
}

pvlc_hip_status pvlc_hip_prefill_plan_check(uint32_t tokens, uint32_t cache_capacity) {
    if (tokens == 0 || tokens > cache_capacity) {
        return invalid(PVLC_HIP_INV_INVALID_DECODER_GEOMETRY,
                       "decoder stack prefill token count " + std::to_string(tokens) + " is outside 1..=" +
                           std::to_string(cache_capacity));
    }
    return ok();
}

void pvlc_hip_f32_to_f16_host(const float *in, uint16_t *out, size_t n) {
    for (size_t i = 0; i < n; ++i) out[i] = f32_to_f16_rne(in[i]);
}

void pvlc_hip_f16_to_f32_host(const uint16_t *in, float *out, size_t n) {
    for (size_t i = 0; i < n; ++i) out[i] = f16_to_f32(in[i]);
}

pvlc_hip_status pvlc_hip_rope_table_f32(float base, uint32_t rotary_dim, uint32_t rows, float *cos_out,
                                        float *sin_out) {
    if (rotary_dim == 0 || rotary_dim % 2 != 0)
        return invalid(PVLC_HIP_INV_INVALID_ROTARY_DIMENSION, "rotary dimension must be nonzero and even");
    if (!std::isfinite(base) || base <= 0.0f)
        return invalid(PVLC_HIP_INV_INVALID_ROPE_BASE, "RoPE base must be positive and finite");
    if (!cos_out || !sin_out) return invalid(PVLC_HIP_INV_LENGTH_MISMATCH, "table pointers are NULL");
    const uint32_t half = rotary_dim / 2;
    for (uint32_t pair = 0; pair < half; ++pair) {
        // apply_rope_neox, cpu-ref lib.rs:459-461, in f32 with the host libm.
        const float exponent = -((2.0f * static_cast<float>(pair)) / static_cast<float>(rotary_dim));
        const float inv_freq = powf(base, exponent);
        for (uint32_t pos = 0; pos < rows; ++pos) {
            const float angle = static_cast<float>(pos) * inv_freq;
            cos_out[static_cast<size_t>(pos) * half + pair] = cosf(angle);
            sin_out[static_cast<size_t>(pos) * half + pair] = sinf(angle);
        }
    }
    return ok();
}

pvlc_hip_status pvlc_hip_mrope_table_f32(const float *raw_cos, const float *raw_sin, uint32_t capacity,
                                         uint32_t section_t, uint32_t section_h, uint32_t section_w, float *cos_out,
                                         float *sin_out) {
    // Section selection of apply_multimodal_rope_f32 (cpu-ref lib.rs:562-672) and decoder_mrope_f32 /
    // decoder_prefill_mrope_f32 (wgsl lib.rs:1185-1234, 1334-1380): frequency pair f of a slot reads axis
    // 0 (temporal) for f < section_t, 1 (height) below section_t + section_h, else 2 (width); the raw tables
    // are [3][capacity][128] and the device rotation reads one cos/sin per pair, so every raw row must
    // repeat its first half (as cat(freqs, freqs) tables do).
    constexpr uint32_t kDim = 128, kHalf = 64;
    if (!raw_cos || !raw_sin || !cos_out || !sin_out)
        return invalid(PVLC_HIP_INV_LENGTH_MISMATCH, "M-RoPE table pointers are NULL");
    if (capacity == 0 || section_t == 0 || section_h == 0 || section_w == 0)
        return invalid(PVLC_HIP_INV_ZERO_DIMENSION, "M-RoPE capacity and sections must be nonzero");
    if (static_cast<uint64_t>(section_t) + section_h + section_w != kHalf)
        return invalid(PVLC_HIP_INV_INVALID_ROTARY_DIMENSION, "M-RoPE sections must sum to head_dim / 2 = 64");
    const size_t n = static_cast<size_t>(3) * capacity * kDim;
    for (size_t i = 0; i < n; ++i)
        if (!std::isfinite(raw_cos[i]) || !std::isfinite(raw_sin[i]))
            return invalid(PVLC_HIP_INV_NON_FINITE_INPUT, "M-RoPE tables contain NaN or infinity");
    for (size_t row = 0; row < static_cast<size_t>(3) * capacity; ++row)
        if (std::memcmp(raw_cos + row * kDim, raw_cos + row * kDim + kHalf, kHalf * sizeof(float)) != 0 ||
            std::memcmp(raw_sin + row * kDim, raw_sin + row * kDim + kHalf, kHalf * sizeof(float)) != 0)
            return invalid(PVLC_HIP_INV_INVALID_ROTARY_DIMENSION,
                           "M-RoPE table row " + std::to_string(row) + " does not repeat its first half");
    for (uint32_t slot = 0; slot < capacity; ++slot)
        for (uint32_t f = 0; f < kHalf; ++f) {
            const uint32_t axis = f < section_t ? 0u : (f < section_t + section_h ? 1u : 2u);
            const size_t src = (static_cast<size_t>(axis) * capacity + slot) * kDim + f;
            cos_out[static_cast<size_t>(slot) * kHalf + f] = raw_cos[src];
            sin_out[static_cast<size_t>(slot) * kHalf + f] = raw_sin[src];
        }
    return ok();
}

}  // extern "C"
