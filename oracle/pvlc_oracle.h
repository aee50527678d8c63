/*
 * CPU oracle for the PaddleOCR-VL decoder KV-cache hot path.
 *
 * TEST INFRASTRUCTURE, NOT PRODUCT CODE.  Only tests/, __graft_entry__.smoke()
 * and bench.py's cpu_baseline leg may load this library, and only as the
 * checker (or as the timed CPU baseline).  The HIP product path never links it.
 *
 * Every compute function restates a function of crates/pvlc-cpu-ref/src/lib.rs
 * (glebkudr/paddleocr-vl-webgpu) with the same loop order and f32 arithmetic:
 * built with -O2 -ffp-contract=off and no fast-math, using glibc expf/powf/
 * sinf/cosf/sqrtf, so every rounding step matches the Rust original.
 *
 * Pinning (how each function is checked, see tests/test_oracle.py):
 *   oracle_decode_gqa_f32   reference digest DIRECT_BOUNDARY_BLAKE3, bounded
 *                           extreme [1.0, 3.0], physical-repeat equality,
 *                           wrong-grouping / missing-scale sensitivity, f64
 *                           softmax closed form.
 *   oracle_causal_gqa_f32   reference digest COMPACT_BLAKE3, row i == decode over
 *                           i+1 tokens (bit-exact), future-poison immunity.
 *   oracle_append_kv_f32    closed form (concatenation), prefix untouched.
 *   oracle_rope_neox_f32    reference closed form at base 500000 / position 17,
 *                           position 0 identity, pair norm preservation.
 *   oracle_mrope_f32        equal-axis M-RoPE == NeoX RoPE bit-exact; section
 *                           selection checked against a brute-force table.
 *   oracle_f32_to_f16       exhaustive comparison with numpy's RNE float16 cast.
 *   oracle_blake3           BLAKE3 specification test vectors, model-lock digests.
 *   oracle_linear_f32       the reference's known answer (vision_contract.rs:433-441),
 *                           its error cases (:444-470), exact small-integer
 *                           products against numpy, an f64 bound.
 *   oracle_top1_f32         an independent numeric comparator (value, sign of
 *                           zero, lowest index) on finite logits, brute force;
 *                           NaN/inf/signed-zero orderings worked by hand.
 */
#ifndef PVLC_ORACLE_H
#define PVLC_ORACLE_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* Mirrors CpuRefErrorCode (crates/pvlc-cpu-ref/src/lib.rs:16-30); 0 = Ok. */
enum {
    ORACLE_OK = 0,
    ORACLE_DIMENSION_MISMATCH = 1,
    ORACLE_NON_POSITIVE_EPSILON = 2,
    ORACLE_ALL_MASKED = 3,
    ORACLE_INVALID_ROTARY_DIMENSION = 4,
    ORACLE_INVALID_ROPE_BASE = 5,
    ORACLE_INVALID_K = 6,
    ORACLE_NON_FINITE_INPUT = 7,
};

/* decode_gqa_f32, lib.rs:858-927.  out has query_heads*head_dim floats. */
int oracle_decode_gqa_f32(const float *query, size_t query_len, const float *key, size_t key_len,
                          const float *value, size_t value_len, size_t cache_tokens, size_t query_heads,
                          size_t key_value_heads, size_t head_dim, float *out);

/* causal_gqa_f32, lib.rs:782-853.  out has tokens*query_heads*head_dim floats. */
int oracle_causal_gqa_f32(const float *query, size_t query_len, const float *key, size_t key_len,
                          const float *value, size_t value_len, size_t tokens, size_t query_heads,
                          size_t key_value_heads, size_t head_dim, float *out);

/* linear_f32 = patch_projection_f32 with patch_size 1, lib.rs:88-128, 131-140:
 * out[r][o] = bias[o] + sum_i input[r][i] * weights[o][i], accumulated in
 * input order from the bias.  weights are output-major [output_width][input_width]. */
int oracle_linear_f32(const float *input, size_t input_len, size_t rows, size_t input_width,
                      const float *weights, size_t weights_len, const float *bias, size_t bias_len,
                      size_t output_width, float *out);

/* decoder_logits_top1_f32 (pvlc-runtime-web decoder_stack_session.rs:308-366)
 * and its host twin top1FromLogitsBytes (web/engine/greedy_generation.mjs:43-79)
 * without the host's finite check: the index of the largest logit under the
 * f32 total order key bits ^ ((u32)(bits >> 31) >> 1), ties to the lowest
 * index; value_bits = the f32 bits of that logit.  n = 0 is a dimension error. */
int oracle_top1_f32(const float *logits, size_t n, uint32_t *index, uint32_t *value_bits);

/* append_decoder_kv_cache, lib.rs:1420-1450: out = prefix rows || one new row. */
int oracle_append_kv_f32(const float *prefix_keys, const float *prefix_values, size_t prefix_tokens,
                         const float *rotated_key, size_t rotated_key_len, const float *value,
                         size_t value_len, size_t key_value_heads, size_t head_dim, float *out_keys,
                         float *out_values);

/* write_decoder_prefill_kv_f32, lib.rs:976-992 (validated clone of the rows). */
int oracle_write_prefill_kv_f32(const float *rotated_key, size_t key_len, const float *value,
                                size_t value_len, size_t tokens, size_t key_value_heads, size_t head_dim,
                                float *out_keys, float *out_values);

/* apply_rope_neox, lib.rs:425-467 (in place). */
int oracle_rope_neox_f32(float *values, size_t values_len, size_t rows, size_t width, size_t rotary_dim,
                         const uint32_t *positions, size_t positions_len, float base);

/* apply_multimodal_rope_f32, lib.rs:562-672.  raw tables are [3, tokens, head_dim]. */
int oracle_mrope_f32(const float *query, size_t query_len, const float *key, size_t key_len, size_t tokens,
                     size_t query_heads, size_t key_value_heads, size_t head_dim, const float *raw_cos,
                     const float *raw_sin, size_t raw_len, const size_t sections[3], float *rotated_query,
                     float *rotated_key);

/* Physically repeated KV oracle of the reference tests
 * (crates/pvlc-cpu-ref/tests/decoder_decode_contract.rs:316-419). */
void oracle_independent_decode_gqa_f32(const float *query, const float *key, const float *value,
                                       size_t cache_tokens, size_t query_heads, size_t key_value_heads,
                                       size_t head_dim, float scale, int rotate_groups, float *out);

/* Replace expf(x) by a fixed result at exact arguments (bit patterns); n = 0
 * restores glibc expf everywhere.  Used only to reproduce a digest that was
 * computed with another platform's libm.  The tables must outlive the calls. */
void oracle_set_expf_overrides(const uint32_t *arg_bits, const uint32_t *result_bits, size_t n);

/* IEEE binary16 conversions: round-to-nearest-even narrowing, exact widening. */
uint16_t oracle_f32_to_f16(float value);
float oracle_f16_to_f32(uint16_t bits);
void oracle_f32_to_f16_array(const float *in, uint16_t *out, size_t n);
void oracle_f16_to_f32_array(const uint16_t *in, float *out, size_t n);

/* Seeded N(0,1) inputs: splitmix64 -> 53-bit uniforms -> Box-Muller in f64 ->
 * f32, then multiplied by `scale` in f32 and rounded to fp16 (RNE). */
void oracle_normal_f16(uint64_t seed, float scale, uint16_t *out, size_t n);
void oracle_normal_f32(uint64_t seed, float *out, size_t n);

/* BLAKE3 of a byte string (32-byte digest). */
void oracle_blake3(const uint8_t *input, size_t len, uint8_t out[32]);

#ifdef __cplusplus
}
#endif

#endif
