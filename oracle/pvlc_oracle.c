/*
 * CPU oracle: C restatement of the decoder KV-cache hot path of
 * crates/pvlc-cpu-ref/src/lib.rs (glebkudr/paddleocr-vl-webgpu).
 *
 * TEST INFRASTRUCTURE, NOT PRODUCT CODE (see pvlc_oracle.h for the rules and
 * for how each function is pinned).  Build flags: -O2 -ffp-contract=off, no
 * fast-math, so `a += b * c` is a rounded product followed by a rounded sum,
 * exactly like Rust's f32 arithmetic (Rust never contracts to FMA).
 */
#include "pvlc_oracle.h"

#include <math.h>
#include <stdlib.h>
#include <string.h>

/* Optional table of exp(x) results that replace glibc's expf at given exact
 * arguments.  Empty by default (pure glibc).  The reference's digest
 * DIRECT_BOUNDARY_BLAKE3 was produced by a platform libm whose expf returns the
 * other neighbour at three arguments that lie ~0.49 ulp from a rounding
 * midpoint; the digest test installs exactly those three values. */
static const uint32_t *g_exp_arg_bits;
static const uint32_t *g_exp_result_bits;
static size_t g_exp_overrides;

void oracle_set_expf_overrides(const uint32_t *arg_bits, const uint32_t *result_bits, size_t n) {
    g_exp_arg_bits = arg_bits;
    g_exp_result_bits = result_bits;
    g_exp_overrides = n;
}

static float oracle_expf(float x) {
    if (g_exp_overrides) {
        uint32_t bits;
        memcpy(&bits, &x, sizeof(bits));
        for (size_t i = 0; i < g_exp_overrides; ++i) {
            if (g_exp_arg_bits[i] == bits) {
                float r;
                memcpy(&r, &g_exp_result_bits[i], sizeof(r));
                return r;
            }
        }
    }
    return expf(x);
}

/* require_finite, lib.rs:3452-3460 */
static int all_finite(const float *values, size_t n) {
    for (size_t i = 0; i < n; ++i) {
        if (!isfinite(values[i])) return 0;
    }
    return 1;
}

/* checked_mul of the Rust original: 0 on overflow. */
static int checked_mul(size_t a, size_t b, size_t *out) {
    if (a != 0 && b > SIZE_MAX / a) return 0;
    *out = a * b;
    return 1;
}

/* require_len, lib.rs:3434-3440 */
static int require_len(size_t actual, size_t rows, size_t columns) {
    size_t expected;
    if (!checked_mul(rows, columns, &expected)) return ORACLE_DIMENSION_MISMATCH;
    return actual == expected ? ORACLE_OK : ORACLE_DIMENSION_MISMATCH;
}

/* attention_index, lib.rs:3424-3432 */
static size_t attention_index(size_t token, size_t head, size_t dim, size_t heads, size_t head_dim) {
    return (token * heads + head) * head_dim + dim;
}

/* validate_gqa_geometry, lib.rs:696-724 (query_rows = tokens) and
 * validate_decode_gqa_geometry, lib.rs:726-754 (query_rows = 1). */
static int validate_attention(size_t query_len, size_t key_len, size_t value_len, size_t query_rows,
                              size_t kv_rows, size_t query_heads, size_t key_value_heads, size_t head_dim,
                              const float *query, const float *key, const float *value) {
    if (kv_rows == 0 || query_heads == 0 || key_value_heads == 0 || head_dim == 0)
        return ORACLE_DIMENSION_MISMATCH;
    if (query_heads % key_value_heads != 0) return ORACLE_DIMENSION_MISMATCH;
    size_t query_width, kv_width;
    if (!checked_mul(query_heads, head_dim, &query_width)) return ORACLE_DIMENSION_MISMATCH;
    if (!checked_mul(key_value_heads, head_dim, &kv_width)) return ORACLE_DIMENSION_MISMATCH;
    int rc;
    if ((rc = require_len(query_len, query_rows, query_width)) != ORACLE_OK) return rc;
    if ((rc = require_len(key_len, kv_rows, kv_width)) != ORACLE_OK) return rc;
    if ((rc = require_len(value_len, kv_rows, kv_width)) != ORACLE_OK) return rc;
    if (!all_finite(query, query_len) || !all_finite(key, key_len) || !all_finite(value, value_len))
        return ORACLE_NON_FINITE_INPUT;
    return ORACLE_OK;
}

/* One (query row, query head) of decode_gqa_f32 / causal_gqa_f32: scores in
 * key order with a sequential dot, max fold, exp and running sum, division,
 * then the dim-outer / token-inner weighted sum (lib.rs:880-924, :806-850). */
static void attend_row(const float *q_row, const float *key, const float *value, size_t keys,
                       size_t key_value_head, size_t key_value_heads, size_t head_dim, float scale,
                       float *probabilities, float *out_row) {
    for (size_t t = 0; t < keys; ++t) {
        float score = 0.0f;
        for (size_t d = 0; d < head_dim; ++d) {
            score += q_row[d] * key[attention_index(t, key_value_head, d, key_value_heads, head_dim)];
        }
        probabilities[t] = score * scale;
    }
    float maximum = -INFINITY;
    for (size_t t = 0; t < keys; ++t) maximum = fmaxf(maximum, probabilities[t]);
    float denominator = 0.0f;
    for (size_t t = 0; t < keys; ++t) {
        probabilities[t] = oracle_expf(probabilities[t] - maximum);
        denominator += probabilities[t];
    }
    for (size_t t = 0; t < keys; ++t) probabilities[t] /= denominator;
    for (size_t d = 0; d < head_dim; ++d) {
        float weighted = 0.0f;
        for (size_t t = 0; t < keys; ++t) {
            weighted += probabilities[t] * value[attention_index(t, key_value_head, d, key_value_heads, head_dim)];
        }
        out_row[d] = weighted;
    }
}

int oracle_decode_gqa_f32(const float *query, size_t query_len, const float *key, size_t key_len,
                          const float *value, size_t value_len, size_t cache_tokens, size_t query_heads,
                          size_t key_value_heads, size_t head_dim, float *out) {
    int rc = validate_attention(query_len, key_len, value_len, 1, cache_tokens, query_heads, key_value_heads,
                                head_dim, query, key, value);
    if (rc != ORACLE_OK) return rc;
    const size_t group = query_heads / key_value_heads;
    /* (head_dim as f32).sqrt().recip(), lib.rs:878 */
    const float scale = 1.0f / sqrtf((float)head_dim);
    float *probabilities = (float *)malloc(cache_tokens * sizeof(float));
    if (!probabilities) return ORACLE_DIMENSION_MISMATCH;
    for (size_t h = 0; h < query_heads; ++h) {
        attend_row(query + h * head_dim, key, value, cache_tokens, h / group, key_value_heads, head_dim, scale,
                   probabilities, out + h * head_dim);
    }
    free(probabilities);
    return ORACLE_OK;
}

int oracle_causal_gqa_f32(const float *query, size_t query_len, const float *key, size_t key_len,
                          const float *value, size_t value_len, size_t tokens, size_t query_heads,
                          size_t key_value_heads, size_t head_dim, float *out) {
    int rc = validate_attention(query_len, key_len, value_len, tokens, tokens, query_heads, key_value_heads,
                                head_dim, query, key, value);
    if (rc != ORACLE_OK) return rc;
    const size_t group = query_heads / key_value_heads;
    const float scale = 1.0f / sqrtf((float)head_dim);
    const size_t query_width = query_heads * head_dim;
    float *probabilities = (float *)malloc(tokens * sizeof(float));
    if (!probabilities) return ORACLE_DIMENSION_MISMATCH;
    for (size_t qt = 0; qt < tokens; ++qt) {
        for (size_t h = 0; h < query_heads; ++h) {
            attend_row(query + attention_index(qt, h, 0, query_heads, head_dim), key, value, qt + 1, h / group,
                       key_value_heads, head_dim, scale, probabilities, out + qt * query_width + h * head_dim);
        }
    }
    free(probabilities);
    return ORACLE_OK;
}

/* validate_kv_geometry, lib.rs:756-774 */
static int validate_kv(const float *key, size_t key_len, const float *value, size_t value_len, size_t tokens,
                       size_t key_value_heads, size_t head_dim) {
    if (tokens == 0 || key_value_heads == 0 || head_dim == 0) return ORACLE_DIMENSION_MISMATCH;
    size_t width;
    if (!checked_mul(key_value_heads, head_dim, &width)) return ORACLE_DIMENSION_MISMATCH;
    int rc;
    if ((rc = require_len(key_len, tokens, width)) != ORACLE_OK) return rc;
    if ((rc = require_len(value_len, tokens, width)) != ORACLE_OK) return rc;
    if (!all_finite(key, key_len) || !all_finite(value, value_len)) return ORACLE_NON_FINITE_INPUT;
    return ORACLE_OK;
}

int oracle_append_kv_f32(const float *prefix_keys, const float *prefix_values, size_t prefix_tokens,
                         const float *rotated_key, size_t rotated_key_len, const float *value,
                         size_t value_len, size_t key_value_heads, size_t head_dim, float *out_keys,
                         float *out_values) {
    int rc = validate_kv(rotated_key, rotated_key_len, value, value_len, 1, key_value_heads, head_dim);
    if (rc != ORACLE_OK) return rc;
    size_t width = key_value_heads * head_dim, prefix_elements;
    if (!checked_mul(prefix_tokens, width, &prefix_elements)) return ORACLE_DIMENSION_MISMATCH;
    /* keys = prefix.keys ++ rotated_key; values = prefix.values ++ value (lib.rs:1437-1442) */
    memcpy(out_keys, prefix_keys, prefix_elements * sizeof(float));
    memcpy(out_keys + prefix_elements, rotated_key, width * sizeof(float));
    memcpy(out_values, prefix_values, prefix_elements * sizeof(float));
    memcpy(out_values + prefix_elements, value, width * sizeof(float));
    return ORACLE_OK;
}

int oracle_linear_f32(const float *input, size_t input_len, size_t rows, size_t input_width,
                      const float *weights, size_t weights_len, const float *bias, size_t bias_len,
                      size_t output_width, float *out) {
    /* patch_projection_f32 validation order (lib.rs:97-111), patch_size 1 */
    if (rows == 0 || input_width == 0 || output_width == 0) return ORACLE_DIMENSION_MISMATCH;
    int rc = require_len(input_len, rows, input_width);
    if (rc != ORACLE_OK) return rc;
    rc = require_len(weights_len, output_width, input_width);
    if (rc != ORACLE_OK) return rc;
    if (bias_len != output_width) return ORACLE_DIMENSION_MISMATCH;
    if (!all_finite(input, input_len) || !all_finite(weights, weights_len) || !all_finite(bias, bias_len))
        return ORACLE_NON_FINITE_INPUT;
    size_t out_len;
    if (!checked_mul(rows, output_width, &out_len)) return ORACLE_DIMENSION_MISMATCH;
    /* lib.rs:117-126: accumulator starts at the bias, += input * coefficient in order */
    for (size_t r = 0; r < rows; ++r) {
        const float *patch = input + r * input_width;
        for (size_t o = 0; o < output_width; ++o) {
            const float *w = weights + o * input_width;
            float accumulator = bias[o];
            for (size_t i = 0; i < input_width; ++i) accumulator += patch[i] * w[i];
            out[r * output_width + o] = accumulator;
        }
    }
    return ORACLE_OK;
}

/* decoder_stack_session.rs:318-321: signed-integer key of an f32 that orders
 * -NaN < -inf < ... < -0 < +0 < ... < +inf < +NaN. */
static int32_t total_order_key(float value) {
    int32_t bits;
    memcpy(&bits, &value, sizeof bits);
    return bits ^ (int32_t)((uint32_t)(bits >> 31) >> 1);
}

int oracle_top1_f32(const float *logits, size_t n, uint32_t *index, uint32_t *value_bits) {
    if (n == 0) return ORACLE_DIMENSION_MISMATCH;
    /* :323-328, :339-346: a candidate replaces the best on a larger key, or an
     * equal key at a lower index; a scan in index order keeps the first of the
     * equal keys, which is the order-independent answer of the tree reduction
     * (:352-366). */
    size_t best = 0;
    int32_t best_key = total_order_key(logits[0]);
    for (size_t i = 1; i < n; ++i) {
        int32_t key = total_order_key(logits[i]);
        if (key > best_key) {
            best_key = key;
            best = i;
        }
    }
    *index = (uint32_t)best;
    memcpy(value_bits, &logits[best], sizeof *value_bits);
    return ORACLE_OK;
}

int oracle_write_prefill_kv_f32(const float *rotated_key, size_t key_len, const float *value,
                                size_t value_len, size_t tokens, size_t key_value_heads, size_t head_dim,
                                float *out_keys, float *out_values) {
    int rc = validate_kv(rotated_key, key_len, value, value_len, tokens, key_value_heads, head_dim);
    if (rc != ORACLE_OK) return rc;
    memcpy(out_keys, rotated_key, key_len * sizeof(float));
    memcpy(out_values, value, value_len * sizeof(float));
    return ORACLE_OK;
}

int oracle_rope_neox_f32(float *values, size_t values_len, size_t rows, size_t width, size_t rotary_dim,
                         const uint32_t *positions, size_t positions_len, float base) {
    int rc = require_len(values_len, rows, width);
    if (rc != ORACLE_OK) return rc;
    if (positions_len != rows) return ORACLE_DIMENSION_MISMATCH;
    if (rotary_dim == 0 || rotary_dim > width || rotary_dim % 2 != 0) return ORACLE_INVALID_ROTARY_DIMENSION;
    if (!isfinite(base) || base <= 0.0f) return ORACLE_INVALID_ROPE_BASE;
    if (!all_finite(values, values_len)) return ORACLE_NON_FINITE_INPUT;
    const size_t half = rotary_dim / 2;
    for (size_t row = 0; row < rows; ++row) {
        const size_t row_start = row * width;
        for (size_t pair = 0; pair < half; ++pair) {
            const size_t first_index = row_start + pair;
            const size_t second_index = row_start + half + pair;
            const float first = values[first_index];
            const float second = values[second_index];
            /* -(2.0 * pair as f32 / rotary_dim as f32), lib.rs:459 */
            const float exponent = -((2.0f * (float)pair) / (float)rotary_dim);
            const float angle = (float)positions[row] * powf(base, exponent);
            const float sine = sinf(angle);
            const float cosine = cosf(angle);
            values[first_index] = first * cosine - second * sine;
            values[second_index] = second * cosine + first * sine;
        }
    }
    return ORACLE_OK;
}

int oracle_mrope_f32(const float *query, size_t query_len, const float *key, size_t key_len, size_t tokens,
                     size_t query_heads, size_t key_value_heads, size_t head_dim, const float *raw_cos,
                     const float *raw_sin, size_t raw_len, const size_t sections[3], float *rotated_query,
                     float *rotated_key) {
    if (tokens == 0 || query_heads == 0 || key_value_heads == 0 || head_dim == 0)
        return ORACLE_DIMENSION_MISMATCH;
    if (query_heads % key_value_heads != 0) return ORACLE_DIMENSION_MISMATCH;
    if (sections[0] == 0 || sections[1] == 0 || sections[2] == 0) return ORACLE_DIMENSION_MISMATCH;
    if (sections[0] + sections[1] + sections[2] != head_dim / 2 || head_dim % 2 != 0)
        return ORACLE_DIMENSION_MISMATCH;
    size_t query_width = query_heads * head_dim, key_width = key_value_heads * head_dim;
    int rc;
    if ((rc = require_len(query_len, tokens, query_width)) != ORACLE_OK) return rc;
    if ((rc = require_len(key_len, tokens, key_width)) != ORACLE_OK) return rc;
    if (raw_len != 3 * tokens * head_dim) return ORACLE_DIMENSION_MISMATCH;
    if (!all_finite(query, query_len) || !all_finite(key, key_len) || !all_finite(raw_cos, raw_len) ||
        !all_finite(raw_sin, raw_len))
        return ORACLE_NON_FINITE_INPUT;

    const size_t repeated[6] = {sections[0], sections[1], sections[2], sections[0], sections[1], sections[2]};
    const size_t half_dim = head_dim / 2;
    float *selected_cos = (float *)malloc(head_dim * sizeof(float));
    float *selected_sin = (float *)malloc(head_dim * sizeof(float));
    if (!selected_cos || !selected_sin) {
        free(selected_cos);
        free(selected_sin);
        return ORACLE_DIMENSION_MISMATCH;
    }
    for (size_t token = 0; token < tokens; ++token) {
        /* Section selection, lib.rs:623-643: chunk i takes axis i % 3. */
        size_t offset = 0;
        for (size_t chunk = 0; chunk < 6; ++chunk) {
            const size_t axis = chunk % 3;
            const size_t axis_base = axis * tokens * head_dim + token * head_dim + offset;
            memcpy(selected_cos + offset, raw_cos + axis_base, repeated[chunk] * sizeof(float));
            memcpy(selected_sin + offset, raw_sin + axis_base, repeated[chunk] * sizeof(float));
            offset += repeated[chunk];
        }
        /* Rotate-half, lib.rs:645-670 */
        for (size_t head = 0; head < query_heads; ++head) {
            const size_t row = attention_index(token, head, 0, query_heads, head_dim);
            for (size_t d = 0; d < head_dim; ++d) {
                const float source = d < half_dim ? -query[row + d + half_dim] : query[row + d - half_dim];
                rotated_query[row + d] = query[row + d] * selected_cos[d] + source * selected_sin[d];
            }
        }
        for (size_t head = 0; head < key_value_heads; ++head) {
            const size_t row = attention_index(token, head, 0, key_value_heads, head_dim);
            for (size_t d = 0; d < head_dim; ++d) {
                const float source = d < half_dim ? -key[row + d + half_dim] : key[row + d - half_dim];
                rotated_key[row + d] = key[row + d] * selected_cos[d] + source * selected_sin[d];
            }
        }
    }
    free(selected_cos);
    free(selected_sin);
    return ORACLE_OK;
}

void oracle_independent_decode_gqa_f32(const float *query, const float *key, const float *value,
                                       size_t cache_tokens, size_t query_heads, size_t key_value_heads,
                                       size_t head_dim, float scale, int rotate_groups, float *out) {
    /* repeat_kv_heads_contiguously / _with_rotated_groups then
     * direct_decode_from_repeated_kv (decoder_decode_contract.rs:316-395). */
    const size_t group = query_heads / key_value_heads;
    float *rk = (float *)malloc(cache_tokens * query_heads * head_dim * sizeof(float));
    float *rv = (float *)malloc(cache_tokens * query_heads * head_dim * sizeof(float));
    float *logits = (float *)malloc((cache_tokens ? cache_tokens : 1) * sizeof(float));
    size_t w = 0;
    for (size_t t = 0; t < cache_tokens; ++t) {
        for (size_t kvh = 0; kvh < key_value_heads; ++kvh) {
            size_t src_head = rotate_groups ? (kvh + 1) % key_value_heads : kvh;
            size_t start = attention_index(t, src_head, 0, key_value_heads, head_dim);
            for (size_t r = 0; r < group; ++r) {
                memcpy(rk + w, key + start, head_dim * sizeof(float));
                memcpy(rv + w, value + start, head_dim * sizeof(float));
                w += head_dim;
            }
        }
    }
    for (size_t h = 0; h < query_heads; ++h) {
        for (size_t t = 0; t < cache_tokens; ++t) {
            float dot = 0.0f;
            for (size_t d = 0; d < head_dim; ++d)
                dot += query[h * head_dim + d] * rk[attention_index(t, h, d, query_heads, head_dim)];
            logits[t] = dot * scale;
        }
        float maximum = -INFINITY;
        for (size_t t = 0; t < cache_tokens; ++t) maximum = fmaxf(maximum, logits[t]);
        for (size_t t = 0; t < cache_tokens; ++t) logits[t] = oracle_expf(logits[t] - maximum);
        /* Rust's f32 Sum folds from -0.0; identical to 0.0 for these positive terms. */
        float denominator = -0.0f;
        for (size_t t = 0; t < cache_tokens; ++t) denominator += logits[t];
        for (size_t t = 0; t < cache_tokens; ++t) logits[t] /= denominator;
        for (size_t d = 0; d < head_dim; ++d) {
            float weighted = 0.0f;
            for (size_t t = 0; t < cache_tokens; ++t)
                weighted += logits[t] * rv[attention_index(t, h, d, query_heads, head_dim)];
            out[h * head_dim + d] = weighted;
        }
    }
    free(rk);
    free(rv);
    free(logits);
}

uint16_t oracle_f32_to_f16(float value) {
    uint32_t x;
    memcpy(&x, &value, sizeof(x));
    const uint32_t sign = (x >> 16) & 0x8000u;
    const uint32_t exponent = (x >> 23) & 0xffu;
    uint32_t mantissa = x & 0x7fffffu;
    if (exponent == 0xffu) {
        if (mantissa == 0) return (uint16_t)(sign | 0x7c00u);
        return (uint16_t)(sign | 0x7e00u | (mantissa >> 13));
    }
    const int e = (int)exponent - 127 + 15;
    if (e >= 31) return (uint16_t)(sign | 0x7c00u);
    if (e <= 0) {
        if (e < -10) return (uint16_t)sign;
        const uint32_t full = mantissa | 0x800000u;
        const uint32_t shift = (uint32_t)(14 - e);
        uint32_t m = full >> shift;
        const uint32_t rem = full & ((1u << shift) - 1u);
        const uint32_t halfway = 1u << (shift - 1u);
        if (rem > halfway || (rem == halfway && (m & 1u))) ++m;
        return (uint16_t)(sign | m);
    }
    uint32_t h = ((uint32_t)e << 10) | (mantissa >> 13);
    const uint32_t rem = mantissa & 0x1fffu;
    if (rem > 0x1000u || (rem == 0x1000u && (h & 1u))) ++h;
    return (uint16_t)(sign | h);
}

float oracle_f16_to_f32(uint16_t bits) {
    const uint32_t sign = ((uint32_t)bits & 0x8000u) << 16;
    const uint32_t exponent = ((uint32_t)bits >> 10) & 0x1fu;
    const uint32_t mantissa = (uint32_t)bits & 0x3ffu;
    uint32_t out;
    if (exponent == 0) {
        float magnitude = (float)mantissa * 0x1.0p-24f;
        memcpy(&out, &magnitude, sizeof(out));
        out |= sign;
    } else if (exponent == 31) {
        out = sign | 0x7f800000u | (mantissa << 13);
    } else {
        out = sign | ((exponent + 112u) << 23) | (mantissa << 13);
    }
    float result;
    memcpy(&result, &out, sizeof(result));
    return result;
}

void oracle_f32_to_f16_array(const float *in, uint16_t *out, size_t n) {
    for (size_t i = 0; i < n; ++i) out[i] = oracle_f32_to_f16(in[i]);
}

void oracle_f16_to_f32_array(const uint16_t *in, float *out, size_t n) {
    for (size_t i = 0; i < n; ++i) out[i] = oracle_f16_to_f32(in[i]);
}

static uint64_t splitmix64_next(uint64_t *state) {
    uint64_t z = (*state += 0x9E3779B97F4A7C15ull);
    z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ull;
    z = (z ^ (z >> 27)) * 0x94D049BB133111EBull;
    return z ^ (z >> 31);
}

void oracle_normal_f32(uint64_t seed, float *out, size_t n) {
    uint64_t state = seed;
    const double two_pi = 6.283185307179586476925286766559;
    for (size_t i = 0; i < n; i += 2) {
        const double u1 = 1.0 - (double)(splitmix64_next(&state) >> 11) * 0x1.0p-53;
        const double u2 = (double)(splitmix64_next(&state) >> 11) * 0x1.0p-53;
        const double r = sqrt(-2.0 * log(u1));
        out[i] = (float)(r * cos(two_pi * u2));
        if (i + 1 < n) out[i + 1] = (float)(r * sin(two_pi * u2));
    }
}

void oracle_normal_f16(uint64_t seed, float scale, uint16_t *out, size_t n) {
    float *tmp = (float *)malloc((n ? n : 1) * sizeof(float));
    oracle_normal_f32(seed, tmp, n);
    for (size_t i = 0; i < n; ++i) out[i] = oracle_f32_to_f16(tmp[i] * scale);
    free(tmp);
}
