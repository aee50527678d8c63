"""Pins the CPU oracle against the reference's own known answers.

Every check here is independent of the oracle's formulas: reference digests,
reference closed forms, textbook identities, or brute force.  A plausible
mistake (dropped scale, wrong KV grouping, off-by-one prefix, swapped rotation
sign, wrong M-RoPE section) fails at least one of them.
"""

import math
import os
import struct

import numpy as np
import pytest

import oracle as O

f32 = np.float32
GOLDEN = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")


def bits(a):
    return np.asarray(a, dtype=np.float32).view(np.uint32)


def modular(n, mul, add, mod, sub, div):
    """(((i*mul + add) % mod) as f32 - sub) / div in f32, as the reference fixtures write it."""
    i = np.arange(n, dtype=np.int64)
    return ((((i * mul + add) % mod).astype(np.float32) - f32(sub)) / f32(div)).astype(np.float32)


def causal_fixture(tokens, qh, kvh, hd):
    # crates/pvlc-cpu-ref/tests/decoder_gqa_contract.rs:14-26
    return (modular(tokens * qh * hd, 17, 3, 37, 18, 11), modular(tokens * kvh * hd, 13, 7, 31, 15, 9),
            modular(tokens * kvh * hd, 19, 5, 41, 20, 7))


def direct_fixture(t, qh, kvh, hd):
    # crates/pvlc-cpu-ref/tests/decoder_decode_contract.rs:289-306
    return (modular(qh * hd, 17, t * 5 + 3, 37, 18, 11), modular(t * kvh * hd, 13, t * 7 + 5, 31, 15, 9),
            modular(t * kvh * hd, 19, t * 11 + 7, 41, 20, 7))


# ---------------------------------------------------------------- BLAKE3 ----

def test_blake3_specification_vectors(golden):
    for n, want in golden["blake3_spec_vectors"].items():
        if n == "cite":
            continue
        data = bytes(i % 251 for i in range(int(n)))
        assert O.blake3_hex(data) == want, n


def test_blake3_model_lock_digests(golden):
    for name, want in golden["blake3_model_lock"].items():
        if name == "cite":
            continue
        with open(os.path.join(GOLDEN, name), "rb") as f:
            assert O.blake3_hex(f.read()) == want, name


# ------------------------------------------------------- causal GQA ----

def test_causal_gqa_reproduces_reference_compact_digest(golden):
    g = golden["compact_blake3"]
    q, k, v = causal_fixture(g["tokens"], g["query_heads"], g["key_value_heads"], g["head_dim"])
    out = O.causal_gqa_f32(q, k, v, g["tokens"], g["query_heads"], g["key_value_heads"], g["head_dim"])
    assert O.blake3_hex(out.astype("<f4").tobytes()) == g["digest"]
    # token 0 attends only to itself: output equals its own value row (test :155-164)
    for qh, kvh in enumerate([0, 0, 1, 1]):
        np.testing.assert_array_equal(out[qh * 3:qh * 3 + 3], v[kvh * 3:kvh * 3 + 3])


def test_causal_row_equals_decode_over_prefix_bit_exact():
    tokens, qh, kvh, hd = 19, 8, 2, 16
    q, k, v = (O.normal_f32(100 + i, n) for i, n in enumerate((tokens * qh * hd, tokens * kvh * hd,
                                                                tokens * kvh * hd)))
    causal = O.causal_gqa_f32(q, k, v, tokens, qh, kvh, hd).reshape(tokens, qh * hd)
    w = kvh * hd
    for i in range(tokens):
        dec = O.decode_gqa_f32(q[i * qh * hd:(i + 1) * qh * hd], k[:(i + 1) * w], v[:(i + 1) * w], i + 1,
                               qh, kvh, hd)
        np.testing.assert_array_equal(bits(causal[i]), bits(dec))


def test_causal_prefix_is_immune_to_future_poison():
    # decoder_gqa_contract.rs:230-262: rows < i never read keys/values >= i+1
    tokens, qh, kvh, hd = 9, 4, 2, 8
    q, k, v = (O.normal_f32(7 + i, n) for i, n in enumerate((tokens * qh * hd, tokens * kvh * hd,
                                                              tokens * kvh * hd)))
    base = O.causal_gqa_f32(q, k, v, tokens, qh, kvh, hd).reshape(tokens, -1)
    k2, v2 = k.copy(), v.copy()
    cut = 5
    k2[cut * kvh * hd:] = 1e4
    v2[cut * kvh * hd:] = -1e4
    poisoned = O.causal_gqa_f32(q, k2, v2, tokens, qh, kvh, hd).reshape(tokens, -1)
    np.testing.assert_array_equal(bits(base[:cut]), bits(poisoned[:cut]))
    assert not np.array_equal(base[cut:], poisoned[cut:])


# ------------------------------------------------------- decode GQA ----

def _direct_digest(golden):
    g = golden["direct_boundary_blake3"]
    h = b""
    for t in g["lengths"]:
        q, k, v = direct_fixture(t, g["query_heads"], g["key_value_heads"], g["head_dim"])
        out = O.decode_gqa_f32(q, k, v, t, g["query_heads"], g["key_value_heads"], g["head_dim"])
        indep = O.independent_decode_gqa_f32(q, k, v, t, g["query_heads"], g["key_value_heads"], g["head_dim"])
        np.testing.assert_array_equal(bits(out), bits(indep))
        h += struct.pack("<Q", t) + out.astype("<f4").tobytes()
    return O.blake3_hex(h)


def test_decode_gqa_reproduces_reference_direct_boundary_digest(golden):
    g = golden["direct_boundary_blake3"]
    # glibc expf everywhere
    O.set_expf_overrides([])
    assert _direct_digest(golden) == g["glibc_digest"]
    # the reference platform's expf at its three near-midpoint arguments
    pairs = [(e["arg_bits"], e["platform_bits"]) for e in g["platform_expf"]]
    for e in g["platform_expf"]:
        x = np.array([e["arg_bits"]], np.uint32).view(np.float32)[0]
        glibc = f32(math.exp(float(x)))  # correctly rounded here (pinned by the glibc digest)
        assert int(bits([glibc])[0]) == e["glibc_bits"]
        assert abs(e["platform_bits"] - e["glibc_bits"]) == 1
    try:
        O.set_expf_overrides(pairs)
        assert _direct_digest(golden) == g["digest"]
    finally:
        O.set_expf_overrides([])


def test_decode_bounded_extreme_is_exact(golden):
    g = golden["bounded_extreme"]
    out = O.decode_gqa_f32(g["query"], g["keys"], g["values"], g["cache_tokens"], g["query_heads"],
                           g["key_value_heads"], g["head_dim"])
    np.testing.assert_array_equal(bits(out), bits(g["expected"]))


def test_decode_group_one_and_single_kv_head_match_physical_repeat():
    for t, qh, kvh, hd in [(7, 2, 2, 5), (9, 4, 1, 3)]:
        q, k, v = direct_fixture(t, qh, kvh, hd)
        np.testing.assert_array_equal(bits(O.decode_gqa_f32(q, k, v, t, qh, kvh, hd)),
                                      bits(O.independent_decode_gqa_f32(q, k, v, t, qh, kvh, hd)))


def test_decode_fixture_is_sensitive_to_grouping_scale_and_truncation():
    t, qh, kvh, hd = 33, 4, 2, 6
    q, k, v = direct_fixture(t, qh, kvh, hd)
    expected = O.decode_gqa_f32(q, k, v, t, qh, kvh, hd)
    wrong = O.independent_decode_gqa_f32(q, k, v, t, qh, kvh, hd, rotate_groups=True)
    noscale = O.independent_decode_gqa_f32(q, k, v, t, qh, kvh, hd, scale=1.0)
    trunc = O.decode_gqa_f32(q, k[kvh * hd:], v[kvh * hd:], t - 1, qh, kvh, hd)
    for other in (wrong, noscale, trunc):
        assert not np.array_equal(bits(other), bits(expected))


def test_decode_matches_float64_softmax_closed_form():
    t, qh, kvh, hd = 300, 16, 2, 128
    q, k, v = O.normal_f32(1, qh * hd), O.normal_f32(2, t * kvh * hd), O.normal_f32(3, t * kvh * hd)
    out = O.decode_gqa_f32(q, k, v, t, qh, kvh, hd).reshape(qh, hd)
    qd, kd, vd = q.reshape(qh, hd).astype(np.float64), k.reshape(t, kvh, hd), v.reshape(t, kvh, hd)
    for h in range(qh):
        g = h // (qh // kvh)
        s = kd[:, g, :].astype(np.float64) @ qd[h] / math.sqrt(hd)
        p = np.exp(s - s.max())
        p /= p.sum()
        ref = p @ vd[:, g, :].astype(np.float64)
        np.testing.assert_allclose(out[h], ref, atol=2e-6, rtol=1e-5)


@pytest.mark.parametrize("case", ["zero_tokens", "zero_heads", "not_divisible", "short_key", "long_value",
                                  "nan_query", "inf_value"])
def test_decode_validation_errors(case):
    qh, kvh, hd, t = 4, 2, 6, 3
    q, k, v = direct_fixture(t, qh, kvh, hd)
    args = dict(query=q, key=k, value=v, cache_tokens=t, query_heads=qh, key_value_heads=kvh, head_dim=hd)
    want = "DimensionMismatch"
    if case == "zero_tokens":
        args["cache_tokens"] = 0
    elif case == "zero_heads":
        args["query_heads"] = 0
    elif case == "not_divisible":
        args["key_value_heads"] = 3
    elif case == "short_key":
        args["key"] = k[:-1]
    elif case == "long_value":
        args["value"] = np.append(v, 0)
    elif case == "nan_query":
        q2 = q.copy()
        q2[3] = np.nan
        args["query"], want = q2, "NonFiniteInput"
    elif case == "inf_value":
        v2 = v.copy()
        v2[0] = np.inf
        args["value"], want = v2, "NonFiniteInput"
    with pytest.raises(O.OracleError) as err:
        O.decode_gqa_f32(**args)
    assert err.value.code == want


# ----------------------------------------------------------- append ----

def test_append_is_concatenation_and_leaves_prefix_untouched():
    prefix, kvh, hd = 5, 2, 4
    pk, pv = O.normal_f32(11, prefix * kvh * hd), O.normal_f32(12, prefix * kvh * hd)
    nk, nv = O.normal_f32(13, kvh * hd), O.normal_f32(14, kvh * hd)
    ok, ov = O.append_kv_f32(pk, pv, prefix, nk, nv, kvh, hd)
    np.testing.assert_array_equal(bits(ok), bits(np.concatenate([pk, nk])))
    np.testing.assert_array_equal(bits(ov), bits(np.concatenate([pv, nv])))
    with pytest.raises(O.OracleError):
        O.append_kv_f32(pk, pv, prefix, nk[:-1], nv, kvh, hd)
    bad = nv.copy()
    bad[1] = np.nan
    with pytest.raises(O.OracleError) as err:
        O.append_kv_f32(pk, pv, prefix, nk, bad, kvh, hd)
    assert err.value.code == "NonFiniteInput"


# ------------------------------------------------------------- RoPE ----

def test_rope_neox_reference_closed_form(golden):
    g = golden["rope_closed_form"]
    orig = np.array(g["values"], np.float32)
    out = O.rope_neox_f32(orig, g["rows"], g["width"], g["rotary_dim"], g["positions"], g["base"])
    np.testing.assert_array_equal(out[:5], orig[:5])  # position 0 is the identity
    assert out[9] == orig[9]  # non-rotary tail untouched
    a0, a1 = f32(17.0), f32(17.0) / np.sqrt(f32(500000.0))
    want = [-2 * np.cos(a0) - 5 * np.sin(a0), -4 * np.cos(a1) - 7 * np.sin(a1),
            5 * np.cos(a0) + -2 * np.sin(a0), 7 * np.cos(a1) + -4 * np.sin(a1)]
    np.testing.assert_allclose(out[5:9], want, atol=g["tolerance"])
    for left, right in [(5, 7), (6, 8)]:
        assert abs((out[left] ** 2 + out[right] ** 2) - (orig[left] ** 2 + orig[right] ** 2)) < 2e-5


def test_rope_neox_matches_float64_rotation_at_base_500000():
    rows, width = 6, 256
    x = O.normal_f32(21, rows * width)
    pos = np.array([0, 1, 17, 1024, 2047, 4095], np.uint32)
    out = O.rope_neox_f32(x, rows, width, 128, pos, 500000.0).reshape(rows, width)
    xr = x.reshape(rows, width).astype(np.float64)
    i = np.arange(64)
    for r in range(rows):
        ang = pos[r] * 500000.0 ** (-2.0 * i / 128)
        f, s = xr[r, :64], xr[r, 64:128]
        np.testing.assert_allclose(out[r, :64], f * np.cos(ang) - s * np.sin(ang), atol=5e-4)
        np.testing.assert_allclose(out[r, 64:128], s * np.cos(ang) + f * np.sin(ang), atol=5e-4)
        np.testing.assert_array_equal(out[r, 128:], x.reshape(rows, width)[r, 128:])


def test_rope_validation_errors():
    x = np.ones(8, np.float32)
    for rd, code in [(0, "InvalidRotaryDimension"), (3, "InvalidRotaryDimension"), (10, "InvalidRotaryDimension")]:
        with pytest.raises(O.OracleError) as err:
            O.rope_neox_f32(x, 2, 4, rd, [0, 1], 10000.0)
        assert err.value.code == code
    for base in (0.0, -1.0, float("inf")):
        with pytest.raises(O.OracleError) as err:
            O.rope_neox_f32(x, 2, 4, 4, [0, 1], base)
        assert err.value.code == "InvalidRopeBase"


def neox_tables(positions, base, head_dim=128):
    """raw M-RoPE tables [3, tokens, head_dim] with all three axes at `positions`,
    cos/sin from the oracle's own RoPE (rotating unit vectors)."""
    tokens = len(positions)
    half = head_dim // 2
    c = np.zeros((tokens, head_dim), np.float32)
    s = np.zeros((tokens, head_dim), np.float32)
    for p in range(half):
        e = np.zeros((tokens, head_dim), np.float32)
        e[:, p] = 1.0
        r = O.rope_neox_f32(e, tokens, head_dim, head_dim, positions, base).reshape(tokens, head_dim)
        c[:, p] = c[:, p + half] = r[:, p]  # first' = 1*cos
        s[:, p] = s[:, p + half] = r[:, p + half]  # second' = 1*sin
    return np.stack([c] * 3), np.stack([s] * 3)


def test_equal_axis_mrope_equals_neox_bit_exact():
    tokens, qh, kvh, hd = 4, 16, 2, 128
    pos = np.array([0, 5, 1024, 2303], np.uint32)
    q, k = O.normal_f32(31, tokens * qh * hd), O.normal_f32(32, tokens * kvh * hd)
    cos, sin = neox_tables(pos, 500000.0)
    rq, rk = O.mrope_f32(q, k, tokens, qh, kvh, hd, cos, sin, (16, 24, 24))
    nq = O.rope_neox_f32(q, tokens * qh, hd, hd, np.repeat(pos, qh), 500000.0)
    nk = O.rope_neox_f32(k, tokens * kvh, hd, hd, np.repeat(pos, kvh), 500000.0)
    np.testing.assert_array_equal(bits(rq), bits(nq))
    np.testing.assert_array_equal(bits(rk), bits(nk))


def test_mrope_section_selection_brute_force():
    tokens, qh, kvh, hd = 3, 2, 1, 128
    rng = np.random.default_rng(5)
    raw_c = rng.standard_normal((3, tokens, hd)).astype(np.float32)
    raw_s = rng.standard_normal((3, tokens, hd)).astype(np.float32)
    q = rng.standard_normal(tokens * qh * hd).astype(np.float32)
    k = rng.standard_normal(tokens * kvh * hd).astype(np.float32)
    rq, rk = O.mrope_f32(q, k, tokens, qh, kvh, hd, raw_c, raw_s, (16, 24, 24))
    # axis of dim d: chunks [16,24,24,16,24,24] take axes 0,1,2,0,1,2
    axis = np.array([0] * 16 + [1] * 24 + [2] * 24 + [0] * 16 + [1] * 24 + [2] * 24)
    for t in range(tokens):
        sc = raw_c[axis, t, np.arange(hd)]
        ss = raw_s[axis, t, np.arange(hd)]
        for heads, src, dst in ((qh, q, rq), (kvh, k, rk)):
            x = src.reshape(tokens, heads, hd)[t]
            rot = np.concatenate([-x[:, 64:], x[:, :64]], axis=1)
            want = (x * sc + rot * ss).astype(np.float32)
            np.testing.assert_array_equal(bits(dst.reshape(tokens, heads, hd)[t]), bits(want))


# ------------------------------------------------------------- fp16 ----

def test_f16_widening_is_exact_for_every_pattern():
    allbits = np.arange(65536, dtype=np.uint32).astype(np.uint16)
    ours = O.f16_to_f32(allbits)
    ref = allbits.view(np.float16).astype(np.float32)
    finite = np.isfinite(ref)
    np.testing.assert_array_equal(bits(ours[finite]), bits(ref[finite]))
    assert np.all(np.isnan(ours[~finite]) == np.isnan(ref[~finite]))


def test_f16_narrowing_is_round_to_nearest_even():
    rng = np.random.default_rng(0)
    # dense coverage of the fp16 range, subnormals, ties and overflow
    x = np.concatenate([
        rng.standard_normal(200000).astype(np.float32) * np.float32(3.0),
        (rng.random(100000).astype(np.float32) - 0.5) * np.float32(1e-4),
        np.array([65504, 65519.99, 65520, 65536, -70000, 2.0 ** -25, 2.0 ** -24, 1.5 * 2.0 ** -24,
                  2.0 ** -14, 1.0 + 2.0 ** -11, 1.0 + 3 * 2.0 ** -11, 0.0, -0.0], np.float32),
        # exact ties between adjacent halves
        (np.arange(-2048, 2048, dtype=np.float32) + np.float32(0.5)) * np.float32(2.0 ** -10),
    ])
    ours = O.f32_to_f16(x)
    with np.errstate(over="ignore"):
        ref = x.astype(np.float16).view(np.uint16)
    np.testing.assert_array_equal(ours, ref)


def test_normal_generator_statistics_and_determinism():
    a = O.normal_f32(123, 1 << 18)
    assert np.array_equal(a, O.normal_f32(123, 1 << 18))
    assert abs(a.mean()) < 0.01 and abs(a.std() - 1) < 0.01
    h = O.normal_f16(123, 1000, 0.5)
    np.testing.assert_array_equal(h, (a[:1000] * np.float32(0.5)).astype(np.float16).view(np.uint16))


def test_write_prefill_kv_is_a_validated_clone():
    # write_decoder_prefill_kv_f32, lib.rs:976-992: rows copied unchanged, geometry and finiteness checked
    tokens, kvh, hd = 7, 2, 8
    k, v = O.normal_f32(51, tokens * kvh * hd), O.normal_f32(52, tokens * kvh * hd)
    ok, ov = O.write_prefill_kv_f32(k, v, tokens, kvh, hd)
    np.testing.assert_array_equal(bits(ok), bits(k))
    np.testing.assert_array_equal(bits(ov), bits(v))
    with pytest.raises(O.OracleError) as err:
        O.write_prefill_kv_f32(k[:-1], v, tokens, kvh, hd)
    assert err.value.code == "DimensionMismatch"
    bad = v.copy()
    bad[4] = np.inf
    with pytest.raises(O.OracleError) as err:
        O.write_prefill_kv_f32(k, bad, tokens, kvh, hd)
    assert err.value.code == "NonFiniteInput"
    with pytest.raises(O.OracleError) as err:
        O.write_prefill_kv_f32(k, v, 0, kvh, hd)
    assert err.value.code == "DimensionMismatch"


def test_linear_reproduces_reference_known_answer():
    # crates/pvlc-cpu-ref/tests/vision_contract.rs:433-441 (output-major weights, bias added first)
    out = O.linear_f32([1.0, 2.0, 3.0, -1.0, 0.0, 2.0], 2, 3, [1.0, 2.0, 3.0, -1.0, 0.5, 2.0], [0.25, -0.5], 2)
    np.testing.assert_array_equal(out, np.array([14.25, 5.5, 5.25, 4.5], np.float32))


def test_linear_validation_errors_follow_reference():
    # vision_contract.rs:444-470: zero dimensions and length mismatches, then non-finite operands
    for rows, width, out_w in [(0, 3, 2), (2, 0, 2), (2, 3, 0)]:
        with pytest.raises(O.OracleError) as err:
            O.linear_f32([], rows, width, [], [], out_w)
        assert err.value.code == "DimensionMismatch"
    for x, w, b in [([1.0, 2.0], [1.0, 2.0, 3.0], [0.0]), ([1.0, 2.0, 3.0], [1.0, 2.0], [0.0]),
                    ([1.0, 2.0, 3.0], [1.0, 2.0, 3.0], [])]:
        with pytest.raises(O.OracleError) as err:
            O.linear_f32(x, 1, 3, w, b, 1)
        assert err.value.code == "DimensionMismatch"
    for x, w, b in [([1.0, np.nan, 3.0], [1.0, 2.0, 3.0], [0.0]), ([1.0, 2.0, 3.0], [1.0, np.inf, 3.0], [0.0]),
                    ([1.0, 2.0, 3.0], [1.0, 2.0, 3.0], [np.nan])]:
        with pytest.raises(O.OracleError) as err:
            O.linear_f32(x, 1, 3, w, b, 1)
        assert err.value.code == "NonFiniteInput"


def test_linear_is_exact_on_small_integers_and_within_f64_bound():
    rng = np.random.default_rng(3)
    # small integers: every partial sum is exactly representable, so any order is exact
    x = rng.integers(-8, 9, (3, 1024)).astype(np.float32)
    w = rng.integers(-8, 9, (40, 1024)).astype(np.float32)
    b = rng.integers(-8, 9, 40).astype(np.float32)
    out = O.linear_f32(x, 3, 1024, w, b, 40).reshape(3, 40)
    want = (x.astype(np.int64) @ w.astype(np.int64).T + b.astype(np.int64)).astype(np.float32)
    np.testing.assert_array_equal(out, want)
    # general values: sequential f32 sum within the classical bound n*eps*sum|terms| of the f64 result
    x = O.normal_f32(61, 2048)
    w = O.f16_to_f32(O.normal_f16(62, 64 * 2048))
    out = O.linear_f32(x, 1, 2048, w, np.zeros(64, np.float32), 64)
    wm = w.reshape(64, 2048).astype(np.float64)
    exact = wm @ x.astype(np.float64)
    bound = 2048 * 2.0 ** -24 * (np.abs(wm) @ np.abs(x.astype(np.float64)))
    assert np.all(np.abs(out - exact) <= bound)
    # a dropped term or a transposed weight layout would not pass
    assert np.max(np.abs(out - (w.reshape(2048, 64).astype(np.float64).T @ x))) > 1.0


# ---------------------------------------------------------------------------
# top-1 over logits (decoder_stack_session.rs:308-366, greedy_generation.mjs:43-79)
# ---------------------------------------------------------------------------

def _f32_bits(x):
    return int(np.array([x], np.float32).view(np.uint32)[0])


def _numeric_top1(values):
    """Independent comparator for non-NaN logits: larger value, then +0 over -0, then the lower index."""
    import math
    return max(range(len(values)), key=lambda i: (float(values[i]), math.copysign(1.0, float(values[i])), -i))


def test_top1_matches_a_numeric_comparator_on_random_logits_with_ties():
    rng = np.random.default_rng(31)
    for n in (1, 2, 3, 17, 256, 1000, 4099):
        for trial in range(4):
            x = rng.standard_normal(n).astype(np.float32)
            if trial >= 1:  # planted ties of the maximum (and quantised values)
                x = np.round(x * 4) / 4
            if trial == 3 and n > 2:
                x[rng.integers(0, n, 3)] = x.max()
            idx, bits = O.top1_f32(x)
            want = _numeric_top1(x)
            assert idx == want and bits == _f32_bits(x[want]), (n, trial)


def test_top1_total_order_on_special_values():
    nan, neg_nan = np.float32(np.nan), -np.float32(np.nan)
    inf = np.float32(np.inf)
    cases = [
        ([-0.0, 0.0], 1), ([0.0, -0.0], 0), ([-0.0, -0.0], 0),
        ([1.0, nan, inf], 1), ([inf, nan], 1), ([neg_nan, -inf], 1), ([neg_nan], 0),
        ([-inf, -inf, -inf], 0), ([-3.0, -1e-45, -1.0], 1), ([1e-45, 0.0, -0.0], 0),
        ([5.0, 7.0, 7.0, 6.0], 1), ([np.float32(3.4028235e38), inf, inf], 1),
    ]
    for values, want in cases:
        x = np.array(values, np.float32)
        idx, bits = O.top1_f32(x)
        assert idx == want, (values, idx)
        assert bits == int(x.view(np.uint32)[want])


def test_top1_rejects_an_empty_logit_row():
    with pytest.raises(O.OracleError) as e:
        O.top1_f32(np.zeros(0, np.float32))
    assert e.value.code == "DimensionMismatch"
