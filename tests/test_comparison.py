"""The restated comparison report (oracle/comparison.py, crates/pvlc-testkit/src/lib.rs:31-330) against the
reference's own contract cases (crates/pvlc-testkit/tests/comparison_contract.rs), so that the metrics the GPU
parity tests assert -- the reference's native decode policy among them -- mean what the reference's do."""

import math

import numpy as np
import pytest

from oracle.comparison import NATIVE_DECODE_POLICY, ComparisonError, ComparisonPolicy, compare_f32

F32MAX = float(np.finfo(np.float32).max)
F32MINPOS = float(np.finfo(np.float32).tiny)


def permissive(**kw):
    base = dict(require_finite=True, max_abs=10.0, max_mean_abs=10.0, max_p99_abs=10.0, max_relative_l2=10.0,
                min_cosine_similarity=-1.0, max_per_token_relative_l2=10.0, max_per_channel_relative_l2=10.0)
    base.update(kw)
    return ComparisonPolicy(**base)


def report_2x2():
    return compare_f32([1.0, -2.0, 0.0, 4.0], [1.1, -2.2, 0.3, 3.6], [2, 2], token_axis=0, channel_axis=1)


def test_every_metric_with_documented_quantiles_and_axes():
    """comparison_contract.rs:24-65 (report_computes_every_required_metric_...)."""
    r = report_2x2()
    assert r.element_count == 4 and r.finite_pair_count == 4
    assert abs(r.max_abs - 0.4) <= 1e-6 and abs(r.mean_abs - 0.25) <= 1e-6
    assert abs(r.p50_abs - 0.2) <= 1e-6 and abs(r.p90_abs - 0.4) <= 1e-6 and abs(r.p99_abs - 0.4) <= 1e-6
    assert abs(r.relative_l2 - math.sqrt(0.3 / 21.0)) <= 1e-6
    assert abs(r.cosine_similarity - 19.9 / math.sqrt(21.0 * 19.1)) <= 1e-6
    assert np.allclose(r.per_token_relative_l2, [0.1, 0.125], atol=1e-6)
    assert np.allclose(r.per_channel_relative_l2, [math.sqrt(0.1), 0.1], atol=1e-6)
    assert r.reference_non_finite == (0, 0, 0) == r.candidate_non_finite and r.non_finite_mismatches == 0


def test_every_policy_metric_fails_independently():
    """comparison_contract.rs:67-144: each threshold one ulp past its metric trips exactly that metric."""
    r = report_2x2()
    assert r.assess(permissive()) == []
    cases = [(permissive(max_abs=math.nextafter(r.max_abs, 0)), "MaxAbs"),
             (permissive(max_mean_abs=math.nextafter(r.mean_abs, 0)), "MeanAbs"),
             (permissive(max_p99_abs=math.nextafter(r.p99_abs, 0)), "P99Abs"),
             (permissive(max_relative_l2=math.nextafter(r.relative_l2, 0)), "RelativeL2"),
             (permissive(min_cosine_similarity=math.nextafter(r.cosine_similarity, 2)), "CosineSimilarity"),
             (permissive(max_per_token_relative_l2=0.124), "PerTokenRelativeL2"),
             (permissive(max_per_channel_relative_l2=0.31), "PerChannelRelativeL2")]
    for policy, want in cases:
        assert r.assess(policy) == [want]


def test_non_finite_values_are_counted_by_kind():
    """comparison_contract.rs:146-183."""
    nan, inf = float("nan"), float("inf")
    r = compare_f32([nan, inf, -inf, 1.0], [nan, -inf, -inf, inf])
    assert r.reference_non_finite == (1, 1, 1) and r.candidate_non_finite == (1, 1, 2)
    assert r.non_finite_mismatches == 2 and r.finite_pair_count == 0
    assert r.assess(permissive()) == ["NonFinite"]
    assert r.assess(permissive(require_finite=False)) == ["NonFiniteMismatch"]
    same = compare_f32([nan, inf, -inf, 1.0], [nan, inf, -inf, 1.0])
    exact = ComparisonPolicy(False, 0.0, 0.0, 0.0, 0.0, 1.0)
    assert same.assess(exact) == []


def test_zero_norm_and_extreme_vectors():
    """comparison_contract.rs:207-230."""
    z = compare_f32([0.0, -0.0], [0.0, 0.0])
    assert z.relative_l2 == 0.0 and z.cosine_similarity == 1.0
    zr = compare_f32([0.0, 0.0], [0.0, 1.0])
    assert math.isinf(zr.relative_l2) and zr.cosine_similarity == 0.0
    ex = compare_f32([F32MAX, F32MINPOS, -F32MAX], [F32MAX, F32MINPOS, -F32MAX])
    assert ex.max_abs == 0.0 and ex.relative_l2 == 0.0 and abs(ex.cosine_similarity - 1.0) <= 1e-15


def test_malformed_shapes_axes_and_policies():
    """comparison_contract.rs:232-330."""
    for args, kw, code in [(([], [], [0]), {}, "EmptyTensor"), (([1.0], [1.0, 2.0], [1]), {}, "LengthMismatch"),
                           (([1.0] * 4, [1.0] * 4, [2, 3]), {}, "ShapeMismatch"),
                           (([1.0], [1.0], [1]), {"token_axis": 1}, "AxisOutOfRange"),
                           (([1.0], [1.0], [1]), {"token_axis": 0, "channel_axis": 0}, "DuplicateAxis")]:
        with pytest.raises(ComparisonError) as e:
            compare_f32(*args, **kw)
        assert e.value.code == code
    r = compare_f32([1.0], [1.0], [1])
    bad = [permissive(max_abs=-1.0), permissive(min_cosine_similarity=1.01)]
    for invalid in (float("nan"), float("-inf"), -1.0):
        bad += [permissive(max_abs=invalid), permissive(max_mean_abs=invalid), permissive(max_p99_abs=invalid),
                permissive(max_relative_l2=invalid), permissive(max_per_token_relative_l2=invalid),
                permissive(max_per_channel_relative_l2=invalid)]
    for c in (float("nan"), float("-inf"), -1.01, 1.01):
        bad.append(permissive(min_cosine_similarity=c))
    for policy in bad:
        with pytest.raises(ComparisonError) as e:
            r.assess(policy)
        assert e.value.code == "InvalidPolicy"


def test_nearest_rank_quantiles_and_threshold_equality():
    """comparison_contract.rs:332-370: nearest-rank p50/p90/p99 over 100 ordered errors; equality passes."""
    ref = np.full(100, 10.0, np.float32)
    cand = np.array([10.0 + k / 100.0 for k in range(1, 101)], np.float32)
    r = compare_f32(ref, cand, [100])
    assert abs(r.p50_abs - 0.50) <= 1e-6 and abs(r.p90_abs - 0.90) <= 1e-6
    assert abs(r.p99_abs - 0.99) <= 1e-6 and abs(r.max_abs - 1.00) <= 1e-6
    eq = ComparisonPolicy(True, r.max_abs, r.mean_abs, r.p99_abs, r.relative_l2, r.cosine_similarity)
    assert r.assess(eq) == []


def test_native_decode_policy_is_the_reference_one():
    """decoder_cached_gqa_native_contract.rs:147-158, and it rejects what it should: an output rounded to fp16
    (one 2^-11 relative step per element) fails its relative L2 on N(0,1)-scale values."""
    p = NATIVE_DECODE_POLICY
    assert (p.require_finite, p.max_abs, p.max_mean_abs, p.max_p99_abs, p.max_relative_l2,
            p.min_cosine_similarity) == (True, 4.0e-4, 6.0e-5, 2.5e-4, 1.5e-4, 0.99999)
    rng = np.random.default_rng(1)
    x = (rng.standard_normal(4096) * 0.05).astype(np.float32)
    assert compare_f32(x, x).assess(p) == []
    assert "RelativeL2" in compare_f32(x, x.astype(np.float16).astype(np.float32)).assess(p)
