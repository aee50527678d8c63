"""The reference's numerical comparison report and policy, restated in numpy.

TEST INFRASTRUCTURE, NOT PRODUCT CODE (the same rule as the rest of ``oracle/``).

Restates ``compare_f32``, ``ComparisonReport::assess`` and ``ComparisonPolicy`` of
crates/pvlc-testkit/src/lib.rs:31-330 (glebkudr/paddleocr-vl-webgpu): every finite pair contributes its
absolute error (in f64) to max / mean / nearest-rank p50, p90, p99; relative L2 and cosine similarity are
taken over the finite pairs with the reference's zero-norm rules; non-finite values are counted by kind, and a
pair whose kinds differ is a mismatch.  The per-token and per-channel relative L2 of the reference are kept
(relative_l2_by_axis, :289-311).  Pinned by the reference's own contract cases
(crates/pvlc-testkit/tests/comparison_contract.rs) in tests/test_comparison.py.
"""

from __future__ import annotations

import math
from dataclasses import dataclass, field

import numpy as np


class ComparisonError(Exception):
    """ComparisonError with the reference's ComparisonErrorCode names (lib.rs, ComparisonErrorCode)."""

    def __init__(self, code: str, message: str):
        super().__init__(message)
        self.code = code


@dataclass(frozen=True)
class ComparisonPolicy:
    """ComparisonPolicy, crates/pvlc-testkit/src/lib.rs:31-41."""
    require_finite: bool
    max_abs: float
    max_mean_abs: float
    max_p99_abs: float
    max_relative_l2: float
    min_cosine_similarity: float
    max_per_token_relative_l2: float | None = None
    max_per_channel_relative_l2: float | None = None


# The policy of the reference's native decode contract tests
# (crates/pvlc-runtime-native/tests/decoder_cached_gqa_native_contract.rs:147-158).
NATIVE_DECODE_POLICY = ComparisonPolicy(require_finite=True, max_abs=4.0e-4, max_mean_abs=6.0e-5, max_p99_abs=2.5e-4,
                                        max_relative_l2=1.5e-4, min_cosine_similarity=0.99999)


@dataclass
class ComparisonReport:
    """ComparisonReport, lib.rs:52-67."""
    element_count: int
    finite_pair_count: int
    max_abs: float
    mean_abs: float
    p50_abs: float
    p90_abs: float
    p99_abs: float
    relative_l2: float
    cosine_similarity: float
    per_token_relative_l2: list | None
    per_channel_relative_l2: list | None
    reference_non_finite: tuple = (0, 0, 0)  # (nan, +inf, -inf)
    candidate_non_finite: tuple = (0, 0, 0)
    non_finite_mismatches: int = 0
    violations: list = field(default_factory=list)

    def assess(self, policy: ComparisonPolicy) -> list:
        """ComparisonReport::assess, lib.rs:172-218: the violated metrics in the reference's order (an empty
        list passes)."""
        _validate_policy(policy)
        out = []
        has_non_finite = self.reference_non_finite != (0, 0, 0) or self.candidate_non_finite != (0, 0, 0)
        if policy.require_finite and has_non_finite:
            out.append("NonFinite")
        elif self.non_finite_mismatches != 0:
            out.append("NonFiniteMismatch")
        if self.max_abs > policy.max_abs:
            out.append("MaxAbs")
        if self.mean_abs > policy.max_mean_abs:
            out.append("MeanAbs")
        if self.p99_abs > policy.max_p99_abs:
            out.append("P99Abs")
        if self.relative_l2 > policy.max_relative_l2:
            out.append("RelativeL2")
        if self.cosine_similarity < policy.min_cosine_similarity:
            out.append("CosineSimilarity")
        if (policy.max_per_token_relative_l2 is not None and self.per_token_relative_l2 is not None
                and any(v > policy.max_per_token_relative_l2 for v in self.per_token_relative_l2)):
            out.append("PerTokenRelativeL2")
        if (policy.max_per_channel_relative_l2 is not None and self.per_channel_relative_l2 is not None
                and any(v > policy.max_per_channel_relative_l2 for v in self.per_channel_relative_l2)):
            out.append("PerChannelRelativeL2")
        return out


def _validate_policy(policy: ComparisonPolicy) -> None:
    """validate_policy, lib.rs:240-266."""
    uppers = [policy.max_abs, policy.max_mean_abs, policy.max_p99_abs, policy.max_relative_l2]
    optional = [v for v in (policy.max_per_token_relative_l2, policy.max_per_channel_relative_l2) if v is not None]
    bad = any(not math.isfinite(v) or v < 0.0 for v in uppers + optional)
    cos = policy.min_cosine_similarity
    if bad or not math.isfinite(cos) or not -1.0 <= cos <= 1.0:
        raise ComparisonError("InvalidPolicy", "comparison policy contains an invalid threshold")


def _relative_l2(error_squared: float, reference_squared: float) -> float:
    """relative_l2, lib.rs:273-283."""
    if reference_squared == 0.0:
        return 0.0 if error_squared == 0.0 else math.inf
    return math.sqrt(error_squared / reference_squared)


def _nearest_rank(sorted_errors: np.ndarray, quantile: float) -> float:
    """nearest_rank, lib.rs:268-271."""
    rank = math.ceil(quantile * len(sorted_errors))
    return float(sorted_errors[max(rank, 1) - 1])


def _non_finite_counts(x: np.ndarray) -> tuple:
    return (int(np.isnan(x).sum()), int(np.sum(x == np.inf)), int(np.sum(x == -np.inf)))


def _kind(x: np.ndarray) -> np.ndarray:
    """0 finite, 1 NaN, 2 +inf, 3 -inf (non_finite_kind, lib.rs:333-343)."""
    k = np.zeros(x.shape, np.int8)
    k[np.isnan(x)] = 1
    k[x == np.inf] = 2
    k[x == -np.inf] = 3
    return k


def _relative_l2_by_axis(reference: np.ndarray, candidate: np.ndarray, shape, axis: int) -> list:
    """relative_l2_by_axis, lib.rs:285-311: finite pairs only, per coordinate of `axis`."""
    ref = reference.reshape(shape).astype(np.float64)
    cand = candidate.reshape(shape).astype(np.float64)
    finite = np.isfinite(ref) & np.isfinite(cand)
    err = np.where(finite, cand - ref, 0.0)
    refz = np.where(finite, ref, 0.0)
    other = tuple(i for i in range(len(shape)) if i != axis)
    e2 = (err * err).sum(axis=other)
    r2 = (refz * refz).sum(axis=other)
    return [_relative_l2(float(a), float(b)) for a, b in zip(np.atleast_1d(e2), np.atleast_1d(r2))]


def compare_f32(reference, candidate, shape=None, token_axis=None, channel_axis=None) -> ComparisonReport:
    """compare_f32, crates/pvlc-testkit/src/lib.rs:69-170."""
    reference = np.asarray(reference, np.float32).ravel()
    candidate = np.asarray(candidate, np.float32).ravel()
    shape = [reference.size] if shape is None else list(shape)
    if reference.size == 0 and candidate.size == 0:
        raise ComparisonError("EmptyTensor", "cannot compare an empty tensor")
    if reference.size != candidate.size:
        raise ComparisonError("LengthMismatch", "reference and candidate lengths differ")
    elements = 1
    for d in shape:
        elements *= int(d)
        if elements > np.iinfo(np.uint64).max:
            raise ComparisonError("ShapeOverflow", "tensor shape product overflowed")
    if elements != reference.size:
        raise ComparisonError("ShapeMismatch", "tensor shape does not match the flat buffer length")
    for axis in (token_axis, channel_axis):
        if axis is not None and axis >= len(shape):
            raise ComparisonError("AxisOutOfRange", "comparison axis is outside the tensor rank")
    if token_axis is not None and token_axis == channel_axis:
        raise ComparisonError("DuplicateAxis", "token and channel axes must differ")

    kr, kc = _kind(reference), _kind(candidate)
    both = (kr == 0) & (kc == 0)
    mismatches = int(np.sum(~both & (kr != kc)))
    exp = reference[both].astype(np.float64)
    act = candidate[both].astype(np.float64)
    err = act - exp
    absolute = np.sort(np.abs(err))
    n = absolute.size
    if n == 0:
        max_abs = mean_abs = p50 = p90 = p99 = 0.0
    else:
        max_abs = float(absolute[-1])
        mean_abs = float(absolute.sum() / n)
        p50, p90, p99 = (_nearest_rank(absolute, q) for q in (0.50, 0.90, 0.99))
    error_l2, reference_l2, candidate_l2 = float(err @ err), float(exp @ exp), float(act @ act)
    dot = float(exp @ act)
    all_equal = bool(np.all(exp == act))
    if all_equal or (reference_l2 == 0.0 and candidate_l2 == 0.0):
        cosine = 1.0
    elif reference_l2 == 0.0 or candidate_l2 == 0.0:
        cosine = 0.0
    else:
        cosine = min(1.0, max(-1.0, dot / (math.sqrt(reference_l2) * math.sqrt(candidate_l2))))
    return ComparisonReport(
        element_count=reference.size, finite_pair_count=n, max_abs=max_abs, mean_abs=mean_abs, p50_abs=p50,
        p90_abs=p90, p99_abs=p99, relative_l2=_relative_l2(error_l2, reference_l2), cosine_similarity=cosine,
        per_token_relative_l2=None if token_axis is None else _relative_l2_by_axis(reference, candidate, shape,
                                                                                    token_axis),
        per_channel_relative_l2=None if channel_axis is None else _relative_l2_by_axis(reference, candidate, shape,
                                                                                        channel_axis),
        reference_non_finite=_non_finite_counts(reference), candidate_non_finite=_non_finite_counts(candidate),
        non_finite_mismatches=mismatches)
