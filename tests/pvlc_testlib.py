"""Shared helpers of the GPU parity tests: seeded fp16 inputs, host packing
into the blocked device layout (independent numpy code), and the tolerance
check of the north star (fp16 output, f32 accumulation: max-abs 2e-3 and
relative L2 1e-2)."""

import sys

import numpy as np

import oracle as O
from oracle.comparison import NATIVE_DECODE_POLICY, compare_f32  # noqa: F401 (re-exported)
from __graft_entry__ import load_package

pvlc = load_package()

ATOL = 2e-3
REL_L2 = 1e-2
W = 256  # one cache row, both kv heads


def f16_bits(seed, n, scale=1.0):
    return O.normal_f16(seed, n, scale)


def widen(bits):
    return O.f16_to_f32(bits)


def check_close(actual, expected, label="", atol=ATOL, rel=REL_L2, policy=None):
    """The reference's comparison report (compare_f32, crates/pvlc-testkit/src/lib.rs:69-170, restated in
    oracle/comparison.py): every metric is printed; the north-star bound (max-abs `atol`, relative L2 `rel`) is
    asserted, and with `policy` (a ComparisonPolicy, e.g. the reference's native decode policy) every metric of
    that policy as well.  Returns (max_abs, rel_l2)."""
    actual = np.asarray(actual, np.float32).ravel()
    expected = np.asarray(expected, np.float32).ravel()
    assert np.all(np.isfinite(actual)), f"{label}: non-finite output"
    r = compare_f32(expected, actual)
    print(f"[parity] {label}: max_abs={r.max_abs:.3e} mean_abs={r.mean_abs:.3e} p99_abs={r.p99_abs:.3e} "
          f"rel_l2={r.relative_l2:.3e} cos={r.cosine_similarity:.8f}", flush=True)
    assert r.max_abs <= atol, f"{label}: max abs {r.max_abs} > {atol}"
    assert r.relative_l2 <= rel, f"{label}: rel L2 {r.relative_l2} > {rel}"
    if policy is not None:
        violations = r.assess(policy)
        assert not violations, f"{label}: violates {violations} of {policy}"
    return r.max_abs, r.relative_l2


def key_slot(t):
    """Slot of token t inside a 16-token block of the key plane: bits 2 and 3 swapped."""
    t = np.asarray(t)
    return (t & 3) | ((t & 4) << 1) | ((t & 8) >> 1)


def scatter_rows(plane_k, plane_v, k_rows, v_rows, tokens, table):
    """Write rows 0..tokens-1 of one sequence into blocked planes through its block table."""
    t = np.arange(tokens)
    blk = np.asarray(table)[t // 16]
    tt = t % 16
    for h in range(2):
        for d in range(128):
            kidx = ((blk * 2 + h) * 16 + d // 8) * 128 + key_slot(tt) * 8 + d % 8
            vidx = ((blk * 2 + h) * 128 + d) * 16 + tt
            plane_k[kidx] = k_rows.reshape(tokens, 2, 128)[:, h, d]
            plane_v[vidx] = v_rows.reshape(tokens, 2, 128)[:, h, d]


def gather_rows(plane_k, plane_v, tokens, table):
    t = np.arange(tokens)
    blk = np.asarray(table)[t // 16]
    tt = t % 16
    k = np.zeros((tokens, 2, 128), np.uint16)
    v = np.zeros((tokens, 2, 128), np.uint16)
    for h in range(2):
        for d in range(128):
            k[:, h, d] = plane_k[((blk * 2 + h) * 16 + d // 8) * 128 + key_slot(tt) * 8 + d % 8]
            v[:, h, d] = plane_v[((blk * 2 + h) * 128 + d) * 16 + tt]
    return k.ravel(), v.ravel()


def rope_k_f16(k_bits, pos, base=500000.0):
    """Oracle rotary on one appended row [2][128] at `pos`, rounded to fp16."""
    rot = O.rope_neox_f32(widen(k_bits), 2, 128, 128, [pos, pos], base)
    return O.f32_to_f16(rot)


def to_dev(bits):
    import torch
    return torch.from_numpy(np.ascontiguousarray(bits).view(np.int16)).cuda()


def to_dev_i32(a):
    import torch
    return torch.from_numpy(np.ascontiguousarray(a, dtype=np.int32)).cuda()


def to_dev_f32(a):
    import torch
    return torch.from_numpy(np.ascontiguousarray(a, dtype=np.float32)).cuda()


def from_dev(t):
    return t.cpu().numpy().view(np.uint16).ravel()


def log(msg):
    print(msg, flush=True)
    sys.stdout.flush()


def dot_error_ratio(got, weights, x, chain):
    """max over rows of |got - W.x (f64)| / (gamma_chain * sum|W*x|): the standard error bound of an f32 dot
    product whose output passes through `chain` roundings (gamma_m = m*u/(1-m*u), u = 2^-24); <= 1 holds for
    any evaluation order of that depth."""
    u = 2.0 ** -24
    g = chain * u / (1 - chain * u)
    w64 = np.asarray(weights, np.float64)
    x64 = np.asarray(x, np.float64)
    exact = w64 @ x64
    mag = np.abs(w64) @ np.abs(x64)
    err = np.abs(np.asarray(got, np.float64) - exact)
    return float((err / np.maximum(g * mag, 1e-300)).max())
