"""GPU parity of the prefill projection with fp16 weights (linear_projection_f16_weights, pvlc-wgsl
lib.rs:1836-1964) against the oracle's linear_f32 with a bias (cpu-ref lib.rs:88-140).

The device computes each product as W.(hi + lo), where hi + lo is the activation row scaled by a power of
two and split exactly into two fp16 values (~22 bits), on MFMA with f32 accumulation; the reference widens
the fp16 weights and accumulates in f32.  Both are held to the standard error bound of an f32 dot product
against an f64 evaluation, |y - y64| <= gamma_m * (sum|w*x| + |b|), gamma_m = m*u/(1-m*u), u = 2^-24 --
m = K + 1 for the oracle's sequential sum, m = 2K + 2 for the device (two MFMA products per term) -- plus
2^-21 * sum|w|*|x| for the split.  A dropped depth chunk, a wrong row or column, or a missing scale or
bias is orders of magnitude outside that."""

import numpy as np
import pytest

import oracle as O
from pvlc_testlib import f16_bits, log, pvlc, to_dev, to_dev_f32, widen

pytestmark = pytest.mark.gpu


def bound_ratio(got, w, x, b, chain, split_term):
    u = 2.0 ** -24
    g = chain * u / (1 - chain * u)
    w64, x64, b64 = np.asarray(w, np.float64), np.asarray(x, np.float64), np.asarray(b, np.float64)
    exact = x64 @ w64.T + b64
    mag = np.abs(x64) @ np.abs(w64).T + np.abs(b64)
    allowed = g * mag + (2.0 ** -21 * (np.abs(x64) @ np.abs(w64).T) if split_term else 0.0)
    err = np.abs(np.asarray(got, np.float64) - exact)
    return float((err / np.maximum(allowed, 1e-300)).max())


def run_projection(rows, k, n, seed, x=None, zero_bias=False):
    import torch
    w = f16_bits(seed, n * k, 0.05)
    if x is None:
        x = O.normal_f32(seed + 1, rows * k).reshape(rows, k)
    b = np.zeros(n, np.float32) if zero_bias else O.normal_f32(seed + 2, n)
    wsb = pvlc.linear_projection_workspace_bytes(rows, k)
    ws = torch.empty(wsb, dtype=torch.uint8, device="cuda")
    sentinel = -7.0
    d_out = torch.full((rows * n + 64,), sentinel, dtype=torch.float32, device="cuda")
    pvlc.linear_projection_f16(to_dev_f32(x), to_dev(w), to_dev_f32(b), d_out, rows, k, n, ws, wsb)
    torch.cuda.synchronize()
    got = d_out.cpu().numpy()
    assert np.all(got[rows * n:] == sentinel), "projection wrote past the output"
    return got[:rows * n].reshape(rows, n), widen(w).reshape(n, k), x, b


def check(rows, k, n, got, wf, x, b, label, oracle_rows=None):
    sel = np.arange(rows) if oracle_rows is None else np.asarray(oracle_rows)
    ratio = bound_ratio(got[sel], wf, x[sel], b, 2 * k + 2, True)
    log(f"[parity] projection {label}: max |gpu - f64| / bound = {ratio:.3f}")
    assert np.all(np.isfinite(got))
    assert ratio <= 1.0
    if oracle_rows is None:
        want = O.linear_f32(x, rows, k, wf, b, n).reshape(rows, n)
        assert bound_ratio(want, wf, x, b, k + 1, False) <= 1.0  # the oracle inside its own bound


# decoder prefill shapes (hidden 1024, q 2048, kv 256, MLP 3072) and ragged tiles
@pytest.mark.parametrize("rows,k,n", [(1, 1024, 4), (37, 1024, 2048), (128, 1024, 256), (129, 1024, 260),
                                      (300, 2048, 1024), (200, 3072, 1024), (77, 1024, 2560), (33, 1024, 6144),
                                      # widths off the K-specialised split (one k step, odd steps) and K = 4096
                                      (130, 32, 132), (9, 96, 36), (140, 1056, 200), (70, 4096, 136)])
def test_projection_matches_linear_oracle(rows, k, n):
    log(f"case: projection rows={rows} k={k} n={n}")
    got, wf, x, b = run_projection(rows, k, n, seed=rows * 31 + k + n)
    check(rows, k, n, got, wf, x, b, f"{rows}x{k}x{n}")


def test_projection_at_prefill_size_sampled_rows():
    rows, k, n = 4096, 1024, 2560  # q|k|v of a 4096-token prefill as one matrix
    log("case: projection 4096x1024x2560 (sampled rows)")
    got, wf, x, b = run_projection(rows, k, n, seed=4096)
    check(rows, k, n, got, wf, x, b, "4096x1024x2560", oracle_rows=[0, 1, 127, 128, 2047, 3000, 4094, 4095])


def test_wide_output_and_ragged_rows_sampled():
    """A wide output (7940 columns, not a multiple of the 128-column tile) over ragged rows (2049: a last row tile
    of one row), sampled rows against the f64 bound."""
    rows, k, n = 2049, 1024, 7940
    log("case: projection 2049x1024x7940 (wide tiles, sampled rows)")
    got, wf, x, b = run_projection(rows, k, n, seed=2049)
    check(rows, k, n, got, wf, x, b, "2049x1024x7940", oracle_rows=[0, 1, 127, 128, 1023, 2047, 2048])


def test_rows_far_outside_the_fp16_range_keep_f32_accuracy():
    rows, k, n = 6, 1024, 64
    rng = np.random.default_rng(9)
    x = rng.standard_normal((rows, k)).astype(np.float32)
    x[0] *= np.float32(1e30)   # beyond fp16 (the power-of-two scaling brings it in range)
    x[1] *= np.float32(1e-20)  # far below fp16 normals
    x[2] = 0.0                 # an all-zero row
    x[3, 5] = np.float32(3e20)  # one huge element among ordinary ones
    x[4] = np.float32(65504.0 * 4)
    log("case: projection dynamic range")
    got, wf, xx, b = run_projection(rows, k, n, seed=77, x=x, zero_bias=True)
    check(rows, k, n, got, wf, xx, b, "dynamic range")
    np.testing.assert_array_equal(got[2], b)


@pytest.mark.parametrize("rows,k,n", [(4096, 1024, 6144),   # gate|up at N=4096: 1024 tiles of 128 x 192, two full rounds
                                      (2049, 256, 7940),    # ragged rows and columns (192): uneven XCD blocks
                                      (1100, 96, 16384),    # 3 k steps (192): the ring's tail without a full period
                                      (2048, 128, 8192),    # 512 tiles of 128 x 256 in one round: 256 columns
                                      (1999, 160, 8000)])   # ragged rows and columns, 5 k steps: 256 columns
def test_wide_kernel_writes_every_tile(rows, k, n):
    """Shapes with at least 512 tiles of 128 x 256 run the wide GEMM, 128 x 192 or 128 x 256 tiles (whichever
    needs fewer columns' worth of rounds of two workgroups per compute unit), whose tiles each XCD takes in one
    block of the output: every output element is written (the output starts as NaN) and two rows of every
    128-row tile (its first and last) are within the f64 bound over all columns."""
    import torch
    log(f"case: wide projection rows={rows} k={k} n={n}")
    seed = rows + k + n
    w = f16_bits(seed, n * k, 0.05)
    x = O.normal_f32(seed + 1, rows * k).reshape(rows, k)
    b = O.normal_f32(seed + 2, n)
    wsb = pvlc.linear_projection_workspace_bytes(rows, k)
    ws = torch.empty(wsb, dtype=torch.uint8, device="cuda")
    d_out = torch.full((rows * n + 64,), float("nan"), dtype=torch.float32, device="cuda")
    pvlc.linear_projection_f16(to_dev_f32(x), to_dev(w), to_dev_f32(b), d_out, rows, k, n, ws, wsb)
    torch.cuda.synchronize()
    got = d_out.cpu().numpy()
    assert np.all(np.isnan(got[rows * n:])), "projection wrote past the output"
    got = got[:rows * n].reshape(rows, n)
    assert np.all(np.isfinite(got)), f"{int(np.sum(~np.isfinite(got)))} outputs never written"
    sel = sorted({r for t in range(0, rows, 128) for r in (t, min(t + 127, rows - 1))})
    wf = widen(w).reshape(n, k)
    ratio = bound_ratio(got[sel], wf, x[sel], b, 2 * k + 2, True)
    log(f"[parity] wide projection {rows}x{k}x{n}: {len(sel)} rows, max |gpu - f64| / bound = {ratio:.3f}")
    assert ratio <= 1.0


@pytest.mark.parametrize("rows,k,n", [(4096, 1024, 2560),   # q|k|v at N=4096: 512 tiles of 128 x 160, one round
                                      (4000, 256, 2560),    # ragged last row tile
                                      (3000, 64, 3200)])    # 2 k steps: the ring's prologue and tail only
def test_160_column_tiles_write_every_output(rows, k, n):
    """Widths that are multiples of 160 with more than 512 tiles of 128 x 128 but at most 512 of 128 x 160 run the
    160-column GEMM (its weight loads: waves 2 and 3 repeat waves 0 and 1's third load): every output element is
    written and the first and last rows of every row tile are within the f64 bound over all columns."""
    import torch
    log(f"case: 160-column projection rows={rows} k={k} n={n}")
    seed = rows * 3 + k + n
    w = f16_bits(seed, n * k, 0.05)
    x = O.normal_f32(seed + 1, rows * k).reshape(rows, k)
    b = O.normal_f32(seed + 2, n)
    wsb = pvlc.linear_projection_workspace_bytes(rows, k)
    ws = torch.empty(wsb, dtype=torch.uint8, device="cuda")
    d_out = torch.full((rows * n + 64,), float("nan"), dtype=torch.float32, device="cuda")
    pvlc.linear_projection_f16(to_dev_f32(x), to_dev(w), to_dev_f32(b), d_out, rows, k, n, ws, wsb)
    torch.cuda.synchronize()
    got = d_out.cpu().numpy()
    assert np.all(np.isnan(got[rows * n:])), "projection wrote past the output"
    got = got[:rows * n].reshape(rows, n)
    assert np.all(np.isfinite(got)), f"{int(np.sum(~np.isfinite(got)))} outputs never written"
    sel = sorted({r for t in range(0, rows, 128) for r in (t, min(t + 127, rows - 1))})
    wf = widen(w).reshape(n, k)
    ratio = bound_ratio(got[sel], wf, x[sel], b, 2 * k + 2, True)
    log(f"[parity] 160-column projection {rows}x{k}x{n}: {len(sel)} rows, max |gpu - f64| / bound = {ratio:.3f}")
    assert ratio <= 1.0

