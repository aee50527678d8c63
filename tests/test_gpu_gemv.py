"""GPU parity of the decoder GEMV with fp16 weights (gemv_tiled_f16_weights, pvlc-wgsl lib.rs:1770-1835)
against the oracle's linear_f32 with a zero bias (cpu-ref lib.rs:131-140).

Both sides accumulate in f32 in different orders, so the test bounds each against an f64 product with the
standard error bound of a recursive f32 dot product: |fl(w.x) - w.x| <= gamma_m * sum|w*x|,
gamma_m = m*u/(1-m*u), u = 2^-24, where m is the longest chain of roundings one output passes through:
m = columns for the oracle's sequential sum, and columns/64 fused multiply-adds per lane plus a 6-level
cross-lane tree for the kernel (64 lanes share a row).  A dropped chunk, a misplaced column or a wrong row
stride breaks that bound by orders of magnitude.  Rows past the end must stay untouched."""

import numpy as np
import pytest

import oracle as O
from pvlc_testlib import dot_error_ratio, f16_bits, log, pvlc, to_dev, to_dev_f32, widen

pytestmark = pytest.mark.gpu
SENTINEL = -12345.0


def run_gemv(rows, columns, seed, scale=0.05, stream=None):
    import torch
    w = f16_bits(seed, rows * columns, scale)
    x = O.normal_f32(seed + 1, columns)
    d_out = torch.full((rows + 64,), SENTINEL, dtype=torch.float32, device="cuda")
    d_w, d_x = to_dev(w), to_dev_f32(x)
    pvlc.gemv_f16(d_w, d_x, d_out, rows, columns, stream=stream)
    torch.cuda.synchronize()
    got = d_out.cpu().numpy()
    assert np.all(got[rows:] == SENTINEL), "GEMV wrote past the last row"
    return got[:rows], widen(w).reshape(rows, columns), x


def check_against_oracle(rows, columns, got, wf, x):
    want = O.linear_f32(x, 1, columns, wf, np.zeros(rows, np.float32), rows)
    assert np.all(np.isfinite(got))
    oracle_ratio = dot_error_ratio(want, wf, x, columns)
    kernel_ratio = dot_error_ratio(got, wf, x, columns // 64 + 6)
    diff = float(np.abs(got.astype(np.float64) - want).max())
    log(f"[parity] gemv {rows}x{columns}: max|gpu-f64|/bound={kernel_ratio:.3f} max|gpu-oracle|={diff:.3e}")
    assert oracle_ratio <= 1.0, "oracle outside its own f32 bound"
    assert kernel_ratio <= 1.0, "kernel outside the f32 bound of its accumulation order"


# the decoder's projection shapes, rows x columns (gemv_tiled_plan_contract.rs real-width cases): keys/values,
# queries, MLP gate/up, attention output, MLP down, LM head
DECODER_SHAPES = [(256, 1024), (2048, 1024), (3072, 1024), (1024, 2048), (1024, 3072), (103_424, 1024)]


@pytest.mark.parametrize("rows,columns", DECODER_SHAPES)
def test_decoder_projections_match_linear_oracle(rows, columns):
    log(f"case: gemv rows={rows} columns={columns}")
    got, wf, x = run_gemv(rows, columns, seed=rows * 7 + columns)
    check_against_oracle(rows, columns, got, wf, x)


@pytest.mark.parametrize("rows", [1, 7, 9, 63, 4095, 4097, 4110])
@pytest.mark.parametrize("columns", [1024, 2048, 3072])
def test_ragged_row_counts_leave_the_tail_untouched(rows, columns):
    log(f"case: gemv ragged rows={rows} columns={columns}")
    got, wf, x = run_gemv(rows, columns, seed=rows + columns)
    check_against_oracle(rows, columns, got, wf, x)


def test_small_integers_are_exact_and_stream_argument_is_honoured():
    import torch
    rows, columns = 40, 2048
    rng = np.random.default_rng(5)
    wi = rng.integers(-4, 5, (rows, columns)).astype(np.float32)
    xi = rng.integers(-4, 5, columns).astype(np.float32)
    d_w = to_dev(pvlc.f32_to_f16(wi))
    d_x = to_dev_f32(xi)
    d_out = torch.zeros(rows, dtype=torch.float32, device="cuda")
    s = torch.cuda.Stream()
    with torch.cuda.stream(s):
        pvlc.gemv_f16(d_w, d_x, d_out, rows, columns, stream=s)
    s.synchronize()
    np.testing.assert_array_equal(d_out.cpu().numpy(), wi @ xi)
    np.testing.assert_array_equal(O.linear_f32(xi, 1, columns, wi, np.zeros(rows, np.float32), rows), wi @ xi)


@pytest.mark.parametrize("columns,rows", [(1024, (2048, 256, 256)), (1024, (3072, 3072)), (2048, (1024,)),
                                          (3072, (1024, 5, 3, 1))])
def test_grouped_gemv_equals_separate_calls(columns, rows):
    """pvlc_hip_gemv_group_f16: every member's output equals pvlc_hip_gemv_f16 on that member bit for bit
    (q, k, v of a layer; gate and up; ragged members); gemv_f16 itself is checked against the linear oracle
    above, and no member writes past its rows."""
    import torch
    log(f"case: grouped GEMV columns={columns} rows={rows}")
    g = torch.Generator(device="cuda").manual_seed(columns + sum(rows))
    ws = [(torch.randn(r * columns, generator=g, device="cuda") * 0.05).half() for r in rows]
    x = torch.randn(columns, generator=g, device="cuda")
    sep = [torch.full((r,), float("nan"), device="cuda") for r in rows]
    grp = [torch.full((r + 4,), float("nan"), device="cuda") for r in rows]
    for w, o, r in zip(ws, sep, rows):
        pvlc.gemv_f16(w, x, o, r, columns)
    pvlc.gemv_group_f16([(w, o, r) for w, o, r in zip(ws, grp, rows)], x, columns)
    torch.cuda.synchronize()
    for i, (a, b, r) in enumerate(zip(sep, grp, rows)):
        assert torch.equal(a, b[:r]), f"member {i}"
        assert torch.isnan(b[r:]).all(), f"member {i} wrote past its rows"
