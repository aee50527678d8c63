"""GPU parity of the greedy top-1 (decoder_logits_top1_f32, pvlc-runtime-web decoder_stack_session.rs:308-366)
and of the LM head fused with it, against the oracle's top-1: index and f32 bits bit-exact, including ties
across workgroups, signed zeros, infinities and NaNs, misaligned rows, grid-stride rows and a workspace reused
by consecutive launches (it must come back zeroed)."""

import numpy as np
import pytest

import oracle as O
from pvlc_testlib import dot_error_ratio, f16_bits, log, pvlc, to_dev, to_dev_f32, widen

pytestmark = pytest.mark.gpu


def _workspace():
    import torch
    nbytes = pvlc.top1_workspace_bytes()
    ws = torch.empty(nbytes, dtype=torch.uint8, device="cuda")
    pvlc.workspace_init(ws, nbytes)
    return ws, nbytes


def device_top1(x, ws, offset=0):
    import torch
    buf = np.zeros(x.size + offset, np.float32)
    buf[offset:] = x
    d = to_dev_f32(buf)
    result = torch.zeros(2, dtype=torch.int32, device="cuda")
    pvlc.logits_top1_f32(d[offset:] if offset else d, x.size, result, ws[0], ws[1])
    torch.cuda.synchronize()
    r = result.cpu().numpy().view(np.uint32)
    return int(r[0]), int(r[1])


@pytest.fixture(scope="module")
def ws():
    return _workspace()


@pytest.mark.parametrize("vocab", [1, 2, 3, 255, 256, 4095, 4096, 4097, 103_424, 103_425, 5_000_003])
def test_top1_matches_oracle_on_random_logits(vocab, ws):
    log(f"case: top1 vocab={vocab}")
    x = O.normal_f32(vocab, vocab)
    assert device_top1(x, ws) == O.top1_f32(x)


def test_top1_ties_across_workgroups_pick_the_lowest_index(ws):
    x = O.normal_f32(9, 103_424)
    peak = np.float32(x.max() + 1)
    for picks in ([90_000, 50_000, 7], [103_423, 4096], [0, 103_423]):
        y = x.copy()
        y[picks] = peak
        got = device_top1(y, ws)
        assert got == O.top1_f32(y) and got[0] == min(picks)


def test_top1_total_order_on_special_values(ws):
    nan = np.float32(np.nan)
    base = np.full(70_000, -5.0, np.float32)
    cases = {"signed zeros": {10: -0.0, 60_000: 0.0}, "zero first": {10: 0.0, 60_000: -0.0},
             "inf": {500: np.inf, 69_999: 1e38}, "nan over inf": {500: np.inf, 69_000: nan},
             "negative nan lowest": {}, "all -inf": None}
    for name, plants in cases.items():
        if plants is None:
            y = np.full(70_000, -np.inf, np.float32)
        else:
            y = base.copy() if name != "signed zeros" and name != "zero first" else np.full(70_000, -1.0, np.float32)
            for i, v in plants.items():
                y[i] = v
            if name == "negative nan lowest":
                y[:] = -np.float32(np.nan)
                y[123] = -np.inf
        got = device_top1(y, ws)
        log(f"case: top1 special {name} -> {got}")
        assert got == O.top1_f32(y), name


@pytest.mark.parametrize("offset", [1, 2, 3])
def test_top1_on_a_misaligned_row(offset, ws):
    x = O.normal_f32(40 + offset, 50_001)
    assert device_top1(x, ws, offset) == O.top1_f32(x)


def test_workspace_comes_back_zeroed_across_consecutive_launches(ws):
    import torch
    results = []
    for vocab, seed in ((5_000_003, 1), (17, 2), (103_424, 3), (1, 4), (300_000, 5)):
        x = O.normal_f32(seed, vocab)
        results.append(device_top1(x, ws) == O.top1_f32(x))
    assert all(results)
    assert int(ws[0].view(torch.int32).abs().sum().item()) == 0


def run_lm_head(rows, columns, seed, ws, plant=None):
    import torch
    w = f16_bits(seed, rows * columns, 0.05)
    x = O.normal_f32(seed + 1, columns)
    if plant is not None:  # identical rows 0.5*sign(x): an exact tie far above every random logit
        wr = w.reshape(rows, columns)
        for r in plant:
            wr[r] = O.f32_to_f16(np.sign(x) * 0.5)
    d_w, d_x = to_dev(w), to_dev_f32(x)
    logits = torch.empty(rows, dtype=torch.float32, device="cuda")
    plain = torch.empty(rows, dtype=torch.float32, device="cuda")
    result = torch.zeros(2, dtype=torch.int32, device="cuda")
    result_no_logits = torch.zeros(2, dtype=torch.int32, device="cuda")
    pvlc.lm_head_top1_f16(d_w, d_x, logits, rows, columns, result, ws[0], ws[1])
    pvlc.lm_head_top1_f16(d_w, d_x, None, rows, columns, result_no_logits, ws[0], ws[1])
    pvlc.gemv_f16(d_w, d_x, plain, rows, columns)
    torch.cuda.synchronize()
    got_logits = logits.cpu().numpy()
    r = tuple(int(v) for v in result.cpu().numpy().view(np.uint32))
    r2 = tuple(int(v) for v in result_no_logits.cpu().numpy().view(np.uint32))
    return got_logits, plain.cpu().numpy(), r, r2, widen(w).reshape(rows, columns), x


@pytest.mark.parametrize("rows,columns", [(1, 1024), (9, 1024), (4096, 1024), (4097, 2048), (103_424, 1024),
                                          (20_000, 3072)])
def test_lm_head_top1_matches_gemv_and_oracle(rows, columns, ws):
    log(f"case: lm_head_top1 rows={rows} columns={columns}")
    logits, plain, r, r2, wf, x = run_lm_head(rows, columns, rows + columns, ws)
    np.testing.assert_array_equal(logits.view(np.uint32), plain.view(np.uint32))
    assert r == O.top1_f32(logits) == r2
    assert dot_error_ratio(logits, wf, x, columns // 64 + 6) <= 1.0


def test_lm_head_tie_picks_the_lowest_row(ws):
    logits, _, r, _, _, _ = run_lm_head(103_424, 1024, 99, ws, plant=(90_001, 77, 50_000))
    assert r == O.top1_f32(logits)
    assert r[0] == 77
