"""GPU parity of the causal prefill (config 4 of the benchmark plan) against
the CPU oracle: rotated keys and values land in the paged cache bit-exactly
(apply_rope_neox then fp16 rounding, cpu-ref lib.rs:425-467), and attention
matches causal_gqa_f32 (cpu-ref lib.rs:782-853) on the rotated fp16 inputs
within max-abs 2e-3 and relative L2 1e-2.  At N = 4096 the oracle checks
sampled rows through the identity `row i of causal == decode over i + 1 keys`
(crates/pvlc-cpu-ref/tests/decoder_decode_contract.rs:888-1047)."""

import numpy as np
import pytest

import oracle as O
from pvlc_testlib import W, check_close, f16_bits, from_dev, gather_rows, log, pvlc, to_dev, to_dev_f32, to_dev_i32, widen

pytestmark = pytest.mark.gpu
BASE = 500000.0


def prefill_workspace(n):
    import torch
    nbytes = pvlc.prefill_workspace_bytes(n)
    ws = torch.empty(max(nbytes, 256), dtype=torch.uint8, device="cuda")
    pvlc.workspace_init(ws, ws.numel())
    return ws, nbytes


def run_prefill(n, seed, table=None, num_blocks=None, scale=0.5, rope=True, with_scratch=False, workspace=None,
                q=None, k=None):
    import torch
    nb = num_blocks or (n + 15) // 16
    q = f16_bits(seed, n * 2048, scale) if q is None else q
    k = f16_bits(seed + 1, n * W, scale) if k is None else k
    v = f16_bits(seed + 2, n * W, scale)
    cos, sin = pvlc.rope_table(BASE, n)
    d_k = torch.zeros(nb * 16 * W, dtype=torch.int16, device="cuda")
    d_v = torch.zeros_like(d_k)
    out = torch.zeros(n * 2048, dtype=torch.int16, device="cuda")
    scratch = torch.zeros(n * 2048, dtype=torch.int16, device="cuda") if with_scratch else None
    err = torch.zeros(1, dtype=torch.int32, device="cuda")
    keep = [to_dev(q), to_dev(k), to_dev(v), to_dev_f32(cos), to_dev_f32(sin)]
    d_t = to_dev_i32(table) if table is not None else None
    pvlc.paged_prefill_f16(tokens=n, num_blocks=nb, key_cache=d_k, value_cache=d_v, query=keep[0], key=keep[1],
                           value=keep[2], out=out, query_scratch=scratch, block_table=d_t,
                           rope_cos=keep[3] if rope else None, rope_sin=keep[4] if rope else None,
                           rope_rows=n if rope else 0, error_word=err,
                           workspace=workspace[0] if workspace else None,
                           workspace_bytes=workspace[1] if workspace else 0)
    torch.cuda.synchronize()
    assert int(err.item()) == 0
    tab = table if table is not None else np.arange(nb)
    gk, gv = gather_rows(from_dev(d_k), from_dev(d_v), n, tab)
    # oracle: rotary in f32, keys stored as fp16
    pos = np.arange(n, dtype=np.uint32)
    if rope:
        qr = O.rope_neox_f32(widen(q), n * 16, 128, 128, np.repeat(pos, 16), BASE)
        kr = O.f32_to_f16(O.rope_neox_f32(widen(k), n * 2, 128, 128, np.repeat(pos, 2), BASE))
    else:
        qr, kr = widen(q), k
    np.testing.assert_array_equal(gk, kr)
    np.testing.assert_array_equal(gv, v)
    return widen(from_dev(out)), qr, widen(kr), widen(v), (from_dev(scratch) if with_scratch else None), q


@pytest.mark.parametrize("n", [1, 2, 15, 16, 17, 63, 64, 65, 100, 257])
def test_prefill_small_matches_causal_oracle(n):
    log(f"case: prefill N={n}")
    out, qr, kr, vr, scratch, q = run_prefill(n, seed=1000 + n)
    want = O.causal_gqa_f32(qr, kr, vr, n, 16, 2, 128)
    check_close(out, want, f"prefill N={n}")


def test_prefill_rotated_query_scratch_is_oracle_rotation_rounded():
    n = 40
    out, qr, kr, vr, scratch, q = run_prefill(n, seed=77, with_scratch=True)
    np.testing.assert_array_equal(scratch, O.f32_to_f16(qr))
    # the attention (which rotates its own query fragments) is unaffected by the scratch
    check_close(out, O.causal_gqa_f32(qr, kr, vr, n, 16, 2, 128), "prefill with scratch")


def test_prefill_without_rotary():
    n = 50
    out, qr, kr, vr, scratch, q = run_prefill(n, seed=88, rope=False)
    check_close(out, O.causal_gqa_f32(qr, kr, vr, n, 16, 2, 128), "prefill no rotary")


def test_prefill_through_permuted_block_table():
    n = 300
    log("case: prefill permuted block table")
    rng = np.random.default_rng(3)
    nb = 40
    table = rng.permutation(nb)[:(n + 15) // 16].astype(np.int32)
    out, qr, kr, vr, scratch, q = run_prefill(n, seed=99, table=table, num_blocks=nb)
    check_close(out, O.causal_gqa_f32(qr, kr, vr, n, 16, 2, 128), "prefill paged")


def test_prefill_config4_sampled_rows_at_4096():
    n = 4096
    log("case: prefill config 4 (N=4096, x0.5, rotary 0..4095)")
    out, qr, kr, vr, scratch, q = run_prefill(n, seed=4096)
    out = out.reshape(n, 2048)
    for i in (0, 1, 15, 16, 17, 255, 1000, 2047, 3333, 4095):
        want = O.decode_gqa_f32(qr[i * 2048:(i + 1) * 2048], kr[:(i + 1) * W], vr[:(i + 1) * W], i + 1, 16, 2, 128)
        check_close(out[i], want, f"config4 row {i}")


def sampled_rows_match_decode(out, qr, kr, vr, n, rows, label):
    out = out.reshape(n, 2048)
    for i in rows:
        want = O.decode_gqa_f32(qr[i * 2048:(i + 1) * 2048], kr[:(i + 1) * W], vr[:(i + 1) * W], i + 1, 16, 2, 128)
        check_close(out[i], want, f"{label} row {i}")


@pytest.mark.parametrize("n", [2049, 2100, 3000, 4096])
def test_split_schedule_matches_the_oracle(n):
    """Long query blocks split over two workgroups and merged by the last one to finish (a workspace is
    given): rows on both sides of the split point and the last rows, against decode over i + 1 keys."""
    log(f"case: split prefill N={n}")
    ws = prefill_workspace(n)
    assert ws[1] > 0
    out, qr, kr, vr, scratch, q = run_prefill(n, seed=5000 + n, workspace=ws)
    rows = sorted({0, 17, 2047, 2048, 2100 % n, n - 17, n - 2, n - 1} | {min(n - 1, 2048 + 64 * k) for k in (1, 7)})
    sampled_rows_match_decode(out, qr, kr, vr, n, rows, f"split N={n}")


def test_split_schedule_through_a_permuted_block_table():
    """The split-K pair schedule (a workspace, N > 2048) over a permuted block table with spare blocks and a
    ragged last block: cache rows through the table bit-exact, sampled rows on both sides of the split point
    against decode over i + 1 keys."""
    n, nb = 2500, 200
    log(f"case: split prefill through a permuted block table, N={n}, {nb} blocks")
    rng = np.random.default_rng(11)
    table = rng.permutation(nb)[:(n + 15) // 16].astype(np.int32)
    ws = prefill_workspace(n)
    assert ws[1] > 0
    out, qr, kr, vr, scratch, q = run_prefill(n, seed=2500, table=table, num_blocks=nb, workspace=ws)
    rows = [0, 15, 16, 1023, 1024, 2047, 2048, 2049, 2300, n - 17, n - 2, n - 1]
    sampled_rows_match_decode(out, qr, kr, vr, n, rows, f"split N={n} permuted table")


def test_split_and_unsplit_schedules_agree_and_the_workspace_is_reusable():
    import torch
    n = 4096
    ws = prefill_workspace(n)
    plain = run_prefill(n, seed=42)[0]
    first = run_prefill(n, seed=42, workspace=ws)[0]
    second = run_prefill(n, seed=42, workspace=ws)[0]
    np.testing.assert_array_equal(first, second)  # two parts merge in a fixed order: bit-identical
    assert float(np.abs(first - plain).max()) <= 1e-3
    # every arrival counter is back to zero
    counters = ws[0][:256 * 2].view(torch.int32)
    assert int(counters.abs().sum().item()) == 0


def causal_gqa_fp32_on_device(qr, kr, vr, n):
    """An fp32 restatement of causal_gqa_f32 (cpu-ref lib.rs:782-853) on the device, one query head at a time:
    scores Q_h K_g^T / sqrt(128) in f32 (query head h reads kv head h // 8), future keys masked, f32 softmax,
    then P V_g.  Inputs are the oracle's rotated f32 query and the fp16 keys and values widened; the products
    run on torch's f32 GEMM (no reduced-precision mode)."""
    import torch
    torch.backends.cuda.matmul.allow_tf32 = False
    q = torch.from_numpy(qr.reshape(n, 16, 128)).cuda()
    k = torch.from_numpy(kr.reshape(n, 2, 128)).cuda()
    v = torch.from_numpy(vr.reshape(n, 2, 128)).cuda()
    future = torch.triu(torch.ones(n, n, dtype=torch.bool, device="cuda"), diagonal=1)
    out = torch.empty(n, 16, 128, device="cuda")
    for h in range(16):
        g = h // 8
        s = torch.matmul(q[:, h, :].contiguous(), k[:, g, :].t().contiguous()) / np.sqrt(128.0)
        s.masked_fill_(future, float("-inf"))
        out[:, h, :] = torch.matmul(torch.softmax(s, dim=1), v[:, g, :].contiguous())
    return out.reshape(-1).cpu().numpy()


@pytest.mark.parametrize("split", [False, True])
def test_config4_every_row_and_a_row_of_every_query_block(split):
    """Config 4 (N=4096) in full, in both schedules: every row of the output against the fp32 restatement on
    the device, and one row of each of the 256 query blocks (position 16b + b mod 16) against the oracle through
    the identity `row i of causal == decode over i + 1 keys` (decoder_decode_contract.rs:888-1047) -- so a fault
    confined to some query blocks or to one side of a split cannot pass."""
    n = 4096
    log(f"case: config 4 every row (N=4096, split={split})")
    ws = prefill_workspace(n) if split else None
    out, qr, kr, vr, scratch, q = run_prefill(n, seed=4097, workspace=ws)
    want = causal_gqa_fp32_on_device(qr, kr, vr, n)
    check_close(out, want, f"config4 split={split} all rows vs fp32 restatement")
    per_row = np.abs(out - want).reshape(n, 2048).max(axis=1)
    assert per_row.max() <= 2e-3, f"worst row {int(per_row.argmax())}: {per_row.max()}"
    rows = [16 * b + b % 16 for b in range(n // 16)]
    sampled_rows_match_decode(out, qr, kr, vr, n, rows, f"config4 split={split} oracle")


@pytest.mark.parametrize("n,split", [(1100, False), (3000, True)])
def test_scores_rising_along_the_sequence_move_the_softmax_reference(n, split):
    """Keys whose scores grow by ~41 log2 units along the sequence: the running maximum of every query passes
    its exponent reference several times (the kernel rescales O and the row sums only when the maximum exceeds
    the reference by 2^8), in both schedules, against decode over i + 1 keys."""
    log(f"case: prefill rising scores N={n} split={split}")
    rng = np.random.default_rng(n)
    q = O.f32_to_f16((0.25 + 0.01 * rng.standard_normal(n * 2048)).astype(np.float32))
    c = (10.0 * np.arange(n) / n).astype(np.float32)
    k = O.f32_to_f16((np.repeat(c, W) * (1.0 + 0.1 * rng.standard_normal(n * W))).astype(np.float32))
    ws = prefill_workspace(n) if split else None
    out, qr, kr, vr, scratch, _ = run_prefill(n, seed=n, rope=False, q=q, k=k, workspace=ws)
    rows = [0, 1, 16, 63, 64, 200, n // 2, n - 65, n - 2, n - 1]
    sampled_rows_match_decode(out, qr, kr, vr, n, rows, f"rising N={n}")
