"""The causal prefill with f32 operands (pvlc_hip_paged_prefill_f32io): query, key, value and output in f32, the
format the reference's prefill chain passes between its dispatches (decoder_prefill_mrope_f32 reads the
projections' f32 q/k/v, decoder_prefill_gqa_f32 writes the f32 output; pvlc-wgsl lib.rs:1262-1416, web
decoder_stack_session.rs:5044-5064).

- With inputs that fp16 holds exactly, the f32 entry point leaves the fp16 one's caches and query scratch bit
  for bit -- one workgroup per query block (N=257) and the split-K pair schedule (N=4096 with a workspace).
  Its output carries the softmax weights as hi + lo fp16 pairs: it meets the reference's native decode policy
  against causal_gqa_f32 (N=257: every row; N=4096: 64 rows spread over the query blocks, through the
  identity `row i == decode over i + 1 keys`), and the fp16 entry point (fp16 weights, fp16 output) stays
  within the north-star bound of it.
- With general f32 inputs the query and the keys are rotated from their f32 values and rounded once: the keys
  in the cache equal the oracle's apply_rope_neox of the f32 keys rounded to fp16, bit for bit, and the output
  is within the prefill tolerance of causal_gqa_f32 over the query rotated and rounded the same way."""

import numpy as np
import pytest

import oracle as O
from pvlc_testlib import (NATIVE_DECODE_POLICY, W, check_close, f16_bits, from_dev, gather_rows, log, pvlc, to_dev,
                          to_dev_f32, widen)

pytestmark = pytest.mark.gpu
BASE = 500000.0


def run(n, q, k, v, f32, split):
    """One prefill on fresh caches; q/k/v are fp16 bits (f32=False) or f32 arrays."""
    import torch
    nb = (n + 15) // 16
    cos, sin = pvlc.rope_table(BASE, n)
    d_k = torch.zeros(nb * 16 * W, dtype=torch.int16, device="cuda")
    d_v = torch.zeros_like(d_k)
    scratch = torch.zeros(n * 2048, dtype=torch.int16, device="cuda")
    err = torch.zeros(1, dtype=torch.int32, device="cuda")
    ws = wsb = None
    if split:
        wsb = pvlc.prefill_workspace_bytes(n)
        ws = torch.empty(max(wsb, 256), dtype=torch.uint8, device="cuda")
        pvlc.workspace_init(ws, ws.numel())
    common = dict(tokens=n, num_blocks=nb, key_cache=d_k, value_cache=d_v, query_scratch=scratch,
                  rope_cos=to_dev_f32(cos), rope_sin=to_dev_f32(sin), rope_rows=n, error_word=err,
                  workspace=ws, workspace_bytes=wsb or 0)
    if f32:
        out = torch.full((n * 2048,), float("nan"), dtype=torch.float32, device="cuda")
        pvlc.paged_prefill_f32io(query=to_dev_f32(q), key=to_dev_f32(k), value=to_dev_f32(v), out=out, **common)
    else:
        out = torch.zeros(n * 2048, dtype=torch.int16, device="cuda")
        pvlc.paged_prefill_f16(query=to_dev(q), key=to_dev(k), value=to_dev(v), out=out, **common)
    torch.cuda.synchronize()
    assert int(err.item()) == 0
    got = out.cpu().numpy() if f32 else from_dev(out)
    return got, from_dev(d_k), from_dev(d_v), from_dev(scratch)


@pytest.mark.parametrize("n,split", [(257, False), (4096, True)])
def test_f32_operands_leave_the_fp16_caches_and_meet_the_native_policy(n, split):
    log(f"case: prefill f32 operands vs fp16 entry point and the oracle, N={n}, split={split}")
    q, k, v = f16_bits(n + 1, n * 2048, 0.5), f16_bits(n + 2, n * W, 0.5), f16_bits(n + 3, n * W, 0.5)
    out16, k16, v16, s16 = run(n, q, k, v, False, split)
    out32, k32, v32, s32 = run(n, widen(q), widen(k), widen(v), True, split)
    np.testing.assert_array_equal(k32, k16)
    np.testing.assert_array_equal(v32, v16)
    np.testing.assert_array_equal(s32, s16)
    assert np.all(np.isfinite(out32))
    pos = np.arange(n, dtype=np.uint32)
    q_rot = widen(O.f32_to_f16(O.rope_neox_f32(widen(q), n * 16, 128, 128, np.repeat(pos, 16), BASE)))
    k_rot = widen(O.f32_to_f16(O.rope_neox_f32(widen(k), n * 2, 128, 128, np.repeat(pos, 2), BASE)))
    if n <= 512:
        want = O.causal_gqa_f32(q_rot, k_rot, widen(v), n, 16, 2, 128)
        check_close(out32, want, f"prefill f32 output N={n}", policy=NATIVE_DECODE_POLICY)
    else:
        rows = [16 * b + b % 16 for b in range(0, n // 16, 4)]
        got = out32.reshape(n, 2048)[rows].ravel()
        want = np.concatenate([O.decode_gqa_f32(q_rot[i * 2048:(i + 1) * 2048], k_rot[:(i + 1) * W],
                                                widen(v)[:(i + 1) * W], i + 1, 16, 2, 128) for i in rows])
        check_close(got, want, f"prefill f32 output N={n}, {len(rows)} rows", policy=NATIVE_DECODE_POLICY)
    check_close(widen(out16), out32, f"prefill fp16 output N={n} vs f32 output")


def test_f32_operands_are_rotated_before_their_rounding():
    n = 200
    log(f"case: prefill f32 operands not representable in fp16, N={n}")
    rng = np.random.default_rng(41)
    q = (rng.standard_normal(n * 2048) * 0.5).astype(np.float32)
    k = (rng.standard_normal(n * W) * 0.5).astype(np.float32)
    v = (rng.standard_normal(n * W) * 0.5).astype(np.float32)
    out, kp, vp, scratch = run(n, q, k, v, True, False)
    pos = np.arange(n, dtype=np.uint32)
    q_rot = O.f32_to_f16(O.rope_neox_f32(q, n * 16, 128, 128, np.repeat(pos, 16), BASE))
    k_rot = O.f32_to_f16(O.rope_neox_f32(k, n * 2, 128, 128, np.repeat(pos, 2), BASE))
    gk, gv = gather_rows(kp, vp, n, np.arange((n + 15) // 16))
    np.testing.assert_array_equal(gk, k_rot)
    np.testing.assert_array_equal(gv, O.f32_to_f16(v))
    np.testing.assert_array_equal(scratch, q_rot)
    want = O.causal_gqa_f32(widen(q_rot), widen(k_rot), widen(O.f32_to_f16(v)), n, 16, 2, 128)
    check_close(out, want, f"prefill f32 operands N={n}", policy=NATIVE_DECODE_POLICY)
