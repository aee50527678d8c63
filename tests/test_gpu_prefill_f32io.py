"""The causal prefill with f32 operands (pvlc_hip_paged_prefill_f32io): query, key, value and output in f32, the
format the reference's prefill chain passes between its dispatches (decoder_prefill_mrope_f32 reads the
projections' f32 q/k/v, decoder_prefill_gqa_f32 writes the f32 output; pvlc-wgsl lib.rs:1262-1416, web
decoder_stack_session.rs:5044-5064).

- With inputs that fp16 holds exactly, the f32 entry point is the fp16 one: bit-identical caches and query
  scratch, and the same f32 output before its last rounding -- one workgroup per query block (N=257) and the
  split-K pair schedule (N=4096 with a workspace). The fp16 entry point rounds the normalised output o * (1/l)
  once, from the exact product (the compiler emits v_fma_mixlo_f16 with a zero addend), while the f32 output
  is that product rounded to f32; the f32 output rounded again to fp16 therefore equals the fp16 output
  except where the f32 product is exactly halfway between two fp16 values, and there the fp16 output must be
  the other neighbour of that midpoint.
- With general f32 inputs the query and the keys are rotated from their f32 values and rounded once: the keys
  in the cache equal the oracle's apply_rope_neox of the f32 keys rounded to fp16, bit for bit, and the output
  is within the prefill tolerance of causal_gqa_f32 over the query rotated and rounded the same way."""

import numpy as np
import pytest

import oracle as O
from pvlc_testlib import W, check_close, f16_bits, from_dev, gather_rows, log, pvlc, to_dev, to_dev_f32, widen

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
def test_f32_operands_match_the_fp16_entry_point(n, split):
    log(f"case: prefill f32 operands vs fp16 entry point, N={n}, split={split}")
    q, k, v = f16_bits(n + 1, n * 2048, 0.5), f16_bits(n + 2, n * W, 0.5), f16_bits(n + 3, n * W, 0.5)
    out16, k16, v16, s16 = run(n, q, k, v, False, split)
    out32, k32, v32, s32 = run(n, widen(q), widen(k), widen(v), True, split)
    np.testing.assert_array_equal(k32, k16)
    np.testing.assert_array_equal(v32, v16)
    np.testing.assert_array_equal(s32, s16)
    assert np.all(np.isfinite(out32))
    assert_single_rounding_of(out32, out16)


def assert_single_rounding_of(out32, out16):
    """out16 is out32's exact product rounded once to fp16: equal to RNE(out32) except at fp16 midpoints."""
    twice = O.f32_to_f16(out32)
    diff = np.nonzero(twice != out16)[0]
    log(f"fp16 outputs on a double-rounding midpoint: {diff.size} of {out16.size}")
    assert diff.size <= out16.size // 1000
    a, b = twice[diff].astype(np.int32), out16[diff].astype(np.int32)
    assert np.all(np.abs(a - b) == 1) and np.all((a >> 15) == (b >> 15)), "not fp16 neighbours"
    mid = (widen(twice[diff]).astype(np.float64) + widen(out16[diff]).astype(np.float64)) / 2
    np.testing.assert_array_equal(out32[diff].astype(np.float64), mid)


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
    check_close(out, want, f"prefill f32 operands N={n}")
