"""The decode step with f32 operands (pvlc_hip_paged_decode_f32io): query, new key and value and output in f32,
the format the reference's chain passes between its dispatches (decoder_mrope_f32 reads the projections' f32
q/k/v, decoder_gqa_split_merge_f32 writes the f32 output the o projection reads; pvlc-wgsl lib.rs:1024-1234,
web decoder_stack_session.rs:4698-4729).

- With inputs that fp16 holds exactly, the caches the f32 entry point leaves are bit-identical to the fp16 entry
  point's -- in the single-shot regime (18 layers, T=2048, the in-kernel merge), with one partition (no merge),
  and in the streaming regime (ragged paged batch: persistent kernel + merge kernel).  Its f32 output carries
  the softmax weights as hi + lo fp16 pairs, so on every sequence it meets the reference's native decode policy
  against decode_gqa_f32 (max-abs 4e-4, mean 6e-5, p99 2.5e-4, relative L2 1.5e-4, cosine 0.99999;
  decoder_cached_gqa_native_contract.rs:147-158); the fp16 entry point (fp16 weights, fp16 output) stays within
  the north-star bound of it.
- With general f32 inputs the query and the new key are rotated from their f32 values and rounded once: the
  appended key row equals the oracle's apply_rope_neox of the f32 key rounded to fp16, bit for bit, and the
  output meets the native policy against decode_gqa_f32 over the query rotated and rounded the same way."""

import numpy as np
import pytest

import oracle as O
from pvlc_testlib import NATIVE_DECODE_POLICY, W, check_close, f16_bits, from_dev, gather_rows, log, pvlc, \
    scatter_rows, to_dev, to_dev_f32, to_dev_i32, widen

pytestmark = pytest.mark.gpu


def build_case(lens, seed, paged):
    """Caches for sequences with lens[s] rows attended after the append (cache_lens = lens - 1): seeded
    permuted block tables when paged, else contiguous per-sequence blocks."""
    rng = np.random.default_rng(seed)
    num_seqs = len(lens)
    cache_lens = np.asarray(lens, np.int64) - 1
    max_context = int(max(lens))
    max_blocks = (max_context + 15) // 16
    if paged:
        need = [(int(t) + 15) // 16 for t in lens]
        num_blocks = sum(need) + 3
        perm = rng.permutation(num_blocks)
        tables = np.full((num_seqs, max_blocks), -1, np.int32)
        off = 0
        for s in range(num_seqs):
            tables[s, :need[s]] = perm[off:off + need[s]]
            off += need[s]
    else:
        num_blocks = num_seqs * max_blocks
        tables = np.arange(num_blocks, dtype=np.int32).reshape(num_seqs, max_blocks)
    kp = np.zeros(num_blocks * 16 * W, np.uint16)
    vp = np.zeros_like(kp)
    rows = []
    for s in range(num_seqs):
        n = int(cache_lens[s])
        rk, rv = f16_bits(seed * 100 + 2 * s, n * W), f16_bits(seed * 100 + 2 * s + 1, n * W)
        if n:
            scatter_rows(kp, vp, rk, rv, n, tables[s])
        rows.append((rk, rv))
    return dict(num_seqs=num_seqs, cache_lens=cache_lens, max_context=max_context, max_blocks=max_blocks,
                num_blocks=num_blocks, tables=tables, kp=kp, vp=vp, rows=rows, paged=paged)


def launch(case, q, nk, nv, f32, rotate_query, partition=0, uniform=False):
    """One step on fresh copies of the case's caches; q/nk/nv are fp16 bits (f32=False) or f32 arrays."""
    import torch
    n, mc = case["num_seqs"], case["max_context"]
    d_k, d_v = to_dev(case["kp"]), to_dev(case["vp"])
    cos, sin = pvlc.rope_table(500000.0, mc + 1)
    keep = [to_dev_f32(cos), to_dev_f32(sin), to_dev_i32(case["cache_lens"])]
    if case["paged"]:
        keep.append(to_dev_i32(case["tables"]))
    wsb = pvlc.decode_workspace_bytes(n, mc, partition)
    ws = torch.empty(wsb, dtype=torch.uint8, device="cuda")
    pvlc.workspace_init(ws, wsb)
    common = dict(num_seqs=n, num_blocks=case["num_blocks"], max_blocks_per_seq=case["max_blocks"], key_cache=d_k,
                  value_cache=d_v, workspace=ws, workspace_bytes=wsb, max_context=mc,
                  block_tables=keep[3] if case["paged"] else None,
                  cache_lens=None if uniform else keep[2], uniform_cache_len=int(case["cache_lens"][0]) if uniform else 0,
                  rope_cos=keep[0], rope_sin=keep[1], rope_rows=mc + 1, rotate_query=rotate_query,
                  partition_tokens=partition)
    if f32:
        d_q, d_nk, d_nv = to_dev_f32(q), to_dev_f32(nk), to_dev_f32(nv)
        d_out = torch.full((n * 2048,), float("nan"), dtype=torch.float32, device="cuda")
        args = pvlc.paged_decode_args(query=None, new_key=None, new_value=None, out=None, **common)
        pvlc.paged_decode_f32io(args, d_q, d_nk, d_nv, d_out)
        torch.cuda.synchronize()
        out = d_out.cpu().numpy()
    else:
        d_q, d_nk, d_nv = to_dev(q), to_dev(nk), to_dev(nv)
        d_out = torch.zeros(n * 2048, dtype=torch.int16, device="cuda")
        args = pvlc.paged_decode_args(query=d_q, new_key=d_nk, new_value=d_nv, out=d_out, **common)
        pvlc.paged_decode_f16(args)
        torch.cuda.synchronize()
        out = from_dev(d_out)
    assert pvlc.workspace_error(ws, wsb) == 0
    return out, from_dev(d_k), from_dev(d_v)


@pytest.mark.parametrize("label,lens,paged,uniform,rotate_query", [
    ("18 layers T=2048 (single shot, in-kernel merge)", [2048] * 18, False, True, True),
    ("4 sequences T=40 (one partition, no merge)", [40] * 4, False, True, False),
    ("12 ragged paged sequences (streaming + merge kernel)", [1, 17, 300, 900, 1500, 2047, 2048, 2500, 3000, 64,
                                                               129, 777], True, False, True),
])
def test_f32_operands_leave_the_fp16_caches_and_meet_the_native_policy(label, lens, paged, uniform, rotate_query):
    log(f"case: f32 operands vs fp16 entry point and the oracle, {label}")
    case = build_case(lens, seed=len(lens) * 7 + 3, paged=paged)
    n = case["num_seqs"]
    q, nk, nv = f16_bits(11, n * 2048), f16_bits(12, n * W), f16_bits(13, n * W)
    out16, k16, v16 = launch(case, q, nk, nv, False, rotate_query, uniform=uniform)
    out32, k32, v32 = launch(case, widen(q), widen(nk), widen(nv), True, rotate_query, uniform=uniform)
    np.testing.assert_array_equal(k32, k16)
    np.testing.assert_array_equal(v32, v16)
    assert np.all(np.isfinite(out32))
    for s in range(n):
        t = int(case["cache_lens"][s])
        gk, gv = gather_rows(k32, v32, t + 1, case["tables"][s])
        qs = widen(q[s * 2048:(s + 1) * 2048])
        if rotate_query:
            qs = widen(O.f32_to_f16(O.rope_neox_f32(qs, 16, 128, 128, [t] * 16, 500000.0)))
        want = O.decode_gqa_f32(qs, widen(gk), widen(gv), t + 1, 16, 2, 128)
        check_close(out32[s * 2048:(s + 1) * 2048], want, f"{label}: f32 output seq {s}", policy=NATIVE_DECODE_POLICY)
        check_close(widen(out16[s * 2048:(s + 1) * 2048]), out32[s * 2048:(s + 1) * 2048],
                    f"{label}: fp16 output seq {s} vs f32 output")


def test_f32_operands_are_rotated_before_their_rounding():
    log("case: f32 operands not representable in fp16, rotated then rounded once")
    lens = [700, 1300, 2048, 5]
    case = build_case(lens, seed=29, paged=True)
    n = case["num_seqs"]
    rng = np.random.default_rng(31)
    q = rng.standard_normal(n * 2048).astype(np.float32)
    nk = rng.standard_normal(n * W).astype(np.float32)
    nv = rng.standard_normal(n * W).astype(np.float32)
    out, kp, vp = launch(case, q, nk, nv, True, rotate_query=True)
    for s in range(n):
        t = int(case["cache_lens"][s])
        gk, gv = gather_rows(kp, vp, t + 1, case["tables"][s])
        k_rot = O.f32_to_f16(O.rope_neox_f32(nk[s * W:(s + 1) * W], 2, 128, 128, [t, t], 500000.0))
        np.testing.assert_array_equal(gk, np.concatenate([case["rows"][s][0], k_rot]))
        np.testing.assert_array_equal(gv, np.concatenate([case["rows"][s][1], O.f32_to_f16(nv[s * W:(s + 1) * W])]))
        q_rot = O.f32_to_f16(O.rope_neox_f32(q[s * 2048:(s + 1) * 2048], 16, 128, 128, [t] * 16, 500000.0))
        want = O.decode_gqa_f32(widen(q_rot), widen(gk), widen(gv), t + 1, 16, 2, 128)
        check_close(out[s * 2048:(s + 1) * 2048], want, f"f32 operands seq {s} T={t + 1}",
                    policy=NATIVE_DECODE_POLICY)
