"""GPU parity at the benchmark's own workloads, and the prefill -> decode chain.

Configs 3 and 5 run at their exact seeded lengths, block tables and partitions (``bench.batched_workload``):
64 sequences with T~U[256,8192] at the automatic partition, and 256 sequences with T~logU[1024,32768] at
512-token partitions (the persistent kernel over ~9,000 items, then the merge kernel).  The caches are drawn on
the device as the bench draws them.  Checks:

- every sequence's cache bit-exact after the step: both planes equal their snapshot with exactly the appended
  rows written, each appended key the oracle's rotation (apply_rope_neox, cpu-ref lib.rs:425-467) rounded to
  fp16, so nothing else moved;
- decode_gqa_f32 (cpu-ref lib.rs:858-927) on 8 sequences spread over the length range, within max-abs 2e-3 and
  relative L2 1e-2;
- every sequence against an fp32 torch restatement of the same attention, at the same tolerance.

The chain test prefills a prompt into a paged cache through a permuted block table and then decodes on that
cache, the way a decoder uses the two (crates/pvlc-cpu-ref/tests/decoder_decode_contract.rs:888-1047: a decode
step equals the last row of a full recompute).
"""

import numpy as np
import pytest

import bench
import oracle as O
from pvlc_testlib import (W, check_close, f16_bits, from_dev, gather_rows, log, pvlc, rope_k_f16, to_dev, to_dev_f32,
                          to_dev_i32, widen)

pytestmark = pytest.mark.gpu
BASE = 500000.0


def appended_index(tables, cache_lens):
    """Element offsets of every sequence's appended row in the key and value planes: [seqs, 2, 128] each."""
    s = np.arange(len(cache_lens))
    n = np.asarray(cache_lens, np.int64)
    blk = tables[s, n // 16].astype(np.int64)[:, None, None]
    t = (n % 16)[:, None, None]
    h = np.arange(2)[None, :, None]
    d = np.arange(128)[None, None, :]
    kidx = ((blk * 2 + h) * 16 + d // 8) * 128 + pvlc.key_slot(t) * 8 + d % 8
    vidx = ((blk * 2 + h) * 128 + d) * 16 + t
    return kidx, vidx


def torch_reference(torch, q, k_rows, v_rows, t):
    """fp32 GQA attention of one sequence over t rows: q [16*128], rows [t*256] fp16 device tensors."""
    qf = q.float().view(16, 128)
    kf = k_rows.float().view(t, 2, 128)
    vf = v_rows.float().view(t, 2, 128)
    out = []
    for g in range(2):
        kt = kf[:, g, :].t().contiguous()
        vg = vf[:, g, :].contiguous()
        s = torch.matmul(qf[g * 8:(g + 1) * 8], kt) / np.sqrt(128.0)
        p = torch.softmax(s, dim=1)
        out.append(torch.matmul(p, vg))
    return torch.cat(out, 0).ravel()


def run_batched_exact(config):
    import torch
    wl = bench.batched_workload(config)
    num_seqs, lens, tables, num_blocks = wl["num_seqs"], wl["lens"], wl["tables"], wl["num_blocks"]
    cache_lens = (lens - 1).astype(np.int32)
    max_context = int(lens.max())
    log(f"case: config {config} exact workload: {num_seqs} seqs, sum T {int(lens.sum())}, max T {max_context}, "
        f"partition {wl['partition']}")
    dev = torch.device("cuda")
    gen = torch.Generator(device=dev).manual_seed(config)
    plane = num_blocks * 16 * W
    kp = torch.randn(plane, generator=gen, device=dev, dtype=torch.float32).half()
    vp = torch.randn(plane, generator=gen, device=dev, dtype=torch.float32).half()
    q = torch.randn(num_seqs * 2048, generator=gen, device=dev, dtype=torch.float32).half()
    nk = torch.randn(num_seqs * W, generator=gen, device=dev, dtype=torch.float32).half()
    nv = torch.randn(num_seqs * W, generator=gen, device=dev, dtype=torch.float32).half()
    snap_k, snap_v = kp.clone(), vp.clone()
    out = torch.zeros(num_seqs * 2048, dtype=torch.float16, device=dev)
    cos, sin = pvlc.rope_table(BASE, max_context)
    d_cos, d_sin = to_dev_f32(cos), to_dev_f32(sin)
    d_tables, d_lens = to_dev_i32(tables), to_dev_i32(cache_lens)
    wsb = pvlc.decode_workspace_bytes(num_seqs, max_context, wl["partition"])
    ws = torch.empty(wsb, dtype=torch.uint8, device=dev)
    pvlc.workspace_init(ws, wsb)
    args = pvlc.paged_decode_args(num_seqs=num_seqs, num_blocks=num_blocks, max_blocks_per_seq=tables.shape[1],
                                  key_cache=kp, value_cache=vp, query=q, new_key=nk, new_value=nv, out=out,
                                  workspace=ws, workspace_bytes=wsb, max_context=max_context, block_tables=d_tables,
                                  cache_lens=d_lens, rope_cos=d_cos, rope_sin=d_sin, rope_rows=max_context,
                                  partition_tokens=wl["partition"])
    pvlc.paged_decode_f16(args)
    torch.cuda.synchronize()
    assert pvlc.workspace_error(ws, wsb) == 0
    if wl["partition"] == 0:
        words = ws[:16].cpu().numpy().view(np.uint32)
        chosen, units = int(words[1]), int(words[2])
        log(f"automatic partition chosen on the device: {chosen} ({units} compute units)")
        assert chosen == pvlc.decode_streaming_partition(cache_lens, max_context, units)

    # Cache: the snapshot with exactly the appended rows written (keys rotated at their position, fp16 RNE).
    host_nk = from_dev(nk.view(torch.int16))
    rot = np.concatenate([rope_k_f16(host_nk[s * W:(s + 1) * W], int(cache_lens[s])) for s in range(num_seqs)])
    kidx, vidx = appended_index(tables, cache_lens)
    want_k, want_v = snap_k.view(torch.int16), snap_v.view(torch.int16)
    want_k[torch.from_numpy(kidx.ravel()).to(dev)] = torch.from_numpy(rot.view(np.int16)).to(dev)
    want_v[torch.from_numpy(vidx.ravel()).to(dev)] = nv.view(torch.int16)
    assert torch.equal(want_k, kp.view(torch.int16)), "key plane differs beyond the appended rows"
    assert torch.equal(want_v, vp.view(torch.int16)), "value plane differs beyond the appended rows"
    del want_k, want_v, snap_k, snap_v

    host_out = widen(from_dev(out.view(torch.int16)))
    host_q = from_dev(q.view(torch.int16))
    order = np.argsort(lens)
    oracle_picks = set(order[np.linspace(0, num_seqs - 1, 8).astype(int)].tolist())
    worst = 0.0
    for s in range(num_seqs):
        t = int(lens[s])
        kr = torch.empty(t * W, dtype=torch.float16, device=dev)
        vr = torch.empty_like(kr)
        pvlc.kv_unpack_f16(kp, vp, t, kr, vr, num_blocks, block_table=d_tables[s])
        got = host_out[s * 2048:(s + 1) * 2048]
        if s in oracle_picks:
            want = O.decode_gqa_f32(widen(host_q[s * 2048:(s + 1) * 2048]), widen(from_dev(kr.view(torch.int16))),
                                    widen(from_dev(vr.view(torch.int16))), t, 16, 2, 128)
            check_close(got, want, f"config {config} seq {s} T={t} (oracle)")
        ref = torch_reference(torch, q[s * 2048:(s + 1) * 2048], kr, vr, t).cpu().numpy()
        err = float(np.abs(got - ref).max())
        rel = float(np.linalg.norm(got - ref) / np.linalg.norm(ref))
        worst = max(worst, err)
        assert np.all(np.isfinite(got)) and err <= 2e-3 and rel <= 1e-2, f"config {config} seq {s} T={t}: {err}"
    log(f"config {config}: all {num_seqs} sequences within tolerance of the fp32 restatement (max abs {worst:.2e})")


def test_config3_exact_workload():
    run_batched_exact(3)


def test_config5_exact_workload():
    run_batched_exact(5)


def test_automatic_partition_lengthened_from_2048():
    """Contexts in (65536, 131072] plan 2048-token partitions; these four make 272 items (two rounds on 256
    compute units) and the kernel lengthens the partition (2560 on 256 units: one round) -- the longest spans
    its 4-wave workgroups cover are exercised only from P0 >= 2048.  Cache rows bit-exact, every sequence
    against the oracle."""
    from test_gpu_decode import paged_case
    lens = [68000, 67000, 67500, 66000]
    log("case: automatic partition lengthened from P0 = 2048 (4 seqs, T ~ 66000-68000)")
    ws = paged_case(4, 0, 0, seed=2048, lens=lens)
    words = ws[:16].cpu().numpy().view(np.uint32)
    chosen, units = int(words[1]), int(words[2])
    cache_lens = np.array(lens, np.int32) - 1
    log(f"{units} compute units: partition {chosen}")
    assert chosen == pvlc.decode_streaming_partition(cache_lens, max(lens), units)
    assert 2048 <= chosen <= 4096
    if units == 256:
        assert chosen == 2560


@pytest.mark.parametrize("n,steps", [(300, 3), (1281, 2), (2048, 2)])
def test_prefill_then_decode_on_the_same_paged_cache(n, steps):
    """Prefill n prompt tokens into a paged cache through a permuted block table, then decode `steps` tokens on
    that cache and table (positions n, n+1, ...).  Checks: each decode's appended row and the prefilled rows
    bit-exact; each decode against decode_gqa_f32 over the rows the prefill wrote plus the appended ones; the
    prefill's last row against decode_gqa_f32 over its n rows; and the reference's identity on the device: a
    prefill of n-1 tokens followed by one decode step of token n-1 gives the prefill-of-n's last row (within
    tolerance) and the same cache rows bit for bit."""
    import torch
    log(f"case: prefill {n} then decode {steps} on one paged cache")
    total = n + steps
    rng = np.random.default_rng(n)
    nb = (total + 15) // 16 + 7
    table = rng.permutation(nb)[:(total + 15) // 16].astype(np.int32)
    q = f16_bits(30 * n, total * 2048, 0.5)
    k = f16_bits(30 * n + 1, total * W, 0.5)
    v = f16_bits(30 * n + 2, total * W, 0.5)
    cos, sin = pvlc.rope_table(BASE, total)
    d_cos, d_sin, d_table = to_dev_f32(cos), to_dev_f32(sin), to_dev_i32(table)

    def prefill(m, d_k, d_v):
        out = torch.zeros(m * 2048, dtype=torch.int16, device="cuda")
        err = torch.zeros(1, dtype=torch.int32, device="cuda")
        nbytes = pvlc.prefill_workspace_bytes(m)
        ws = None
        if nbytes:
            ws = torch.empty(nbytes, dtype=torch.uint8, device="cuda")
            pvlc.workspace_init(ws, nbytes)
        keep = [to_dev(q[:m * 2048]), to_dev(k[:m * W]), to_dev(v[:m * W])]
        pvlc.paged_prefill_f16(tokens=m, num_blocks=nb, key_cache=d_k, value_cache=d_v, query=keep[0], key=keep[1],
                               value=keep[2], out=out, block_table=d_table, rope_cos=d_cos, rope_sin=d_sin,
                               rope_rows=total, error_word=err, workspace=ws, workspace_bytes=nbytes)
        torch.cuda.synchronize()
        assert int(err.item()) == 0
        return widen(from_dev(out))

    def decode(pos, d_k, d_v, ragged=False):
        """One decode step at `pos`: a uniform length runs the single-shot kernel through the block table, a
        ragged one (cache_lens given) the persistent kernel and the merge kernel."""
        out = torch.zeros(2048, dtype=torch.int16, device="cuda")
        wsb = pvlc.decode_workspace_bytes(1, total)
        ws = torch.empty(wsb, dtype=torch.uint8, device="cuda")
        pvlc.workspace_init(ws, wsb)
        keep = [to_dev(q[pos * 2048:(pos + 1) * 2048]), to_dev(k[pos * W:(pos + 1) * W]),
                to_dev(v[pos * W:(pos + 1) * W]), to_dev_i32(np.array([pos], np.int32))]
        a = pvlc.paged_decode_args(num_seqs=1, num_blocks=nb, max_blocks_per_seq=len(table), key_cache=d_k,
                                   value_cache=d_v, query=keep[0], new_key=keep[1], new_value=keep[2], out=out,
                                   workspace=ws, workspace_bytes=wsb, max_context=total, block_tables=d_table,
                                   cache_lens=keep[3] if ragged else None, uniform_cache_len=pos, rope_cos=d_cos,
                                   rope_sin=d_sin, rope_rows=total, rotate_query=True)
        pvlc.paged_decode_f16(a)
        torch.cuda.synchronize()
        assert pvlc.workspace_error(ws, wsb) == 0
        return widen(from_dev(out))

    # oracle inputs: rotated queries (f32) and rotated keys rounded to fp16, as both kernels store them
    pos = np.arange(total, dtype=np.uint32)
    qr = O.rope_neox_f32(widen(q), total * 16, 128, 128, np.repeat(pos, 16), BASE)
    kr = O.f32_to_f16(O.rope_neox_f32(widen(k), total * 2, 128, 128, np.repeat(pos, 2), BASE))

    d_k = torch.zeros(nb * 16 * W, dtype=torch.int16, device="cuda")
    d_v = torch.zeros_like(d_k)
    pre = prefill(n, d_k, d_v).reshape(n, 2048)
    check_close(pre[n - 1], O.decode_gqa_f32(qr[(n - 1) * 2048:n * 2048], widen(kr[:n * W]), widen(v[:n * W]), n,
                                             16, 2, 128), f"prefill {n} last row")
    for i in range(steps):
        p = n + i
        got = decode(p, d_k, d_v, ragged=i % 2 == 1)
        gk, gv = gather_rows(from_dev(d_k), from_dev(d_v), p + 1, table)
        np.testing.assert_array_equal(gk, kr[:(p + 1) * W])
        np.testing.assert_array_equal(gv, v[:(p + 1) * W])
        want = O.decode_gqa_f32(qr[p * 2048:(p + 1) * 2048], widen(kr[:(p + 1) * W]), widen(v[:(p + 1) * W]),
                                p + 1, 16, 2, 128)
        check_close(got, want, f"decode at position {p} after prefill {n}")

    # prefill(n-1) + decode(n-1) == prefill(n): last row within tolerance, cache rows bit for bit
    e_k = torch.zeros(nb * 16 * W, dtype=torch.int16, device="cuda")
    e_v = torch.zeros_like(e_k)
    prefill(n - 1, e_k, e_v)
    step = decode(n - 1, e_k, e_v)
    check_close(step, pre[n - 1], f"decode step {n - 1} vs prefill-of-{n} last row")
    f_k = torch.zeros_like(e_k)
    f_v = torch.zeros_like(e_k)
    prefill(n, f_k, f_v)
    ek, ev = gather_rows(from_dev(e_k), from_dev(e_v), n, table)
    fk, fv = gather_rows(from_dev(f_k), from_dev(f_v), n, table)
    np.testing.assert_array_equal(ek, fk)
    np.testing.assert_array_equal(ev, fv)
