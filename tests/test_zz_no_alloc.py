"""pvlc_hip_paged_decode_f16_no_alloc against pvlc_hip_paged_decode_f16.

The no-alloc entry point runs the same kernels with the split-K state in the library's per-device scratch array;
its outputs and caches must equal the workspace entry point's bit for bit, call after call, whatever the previous
call left in the shared scratch: an 18-layer single-shot step (in-kernel merge through the counters), then smaller
launches -- a ragged paged batch on the streaming kernel with an automatic partition (status words, merge kernel)
and a 4-layer single-shot step whose counters are the ones the first call left.  Each call is also checked against
the oracle on a sampled sequence.  Launches beyond the scratch are rejected before any GPU effect.
"""

import numpy as np
import pytest

import oracle as O
from pvlc_testlib import W, check_close, f16_bits, from_dev, gather_rows, log, pvlc, rope_k_f16, scatter_rows, widen

pytestmark = pytest.mark.gpu
BASE = 500000.0


def make_case(num_seqs, lens, seed, paged):
    """Host inputs of one decode launch: lens are rows attended after the append."""
    rng = np.random.default_rng(seed)
    lens = np.asarray(lens, np.int64)
    cache_lens = (lens - 1).astype(np.int32)
    max_context = int(lens.max())
    max_blocks = (max_context + 15) // 16
    if paged:
        need = (lens + 15) // 16
        num_blocks = int(need.sum()) + 3
        perm = rng.permutation(num_blocks).astype(np.int32)
        tables = np.zeros((num_seqs, max_blocks), np.int32)
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
        rk, rv = f16_bits(seed * 50 + 2 * s, n * W), f16_bits(seed * 50 + 2 * s + 1, n * W)
        scatter_rows(kp, vp, rk, rv, n, tables[s])
        rows.append((rk, rv))
    return dict(num_seqs=num_seqs, lens=lens, cache_lens=cache_lens, max_context=max_context, max_blocks=max_blocks,
                num_blocks=num_blocks, tables=tables, paged=paged, kp=kp, vp=vp, rows=rows,
                q=f16_bits(seed + 1, num_seqs * 2048), nk=f16_bits(seed + 2, num_seqs * W),
                nv=f16_bits(seed + 3, num_seqs * W))


def launch(case, no_alloc):
    """Run one decode of `case` through either entry point on fresh copies of its caches."""
    import torch
    from pvlc_testlib import to_dev, to_dev_f32, to_dev_i32
    d_k, d_v = to_dev(case["kp"]), to_dev(case["vp"])
    out = torch.zeros(case["num_seqs"] * 2048, dtype=torch.int16, device="cuda")
    cos, sin = pvlc.rope_table(BASE, case["max_context"])
    keep = [to_dev(case["q"]), to_dev(case["nk"]), to_dev(case["nv"]), to_dev_f32(cos), to_dev_f32(sin),
            to_dev_i32(case["tables"]), to_dev_i32(case["cache_lens"])]
    common = dict(num_seqs=case["num_seqs"], num_blocks=case["num_blocks"], max_blocks_per_seq=case["max_blocks"],
                  key_cache=d_k, value_cache=d_v, query=keep[0], new_key=keep[1], new_value=keep[2], out=out,
                  max_context=case["max_context"], rope_cos=keep[3], rope_sin=keep[4],
                  rope_rows=case["max_context"])
    if case["paged"]:
        common.update(block_tables=keep[5], cache_lens=keep[6])
    else:
        common.update(uniform_cache_len=int(case["cache_lens"][0]))
    if no_alloc:
        err = torch.zeros(1, dtype=torch.int32, device="cuda")
        pvlc.paged_decode_f16_no_alloc(pvlc.paged_decode_args(workspace=None, workspace_bytes=0, **common), err)
        torch.cuda.synchronize()
        error = int(err.item())
    else:
        wsb = pvlc.decode_workspace_bytes(case["num_seqs"], case["max_context"])
        ws = torch.empty(wsb, dtype=torch.uint8, device="cuda")
        pvlc.workspace_init(ws, wsb)
        pvlc.paged_decode_f16(pvlc.paged_decode_args(workspace=ws, workspace_bytes=wsb, **common))
        torch.cuda.synchronize()
        error = pvlc.workspace_error(ws, wsb)
    return from_dev(out), from_dev(d_k), from_dev(d_v), error


def check_pair(case, label):
    ref_out, ref_k, ref_v, ref_err = launch(case, no_alloc=False)
    out, kp, vp, err = launch(case, no_alloc=True)
    assert ref_err == 0 and err == 0
    np.testing.assert_array_equal(out, ref_out, err_msg=f"{label}: attention differs from the workspace entry point")
    np.testing.assert_array_equal(kp, ref_k, err_msg=f"{label}: key plane differs")
    np.testing.assert_array_equal(vp, ref_v, err_msg=f"{label}: value plane differs")
    # one sequence against the oracle: appended row bit-exact, attention within tolerance
    s = int(np.argmax(case["lens"]))
    n = int(case["cache_lens"][s])
    gk, gv = gather_rows(kp, vp, n + 1, case["tables"][s])
    np.testing.assert_array_equal(gk, np.concatenate([case["rows"][s][0], rope_k_f16(case["nk"][s * W:(s + 1) * W], n)]))
    np.testing.assert_array_equal(gv, np.concatenate([case["rows"][s][1], case["nv"][s * W:(s + 1) * W]]))
    want = O.decode_gqa_f32(widen(case["q"][s * 2048:(s + 1) * 2048]), widen(gk), widen(gv), n + 1, 16, 2, 128)
    check_close(widen(out[s * 2048:(s + 1) * 2048]), want, f"{label} seq {s}")


def test_no_alloc_matches_the_workspace_entry_point_call_after_call():
    log("case: no-alloc call 1: 18 layers, T=2048, single shot")
    check_pair(make_case(18, [2048] * 18, seed=31, paged=False), "no-alloc 18 layers T=2048")
    log("case: no-alloc call 2 (smaller): 6 ragged paged sequences, automatic streaming partition")
    check_pair(make_case(6, [700, 3100, 90, 1600, 2999, 17], seed=32, paged=True), "no-alloc ragged 6")
    log("case: no-alloc call 3 (smaller): 4 layers, T=300, single shot")
    check_pair(make_case(4, [300] * 4, seed=33, paged=False), "no-alloc 4 layers T=300")


def test_no_alloc_rejects_launches_beyond_its_scratch():
    import torch
    log("case: no-alloc rejections")
    dummy = torch.zeros(16, dtype=torch.int16, device="cuda")
    err = torch.zeros(1, dtype=torch.int32, device="cuda")
    lens = torch.zeros(256, dtype=torch.int32, device="cuda")
    big = pvlc.paged_decode_args(num_seqs=256, num_blocks=600000, max_blocks_per_seq=2048, key_cache=dummy,
                                 value_cache=dummy, query=dummy, new_key=dummy, new_value=dummy, out=dummy,
                                 workspace=None, workspace_bytes=0, max_context=32768, block_tables=lens,
                                 cache_lens=lens, partition_tokens=512)
    with pytest.raises(pvlc.PvlcHipError) as e:  # 256 x 64 partitions: 132 MiB of split-K state
        pvlc.paged_decode_f16_no_alloc(big, err)
    assert e.value.invocation_code == "InvalidDecoderGeometry" and "bytes of scratch" in str(e.value)
    ws = torch.empty(256, dtype=torch.uint8, device="cuda")
    small = pvlc.paged_decode_args(num_seqs=1, num_blocks=1, max_blocks_per_seq=1, key_cache=dummy,
                                   value_cache=dummy, query=dummy, new_key=dummy, new_value=dummy, out=dummy,
                                   workspace=ws, workspace_bytes=256, max_context=16, uniform_cache_len=3)
    with pytest.raises(pvlc.PvlcHipError) as e:
        pvlc.paged_decode_f16_no_alloc(small, err)
    assert e.value.invocation_code == "LengthMismatch" and "takes no workspace" in str(e.value)
    torch.cuda.synchronize()
    assert int(err.item()) == 0


def _first_call_captured_child():
    """Body of the child process of test_no_alloc_first_call_inside_graph_capture: the process's first
    no-alloc call is made while torch captures its stream into a HIP graph."""
    import torch
    from pvlc_testlib import to_dev, to_dev_f32, to_dev_i32
    case = make_case(4, [2048] * 4, seed=36, paged=False)
    ref_out, ref_k, ref_v, ref_err = launch(case, no_alloc=False)  # workspace entry point, fresh caches
    assert ref_err == 0
    d_k, d_v = to_dev(case["kp"]), to_dev(case["vp"])
    out = torch.zeros(case["num_seqs"] * 2048, dtype=torch.int16, device="cuda")
    err = torch.zeros(1, dtype=torch.int32, device="cuda")
    cos, sin = pvlc.rope_table(BASE, case["max_context"])
    keep = [to_dev(case["q"]), to_dev(case["nk"]), to_dev(case["nv"]), to_dev_f32(cos), to_dev_f32(sin)]
    args = pvlc.paged_decode_args(num_seqs=case["num_seqs"], num_blocks=case["num_blocks"],
                                  max_blocks_per_seq=case["max_blocks"], key_cache=d_k, value_cache=d_v,
                                  query=keep[0], new_key=keep[1], new_value=keep[2], out=out, workspace=None,
                                  workspace_bytes=0, max_context=case["max_context"], rope_cos=keep[3],
                                  rope_sin=keep[4], rope_rows=case["max_context"],
                                  uniform_cache_len=int(case["cache_lens"][0]))
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        pvlc.paged_decode_f16_no_alloc(args, err, torch.cuda.current_stream())
    torch.cuda.synchronize()
    for i in range(3):
        out.zero_()
        graph.replay()
        torch.cuda.synchronize()
        assert int(err.item()) == 0, f"replay {i}: device error bits {int(err.item())}"
        np.testing.assert_array_equal(from_dev(out), ref_out, err_msg=f"replay {i}: attention differs")
        np.testing.assert_array_equal(from_dev(d_k), ref_k, err_msg=f"replay {i}: key plane differs")
        np.testing.assert_array_equal(from_dev(d_v), ref_v, err_msg=f"replay {i}: value plane differs")
        torch.randn(1 << 20, device="cuda").sum().item()  # eager work between replays
    print("capture child ok", flush=True)


def test_no_alloc_first_call_inside_graph_capture():
    """A fresh process whose first no-alloc call (the per-device set-up included) is made under HIP graph
    capture: the set-up launches and waits for nothing, so the call is captured like any other, and three
    replays (eager work and synchronisations between them) equal the workspace entry point bit for bit."""
    import os
    import subprocess
    import sys
    log("case: no-alloc first call inside graph capture (child process)")
    here = os.path.dirname(os.path.abspath(__file__))
    code = (f"import sys; sys.path[:0] = [{here!r}, {os.path.dirname(here)!r}]; "
            "import test_zz_no_alloc as t; t._first_call_captured_child()")
    proc = subprocess.run([sys.executable, "-c", code], capture_output=True, text=True, timeout=100)
    print(proc.stdout[-2000:], proc.stderr[-2000:], flush=True)
    assert proc.returncode == 0, f"child failed ({proc.returncode}): {proc.stderr[-1500:]}"
    assert "capture child ok" in proc.stdout
