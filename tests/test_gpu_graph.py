"""HIP-graph replay of the device entry points that a decode loop captures: a dependent GEMV chain ending in
the LM head fused with the greedy top-1, and the fused 18-layer rotary-append + GQA decode step.  The entry
points allocate nothing and clear their own counters and slots with kernels (no memset nodes), so a graph
captured once is replayed; every replay, with eager work and synchronisations between replays, must equal the
eager launches bit for bit."""

import numpy as np
import pytest

from pvlc_testlib import W, f16_bits, log, pvlc, to_dev, to_dev_f32

pytestmark = pytest.mark.gpu


def _capture(fn):
    """Capture fn(stream) into a graph on a side stream (after one warm-up launch there)."""
    import torch
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        fn(side)
    torch.cuda.current_stream().wait_stream(side)
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        fn(torch.cuda.current_stream())
    torch.cuda.synchronize()
    return graph


def test_gemv_chain_and_lm_head_top1_replay_from_a_graph():
    import torch
    log("case: graph replay of x -> W1 x -> W2 (W1 x) -> LM head + top-1")
    w1 = to_dev(f16_bits(1, 2048 * 1024, 0.03))
    w2 = to_dev(f16_bits(2, 1024 * 2048, 0.03))
    head = to_dev(f16_bits(3, 20_000 * 1024, 0.05))
    x = torch.zeros(1024, dtype=torch.float32, device="cuda")
    y1 = torch.empty(2048, dtype=torch.float32, device="cuda")
    y2 = torch.empty(1024, dtype=torch.float32, device="cuda")
    logits = torch.empty(20_000, dtype=torch.float32, device="cuda")
    result = torch.zeros(2, dtype=torch.int32, device="cuda")
    nbytes = pvlc.top1_workspace_bytes()
    ws = torch.empty(nbytes, dtype=torch.uint8, device="cuda")
    pvlc.workspace_init(ws, nbytes)

    def chain(stream):
        pvlc.gemv_f16(w1, x, y1, 2048, 1024, stream)
        pvlc.gemv_f16(w2, y1, y2, 1024, 2048, stream)
        pvlc.lm_head_top1_f16(head, y2, logits, 20_000, 1024, result, ws, nbytes, stream)

    graph = _capture(chain)
    for rep in range(4):
        x.copy_(to_dev_f32(np.random.default_rng(rep).standard_normal(1024).astype(np.float32)))  # eager work
        graph.replay()
        torch.cuda.synchronize()
        got = (y2.clone(), logits.clone(), result.clone())
        result.zero_()
        chain(torch.cuda.current_stream())  # eager launches of the same chain
        torch.cuda.synchronize()
        assert torch.equal(got[0], y2) and torch.equal(got[1], logits), f"replay {rep}"
        assert torch.equal(got[2], result), f"replay {rep}: top-1"
    assert int(ws.view(torch.int32).abs().sum().item()) == 0  # the slots come back cleared


def test_grouped_gemv_stage_replays_from_a_graph():
    """x -> (q, k, v) as one grouped launch -> o over q -> (gate, up) grouped over o's output: every replay,
    with new inputs written eagerly in between, equals the same launches made eagerly."""
    import torch
    log("case: graph replay of grouped q|k|v -> o -> grouped gate|up")
    wq, wk, wv = (to_dev(f16_bits(s, r * 1024, 0.03)) for s, r in ((11, 2048), (12, 256), (13, 256)))
    wo = to_dev(f16_bits(14, 1024 * 2048, 0.03))
    wg, wu = (to_dev(f16_bits(s, 3072 * 1024, 0.03)) for s in (15, 16))
    x = torch.zeros(1024, dtype=torch.float32, device="cuda")
    q, k, v = (torch.empty(r, dtype=torch.float32, device="cuda") for r in (2048, 256, 256))
    o = torch.empty(1024, dtype=torch.float32, device="cuda")
    gate, up = (torch.empty(3072, dtype=torch.float32, device="cuda") for _ in range(2))

    def chain(stream):
        pvlc.gemv_group_f16([(wq, q, 2048), (wk, k, 256), (wv, v, 256)], x, 1024, stream)
        pvlc.gemv_f16(wo, q, o, 1024, 2048, stream)
        pvlc.gemv_group_f16([(wg, gate, 3072), (wu, up, 3072)], o, 1024, stream)

    graph = _capture(chain)
    for rep in range(4):
        x.copy_(to_dev_f32(np.random.default_rng(50 + rep).standard_normal(1024).astype(np.float32)))
        graph.replay()
        torch.cuda.synchronize()
        got = [t.clone() for t in (q, k, v, o, gate, up)]
        chain(torch.cuda.current_stream())
        torch.cuda.synchronize()
        for name, a, b in zip("q k v o gate up".split(), got, (q, k, v, o, gate, up)):
            assert torch.equal(a, b), f"replay {rep}: {name}"


def test_decode_step_replays_from_a_graph():
    import torch
    layers, prefix, capacity = 18, 2047, 2304
    log(f"case: graph replay of the decode step ({layers} layers, T={prefix + 1})")
    nb_per = (capacity + 15) // 16
    kp = torch.zeros(layers * nb_per * 16 * W, dtype=torch.int16, device="cuda")
    vp = torch.zeros_like(kp)
    kp.copy_(to_dev(f16_bits(11, kp.numel(), 0.5)))
    vp.copy_(to_dev(f16_bits(12, vp.numel(), 0.5)))
    q = torch.empty(layers * 2048, dtype=torch.int16, device="cuda")
    nk, nv = to_dev(f16_bits(13, layers * W)), to_dev(f16_bits(14, layers * W))
    out = torch.zeros(layers * 2048, dtype=torch.int16, device="cuda")
    cos, sin = pvlc.rope_table(500000.0, capacity + 8)
    d_cos, d_sin = to_dev_f32(cos), to_dev_f32(sin)
    wsb = pvlc.decode_workspace_bytes(layers, capacity, 0)
    ws = torch.empty(wsb, dtype=torch.uint8, device="cuda")
    pvlc.workspace_init(ws, wsb)
    args = pvlc.paged_decode_args(num_seqs=layers, num_blocks=layers * nb_per, max_blocks_per_seq=nb_per,
                                  key_cache=kp, value_cache=vp, query=q, new_key=nk, new_value=nv, out=out,
                                  workspace=ws, workspace_bytes=wsb, max_context=capacity, uniform_cache_len=prefix,
                                  rope_cos=d_cos, rope_sin=d_sin, rope_rows=capacity + 8)
    q.copy_(to_dev(f16_bits(20, q.numel())))
    graph = _capture(lambda stream: pvlc.paged_decode_f16(args, stream))
    for rep in range(4):
        q.copy_(to_dev(f16_bits(30 + rep, q.numel())))  # eager work: a new query for every replay
        graph.replay()
        torch.cuda.synchronize()
        got = out.clone()
        out.zero_()
        pvlc.paged_decode_f16(args, torch.cuda.current_stream())  # the same step launched eagerly
        torch.cuda.synchronize()
        assert torch.equal(got, out), f"replay {rep}"
        assert pvlc.workspace_error(ws, wsb) == 0
