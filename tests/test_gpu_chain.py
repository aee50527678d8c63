"""The decoder token step on this backend's entry points (bench.TokenChain): per layer a grouped q|k|v GEMV, the
single-layer paged decode (rotary on q and the new key, append, GQA), the o GEMV, a grouped gate|up GEMV and the
down GEMV, then the LM head fused with the greedy top-1 -- the per-layer chain the reference's stack session
issues (crates/pvlc-runtime-web/src/web/decoder_stack_session.rs:4625-4797).  The decode runs on the f32 operands
the projections write (pvlc_hip_paged_decode_f32io), or through fp16 conversions and the fp16 entry point.
Checks, at 3 layers and T=300 and at the bench's shape (18 layers, T=2048, the 103424-row LM head):

- every layer's attention against decode_gqa_f32 (cpu-ref lib.rs:858-927) over that layer's cached rows plus
  the appended row, on the q|k|v the chain computed (q rotated with apply_rope_neox and rounded to fp16 -- from
  its f32 value with f32 operands --, the key likewise), within max-abs 2e-3 and relative L2 1e-2; every layer's
  cache rows bit-exact after the append;
- the top-1 result names a maximal logit and carries its bits;
- replays of the step captured in a HIP graph, with eager work and synchronisations between them, equal the
  eager step bit for bit in every buffer the step writes.
"""

import numpy as np
import pytest

import bench
import oracle as O
from pvlc_testlib import W, check_close, from_dev, log, pvlc, rope_k_f16, widen

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("layers,context,capacity,head_rows,f32_operands",
                         [(3, 300, 320, 20_000, True), (3, 300, 320, 20_000, False),
                          (18, 2048, 2304, 103_424, True), (18, 2048, 2304, 103_424, False)])
def test_token_chain_against_the_oracle_and_replayed_from_a_graph(layers, context, capacity, head_rows,
                                                                  f32_operands):
    import torch
    log(f"case: decoder token chain, {layers} layers, T={context}, f32 operands {f32_operands}")
    chain = bench.TokenChain(pvlc, torch, layers, context, capacity, head_rows=head_rows, seed=5,
                             f32_operands=f32_operands)
    stream = torch.cuda.current_stream()
    before = []
    for l in range(layers):
        kr = torch.empty((context - 1) * W, dtype=torch.float16, device="cuda")
        vr = torch.empty_like(kr)
        off = l * chain.nb * 16 * W
        pvlc.kv_unpack_f16(chain.kp[off:], chain.vp[off:], context - 1, kr, vr, chain.nb)
        before.append((from_dev(kr.view(torch.int16)), from_dev(vr.view(torch.int16))))
    chain.step(stream)
    torch.cuda.synchronize()
    pos = context - 1
    for l in range(layers):
        if f32_operands:
            qkv = chain.qkv32[l].cpu().numpy()
            q = widen(O.f32_to_f16(O.rope_neox_f32(qkv[:2048], 16, 128, 128, [pos] * 16, 500000.0)))
            k_new = O.f32_to_f16(O.rope_neox_f32(qkv[2048:2304], 2, 128, 128, [pos] * 2, 500000.0))
            v_new = O.f32_to_f16(qkv[2304:2560])
            got = chain.attn32[l].cpu().numpy()
        else:
            qkv = from_dev(chain.qkv16[l].view(torch.int16))
            q = O.rope_neox_f32(widen(qkv[:2048]), 16, 128, 128, [pos] * 16, 500000.0)
            k_new = rope_k_f16(qkv[2048:2304], pos)
            v_new = qkv[2304:2560]
            got = widen(from_dev(chain.attn16[l].view(torch.int16)))
        keys = np.concatenate([before[l][0], k_new])
        values = np.concatenate([before[l][1], v_new])
        want = O.decode_gqa_f32(q, widen(keys), widen(values), context, 16, 2, 128)
        check_close(got, want, f"chain layer {l}")
        kr = torch.empty(context * W, dtype=torch.float16, device="cuda")
        vr = torch.empty_like(kr)
        off = l * chain.nb * 16 * W
        pvlc.kv_unpack_f16(chain.kp[off:], chain.vp[off:], context, kr, vr, chain.nb)
        np.testing.assert_array_equal(from_dev(kr.view(torch.int16)), keys)
        np.testing.assert_array_equal(from_dev(vr.view(torch.int16)), values)
    logits = chain.logits.cpu().numpy()
    index, bits = (int(v) for v in chain.result.cpu().numpy().view(np.uint32))
    assert logits[index] == logits.max() and logits[:index].max(initial=-np.inf) < logits[index]
    assert np.float32(logits[index]).view(np.uint32) == bits

    eager = chain.state()
    graph = chain.capture(chain.step)
    for rep in range(3):
        for t in chain.attn16 + chain.qkv16 + chain.attn32 + chain.qkv32:
            t.zero_()  # eager work between replays
        chain.result.zero_()
        graph.replay()
        torch.cuda.synchronize()
        got = chain.state()
        assert all(torch.equal(a, b) for a, b in zip(eager, got)), f"replay {rep} differs from the eager step"
