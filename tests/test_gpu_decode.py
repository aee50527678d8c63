"""GPU parity of the decode hot path against the CPU oracle.

Inputs are seeded N(0,1) drawn as fp16; the oracle runs on the same values
widened exactly to f32 (decode_gqa_f32, cpu-ref lib.rs:858-927).  Bars:
appended rows and cache gathers bit-exact; attention within max-abs 2e-3 and
relative L2 1e-2.  Mirrors the reference's native contract tests
(crates/pvlc-runtime-native/tests/decoder_cached_gqa_native_contract.rs,
decoder_kv_session_native_contract.rs).
"""

import numpy as np
import pytest

import oracle as O
from pvlc_testlib import (NATIVE_DECODE_POLICY, W, check_close, f16_bits, from_dev, gather_rows, log, pvlc, rope_k_f16,
                          scatter_rows, to_dev, to_dev_f32, to_dev_i32, widen)

pytestmark = pytest.mark.gpu
POISON = np.array([0x7FC051A7], np.uint32).view(np.float32)[0]  # runtime-core lib.rs:184


@pytest.fixture(scope="module")
def runtime():
    rt = pvlc.NativeRuntime(0)
    yield rt
    rt.close()


def session_inputs(seed, prefix, capacity):
    keys = widen(f16_bits(seed, capacity * W))
    values = widen(f16_bits(seed + 1, capacity * W))
    keys[prefix * W:] = POISON
    values[prefix * W:] = POISON
    return keys, values


def step_inputs(seed):
    return widen(f16_bits(seed, 2048)), widen(f16_bits(seed + 1, W)), widen(f16_bits(seed + 2, W))


def bits32(a):
    return np.asarray(a, np.float32).view(np.uint32)


def test_session_single_step_config1_shape(runtime):
    prefix, capacity = 1024, 1040
    log(f"case: session step prefix={prefix} capacity={capacity}")
    keys, values = session_inputs(10, prefix, capacity)
    q, k, v = step_inputs(20)
    s = runtime.begin_decoder_kv_session(pvlc.DecoderKvSessionDescriptor(prefix, capacity, keys, values))
    ex = s.step(pvlc.DecoderKvSessionStep(q, k, v))
    assert ex.cache_tokens == prefix + 1 and s.cache_tokens == prefix + 1
    ka = np.concatenate([keys[:prefix * W], k])
    va = np.concatenate([values[:prefix * W], v])
    check_close(ex.attention, O.decode_gqa_f32(q, ka, va, prefix + 1, 16, 2, 128), "session T=1025",
                policy=NATIVE_DECODE_POLICY)
    snap = s.finish()
    assert snap.cache_tokens == prefix + 1 and snap.cache_capacity == capacity
    np.testing.assert_array_equal(bits32(snap.key_cache[:(prefix + 1) * W]), bits32(ka))
    np.testing.assert_array_equal(bits32(snap.value_cache[:(prefix + 1) * W]), bits32(va))
    # The poison tail comes back with its f32 payload.
    assert np.all(bits32(snap.key_cache[(prefix + 1) * W:]) == bits32(POISON))
    assert np.all(bits32(snap.value_cache[(prefix + 1) * W:]) == bits32(POISON))


def rounded(x):
    return np.asarray(x, np.float32).astype(np.float16).astype(np.float32)


@pytest.mark.parametrize("prefix,capacity", [(37, 45), (2047, 2060)])
def test_session_finish_returns_f32_rows_as_given(runtime, prefix, capacity):
    """Rows that fp16 does not hold exactly: finish returns every row bit for bit as it was given (the
    descriptor's and each appended one), as the reference's f32 cache does; the attention is the decode of the
    operands rounded to fp16 once (RNE), checked against the oracle on those rounded values."""
    log(f"case: session f32 rows prefix={prefix} capacity={capacity}")
    rng = np.random.default_rng(prefix)
    keys = rng.standard_normal(capacity * W, dtype=np.float32)
    values = rng.standard_normal(capacity * W, dtype=np.float32)
    keys[prefix * W:] = POISON
    values[prefix * W:] = POISON
    assert np.any(rounded(keys[:prefix * W]) != keys[:prefix * W])
    s = runtime.begin_decoder_kv_session(pvlc.DecoderKvSessionDescriptor(prefix, capacity, keys, values))
    ka, va = keys[:prefix * W].copy(), values[:prefix * W].copy()
    for i in range(3):
        q = rng.standard_normal(2048, dtype=np.float32)
        k = rng.standard_normal(W, dtype=np.float32)
        v = rng.standard_normal(W, dtype=np.float32)
        out = s.step(pvlc.DecoderKvSessionStep(q, k, v)).attention
        ka, va = np.concatenate([ka, k]), np.concatenate([va, v])
        t = prefix + 1 + i
        check_close(out, O.decode_gqa_f32(rounded(q), rounded(ka), rounded(va), t, 16, 2, 128), f"step {i} T={t}",
                    policy=NATIVE_DECODE_POLICY)
    snap = s.finish()
    assert snap.cache_tokens == prefix + 3
    np.testing.assert_array_equal(bits32(snap.key_cache[:(prefix + 3) * W]), bits32(ka))
    np.testing.assert_array_equal(bits32(snap.value_cache[:(prefix + 3) * W]), bits32(va))
    assert np.all(bits32(snap.key_cache[(prefix + 3) * W:]) == bits32(POISON))


@pytest.mark.parametrize("prefix", [1, 2, 15, 16, 17, 63, 64, 65, 127, 128, 129, 255, 256, 257, 511, 1023, 2047])
def test_session_prefix_sweep(runtime, prefix):
    capacity = prefix + 1 + (prefix % 7)
    log(f"case: prefix sweep prefix={prefix} capacity={capacity}")
    keys, values = session_inputs(1000 + prefix, prefix, capacity)
    q, k, v = step_inputs(2000 + prefix)
    s = runtime.begin_decoder_kv_session(pvlc.DecoderKvSessionDescriptor(prefix, capacity, keys, values))
    out = s.step(pvlc.DecoderKvSessionStep(q, k, v)).attention
    ka = np.concatenate([keys[:prefix * W], k])
    va = np.concatenate([values[:prefix * W], v])
    check_close(out, O.decode_gqa_f32(q, ka, va, prefix + 1, 16, 2, 128), f"prefix={prefix}",
                policy=NATIVE_DECODE_POLICY)


def test_session_persistent_steps_and_finish_snapshot(runtime):
    prefix, capacity, steps = 300, 310, 5
    log("case: persistent session 5 steps")
    keys, values = session_inputs(30, prefix, capacity)
    s = runtime.begin_decoder_kv_session(pvlc.DecoderKvSessionDescriptor(prefix, capacity, keys, values))
    ka, va = keys[:prefix * W].copy(), values[:prefix * W].copy()
    for i in range(steps):
        q, k, v = step_inputs(40 + 3 * i)
        out = s.step(pvlc.DecoderKvSessionStep(q, k, v)).attention
        ka, va = np.concatenate([ka, k]), np.concatenate([va, v])
        t = prefix + 1 + i
        check_close(out, O.decode_gqa_f32(q, ka, va, t, 16, 2, 128), f"step {i} T={t}", policy=NATIVE_DECODE_POLICY)
    snap = s.finish()
    assert snap.cache_tokens == prefix + steps
    np.testing.assert_array_equal(bits32(snap.key_cache[:(prefix + steps) * W]), bits32(ka))
    np.testing.assert_array_equal(bits32(snap.value_cache[:(prefix + steps) * W]), bits32(va))
    with pytest.raises(pvlc.PvlcHipError):
        s.step(pvlc.DecoderKvSessionStep(*step_inputs(99)))  # consumed by finish


def test_session_invalid_step_has_no_effect_and_capacity_exhaustion(runtime):
    prefix, capacity = 5, 7
    log("case: invalid step / exhaustion")
    keys, values = session_inputs(50, prefix, capacity)
    s = runtime.begin_decoder_kv_session(pvlc.DecoderKvSessionDescriptor(prefix, capacity, keys, values))
    q, k, v = step_inputs(60)
    bad = q.copy()
    bad[0] = np.nan
    with pytest.raises(pvlc.PvlcHipError) as e:
        s.step(pvlc.DecoderKvSessionStep(bad, k, v))
    assert e.value.invocation_code == "NonFiniteInput" and s.cache_tokens == prefix and not s.poisoned
    with pytest.raises(pvlc.PvlcHipError) as e:
        s.step(pvlc.DecoderKvSessionStep(q, k[:-1], v))
    assert e.value.invocation_code == "LengthMismatch" and s.cache_tokens == prefix
    big = k.copy()
    big[3] = 1e6  # finite f32 outside fp16 storage
    with pytest.raises(pvlc.PvlcHipError) as e:
        s.step(pvlc.DecoderKvSessionStep(q, big, v))
    assert e.value.invocation_code == "NonFiniteInput" and s.cache_tokens == prefix
    s.step(pvlc.DecoderKvSessionStep(q, k, v))
    s.step(pvlc.DecoderKvSessionStep(q, k, v))
    assert s.cache_tokens == capacity
    with pytest.raises(pvlc.PvlcHipError) as e:
        s.step(pvlc.DecoderKvSessionStep(q, k, v))
    assert e.value.invocation_code == "InvalidDecoderGeometry" and s.cache_tokens == capacity
    snap = s.finish()
    np.testing.assert_array_equal(bits32(snap.key_cache[:prefix * W]), bits32(keys[:prefix * W]))


def test_session_failure_after_submission_poisons(runtime):
    log("case: injected failure poisons")
    keys, values = session_inputs(70, 4, 8)
    s = runtime.begin_decoder_kv_session(pvlc.DecoderKvSessionDescriptor(4, 8, keys, values))
    s.fail_next_step_after_submit()
    with pytest.raises(pvlc.PvlcHipError) as e:
        s.step(pvlc.DecoderKvSessionStep(*step_inputs(80)))
    assert e.value.code == "Operation" and s.poisoned and s.cache_tokens == 4
    with pytest.raises(pvlc.PvlcHipError) as e:
        s.step(pvlc.DecoderKvSessionStep(*step_inputs(81)))
    assert e.value.code == "Operation"
    with pytest.raises(pvlc.PvlcHipError) as e:
        s.finish()
    assert e.value.code == "Operation"


def test_expired_gpu_wait_poisons_the_session(runtime):
    """The reference bounds every wait by GPU_WAIT_TIMEOUT (native lib.rs:56) and fails the step with Operation
    (decoder_kv_session.rs:729-735); the step had marked the session poisoned before submitting
    (:513-528).  The hook reports the next wait's deadline as passed while the GPU work runs to completion, so
    no GPU hangs.  A finish whose wait expires fails the same way; a fresh session on the runtime works."""
    log("case: expired GPU wait poisons")
    keys, values = session_inputs(75, 6, 12)
    s = runtime.begin_decoder_kv_session(pvlc.DecoderKvSessionDescriptor(6, 12, keys, values))
    s.step(pvlc.DecoderKvSessionStep(*step_inputs(76)))
    s.expire_next_wait()
    with pytest.raises(pvlc.PvlcHipError) as e:
        s.step(pvlc.DecoderKvSessionStep(*step_inputs(77)))
    assert e.value.code == "Operation" and "did not complete within 30000 ms" in str(e.value)
    assert s.poisoned and s.cache_tokens == 7
    with pytest.raises(pvlc.PvlcHipError) as e:
        s.step(pvlc.DecoderKvSessionStep(*step_inputs(78)))
    assert e.value.code == "Operation"
    del s
    t = runtime.begin_decoder_kv_session(pvlc.DecoderKvSessionDescriptor(6, 12, keys, values))
    q, k, v = step_inputs(79)
    out = t.step(pvlc.DecoderKvSessionStep(q, k, v)).attention
    check_close(out, O.decode_gqa_f32(q, np.concatenate([keys[:6 * W], k]), np.concatenate([values[:6 * W], v]), 7,
                                      16, 2, 128), "after an expired wait")
    t.expire_next_wait()
    with pytest.raises(pvlc.PvlcHipError) as e:
        t.finish()
    assert e.value.code == "Operation"


def test_wait_bound_is_a_runtime_option():
    rt = pvlc.NativeRuntime(0, gpu_wait_timeout_ns=1_500_000_000)
    keys, values = session_inputs(85, 3, 5)
    s = rt.begin_decoder_kv_session(pvlc.DecoderKvSessionDescriptor(3, 5, keys, values))
    s.expire_next_wait()
    with pytest.raises(pvlc.PvlcHipError) as e:
        s.step(pvlc.DecoderKvSessionStep(*step_inputs(86)))
    assert "within 1500 ms" in str(e.value)
    del s
    rt.close()


def test_runtime_destroyed_before_its_sessions():
    """Sessions borrow their runtime (NativeDecoderKvSession<'runtime>, decoder_kv_session.rs:23-30): a runtime
    destroyed while sessions live is released by the last of them, and they keep working until then -- also a
    session kept alive only by an exception's traceback, which is dropped after the runtime."""
    rt = pvlc.NativeRuntime(0)
    keys, values = session_inputs(87, 9, 20)
    a = rt.begin_decoder_kv_session(pvlc.DecoderKvSessionDescriptor(9, 20, keys, values))
    b = rt.begin_decoder_kv_session(pvlc.DecoderKvSessionDescriptor(9, 20, keys, values))
    b.expire_next_wait()
    with pytest.raises(pvlc.PvlcHipError) as e:
        b.step(pvlc.DecoderKvSessionStep(*step_inputs(88)))
    del b
    rt.close()
    q, k, v = step_inputs(89)
    out = a.step(pvlc.DecoderKvSessionStep(q, k, v)).attention
    check_close(out, O.decode_gqa_f32(q, np.concatenate([keys[:9 * W], k]), np.concatenate([values[:9 * W], v]), 10,
                                      16, 2, 128), "session after its runtime was destroyed")
    snap = a.finish()
    assert snap.cache_tokens == 10
    del e  # drops the last reference to the poisoned session, after its runtime


def counter_delta(before, after):
    return {k: after[k] - before[k] for k in before}


@pytest.mark.parametrize("prefix,capacity,launches", [(7, 13, 1), (7000, 7100, 2)])
def test_session_effect_topology(prefix, capacity, launches):
    """Exact per-call effects, as decoder_kv_session_native_contract.rs:411 asserts through its observer:
    creation uploads both planes, clears the workspace with one fill kernel and waits once; a step uploads its
    operands once, launches the decode (one kernel, or the persistent kernel and its merge kernel for contexts
    beyond one round of single-shot workgroups), reads the attention back once and waits once; finish reads both
    planes back and waits once; an invalid step has no effect at all."""
    rt = pvlc.NativeRuntime(0)
    keys, values = session_inputs(140, prefix, capacity)
    c0 = rt.counters()
    s = rt.begin_decoder_kv_session(pvlc.DecoderKvSessionDescriptor(prefix, capacity, keys, values))
    c1 = rt.counters()
    assert counter_delta(c0, c1) == {"kernel_launches": 1, "host_to_device_copies": 2, "device_to_host_copies": 0,
                                     "synchronizations": 1, "sessions_created": 1}
    q, k, v = step_inputs(141)
    ex = s.step(pvlc.DecoderKvSessionStep(q, k, v))
    c2 = rt.counters()
    assert ex.dispatch_count == launches
    assert counter_delta(c1, c2) == {"kernel_launches": launches, "host_to_device_copies": 1,
                                     "device_to_host_copies": 1, "synchronizations": 1, "sessions_created": 0}
    bad = q.copy()
    bad[5] = np.inf
    with pytest.raises(pvlc.PvlcHipError):
        s.step(pvlc.DecoderKvSessionStep(bad, k, v))
    assert rt.counters() == c2
    s.finish()
    c3 = rt.counters()
    assert counter_delta(c2, c3) == {"kernel_launches": 0, "host_to_device_copies": 0, "device_to_host_copies": 2,
                                     "synchronizations": 1, "sessions_created": 0}
    rt.close()


def test_interleaved_sessions_stay_independent(runtime):
    log("case: interleaved sessions")
    a_k, a_v = session_inputs(90, 33, 40)
    b_k, b_v = session_inputs(91, 70, 80)
    a = runtime.begin_decoder_kv_session(pvlc.DecoderKvSessionDescriptor(33, 40, a_k, a_v))
    b = runtime.begin_decoder_kv_session(pvlc.DecoderKvSessionDescriptor(70, 80, b_k, b_v))
    qa, ka, va = step_inputs(92)
    qb, kb, vb = step_inputs(93)
    oa = a.step(pvlc.DecoderKvSessionStep(qa, ka, va)).attention
    ob = b.step(pvlc.DecoderKvSessionStep(qb, kb, vb)).attention
    check_close(oa, O.decode_gqa_f32(qa, np.concatenate([a_k[:33 * W], ka]), np.concatenate([a_v[:33 * W], va]),
                                     34, 16, 2, 128), "session a")
    check_close(ob, O.decode_gqa_f32(qb, np.concatenate([b_k[:70 * W], kb]), np.concatenate([b_v[:70 * W], vb]),
                                     71, 16, 2, 128), "session b")


def test_cached_gqa_one_shot(runtime):
    prefix, capacity = 200, 256
    log("case: run_decoder_cached_gqa")
    keys, values = session_inputs(100, prefix, capacity)
    q, k, v = step_inputs(110)
    ex = runtime.run_decoder_cached_gqa(pvlc.DecoderCachedGqaInvocation(prefix, capacity, q, k, v, keys, values))
    assert ex.cache_tokens == prefix + 1 and ex.cache_capacity == capacity
    ka = np.concatenate([keys[:prefix * W], k])
    va = np.concatenate([values[:prefix * W], v])
    check_close(ex.attention, O.decode_gqa_f32(q, ka, va, prefix + 1, 16, 2, 128), "cached gqa",
                policy=NATIVE_DECODE_POLICY)
    np.testing.assert_array_equal(bits32(ex.key_cache[:(prefix + 1) * W]), bits32(ka))
    np.testing.assert_array_equal(bits32(ex.value_cache[:(prefix + 1) * W]), bits32(va))


def test_wrong_grouping_would_be_detected(runtime):
    # decoder_cached_gqa_native_contract.rs:248-272: the GPU result is far from a
    # swapped-group oracle, so the tolerance check has teeth.
    prefix, capacity = 64, 80
    keys, values = session_inputs(120, prefix, capacity)
    q, k, v = step_inputs(130)
    out = runtime.run_decoder_cached_gqa(
        pvlc.DecoderCachedGqaInvocation(prefix, capacity, q, k, v, keys, values)).attention
    ka = np.concatenate([keys[:prefix * W], k])
    va = np.concatenate([values[:prefix * W], v])
    wrong = O.independent_decode_gqa_f32(q, ka, va, prefix + 1, 16, 2, 128, rotate_groups=True)
    assert np.max(np.abs(out - wrong)) > 0.05


def device_decode(layers, prefix, capacity, seed, rope=True, rotate_query=False, partition=0, positions=None,
                  workspace=None):
    """Contiguous per-layer caches (block_tables NULL), one launch for all layers."""
    import torch
    nb_per = (capacity + 15) // 16
    kp = np.zeros(layers * nb_per * 16 * W, np.uint16)
    vp = np.zeros_like(kp)
    rows_k, rows_v = [], []
    for l in range(layers):
        rk, rv = f16_bits(seed + 10 * l, prefix * W), f16_bits(seed + 10 * l + 1, prefix * W)
        table = np.arange(l * nb_per, (l + 1) * nb_per)
        scatter_rows(kp, vp, rk, rv, prefix, table)
        rows_k.append(rk)
        rows_v.append(rv)
    q = f16_bits(seed + 7, layers * 2048)
    nk = f16_bits(seed + 8, layers * W)
    nv = f16_bits(seed + 9, layers * W)
    rows = max(capacity, 1 if positions is None else int(np.max(positions)) + 1) + 8
    cos, sin = pvlc.rope_table(500000.0, rows)
    d_k, d_v, d_q, d_nk, d_nv = to_dev(kp), to_dev(vp), to_dev(q), to_dev(nk), to_dev(nv)
    d_out = torch.zeros(layers * 2048, dtype=torch.int16, device="cuda")
    d_cos, d_sin = to_dev_f32(cos), to_dev_f32(sin)
    d_pos = to_dev_i32(positions) if positions is not None else None
    if workspace is None:
        wsb = pvlc.decode_workspace_bytes(layers, capacity, partition)
        ws = torch.empty(wsb, dtype=torch.uint8, device="cuda")
        pvlc.workspace_init(ws, wsb)
    else:
        ws, wsb = workspace
    args = pvlc.paged_decode_args(num_seqs=layers, num_blocks=layers * nb_per, max_blocks_per_seq=nb_per,
                                  key_cache=d_k, value_cache=d_v, query=d_q, new_key=d_nk, new_value=d_nv,
                                  out=d_out, workspace=ws, workspace_bytes=wsb, max_context=capacity,
                                  uniform_cache_len=prefix, rope_cos=d_cos if rope else None,
                                  rope_sin=d_sin if rope else None, rope_rows=rows if rope else 0,
                                  positions=d_pos, rotate_query=rotate_query, partition_tokens=partition)
    pvlc.paged_decode_f16(args)
    torch.cuda.synchronize()
    assert pvlc.workspace_error(ws, wsb) == 0
    out = from_dev(d_out)
    kp2, vp2 = from_dev(d_k), from_dev(d_v)
    return dict(q=q, nk=nk, nv=nv, rows_k=rows_k, rows_v=rows_v, out=out, kp=kp2, vp=vp2, nb_per=nb_per,
                cos=cos, sin=sin)


def check_device_layers(r, layers, prefix, rope=True, rotate_query=False, positions=None, label=""):
    for l in range(layers):
        pos = prefix if positions is None else int(positions[l])
        nk = r["nk"][l * W:(l + 1) * W]
        nk_rot = rope_k_f16(nk, pos) if rope else nk
        table = np.arange(l * r["nb_per"], (l + 1) * r["nb_per"])
        gk, gv = gather_rows(r["kp"], r["vp"], prefix + 1, table)
        # cache: prefix untouched, appended (rotated) row bit-exact
        np.testing.assert_array_equal(gk, np.concatenate([r["rows_k"][l], nk_rot]))
        np.testing.assert_array_equal(gv, np.concatenate([r["rows_v"][l], r["nv"][l * W:(l + 1) * W]]))
        q = widen(r["q"][l * 2048:(l + 1) * 2048])
        if rotate_query:
            q = O.rope_neox_f32(q, 16, 128, 128, [pos] * 16, 500000.0)
        want = O.decode_gqa_f32(q, widen(gk), widen(gv), prefix + 1, 16, 2, 128)
        check_close(widen(r["out"][l * 2048:(l + 1) * 2048]), want, f"{label} layer {l}")


def test_config1_rotary_append_at_1024():
    log("case: config 1 (prefix 1024, rotary K at pos 1024, base 500000)")
    r = device_decode(1, 1024, 1040, seed=500)
    check_device_layers(r, 1, 1024, label="config1")


@pytest.mark.parametrize("partition", [0, 48, 64, 128, 160, 192, 256, 304, 320, 336, 384, 512, 1024])
def test_config2_18_layers_at_2048(partition):
    log(f"case: config 2 step (18 layers, T=2048, partition={partition})")
    r = device_decode(18, 2047, 2304, seed=600, partition=partition)
    check_device_layers(r, 18, 2047, label=f"config2 p={partition}")


@pytest.mark.parametrize("prefix,planned", [(1280, 192), (1343, 192), (1344, 256), (1600, 256), (1791, 256),
                                            (1792, 320), (2047, 320), (2239, 320), (2240, 384), (2303, 384)])
def test_config2_sweep_automatic_shapes(prefix, planned):
    """The config-2 sweep (T = 1281..2304, 18 layers, capacity 2304) runs four automatic single-shot shapes:
    192-token partitions (6 waves) up to T = 1344, 256 (8 waves) up to 1792, 320 (10 waves) up to 2240 (the
    headline T = 2048 among them), 384 (12 waves) beyond.  Both ends of each range, against the oracle on every
    layer."""
    assert pvlc.decode_partition(18, prefix + 1) == planned
    log(f"case: config 2 sweep shape T={prefix + 1} (automatic partition {planned})")
    r = device_decode(18, prefix, 2304, seed=3000 + prefix)
    check_device_layers(r, 18, prefix, label=f"sweep T={prefix + 1}")


@pytest.mark.parametrize("layers,prefix,partition", [(1, 2047, 0), (1, 2047, 32), (1, 1999, 32), (1, 2047, 64),
                                                     (1, 299, 16), (1, 1024, 128), (1, 4095, 64), (4, 2047, 0),
                                                     (2, 700, 48), (1, 127, 16)])
def test_many_partitions_and_one_wave_partitions(layers, prefix, partition):
    """Single-shot launches with up to 64 partitions per (layer, kv head) -- the last to arrive merges them all
    (16-byte partials, batches of 4 partials with the 16 elements a thread of the one-wave shape owns) -- and
    partitions of one or two tiles, which run on one-wave workgroups.  Every layer against the oracle, caches
    bit-exact."""
    log(f"case: many partitions layers={layers} T={prefix + 1} partition={partition}")
    r = device_decode(layers, prefix, prefix + 1, seed=4100 + prefix + partition, partition=partition)
    check_device_layers(r, layers, prefix, label=f"parts T={prefix + 1} p={partition}")


def test_arrival_counters_across_launches():
    """One workspace through launches whose partition counts change from launch to launch (up to 64 partitions,
    single partitions between them): the arrival counters are never reset -- every launch adds one generation
    (1024) to each counter it uses -- so every launch finds them ready whatever the previous one left."""
    import torch
    capacity = 2048
    wsb = pvlc.decode_workspace_bytes(2, capacity, 32)
    ws = torch.empty(wsb, dtype=torch.uint8, device="cuda")
    pvlc.workspace_init(ws, wsb)
    for i, (prefix, partition) in enumerate([(2047, 32), (2047, 512), (100, 0), (1500, 48), (33, 32), (2040, 0),
                                             (15, 0), (2047, 64), (999, 320), (2047, 0)]):
        log(f"case: shared workspace launch {i}: T={prefix + 1} partition={partition}")
        r = device_decode(2, prefix, capacity, seed=4300 + i, partition=partition, workspace=(ws, wsb))
        check_device_layers(r, 2, prefix, label=f"shared ws {i} T={prefix + 1} p={partition}")
    counters = ws[256:256 + 16].view(torch.int32).cpu().numpy()
    assert np.all(counters % 1024 == 0) and np.all(counters > 0), counters


def test_rotated_query_and_explicit_positions():
    log("case: rotate query, explicit positions")
    positions = np.array([3, 900, 17], np.int32)
    r = device_decode(3, 700, 720, seed=700, rotate_query=True, positions=positions)
    check_device_layers(r, 3, 700, rotate_query=True, positions=positions, label="rotq")


def test_no_rotary_small_contexts():
    for prefix in (0, 1, 15, 16, 63, 64):
        log(f"case: no rotary prefix={prefix}")
        r = device_decode(2, prefix, max(prefix + 1, 16), seed=800 + prefix, rope=False)
        check_device_layers(r, 2, prefix, rope=False, label=f"norope p={prefix}")


def paged_case(num_seqs, lo, hi, seed, partition=0, log_uniform=False, workspace=None, lens=None):
    """Ragged batch over a shared paged cache with seeded permuted block tables.  Returns the workspace."""
    import torch
    rng = np.random.default_rng(seed)
    if lens is not None:
        lens = np.asarray(lens, np.int64)
    elif log_uniform:
        lens = np.exp(rng.uniform(np.log(lo), np.log(hi), num_seqs)).astype(np.int64)
    else:
        lens = rng.integers(lo, hi + 1, num_seqs)
    cache_lens = lens - 1  # rows already cached; the step appends one
    max_context = int(lens.max())
    max_blocks = (max_context + 15) // 16
    need = [(int(t) + 15) // 16 for t in lens]
    num_blocks = sum(need) + 5
    perm = rng.permutation(num_blocks)
    tables = np.full((num_seqs, max_blocks), -1, np.int32)
    kp = np.zeros(num_blocks * 16 * W, np.uint16)
    vp = np.zeros_like(kp)
    off = 0
    rows = []
    for s in range(num_seqs):
        tables[s, :need[s]] = perm[off:off + need[s]]
        off += need[s]
        n = int(cache_lens[s])
        rk, rv = f16_bits(seed * 100 + 2 * s, n * W), f16_bits(seed * 100 + 2 * s + 1, n * W)
        if n:
            scatter_rows(kp, vp, rk, rv, n, tables[s])
        rows.append((rk, rv))
    q = f16_bits(seed + 1, num_seqs * 2048)
    nk = f16_bits(seed + 2, num_seqs * W)
    nv = f16_bits(seed + 3, num_seqs * W)
    cos, sin = pvlc.rope_table(500000.0, max_context + 1)
    d_k, d_v = to_dev(kp), to_dev(vp)
    d_out = torch.zeros(num_seqs * 2048, dtype=torch.int16, device="cuda")
    if workspace is None:
        wsb = pvlc.decode_workspace_bytes(num_seqs, max_context, partition)
        ws = torch.empty(wsb, dtype=torch.uint8, device="cuda")
        pvlc.workspace_init(ws, wsb)
    else:
        ws, wsb = workspace
    keep = [to_dev(q), to_dev(nk), to_dev(nv), to_dev_i32(tables), to_dev_i32(cache_lens), to_dev_f32(cos),
            to_dev_f32(sin)]
    args = pvlc.paged_decode_args(num_seqs=num_seqs, num_blocks=num_blocks, max_blocks_per_seq=max_blocks,
                                  key_cache=d_k, value_cache=d_v, query=keep[0], new_key=keep[1], new_value=keep[2],
                                  out=d_out, workspace=ws, workspace_bytes=wsb, max_context=max_context,
                                  block_tables=keep[3], cache_lens=keep[4], rope_cos=keep[5], rope_sin=keep[6],
                                  rope_rows=max_context + 1, partition_tokens=partition)
    pvlc.paged_decode_f16(args)
    torch.cuda.synchronize()
    assert pvlc.workspace_error(ws, wsb) == 0
    out, kp2, vp2 = from_dev(d_out), from_dev(d_k), from_dev(d_v)
    for s in range(num_seqs):
        n = int(cache_lens[s])
        gk, gv = gather_rows(kp2, vp2, n + 1, tables[s])
        nk_rot = rope_k_f16(nk[s * W:(s + 1) * W], n)
        np.testing.assert_array_equal(gk, np.concatenate([rows[s][0], nk_rot]))
        np.testing.assert_array_equal(gv, np.concatenate([rows[s][1], nv[s * W:(s + 1) * W]]))
        want = O.decode_gqa_f32(widen(q[s * 2048:(s + 1) * 2048]), widen(gk), widen(gv), n + 1, 16, 2, 128)
        check_close(widen(out[s * 2048:(s + 1) * 2048]), want, f"paged seq {s} T={n + 1}")
    return ws


@pytest.mark.parametrize("partition", [0, 64, 80, 512])
def test_paged_ragged_batch(partition):
    log(f"case: paged ragged 12 seqs partition={partition}")
    paged_case(12, 1, 3000, seed=900 + partition, partition=partition)


def test_automatic_partition_balances_the_compute_units():
    """Ragged lengths whose 512-token partitions make two items more than two per compute unit (on 256 units):
    with an automatic partition the kernel picks, among P0 + c*P0/4 (c = 0..4), the one with the least
    ceil(items / units) * P, and the merge kernel uses the same partition.  The choice and the unit count are read
    back from the workspace header; outputs match the oracle whatever the choice."""
    lens = [8192] * 15 + [8300]  # 15 * 16 + 17 = 257 partitions of 512 -> 514 items
    log("case: automatic streaming partition, 16 seqs (15 x 8192, 8300)")
    ws = paged_case(16, 0, 0, seed=990, lens=lens)
    words = ws[:16].cpu().numpy().view(np.uint32)
    chosen, units = int(words[1]), int(words[2])
    assert units > 0
    best, expected = None, None
    for c in range(5):
        pc = 512 + c * 128
        items = 2 * sum((t + pc - 1) // pc for t in lens)
        cost = -(-items // units) * pc
        if best is None or cost < best:
            best, expected = cost, pc
    log(f"{units} compute units: partition {chosen} (expected {expected})")
    assert chosen == expected
    if units == 256:
        assert chosen == 640  # 514 items at 512 (3 per unit), 416 at 640 (2 per unit)


def test_paged_maximum_merge_width():
    """Config 5's longest contexts: 32768 rows at 512-token partitions is 64 partitions, the most one merge
    combines (the plan rejects more); a neighbour at 32767 rows and a short one share the launch.  Cache rows
    bit-exact, attention within tolerance of the oracle."""
    log("case: paged decode at 64 partitions per merge (T = 32768, 32767, 1500; partition 512)")
    paged_case(3, 0, 0, seed=970, partition=512, lens=[32768, 32767, 1500])


def test_paged_long_context_split_k():
    log("case: paged long context (8 seqs, log-uniform [1024, 9000], partition 512)")
    paged_case(8, 1024, 9000, seed=950, partition=512, log_uniform=True)


@pytest.mark.parametrize("partition", [0, 32])
def test_more_ragged_sequences_than_the_persistent_kernel_numbers(partition):
    """A ragged batch of 2049 sequences, one more than the persistent kernel numbers in LDS, runs one workgroup
    per (partition, kv head, sequence) at the planned partition, with each sequence's own length and the
    in-kernel merge.  Every sequence's cache rows are checked bit-exact and its attention against the oracle."""
    log(f"case: 2049 ragged seqs T in [1, 48], partition={partition}")
    paged_case(2049, 1, 48, seed=880 + partition, partition=partition)


def test_one_workspace_across_launch_paths_and_partitions():
    # The split-K merge relies on the workspace's sentinels; every launch must restore them, whichever path
    # (single-shot in-kernel merge or streaming partials + merge kernel) and partition stride it used.
    import torch
    wsb = max(pvlc.decode_workspace_bytes(18, 2304, p) for p in (0, 64, 512))
    wsb = max(wsb, pvlc.decode_workspace_bytes(12, 3000, 0), pvlc.decode_workspace_bytes(12, 3000, 64))
    ws = torch.empty(wsb, dtype=torch.uint8, device="cuda")
    pvlc.workspace_init(ws, wsb)
    for i, (kind, part) in enumerate([("uniform", 0), ("ragged", 0), ("uniform", 64), ("uniform", 0),
                                      ("ragged", 64), ("uniform", 512), ("uniform", 0)]):
        log(f"case: shared workspace launch {i}: {kind} partition={part}")
        if kind == "uniform":
            r = device_decode(18, 2047, 2304, seed=1200 + i, partition=part, workspace=(ws, wsb))
            check_device_layers(r, 18, 2047, label=f"shared ws {i}")
        else:
            paged_case(12, 1, 3000, seed=1300 + i, partition=part, workspace=(ws, wsb))


def test_pack_unpack_roundtrip_through_block_table():
    import torch
    log("case: pack/unpack")
    tokens, num_blocks = 100, 12
    rng = np.random.default_rng(5)
    table = rng.permutation(num_blocks)[:7].astype(np.int32)
    k, v = f16_bits(1, tokens * W), f16_bits(2, tokens * W)
    d_k = torch.zeros(num_blocks * 16 * W, dtype=torch.int16, device="cuda")
    d_v = torch.zeros_like(d_k)
    d_t = to_dev_i32(table)
    pvlc.kv_pack_f16(to_dev(k), to_dev(v), tokens, d_k, d_v, num_blocks, block_table=d_t)
    kp, vp = np.zeros(num_blocks * 16 * W, np.uint16), np.zeros(num_blocks * 16 * W, np.uint16)
    scatter_rows(kp, vp, k, v, tokens, table)
    np.testing.assert_array_equal(from_dev(d_k), kp)
    np.testing.assert_array_equal(from_dev(d_v), vp)
    ok, ov = torch.zeros(tokens * W, dtype=torch.int16, device="cuda"), torch.zeros(tokens * W, dtype=torch.int16,
                                                                                      device="cuda")
    pvlc.kv_unpack_f16(d_k, d_v, tokens, ok, ov, num_blocks, block_table=d_t)
    np.testing.assert_array_equal(from_dev(ok), k)
    np.testing.assert_array_equal(from_dev(ov), v)
