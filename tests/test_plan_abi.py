"""Host-only tests of the C ABI: every declared symbol is exported, and the
plan layer reproduces runtime-core's admission rules and error precedence
(crates/pvlc-runtime-core/tests/decoder_kv_session_plan_contract.rs,
decoder_gqa_split_plan_contract.rs, decoder_cached_gqa_plan_contract.rs)."""

import ctypes
import os
import re

import numpy as np
import pytest

from __graft_entry__ import REPO, load_package

pvlc = load_package()
HEADER = os.path.join(REPO, "include", "pvlc_hip.h")
CAP = 40
WIDTH = 256


def declared_functions():
    text = open(HEADER).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(pvlc_hip_\w+)\s*\(", text)) - {"pvlc_hip_status"})


def test_library_exports_every_declared_symbol():
    names = declared_functions()
    assert len(names) >= 25
    lib = ctypes.CDLL(pvlc.LIBRARY_PATH)
    missing = [n for n in names if not hasattr(lib, n)]
    assert not missing, missing
    # and the Python mirror binds each of them with a signature
    assert set(names) <= set(pvlc.SIGNATURES), set(names) - set(pvlc.SIGNATURES)


def caches(prefix=8, cap=CAP, poison=True):
    k = np.arange(cap * WIDTH, dtype=np.float32) / 1024
    v = -np.arange(cap * WIDTH, dtype=np.float32) / 2048
    if poison:  # the reference admits NaN poison after the semantic prefix (runtime-core :925-929)
        k[prefix * WIDTH:] = np.nan
        v[prefix * WIDTH:] = np.nan
    return k, v


def desc(prefix=8, cap=CAP, poison=True, **kw):
    k, v = caches(prefix, cap, poison)
    d = dict(prefix_tokens=prefix, cache_capacity=cap, key_cache=k, value_cache=v)
    d.update(kw)
    return pvlc.DecoderKvSessionDescriptor(**d)


def code(excinfo):
    return excinfo.value.code, excinfo.value.invocation_code


def test_session_plan_pinned_geometry_and_sizes():
    plan = pvlc.plan_kv_session(desc())
    assert (plan.initial_cache_tokens, plan.cache_capacity) == (8, CAP)
    assert (plan.query_elements, plan.key_value_width, plan.cache_elements) == (2048, 256, CAP * 256)
    assert (plan.cache_bytes, plan.attention_bytes) == (CAP * 1024, 8192)
    # split partials at the full capacity: 16 heads x ceil(40/32) chunks x 192 f32
    assert plan.split_partials_bytes == 16 * 2 * 192 * 4


@pytest.mark.parametrize("kw,want", [
    (dict(query_heads=0), ("InvalidInvocation", "ZeroDimension")),
    (dict(prefix_tokens=0), ("InvalidInvocation", "ZeroDimension")),
    (dict(cache_capacity=0), ("InvalidInvocation", "ZeroDimension")),
    (dict(head_dim=256), ("InvalidInvocation", "UnsupportedHeadDimension")),
    (dict(head_dim=64), ("InvalidInvocation", "InvalidDecoderGeometry")),
    (dict(query_heads=8), ("InvalidInvocation", "InvalidDecoderGeometry")),
    (dict(key_value_heads=4), ("InvalidInvocation", "InvalidDecoderGeometry")),
    (dict(query_heads=15), ("InvalidInvocation", "InvalidDecoderGeometry")),
    (dict(prefix_tokens=CAP), ("InvalidInvocation", "InvalidDecoderGeometry")),
])
def test_session_plan_geometry_errors(kw, want):
    with pytest.raises(pvlc.PvlcHipError) as e:
        pvlc.plan_kv_session(desc(**kw))
    assert code(e) == want


def test_session_plan_length_and_finite_precedence():
    k, v = caches()
    with pytest.raises(pvlc.PvlcHipError) as e:
        pvlc.plan_kv_session(pvlc.DecoderKvSessionDescriptor(8, CAP, k[:-1], v))
    assert code(e) == ("InvalidInvocation", "LengthMismatch")
    k2 = k.copy()
    k2[3] = np.inf  # inside the semantic prefix
    with pytest.raises(pvlc.PvlcHipError) as e:
        pvlc.plan_kv_session(pvlc.DecoderKvSessionDescriptor(8, CAP, k2, v[:-1]))
    assert code(e) == ("InvalidInvocation", "LengthMismatch")  # lengths are checked before finiteness
    with pytest.raises(pvlc.PvlcHipError) as e:
        pvlc.plan_kv_session(pvlc.DecoderKvSessionDescriptor(8, CAP, k2, v))
    assert code(e) == ("InvalidInvocation", "NonFiniteInput")
    # poison after the prefix is admitted
    pvlc.plan_kv_session(pvlc.DecoderKvSessionDescriptor(8, CAP, k, v))


def step(q=2048, k=256, v=256):
    return pvlc.DecoderKvSessionStep(np.zeros(q, np.float32), np.zeros(k, np.float32), np.zeros(v, np.float32))


def test_step_plan_uniform_words_and_transition_bounds():
    plan = pvlc.plan_kv_session(desc(prefix=8))
    sp = pvlc.plan_kv_step(plan, 8, step())
    assert sp["cache_tokens_before"] == 8 and sp["cache_tokens_after"] == 9
    assert sp["append_uniform_words"] == [8, 2, 128, CAP]
    assert sp["attention_uniform_words"] == [9, 16, 2, 128]
    assert sp["valid_cache_elements"] == 9 * 256
    assert sp["split_gqa"]["chunk_count"] == 1 and sp["split_gqa"]["uniform_words"][:2] == [9, 1]
    # last append slot, then exhaustion
    assert pvlc.plan_kv_step(plan, CAP - 1)["cache_tokens_after"] == CAP
    for bad in (CAP, 7):
        with pytest.raises(pvlc.PvlcHipError) as e:
            pvlc.plan_kv_step(plan, bad, step())
        assert code(e) == ("InvalidInvocation", "InvalidDecoderGeometry")


@pytest.mark.parametrize("s,want", [
    (step(q=2047), "LengthMismatch"), (step(k=255), "LengthMismatch"), (step(v=257), "LengthMismatch"),
])
def test_step_plan_length_errors(s, want):
    plan = pvlc.plan_kv_session(desc())
    with pytest.raises(pvlc.PvlcHipError) as e:
        pvlc.plan_kv_step(plan, 8, s)
    assert code(e) == ("InvalidInvocation", want)


def test_step_plan_non_finite_operands():
    plan = pvlc.plan_kv_session(desc())
    s = step()
    s.appended_value[5] = np.nan
    with pytest.raises(pvlc.PvlcHipError) as e:
        pvlc.plan_kv_step(plan, 8, s)
    assert code(e) == ("InvalidInvocation", "NonFiniteInput")


def test_split_plan_matches_reference_dispatch_and_span_bound():
    # decoder_gqa_split_plan_contract.rs: 16*ceil(T/32) partial workgroups, 192-f32 records
    p = pvlc.plan_gqa_split(1025)
    assert (p["chunk_size"], p["chunk_count"], p["partial_workgroups"]) == (32, 33, 528)
    assert p["partials_bytes"] == 528 * 192 * 4 and p["merge_workgroups"] == 32
    assert pvlc.plan_gqa_split(2048)["partial_workgroups"] == 1024
    assert pvlc.plan_gqa_split(131040)["partial_workgroups"] == 65520  # the widest admitted span
    with pytest.raises(pvlc.PvlcHipError) as e:
        pvlc.plan_gqa_split(131041)
    assert code(e) == ("InvalidInvocation", "InvalidDecoderGeometry")
    for args in ((0,), (16, 16, 2, 64), (16, 12, 5, 128), (16, 8, 2, 128)):
        with pytest.raises(pvlc.PvlcHipError):
            pvlc.plan_gqa_split(*args)


def test_session_capacity_bound_follows_split_span():
    pvlc.plan_kv_session(desc(prefix=1, cap=131040, poison=False))
    with pytest.raises(pvlc.PvlcHipError) as e:
        pvlc.plan_kv_session(desc(prefix=1, cap=131041, poison=False))
    assert code(e) == ("InvalidInvocation", "InvalidDecoderGeometry")


def test_prefill_token_bound():
    pvlc.plan_prefill(1, 1)
    pvlc.plan_prefill(4096, 4096)
    for tokens, cap in ((0, 10), (11, 10)):
        with pytest.raises(pvlc.PvlcHipError) as e:
            pvlc.plan_prefill(tokens, cap)
        assert code(e) == ("InvalidInvocation", "InvalidDecoderGeometry")


def test_host_fp16_rounding_is_ieee_rne():
    rng = np.random.default_rng(3)
    x = np.concatenate([rng.standard_normal(100000).astype(np.float32) * 7,
                        (rng.random(50000).astype(np.float32) - 0.5) * np.float32(2e-4),
                        np.array([65504, 65519.99, 65520, 1e6, -1e6, 2 ** -25, 2 ** -24, 1.5 * 2 ** -24, 0, -0.0],
                                 np.float32),
                        (np.arange(-2048, 2048, dtype=np.float32) + 0.5) * np.float32(2 ** -10)])
    with np.errstate(over="ignore"):
        want = x.astype(np.float16).view(np.uint16)
    np.testing.assert_array_equal(pvlc.f32_to_f16(x), want)
    allbits = np.arange(65536, dtype=np.uint32).astype(np.uint16)
    back = pvlc.f16_to_f32(allbits)
    ref = allbits.view(np.float16).astype(np.float32)
    fin = np.isfinite(ref)
    np.testing.assert_array_equal(back[fin].view(np.uint32), ref[fin].view(np.uint32))


def test_rope_table_matches_reference_angle_formula():
    import oracle as O
    cos, sin = pvlc.rope_table(500000.0, 64)
    # the oracle's apply_rope_neox rotating unit vectors yields cos/sin of the same angles, bit-exact
    for pos in (0, 1, 17, 63):
        for pair in (0, 1, 31, 63):
            e = np.zeros(128, np.float32)
            e[pair] = 1.0
            r = O.rope_neox_f32(e, 1, 128, 128, [pos], 500000.0)
            assert r[pair].view(np.uint32) == cos[pos, pair].view(np.uint32)
            assert r[pair + 64].view(np.uint32) == sin[pos, pair].view(np.uint32)


def test_decode_workspace_and_partition_rules():
    # balanced single-shot partitions: about 256 workgroups (one per compute unit) in one round,
    # at most 16 partitions per (sequence, kv head), whole 16-token tiles
    # rounded up to the tile capacity of a single-shot shape (4, 8, 12, 16, 20 or 24 tiles)
    assert pvlc.decode_partition(1, 1025) == 128         # 2 units: 5 tiles -> 8, 9 partitions
    assert pvlc.decode_partition(18, 2048) == 320        # 36 units: 19 tiles -> 20, 7 partitions (252 workgroups)
    assert pvlc.decode_partition(18, 2304) == 384        # 36 units: 21 tiles -> 24, 6 partitions
    assert pvlc.decode_partition(64, 512) == 256         # 128 units x 2 partitions of 16 tiles
    assert pvlc.decode_partition(128, 96) == 128         # 256 units: one partition of 6 tiles -> 8
    # streaming partitions once one workgroup would need more than 32 tiles
    assert pvlc.decode_partition(64, 8192) == 512
    assert pvlc.decode_partition(256, 32768) == 512      # at most 64 partitions per merge
    assert pvlc.decode_partition(1, 131040) == 2048
    assert pvlc.decode_workspace_bytes(18, 2048, 256) % 256 == 0
    assert pvlc.decode_workspace_bytes(18, 2048, 63) == 0
    assert pvlc.decode_workspace_bytes(18, 2048, 48) > 0


FAKE = 1 << 20  # a 16-byte-aligned placeholder address, never dereferenced: validation fails first


def _workspace_status(num_seqs, max_context, cache_len, workspace_bytes, partition=0):
    """Status of a launch whose only possible validation failure is the workspace size (the launch
    itself fails without a GPU, after validation)."""
    blocks = (max_context + 15) // 16
    args = pvlc.paged_decode_args(num_seqs=num_seqs, num_blocks=num_seqs * blocks, max_blocks_per_seq=blocks,
                                  key_cache=FAKE, value_cache=FAKE, query=FAKE, new_key=FAKE, new_value=FAKE,
                                  out=FAKE, workspace=FAKE, workspace_bytes=workspace_bytes, max_context=max_context,
                                  uniform_cache_len=cache_len, partition_tokens=partition)
    try:
        pvlc.paged_decode_f16(args)
    except pvlc.PvlcHipError as e:
        return e.code, e.invocation_code
    return None


@pytest.mark.parametrize("num_seqs,max_context", [(1, 1040), (1, 131040), (18, 2304), (7, 300), (64, 8192),
                                                  (100, 40), (256, 4096), (2, 70000)])
def test_auto_workspace_covers_every_uniform_length(num_seqs, max_context):
    # The workspace sized for max_context holds every automatic launch with a shorter uniform
    # cache length (those pick balanced partitions for the rows they attend).
    import torch
    if torch.cuda.is_available():
        pytest.skip("this check relies on the launch failing without a GPU")
    wsb = pvlc.decode_workspace_bytes(num_seqs, max_context, 0)
    for t in sorted({1, 2, 16, 17, 33, 100, 511, 1000, 1025, 2047, 4097, max_context // 3, max_context}):
        if t > max_context:
            continue
        st = _workspace_status(num_seqs, max_context, t - 1, wsb)
        assert st != ("InvalidInvocation", "LengthMismatch"), (num_seqs, max_context, t)
        assert st != ("InvalidInvocation", "InvalidDecoderGeometry"), (num_seqs, max_context, t)
    assert _workspace_status(num_seqs, max_context, max_context - 1, 256) == ("InvalidInvocation", "LengthMismatch")


def test_device_entry_points_validate_before_touching_the_gpu():
    args = pvlc.paged_decode_args(num_seqs=0, num_blocks=1, max_blocks_per_seq=1, key_cache=FAKE, value_cache=FAKE,
                                  query=FAKE, new_key=FAKE, new_value=FAKE, out=FAKE, workspace=FAKE, workspace_bytes=1 << 20,
                                  max_context=16)
    with pytest.raises(pvlc.PvlcHipError) as e:
        pvlc.paged_decode_f16(args)
    assert code(e) == ("InvalidInvocation", "ZeroDimension")
    args = pvlc.paged_decode_args(num_seqs=1, num_blocks=1, max_blocks_per_seq=1, key_cache=FAKE, value_cache=FAKE,
                                  query=FAKE, new_key=FAKE, new_value=FAKE, out=FAKE, workspace=FAKE, workspace_bytes=1 << 20,
                                  max_context=32)
    with pytest.raises(pvlc.PvlcHipError) as e:
        pvlc.paged_decode_f16(args)
    assert code(e) == ("InvalidInvocation", "InvalidDecoderGeometry")
    args = pvlc.paged_decode_args(num_seqs=1, num_blocks=4, max_blocks_per_seq=4, key_cache=FAKE, value_cache=FAKE,
                                  query=FAKE, new_key=FAKE, new_value=FAKE, out=FAKE, workspace=FAKE, workspace_bytes=16,
                                  max_context=64, uniform_cache_len=10)
    with pytest.raises(pvlc.PvlcHipError) as e:
        pvlc.paged_decode_f16(args)
    assert code(e) == ("InvalidInvocation", "LengthMismatch")


def test_runtime_without_gpu_reports_adapter_unavailable():
    import torch
    if torch.cuda.is_available():
        pytest.skip("a GPU is visible")
    with pytest.raises(pvlc.PvlcHipError) as e:
        pvlc.NativeRuntime(0)
    assert e.value.code == "AdapterUnavailable"


def test_prefill_workspace_is_only_needed_for_long_blocks():
    # up to 2048 tokens every query block attends at most 32 steps of 64 keys and runs whole; beyond, block l
    # and block qblocks-1-l share two workgroups: a counter and two partial slabs of 75776 bytes per pair and
    # kv head
    for n in (1, 16, 1000, 2048):
        assert pvlc.prefill_workspace_bytes(n) == 0, n
    for n in (2049, 3000, 4096, 8192):
        pairs = ((n + 15) // 16 + 1) // 2
        counters = -(-(2 * pairs * 4) // 256) * 256
        assert pvlc.prefill_workspace_bytes(n) == counters + 2 * pairs * 2 * 75776, n


def test_prefill_rejects_a_short_or_misaligned_workspace():
    need = pvlc.prefill_workspace_bytes(4096)
    fake = 1 << 20  # never dereferenced: validation fails first
    common = dict(tokens=4096, num_blocks=256, key_cache=fake, value_cache=fake, query=fake, key=fake, value=fake,
                  out=fake)
    with pytest.raises(pvlc.PvlcHipError) as e:
        pvlc.paged_prefill_f16(**common, workspace=fake, workspace_bytes=need - 4)
    assert e.value.invocation_code == "LengthMismatch"
    with pytest.raises(pvlc.PvlcHipError) as e:
        pvlc.paged_prefill_f16(**common, workspace=fake + 4, workspace_bytes=need)
    assert e.value.invocation_code == "LengthMismatch"


def test_f32_operand_decode_rejects_mixed_or_missing_operands():
    """pvlc_hip_paged_decode_f32io takes the query, new key and value and output as f32 arguments: fp16 ones left
    in the args, or a missing f32 one, are rejected before any GPU effect (placeholder addresses, never read)."""
    fake = 1 << 20
    common = dict(num_seqs=1, num_blocks=1, max_blocks_per_seq=1, key_cache=fake, value_cache=fake, workspace=fake,
                  workspace_bytes=1 << 20, max_context=16, uniform_cache_len=0)
    mixed = pvlc.paged_decode_args(query=fake, new_key=None, new_value=None, out=None, **common)
    with pytest.raises(pvlc.PvlcHipError) as e:
        pvlc.paged_decode_f32io(mixed, fake, fake, fake, fake)
    assert code(e) == ("InvalidInvocation", "LengthMismatch") and "must be NULL" in str(e.value)
    bare = pvlc.paged_decode_args(query=None, new_key=None, new_value=None, out=None, **common)
    for missing in range(4):
        ptrs = [fake] * 4
        ptrs[missing] = None
        with pytest.raises(pvlc.PvlcHipError) as e:
            pvlc.paged_decode_f32io(bare, *ptrs)
        assert code(e) == ("InvalidInvocation", "LengthMismatch") and "f32 operand pointer is NULL" in str(e.value)
    # and the fp16 entry point still requires its own operands
    with pytest.raises(pvlc.PvlcHipError) as e:
        pvlc.paged_decode_f16(bare)
    assert code(e) == ("InvalidInvocation", "LengthMismatch")


@pytest.mark.parametrize("operand", ["query", "new_key", "new_value", "out", "key_cache", "value_cache", "workspace"])
def test_decode_rejects_unaligned_operands(operand):
    """The decode reads the query and the cache planes as 16-byte vectors and moves split-K partials with 16-byte
    accesses: an operand that is not 16-byte aligned (a 4-byte-aligned float sub-view, say) is rejected before any
    GPU effect, in the fp16 and the f32 forms."""
    common = dict(num_seqs=1, num_blocks=4, max_blocks_per_seq=4, key_cache=FAKE, value_cache=FAKE, query=FAKE,
                  new_key=FAKE, new_value=FAKE, out=FAKE, workspace=FAKE, workspace_bytes=1 << 20, max_context=64,
                  uniform_cache_len=10)
    common[operand] = FAKE + 4
    with pytest.raises(pvlc.PvlcHipError) as e:
        pvlc.paged_decode_f16(pvlc.paged_decode_args(**common))
    assert code(e) == ("InvalidInvocation", "LengthMismatch") and "16-byte aligned" in str(e.value)
    if operand in ("query", "new_key", "new_value", "out"):
        f32 = dict(query=FAKE, new_key=FAKE, new_value=FAKE, out=FAKE)
        f32[operand] = FAKE + 4
        args = pvlc.paged_decode_args(**{**common, operand: FAKE, "query": None, "new_key": None,
                                         "new_value": None, "out": None})
        with pytest.raises(pvlc.PvlcHipError) as e:
            pvlc.paged_decode_f32io(args, f32["query"], f32["new_key"], f32["new_value"], f32["out"])
        assert code(e) == ("InvalidInvocation", "LengthMismatch") and "16-byte aligned" in str(e.value)


def test_f32_operand_prefill_rejects_mixed_or_missing_operands():
    """pvlc_hip_paged_prefill_f32io takes the query, key, value and output as f32 arguments: fp16 ones left in the
    args, or a missing f32 one, are rejected before any GPU effect (placeholder addresses, never read)."""
    fake = 1 << 20
    mixed = pvlc.PagedPrefillArgsC(16, 1, None, fake, fake, fake, None, None, None, None, None, 0, None, None, None,
                                   None, 0)
    with pytest.raises(pvlc.PvlcHipError) as e:
        pvlc._check(pvlc.lib.pvlc_hip_paged_prefill_f32io(ctypes.byref(mixed), fake, fake, fake, fake, None))
    assert code(e) == ("InvalidInvocation", "LengthMismatch") and "must be NULL" in str(e.value)
    for missing in range(4):
        ptrs = [fake] * 4
        ptrs[missing] = None
        with pytest.raises(pvlc.PvlcHipError) as e:
            pvlc.paged_prefill_f32io(tokens=16, num_blocks=1, key_cache=fake, value_cache=fake, query=ptrs[0],
                                     key=ptrs[1], value=ptrs[2], out=ptrs[3])
        assert code(e) == ("InvalidInvocation", "LengthMismatch") and "f32 operand pointer is NULL" in str(e.value)
    # and the fp16 entry point still requires its own operands
    with pytest.raises(pvlc.PvlcHipError) as e:
        pvlc.paged_prefill_f16(tokens=16, num_blocks=1, key_cache=fake, value_cache=fake, query=None, key=None,
                               value=None, out=None)
    assert code(e) == ("InvalidInvocation", "LengthMismatch")


def test_prefill_rejects_unaligned_rows():
    """The prefill kernels move query, key, value, output, cache and scratch rows as 16-byte vectors: a pointer off
    that alignment is rejected before any GPU effect (placeholder addresses, never read)."""
    fake = 1 << 20
    base = dict(tokens=16, num_blocks=1, key_cache=fake, value_cache=fake, query=fake, key=fake, value=fake, out=fake)
    for name in ("query", "key", "value", "out", "key_cache", "value_cache", "query_scratch"):
        kw = dict(base, **{name: fake + 2})
        with pytest.raises(pvlc.PvlcHipError) as e:
            pvlc.paged_prefill_f16(**kw)
        assert code(e) == ("InvalidInvocation", "LengthMismatch") and "16-byte aligned" in str(e.value), name
    with pytest.raises(pvlc.PvlcHipError) as e:
        pvlc.paged_prefill_f32io(tokens=16, num_blocks=1, key_cache=fake, value_cache=fake, query=fake, key=fake + 4,
                                 value=fake, out=fake)
    assert "16-byte aligned" in str(e.value)
