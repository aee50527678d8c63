"""MI355X (gfx950) backend for the PaddleOCR-VL decoder KV-cache hot path.

Python host mirror of the reference's operator surface, over the C ABI of
``libpvlc_hip.so`` (``include/pvlc_hip.h``):

* plan authority of ``crates/pvlc-runtime-core`` -- :func:`plan_kv_session`,
  :func:`plan_kv_step`, :func:`plan_gqa_split`, :func:`plan_prefill`;
* executor of ``crates/pvlc-runtime-native`` -- :class:`NativeRuntime` with
  ``run_decoder_cached_gqa`` and ``begin_decoder_kv_session``, and
  :class:`NativeDecoderKvSession` with ``step`` / ``finish``;
* the device-resident hot path -- :func:`paged_decode_f16`,
  :func:`paged_prefill_f16`, :func:`kv_pack_f16`, :func:`kv_unpack_f16`.

Names, argument meaning and error behaviour follow the reference; failures
raise :class:`PvlcHipError` carrying the reference's ``RuntimeErrorCode`` and,
for plan failures, its ``InvocationErrorCode``.  There is no fallback: if the
HIP library is missing, importing this package fails.
"""

from __future__ import annotations

import ctypes
import os
from dataclasses import dataclass

import numpy as np

_HERE = os.path.dirname(os.path.abspath(__file__))
# PVLC_HIP_LIBRARY selects another build of the same C ABI (default: in-tree).
LIBRARY_PATH = os.environ.get("PVLC_HIP_LIBRARY", os.path.join(_HERE, "libpvlc_hip.so"))

QUERY_HEADS = 16
KV_HEADS = 2
HEAD_DIM = 128
BLOCK_TOKENS = 16

RUNTIME_ERROR_CODES = {
    1: "AdapterUnavailable", 2: "DeviceRequest", 3: "InvalidInvocation", 4: "Validation", 5: "OutOfMemory",
    6: "Internal", 7: "Operation", 8: "Mapping", 9: "Capture",
}
INVOCATION_ERROR_CODES = {
    0: None, 1: "ZeroDimension", 2: "LengthMismatch", 3: "ArithmeticOverflow", 4: "InvalidEpsilon",
    5: "InvalidRotaryDimension", 6: "InvalidRopeBase", 7: "UnsupportedHeadDimension",
    8: "InvalidDecoderGeometry", 9: "InvalidVisionGeometry", 10: "InvalidProjectorGeometry",
    11: "InvalidSequenceBoundaries", 12: "InvalidCheckpointSelection", 13: "InvalidActivationLayout",
    14: "InvalidFusionTarget", 15: "NonFiniteInput",
}


class PvlcHipError(Exception):
    """RuntimeError of pvlc-runtime-native (lib.rs:285-349) with the nested
    InvocationErrorCode of pvlc-runtime-core (lib.rs:5335-5351) when a plan
    rejected the call."""

    def __init__(self, status: int, message: str):
        self.status = status
        self.code = RUNTIME_ERROR_CODES.get(status >> 8, str(status >> 8))
        self.invocation_code = INVOCATION_ERROR_CODES.get(status & 0xFF, str(status & 0xFF))
        detail = f"{self.code}" + (f"/{self.invocation_code}" if self.invocation_code else "")
        super().__init__(f"native runtime error {detail}: {message}")


# --------------------------------------------------------------------------
# C ABI
# --------------------------------------------------------------------------

_F = ctypes.POINTER(ctypes.c_float)
_U16 = ctypes.POINTER(ctypes.c_uint16)
_I32 = ctypes.POINTER(ctypes.c_int32)
_VP = ctypes.c_void_p
_SZ = ctypes.c_size_t
_U32 = ctypes.c_uint32


class KvSessionDescriptorC(ctypes.Structure):
    _fields_ = [("query_heads", _U32), ("key_value_heads", _U32), ("head_dim", _U32), ("prefix_tokens", _U32),
                ("cache_capacity", _U32), ("key_cache", _F), ("key_cache_len", _SZ), ("value_cache", _F),
                ("value_cache_len", _SZ)]


class KvSessionPlanC(ctypes.Structure):
    _fields_ = [("initial_cache_tokens", _U32), ("cache_capacity", _U32), ("query_heads", _U32),
                ("key_value_heads", _U32), ("head_dim", _U32), ("query_elements", ctypes.c_uint64),
                ("key_value_width", ctypes.c_uint64), ("cache_elements", ctypes.c_uint64),
                ("cache_bytes", ctypes.c_uint64), ("attention_bytes", ctypes.c_uint64),
                ("split_partials_bytes", ctypes.c_uint64)]


class KvStepOperandsC(ctypes.Structure):
    _fields_ = [("query", _F), ("query_len", _SZ), ("appended_key", _F), ("appended_key_len", _SZ),
                ("appended_value", _F), ("appended_value_len", _SZ)]


class GqaSplitPlanC(ctypes.Structure):
    _fields_ = [("chunk_size", _U32), ("chunk_count", _U32), ("partials_elements", ctypes.c_uint64),
                ("partials_bytes", ctypes.c_uint64), ("partial_stride_f32", _U32), ("partial_workgroups", _U32),
                ("merge_workgroups", _U32), ("uniform_words", _U32 * 4)]


class ProjectionPlanC(ctypes.Structure):
    _fields_ = [("kernel", _U32), ("weight_storage", _U32), ("input_bytes", ctypes.c_uint64),
                ("weight_bytes", ctypes.c_uint64), ("bias_bytes", ctypes.c_uint64), ("output_bytes", ctypes.c_uint64),
                ("dispatch", _U32 * 3)]


# VisionPatchProjectionBytesErrorCode (runtime-core lib.rs:1751-1759).
PROJECTION_ERROR_CODES = {1: "InvalidGeometry", 2: "Overflow", 3: "LengthMismatch", 4: "NonFinite",
                          5: "MissingShaderF16", 6: "DispatchLimitExceeded"}


class ProjectionPlanError(Exception):
    """VisionPatchProjectionBytesError (runtime-core lib.rs:1761-1766)."""

    def __init__(self, code: int):
        self.code = PROJECTION_ERROR_CODES.get(code, str(code))
        super().__init__(f"vision patch-projection bytes error {self.code}")


class GemvTiledPlanC(ctypes.Structure):
    _fields_ = [("tile_rows", _U32), ("threads_per_row", _U32), ("vector_width", _U32), ("shared_capacity", _U32),
                ("workgroup_storage_bytes", _U32), ("dispatch", _U32 * 3), ("workgroup_size", _U32 * 3),
                ("uniform_words", _U32 * 4), ("output_elements", ctypes.c_uint64), ("output_bytes", ctypes.c_uint64)]


class KvStepPlanC(ctypes.Structure):
    _fields_ = [("cache_tokens_before", _U32), ("cache_tokens_after", _U32),
                ("valid_cache_elements", ctypes.c_uint64), ("append_uniform_words", _U32 * 4),
                ("attention_uniform_words", _U32 * 4), ("split_gqa", GqaSplitPlanC)]


class RuntimeOptionsC(ctypes.Structure):
    _fields_ = [("device", ctypes.c_int32), ("gpu_wait_timeout_ns", ctypes.c_uint64)]


class RuntimeCountersC(ctypes.Structure):
    _fields_ = [("kernel_launches", ctypes.c_uint64), ("host_to_device_copies", ctypes.c_uint64),
                ("device_to_host_copies", ctypes.c_uint64), ("synchronizations", ctypes.c_uint64),
                ("sessions_created", ctypes.c_uint64)]


class CachedGqaInvocationC(ctypes.Structure):
    _fields_ = [("query_heads", _U32), ("key_value_heads", _U32), ("head_dim", _U32), ("prefix_tokens", _U32),
                ("cache_capacity", _U32), ("query", _F), ("query_len", _SZ), ("appended_key", _F),
                ("appended_key_len", _SZ), ("appended_value", _F), ("appended_value_len", _SZ),
                ("key_cache", _F), ("key_cache_len", _SZ), ("value_cache", _F), ("value_cache_len", _SZ)]


class CachedGqaExecutionC(ctypes.Structure):
    _fields_ = [("attention", _F), ("attention_len", _SZ), ("key_cache", _F), ("key_cache_len", _SZ),
                ("value_cache", _F), ("value_cache_len", _SZ), ("cache_tokens", _U32), ("cache_capacity", _U32),
                ("queue_wall_time_ns", ctypes.c_uint64)]


class KvStepExecutionC(ctypes.Structure):
    _fields_ = [("cache_tokens_before", _U32), ("cache_tokens_after", _U32),
                ("queue_wall_time_ns", ctypes.c_uint64), ("dispatch_count", _U32)]


class PagedDecodeArgsC(ctypes.Structure):
    _fields_ = [("num_seqs", _U32), ("num_blocks", _U32), ("max_blocks_per_seq", _U32), ("block_tables", _VP),
                ("cache_lens", _VP), ("uniform_cache_len", _U32), ("max_context", _U32), ("key_cache", _VP),
                ("value_cache", _VP), ("query", _VP), ("new_key", _VP), ("new_value", _VP), ("out", _VP),
                ("rope_cos", _VP), ("rope_sin", _VP), ("rope_rows", _U32), ("positions", _VP),
                ("rotate_query", _U32), ("partition_tokens", _U32), ("workspace", _VP), ("workspace_bytes", _SZ)]


class PagedPrefillArgsC(ctypes.Structure):
    _fields_ = [("tokens", _U32), ("num_blocks", _U32), ("block_table", _VP), ("key_cache", _VP),
                ("value_cache", _VP), ("query", _VP), ("key", _VP), ("value", _VP), ("out", _VP),
                ("rope_cos", _VP), ("rope_sin", _VP), ("rope_rows", _U32), ("positions", _VP),
                ("query_scratch", _VP), ("error_word", _VP), ("workspace", _VP), ("workspace_bytes", ctypes.c_uint64)]


# Exported symbols with their C signatures (argtypes, restype).
SIGNATURES = {
    "pvlc_hip_last_error_message": ([], ctypes.c_char_p),
    "pvlc_hip_kv_session_plan_create": ([ctypes.POINTER(KvSessionDescriptorC), ctypes.POINTER(KvSessionPlanC)],
                                        ctypes.c_int32),
    "pvlc_hip_kv_session_plan_step": ([ctypes.POINTER(KvSessionPlanC), _U32, ctypes.POINTER(KvStepOperandsC),
                                      ctypes.POINTER(KvStepPlanC)], ctypes.c_int32),
    "pvlc_hip_gqa_split_plan_create": ([_U32, _U32, _U32, _U32, ctypes.POINTER(GqaSplitPlanC)], ctypes.c_int32),
    "pvlc_hip_prefill_plan_check": ([_U32, _U32], ctypes.c_int32),
    "pvlc_hip_runtime_create": ([ctypes.POINTER(RuntimeOptionsC), ctypes.POINTER(_VP)], ctypes.c_int32),
    "pvlc_hip_runtime_destroy": ([_VP], None),
    "pvlc_hip_runtime_counters_get": ([_VP, ctypes.POINTER(RuntimeCountersC)], ctypes.c_int32),
    "pvlc_hip_run_decoder_cached_gqa": ([_VP, ctypes.POINTER(CachedGqaInvocationC),
                                        ctypes.POINTER(CachedGqaExecutionC)], ctypes.c_int32),
    "pvlc_hip_begin_decoder_kv_session": ([_VP, ctypes.POINTER(KvSessionDescriptorC), ctypes.POINTER(_VP)],
                                          ctypes.c_int32),
    "pvlc_hip_kv_session_cache_tokens": ([_VP], _U32),
    "pvlc_hip_kv_session_cache_capacity": ([_VP], _U32),
    "pvlc_hip_kv_session_is_poisoned": ([_VP], ctypes.c_int32),
    "pvlc_hip_kv_session_step": ([_VP, ctypes.POINTER(KvStepOperandsC), _F, _SZ, ctypes.POINTER(KvStepExecutionC)],
                                 ctypes.c_int32),
    "pvlc_hip_kv_session_finish": ([_VP, _F, _SZ, _F, _SZ, ctypes.POINTER(_U32), ctypes.POINTER(_U32)],
                                   ctypes.c_int32),
    "pvlc_hip_kv_session_destroy": ([_VP], None),
    "pvlc_hip_kv_session_fail_next_step_after_submit": ([_VP], None),
    "pvlc_hip_kv_session_expire_next_wait": ([_VP], None),
    "pvlc_hip_rope_table_f32": ([ctypes.c_float, _U32, _U32, _F, _F], ctypes.c_int32),
    "pvlc_hip_mrope_table_f32": ([_F, _F, _U32, _U32, _U32, _U32, _F, _F], ctypes.c_int32),
    "pvlc_hip_f32_to_f16_host": ([_F, _U16, _SZ], None),
    "pvlc_hip_f16_to_f32_host": ([_U16, _F, _SZ], None),
    "pvlc_hip_paged_decode_partition": ([_U32, _U32], _U32),
    "pvlc_hip_paged_decode_streaming_partition": ([ctypes.POINTER(ctypes.c_int32), _U32, _U32, _U32], _U32),
    "pvlc_hip_paged_decode_workspace_bytes": ([_U32, _U32, _U32], _SZ),
    "pvlc_hip_workspace_init": ([_VP, _SZ, _VP], ctypes.c_int32),
    "pvlc_hip_workspace_error": ([_VP, _SZ, _VP, ctypes.POINTER(_U32)], ctypes.c_int32),
    "pvlc_hip_paged_decode_f16": ([ctypes.POINTER(PagedDecodeArgsC), _VP], ctypes.c_int32),
    "pvlc_hip_paged_decode_f16_no_alloc": ([ctypes.POINTER(PagedDecodeArgsC), _VP, _VP], ctypes.c_int32),
    "pvlc_hip_paged_decode_f32io": ([ctypes.POINTER(PagedDecodeArgsC), _VP, _VP, _VP, _VP, _VP], ctypes.c_int32),
    "pvlc_hip_paged_prefill_f16": ([ctypes.POINTER(PagedPrefillArgsC), _VP], ctypes.c_int32),
    "pvlc_hip_paged_prefill_f32io": ([ctypes.POINTER(PagedPrefillArgsC), _VP, _VP, _VP, _VP, _VP], ctypes.c_int32),
    "pvlc_hip_kv_pack_f16": ([_VP, _VP, _U32, _VP, _U32, _VP, _VP, _VP], ctypes.c_int32),
    "pvlc_hip_kv_unpack_f16": ([_VP, _VP, _U32, _VP, _U32, _VP, _VP, _VP], ctypes.c_int32),
    "pvlc_hip_gemv_tiled_plan_create": ([_U32, _U32, ctypes.POINTER(GemvTiledPlanC)], ctypes.c_int32),
    "pvlc_hip_gemv_f16": ([_VP, _VP, _VP, _U32, _U32, _VP], ctypes.c_int32),
    "pvlc_hip_gemv_group_f16": ([_VP, _U32, _VP, _U32, _VP], ctypes.c_int32),
    "pvlc_hip_top1_workspace_bytes": ([], _SZ),
    "pvlc_hip_paged_prefill_workspace_bytes": ([_U32], _SZ),
    "pvlc_hip_projection_plan_create": ([_U32, _U32, _U32, _U32, ctypes.POINTER(ProjectionPlanC)], ctypes.c_int32),
    "pvlc_hip_projection_validate_capabilities": ([ctypes.POINTER(ProjectionPlanC), ctypes.c_int32, _U32],
                                                  ctypes.c_int32),
    "pvlc_hip_projection_validate_operands": ([ctypes.POINTER(ProjectionPlanC), _VP, _SZ, _VP, _SZ, _VP, _SZ],
                                              ctypes.c_int32),
    "pvlc_hip_linear_projection_workspace_bytes": ([_U32, _U32], _SZ),
    "pvlc_hip_linear_projection_f16": ([_VP, _VP, _VP, _VP, _U32, _U32, _U32, _VP, _SZ, _VP], ctypes.c_int32),
    "pvlc_hip_logits_top1_f32": ([_VP, _U32, _VP, _VP, _SZ, _VP], ctypes.c_int32),
    "pvlc_hip_lm_head_top1_f16": ([_VP, _VP, _VP, _U32, _U32, _VP, _VP, _SZ, _VP], ctypes.c_int32),
}


def _load() -> ctypes.CDLL:
    if not os.path.exists(LIBRARY_PATH):
        raise ImportError(f"{LIBRARY_PATH} is missing: build it with __graft_entry__.build() "
                          "(there is no CPU fallback for this backend)")
    # One HIP runtime per process: PyTorch bundles its own libamdhip64.so.7.
    # Loading it first lets this library's libamdhip64.so.7 dependency bind to
    # that copy (same SONAME) instead of mapping a second runtime, which would
    # leave one of the two without devices.
    try:
        import torch  # noqa: F401
    except ImportError:
        pass
    lib = ctypes.CDLL(LIBRARY_PATH)
    for name, (argtypes, restype) in SIGNATURES.items():
        fn = getattr(lib, name)
        fn.argtypes = argtypes
        fn.restype = restype
    return lib


lib = _load()


def _check(status: int) -> None:
    if status != 0:
        msg = lib.pvlc_hip_last_error_message()
        raise PvlcHipError(status, msg.decode() if msg else "")


def _f32(a) -> np.ndarray:
    return np.ascontiguousarray(np.asarray(a, dtype=np.float32).ravel())


def _fp(a: np.ndarray):
    return a.ctypes.data_as(_F) if a.size else ctypes.cast(None, _F)


# --------------------------------------------------------------------------
# Reference-shaped operands
# --------------------------------------------------------------------------

@dataclass
class DecoderKvSessionDescriptor:
    """runtime-core DecoderKvSessionDescriptor (lib.rs:833-843)."""

    prefix_tokens: int
    cache_capacity: int
    key_cache: np.ndarray
    value_cache: np.ndarray
    query_heads: int = QUERY_HEADS
    key_value_heads: int = KV_HEADS
    head_dim: int = HEAD_DIM

    def _c(self):
        k, v = _f32(self.key_cache), _f32(self.value_cache)
        c = KvSessionDescriptorC(self.query_heads, self.key_value_heads, self.head_dim, self.prefix_tokens,
                                 self.cache_capacity, _fp(k), k.size, _fp(v), v.size)
        return c, (k, v)


@dataclass
class DecoderKvSessionStep:
    """runtime-core DecoderKvSessionStep (lib.rs:845-851)."""

    query: np.ndarray
    appended_key: np.ndarray
    appended_value: np.ndarray

    def _c(self):
        q, k, v = _f32(self.query), _f32(self.appended_key), _f32(self.appended_value)
        return KvStepOperandsC(_fp(q), q.size, _fp(k), k.size, _fp(v), v.size), (q, k, v)


@dataclass
class DecoderCachedGqaInvocation:
    """runtime-core DecoderCachedGqaInvocation (lib.rs:883-900)."""

    prefix_tokens: int
    cache_capacity: int
    query: np.ndarray
    appended_key: np.ndarray
    appended_value: np.ndarray
    key_cache: np.ndarray
    value_cache: np.ndarray
    query_heads: int = QUERY_HEADS
    key_value_heads: int = KV_HEADS
    head_dim: int = HEAD_DIM


@dataclass
class DecoderCachedGqaExecution:
    """pvlc-runtime-native DecoderCachedGqaExecution (lib.rs:519-526)."""

    attention: np.ndarray
    key_cache: np.ndarray
    value_cache: np.ndarray
    cache_tokens: int
    cache_capacity: int
    queue_wall_time_ns: int


@dataclass
class DecoderKvSessionStepExecution:
    """pvlc-runtime-native DecoderKvSessionStepExecution (lib.rs:590-594)."""

    attention: np.ndarray
    cache_tokens: int
    queue_wall_time_ns: int
    dispatch_count: int


@dataclass
class DecoderKvSessionSnapshot:
    """pvlc-runtime-native DecoderKvSessionSnapshot (lib.rs:610-616)."""

    key_cache: np.ndarray
    value_cache: np.ndarray
    cache_tokens: int
    cache_capacity: int


# --------------------------------------------------------------------------
# Plans (host only)
# --------------------------------------------------------------------------

def _struct_dict(s) -> dict:
    out = {}
    for name, _ in s._fields_:
        v = getattr(s, name)
        if isinstance(v, ctypes.Structure):
            v = _struct_dict(v)
        elif isinstance(v, ctypes.Array):
            v = list(v)
        out[name] = v
    return out


def plan_kv_session(descriptor: DecoderKvSessionDescriptor) -> KvSessionPlanC:
    """DecoderKvSessionDescriptor::plan (runtime-core lib.rs:952-968)."""
    c, keep = descriptor._c()
    plan = KvSessionPlanC()
    _check(lib.pvlc_hip_kv_session_plan_create(ctypes.byref(c), ctypes.byref(plan)))
    del keep
    return plan


def plan_kv_step(plan: KvSessionPlanC, cache_tokens: int, step: DecoderKvSessionStep | None = None) -> dict:
    """DecoderKvSessionPlan::plan_step / plan_cache_transition (lib.rs:976-1054)."""
    out = KvStepPlanC()
    if step is None:
        _check(lib.pvlc_hip_kv_session_plan_step(ctypes.byref(plan), cache_tokens, None, ctypes.byref(out)))
    else:
        c, keep = step._c()
        _check(lib.pvlc_hip_kv_session_plan_step(ctypes.byref(plan), cache_tokens, ctypes.byref(c),
                                                 ctypes.byref(out)))
        del keep
    return _struct_dict(out)


def plan_gqa_split(cache_tokens: int, query_heads: int = QUERY_HEADS, key_value_heads: int = KV_HEADS,
                   head_dim: int = HEAD_DIM) -> dict:
    """DecoderGqaSplitDescriptor::plan (runtime-core lib.rs:2889-2978)."""
    out = GqaSplitPlanC()
    _check(lib.pvlc_hip_gqa_split_plan_create(cache_tokens, query_heads, key_value_heads, head_dim,
                                              ctypes.byref(out)))
    return _struct_dict(out)


def plan_gemv_tiled(rows: int, columns: int) -> dict:
    """GemvTiledDescriptor::plan (runtime-core lib.rs:753-785)."""
    out = GemvTiledPlanC()
    _check(lib.pvlc_hip_gemv_tiled_plan_create(rows, columns, ctypes.byref(out)))
    return _struct_dict(out)


def gemv_f16(weights, vector, out, rows: int, columns: int, stream=None) -> None:
    """out[r] = sum_c weights[r][c] * vector[c] (fp16 weights, f32 vector and output): replaces
    gemv_tiled_f16_weights (pvlc-wgsl lib.rs:1770-1835); admission as plan_gemv_tiled."""
    _check(lib.pvlc_hip_gemv_f16(_ptr(weights), _ptr(vector), _ptr(out), rows, columns, _stream(stream)))


class GemvMemberC(ctypes.Structure):
    _fields_ = [("weights", ctypes.c_void_p), ("out", ctypes.c_void_p), ("rows", ctypes.c_uint32)]


class GemvMembers:
    """The members of a grouped GEMV as the C array pvlc_hip_gemv_group_f16 reads, built once (a decode loop
    reuses its groups every token)."""

    def __init__(self, members):
        self.count = len(members)
        self.array = (GemvMemberC * max(1, self.count))()
        for i, (w, o, r) in enumerate(members):
            self.array[i] = GemvMemberC(_ptr(w), _ptr(o), r)
        self.keep = list(members)  # the tensors stay alive while the array points at them
        self.pointer = ctypes.cast(self.array, ctypes.c_void_p) if self.count else None


def gemv_group_f16(members, vector, columns: int, stream=None) -> None:
    """Up to 4 GEMVs (weights, out, rows) of one width reading the same vector, in one launch; each member's
    output is bit-identical to gemv_f16 on it (the projections sharing a hidden state: q, k, v; gate, up).
    `members` is a list of (weights, out, rows) or a prebuilt GemvMembers."""
    if not isinstance(members, GemvMembers):
        members = GemvMembers(members)
    _check(lib.pvlc_hip_gemv_group_f16(members.pointer, members.count, _ptr(vector), columns, _stream(stream)))


def top1_workspace_bytes() -> int:
    """Bytes of the top-1 workspace (arrival counter + candidate slots); zero it once with workspace_init."""
    return int(lib.pvlc_hip_top1_workspace_bytes())


def logits_top1_f32(logits, vocab: int, result, workspace, workspace_bytes: int, stream=None) -> None:
    """decoder_logits_top1_f32 (decoder_stack_session.rs:308-366): result[0] = index of the largest logit
    under the f32 total order (ties to the lowest index), result[1] = its f32 bits."""
    _check(lib.pvlc_hip_logits_top1_f32(_ptr(logits), vocab, _ptr(result), _ptr(workspace), workspace_bytes,
                                        _stream(stream)))


def lm_head_top1_f16(weights, hidden, logits, rows: int, columns: int, result, workspace, workspace_bytes: int,
                     stream=None) -> None:
    """LM-head GEMV (gemv_f16 semantics) and the top-1 of its logits in one launch; logits may be None."""
    _check(lib.pvlc_hip_lm_head_top1_f16(_ptr(weights), _ptr(hidden), _ptr(logits), rows, columns, _ptr(result),
                                         _ptr(workspace), workspace_bytes, _stream(stream)))


class ProjectionPlan:
    """VisionPatchProjectionBytesPlan (runtime-core lib.rs:1741-1749) and its checks (:1853-1913)."""

    def __init__(self, raw: ProjectionPlanC):
        self._raw = raw
        self.kernel = "linear_projection_f16_weights" if raw.kernel == 1 else "vision_patch_projection_f32"
        self.weight_storage = "f16" if raw.weight_storage == 1 else "f32"
        self.input_bytes, self.weight_bytes = raw.input_bytes, raw.weight_bytes
        self.bias_bytes, self.output_bytes = raw.bias_bytes, raw.output_bytes
        self.dispatch = list(raw.dispatch)

    def requires_shader_f16(self) -> bool:
        return self.weight_storage == "f16"

    def validate_capabilities(self, shader_f16_available: bool, max_compute_workgroups_per_dimension: int) -> None:
        rc = lib.pvlc_hip_projection_validate_capabilities(ctypes.byref(self._raw), int(shader_f16_available),
                                                           max_compute_workgroups_per_dimension)
        if rc:
            raise ProjectionPlanError(rc)

    def validate_operands(self, input: bytes, weight: bytes, bias: bytes) -> None:
        args = []
        keep = []
        for data in (input, weight, bias):
            data = bytes(data)
            buf = ctypes.create_string_buffer(data, len(data)) if data else None
            keep.append(buf)
            args += [ctypes.cast(buf, _VP) if buf is not None else None, len(data)]
        rc = lib.pvlc_hip_projection_validate_operands(ctypes.byref(self._raw), *args)
        if rc:
            raise ProjectionPlanError(rc)


def plan_projection(patch_count: int, input_width: int, output_width: int, weight_storage: str = "f16") -> ProjectionPlan:
    """VisionPatchProjectionBytesDescriptor::plan (runtime-core lib.rs:1768-1840)."""
    raw = ProjectionPlanC()
    rc = lib.pvlc_hip_projection_plan_create(patch_count, input_width, output_width,
                                             1 if weight_storage == "f16" else 0, ctypes.byref(raw))
    if rc:
        raise ProjectionPlanError(rc)
    return ProjectionPlan(raw)


def linear_projection_workspace_bytes(rows: int, input_width: int) -> int:
    return int(lib.pvlc_hip_linear_projection_workspace_bytes(rows, input_width))


def linear_projection_f16(input, weight, bias, out, rows: int, input_width: int, output_width: int, workspace,
                          workspace_bytes: int, stream=None) -> None:
    """out = input . weight^T + bias with fp16 weights and f32 activations (linear_projection_f16_weights,
    pvlc-wgsl lib.rs:1836-1964), f32-grade products on MFMA."""
    _check(lib.pvlc_hip_linear_projection_f16(_ptr(input), _ptr(weight), _ptr(bias), _ptr(out), rows, input_width,
                                              output_width, _ptr(workspace), workspace_bytes, _stream(stream)))


def plan_prefill(tokens: int, cache_capacity: int) -> None:
    """Token bound of DecoderStackGeometryDescriptor::plan_prefill (lib.rs:2293-2297, 2491-2498)."""
    _check(lib.pvlc_hip_prefill_plan_check(tokens, cache_capacity))


def rope_table(base: float, rows: int, rotary_dim: int = HEAD_DIM) -> tuple[np.ndarray, np.ndarray]:
    """cos/sin tables [rows][rotary_dim/2] of apply_rope_neox's angles (cpu-ref lib.rs:459-461)."""
    half = rotary_dim // 2
    cos = np.zeros(rows * half, np.float32)
    sin = np.zeros(rows * half, np.float32)
    _check(lib.pvlc_hip_rope_table_f32(ctypes.c_float(base), rotary_dim, rows, _fp(cos), _fp(sin)))
    return cos.reshape(rows, half), sin.reshape(rows, half)


def mrope_table(raw_cos, raw_sin, capacity: int, sections=(16, 24, 24)) -> tuple[np.ndarray, np.ndarray]:
    """[capacity][64] cos/sin tables from raw M-RoPE tables [3][capacity][128] (decoder_mrope_f32's section
    selection, pvlc-wgsl lib.rs:1185-1234)."""
    rc = np.ascontiguousarray(raw_cos, dtype=np.float32).ravel()
    rs = np.ascontiguousarray(raw_sin, dtype=np.float32).ravel()
    if rc.size != 3 * capacity * HEAD_DIM or rs.size != rc.size:
        raise PvlcHipError(0x300 | 2, "raw M-RoPE tables must hold 3 x capacity x 128 values")
    half = HEAD_DIM // 2
    cos = np.zeros(capacity * half, np.float32)
    sin = np.zeros(capacity * half, np.float32)
    _check(lib.pvlc_hip_mrope_table_f32(_fp(rc), _fp(rs), capacity, sections[0], sections[1], sections[2], _fp(cos),
                                        _fp(sin)))
    return cos.reshape(capacity, half), sin.reshape(capacity, half)


def f32_to_f16(values) -> np.ndarray:
    """Host round-to-nearest-even fp16 (bit patterns as uint16)."""
    x = _f32(values)
    out = np.zeros(x.size, np.uint16)
    lib.pvlc_hip_f32_to_f16_host(_fp(x), out.ctypes.data_as(_U16), x.size)
    return out


def f16_to_f32(bits) -> np.ndarray:
    b = np.ascontiguousarray(np.asarray(bits, dtype=np.uint16).ravel())
    out = np.zeros(b.size, np.float32)
    lib.pvlc_hip_f16_to_f32_host(b.ctypes.data_as(_U16), _fp(out), b.size)
    return out


# --------------------------------------------------------------------------
# Runtime and sessions (pvlc-runtime-native surface)
# --------------------------------------------------------------------------

class NativeRuntime:
    """pvlc-runtime-native NativeRuntime (lib.rs:724-745, 912-1018) on one HIP device.

    Every wait for submitted GPU work is bounded by ``gpu_wait_timeout_ns`` (0: 30 s, GPU_WAIT_TIMEOUT of
    lib.rs:56); an expired wait raises Operation and poisons the session that waited."""

    def __init__(self, device: int = 0, gpu_wait_timeout_ns: int = 0):
        handle = _VP()
        _check(lib.pvlc_hip_runtime_create(ctypes.byref(RuntimeOptionsC(device, gpu_wait_timeout_ns)),
                                           ctypes.byref(handle)))
        self._handle = handle

    def close(self) -> None:
        if getattr(self, "_handle", None):
            lib.pvlc_hip_runtime_destroy(self._handle)
            self._handle = None

    def __del__(self):
        self.close()

    def counters(self) -> dict:
        c = RuntimeCountersC()
        _check(lib.pvlc_hip_runtime_counters_get(self._handle, ctypes.byref(c)))
        return _struct_dict(c)

    def run_decoder_cached_gqa(self, inv: DecoderCachedGqaInvocation) -> DecoderCachedGqaExecution:
        """NativeRuntime::run_decoder_cached_gqa (lib.rs:1259-1264)."""
        q, k, v = _f32(inv.query), _f32(inv.appended_key), _f32(inv.appended_value)
        kc, vc = _f32(inv.key_cache), _f32(inv.value_cache)
        c = CachedGqaInvocationC(inv.query_heads, inv.key_value_heads, inv.head_dim, inv.prefix_tokens,
                                 inv.cache_capacity, _fp(q), q.size, _fp(k), k.size, _fp(v), v.size, _fp(kc),
                                 kc.size, _fp(vc), vc.size)
        cache_elems = inv.cache_capacity * inv.key_value_heads * inv.head_dim
        att = np.zeros(inv.query_heads * inv.head_dim, np.float32)
        ko, vo = np.zeros(cache_elems, np.float32), np.zeros(cache_elems, np.float32)
        e = CachedGqaExecutionC(_fp(att), att.size, _fp(ko), ko.size, _fp(vo), vo.size, 0, 0, 0)
        _check(lib.pvlc_hip_run_decoder_cached_gqa(self._handle, ctypes.byref(c), ctypes.byref(e)))
        return DecoderCachedGqaExecution(att, ko, vo, e.cache_tokens, e.cache_capacity, e.queue_wall_time_ns)

    def begin_decoder_kv_session(self, descriptor: DecoderKvSessionDescriptor) -> "NativeDecoderKvSession":
        """NativeRuntime::begin_decoder_kv_session (lib.rs:1266-1271)."""
        c, keep = descriptor._c()
        handle = _VP()
        _check(lib.pvlc_hip_begin_decoder_kv_session(self._handle, ctypes.byref(c), ctypes.byref(handle)))
        del keep
        return NativeDecoderKvSession(self, handle)


class NativeDecoderKvSession:
    """pvlc-runtime-native NativeDecoderKvSession (decoder_kv_session.rs:23-545).

    ``finish`` consumes the session; using it afterwards raises Operation."""

    def __init__(self, runtime: NativeRuntime, handle):
        self._runtime = runtime  # the session borrows its runtime
        self._handle = handle

    def _live(self):
        if not self._handle:
            raise PvlcHipError(7 << 8, "decoder KV session was consumed by finish")
        return self._handle

    @property
    def cache_tokens(self) -> int:
        return lib.pvlc_hip_kv_session_cache_tokens(self._live())

    @property
    def cache_capacity(self) -> int:
        return lib.pvlc_hip_kv_session_cache_capacity(self._live())

    @property
    def poisoned(self) -> bool:
        return bool(lib.pvlc_hip_kv_session_is_poisoned(self._live()))

    def step(self, step: DecoderKvSessionStep) -> DecoderKvSessionStepExecution:
        c, keep = step._c()
        att = np.zeros(QUERY_HEADS * HEAD_DIM, np.float32)
        ex = KvStepExecutionC()
        _check(lib.pvlc_hip_kv_session_step(self._live(), ctypes.byref(c), _fp(att), att.size, ctypes.byref(ex)))
        del keep
        return DecoderKvSessionStepExecution(att, ex.cache_tokens_after, ex.queue_wall_time_ns, ex.dispatch_count)

    def finish(self) -> DecoderKvSessionSnapshot:
        handle = self._live()
        self._handle = None
        cap = lib.pvlc_hip_kv_session_cache_capacity(handle)
        n = cap * KV_HEADS * HEAD_DIM
        ko, vo = np.zeros(n, np.float32), np.zeros(n, np.float32)
        tokens, capacity = _U32(), _U32()
        _check(lib.pvlc_hip_kv_session_finish(handle, _fp(ko), n, _fp(vo), n, ctypes.byref(tokens),
                                              ctypes.byref(capacity)))
        return DecoderKvSessionSnapshot(ko, vo, tokens.value, capacity.value)

    def fail_next_step_after_submit(self) -> None:
        lib.pvlc_hip_kv_session_fail_next_step_after_submit(self._live())

    def expire_next_wait(self) -> None:
        """Test hook: the next bounded GPU wait (step or finish) reports its deadline as passed."""
        lib.pvlc_hip_kv_session_expire_next_wait(self._live())

    def __del__(self):
        if getattr(self, "_handle", None):
            lib.pvlc_hip_kv_session_destroy(self._handle)
            self._handle = None


# --------------------------------------------------------------------------
# Device-resident hot path (pointers from torch tensors or plain ints)
# --------------------------------------------------------------------------

def _ptr(x) -> int | None:
    if x is None:
        return None
    if isinstance(x, int):
        return x
    return x.data_ptr()


def _stream(stream) -> int | None:
    if stream is None:
        return None
    if isinstance(stream, int):
        return stream
    return stream.cuda_stream


def decode_partition(num_seqs: int, max_context: int) -> int:
    return lib.pvlc_hip_paged_decode_partition(num_seqs, max_context)


def decode_streaming_partition(cache_lens, max_context: int, compute_units: int) -> int:
    """Partition an automatic launch over these ragged cache lengths settles on (host replay of the device rule)."""
    lens = np.ascontiguousarray(np.asarray(cache_lens, dtype=np.int32).ravel())
    return lib.pvlc_hip_paged_decode_streaming_partition(lens.ctypes.data_as(ctypes.POINTER(ctypes.c_int32)),
                                                         len(lens), max_context, compute_units)


def decode_workspace_bytes(num_seqs: int, max_context: int, partition_tokens: int = 0) -> int:
    return lib.pvlc_hip_paged_decode_workspace_bytes(num_seqs, max_context, partition_tokens)


def workspace_init(workspace, nbytes: int, stream=None) -> None:
    _check(lib.pvlc_hip_workspace_init(_ptr(workspace), nbytes, _stream(stream)))


def workspace_error(workspace, nbytes: int, stream=None) -> int:
    out = _U32()
    _check(lib.pvlc_hip_workspace_error(_ptr(workspace), nbytes, _stream(stream), ctypes.byref(out)))
    return out.value


def paged_decode_args(*, num_seqs, num_blocks, max_blocks_per_seq, key_cache, value_cache, query, new_key,
                      new_value, out, workspace, workspace_bytes, max_context, block_tables=None, cache_lens=None,
                      uniform_cache_len=0, rope_cos=None, rope_sin=None, rope_rows=0, positions=None,
                      rotate_query=False, partition_tokens=0) -> PagedDecodeArgsC:
    return PagedDecodeArgsC(num_seqs, num_blocks, max_blocks_per_seq, _ptr(block_tables), _ptr(cache_lens),
                            uniform_cache_len, max_context, _ptr(key_cache), _ptr(value_cache), _ptr(query),
                            _ptr(new_key), _ptr(new_value), _ptr(out), _ptr(rope_cos), _ptr(rope_sin), rope_rows,
                            _ptr(positions), int(rotate_query), partition_tokens, _ptr(workspace), workspace_bytes)


def paged_decode_f16(args: PagedDecodeArgsC, stream=None) -> None:
    """One fused rotary+append+attention decode step for every sequence
    (replaces decoder_mrope/kv_append/gqa_split_partial/merge, wgsl lib.rs:927-1234)."""
    _check(lib.pvlc_hip_paged_decode_f16(ctypes.byref(args), _stream(stream)))


def paged_decode_f32io(args: PagedDecodeArgsC, query, new_key, new_value, out, stream=None) -> None:
    """paged_decode_f16 with f32 query, new key and value and output, the reference chain's operand format
    (the args' fp16 operand pointers must be None)."""
    _check(lib.pvlc_hip_paged_decode_f32io(ctypes.byref(args), _ptr(query), _ptr(new_key), _ptr(new_value),
                                           _ptr(out), _stream(stream)))


def paged_decode_f16_no_alloc(args: PagedDecodeArgsC, error_word, stream=None) -> None:
    """paged_decode_f16 with its split-K state in the library's per-device scratch (no workspace, no
    allocation); the device error bits are OR-ed into ``error_word`` (a caller-zeroed device word)."""
    _check(lib.pvlc_hip_paged_decode_f16_no_alloc(ctypes.byref(args), _ptr(error_word), _stream(stream)))


def prefill_workspace_bytes(tokens: int) -> int:
    """Bytes of the split-K prefill workspace (0 when no query block splits)."""
    return int(lib.pvlc_hip_paged_prefill_workspace_bytes(tokens))


def paged_prefill_f16(*, tokens, num_blocks, key_cache, value_cache, query, key, value, out, query_scratch=None,
                      block_table=None, rope_cos=None, rope_sin=None, rope_rows=0, positions=None,
                      error_word=None, workspace=None, workspace_bytes=0, stream=None) -> None:
    """Causal prefill with rotary and paged range append
    (replaces decoder_prefill_mrope/kv_append_range/prefill_gqa, wgsl lib.rs:1262-1416); with a workspace the
    long query blocks are split over several workgroups and merged (split-K)."""
    a = PagedPrefillArgsC(tokens, num_blocks, _ptr(block_table), _ptr(key_cache), _ptr(value_cache), _ptr(query),
                          _ptr(key), _ptr(value), _ptr(out), _ptr(rope_cos), _ptr(rope_sin), rope_rows,
                          _ptr(positions), _ptr(query_scratch), _ptr(error_word), _ptr(workspace), workspace_bytes)
    _check(lib.pvlc_hip_paged_prefill_f16(ctypes.byref(a), _stream(stream)))


def paged_prefill_f32io(*, tokens, num_blocks, key_cache, value_cache, query, key, value, out, query_scratch=None,
                        block_table=None, rope_cos=None, rope_sin=None, rope_rows=0, positions=None,
                        error_word=None, workspace=None, workspace_bytes=0, stream=None) -> None:
    """paged_prefill_f16 with f32 query, key, value and output, the reference chain's operand format."""
    a = PagedPrefillArgsC(tokens, num_blocks, _ptr(block_table), _ptr(key_cache), _ptr(value_cache), None, None,
                          None, None, _ptr(rope_cos), _ptr(rope_sin), rope_rows, _ptr(positions),
                          _ptr(query_scratch), _ptr(error_word), _ptr(workspace), workspace_bytes)
    _check(lib.pvlc_hip_paged_prefill_f32io(ctypes.byref(a), _ptr(query), _ptr(key), _ptr(value), _ptr(out),
                                            _stream(stream)))


def kv_pack_f16(key_rows, value_rows, tokens, key_cache, value_cache, num_blocks, block_table=None,
                stream=None) -> None:
    _check(lib.pvlc_hip_kv_pack_f16(_ptr(key_rows), _ptr(value_rows), tokens, _ptr(block_table), num_blocks,
                                    _ptr(key_cache), _ptr(value_cache), _stream(stream)))


def kv_unpack_f16(key_cache, value_cache, tokens, key_rows, value_rows, num_blocks, block_table=None,
                  stream=None) -> None:
    _check(lib.pvlc_hip_kv_unpack_f16(_ptr(key_cache), _ptr(value_cache), tokens, _ptr(block_table), num_blocks,
                                      _ptr(key_rows), _ptr(value_rows), _stream(stream)))


def key_slot(t):
    """Slot of token t (0..15) inside a 16-token block of the key plane: bits 2 and 3 swapped."""
    return (t & 3) | ((t & 4) << 1) | ((t & 8) >> 1)


def blocked_key_index(token: np.ndarray, head: np.ndarray, dim: np.ndarray) -> np.ndarray:
    """Element offset of key (token, head, dim) in contiguous blocked planes."""
    b, t = token // BLOCK_TOKENS, token % BLOCK_TOKENS
    return ((b * KV_HEADS + head) * (HEAD_DIM // 8) + dim // 8) * (BLOCK_TOKENS * 8) + key_slot(t) * 8 + dim % 8


def blocked_value_index(token: np.ndarray, head: np.ndarray, dim: np.ndarray) -> np.ndarray:
    b, t = token // BLOCK_TOKENS, token % BLOCK_TOKENS
    return ((b * KV_HEADS + head) * HEAD_DIM + dim) * BLOCK_TOKENS + t
