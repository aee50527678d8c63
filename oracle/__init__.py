"""ctypes front end of the CPU oracle (``libpvlc_oracle.so``).

TEST INFRASTRUCTURE, NOT PRODUCT CODE.  Only ``tests/``,
``__graft_entry__.smoke()`` and the ``cpu_baseline`` leg of ``bench.py`` may
import this package, and only as the checker or the timed CPU baseline.

Each wrapper calls the C restatement of one function of
``crates/pvlc-cpu-ref/src/lib.rs`` (glebkudr/paddleocr-vl-webgpu); the citations
are on the C functions in ``pvlc_oracle.c``.
"""

from __future__ import annotations

import ctypes
import os
import subprocess

import numpy as np

_HERE = os.path.dirname(os.path.abspath(__file__))
_LIB_PATH = os.path.join(_HERE, "libpvlc_oracle.so")

# Mirrors CpuRefErrorCode (crates/pvlc-cpu-ref/src/lib.rs:16-30).
ERROR_NAMES = {
    0: "Ok",
    1: "DimensionMismatch",
    2: "NonPositiveEpsilon",
    3: "AllMasked",
    4: "InvalidRotaryDimension",
    5: "InvalidRopeBase",
    6: "InvalidK",
    7: "NonFiniteInput",
}


class OracleError(Exception):
    def __init__(self, code: int):
        super().__init__(f"CPU reference error {ERROR_NAMES.get(code, code)}")
        self.code = ERROR_NAMES.get(code, str(code))


def build() -> str:
    """Compile the oracle with its Makefile (gcc, -O2 -ffp-contract=off)."""
    subprocess.run(["make", "-s", "-B", "-C", _HERE], check=True)
    return _LIB_PATH


_lib = None


def lib() -> ctypes.CDLL:
    global _lib
    if _lib is None:
        if not os.path.exists(_LIB_PATH):
            build()
        _lib = ctypes.CDLL(_LIB_PATH)
        _declare(_lib)
    return _lib


_F = ctypes.POINTER(ctypes.c_float)
_U16 = ctypes.POINTER(ctypes.c_uint16)
_U32 = ctypes.POINTER(ctypes.c_uint32)
_U8 = ctypes.POINTER(ctypes.c_uint8)
_SZ = ctypes.c_size_t


def _declare(l: ctypes.CDLL) -> None:
    l.oracle_decode_gqa_f32.argtypes = [_F, _SZ, _F, _SZ, _F, _SZ, _SZ, _SZ, _SZ, _SZ, _F]
    l.oracle_causal_gqa_f32.argtypes = [_F, _SZ, _F, _SZ, _F, _SZ, _SZ, _SZ, _SZ, _SZ, _F]
    l.oracle_append_kv_f32.argtypes = [_F, _F, _SZ, _F, _SZ, _F, _SZ, _SZ, _SZ, _F, _F]
    l.oracle_linear_f32.argtypes = [_F, _SZ, _SZ, _SZ, _F, _SZ, _F, _SZ, _SZ, _F]
    l.oracle_top1_f32.argtypes = [_F, _SZ, ctypes.POINTER(ctypes.c_uint32), ctypes.POINTER(ctypes.c_uint32)]
    l.oracle_write_prefill_kv_f32.argtypes = [_F, _SZ, _F, _SZ, _SZ, _SZ, _SZ, _F, _F]
    l.oracle_rope_neox_f32.argtypes = [_F, _SZ, _SZ, _SZ, _SZ, _U32, _SZ, ctypes.c_float]
    l.oracle_mrope_f32.argtypes = [_F, _SZ, _F, _SZ, _SZ, _SZ, _SZ, _SZ, _F, _F, _SZ,
                                   ctypes.POINTER(ctypes.c_size_t), _F, _F]
    l.oracle_independent_decode_gqa_f32.argtypes = [_F, _F, _F, _SZ, _SZ, _SZ, _SZ, ctypes.c_float,
                                                    ctypes.c_int, _F]
    l.oracle_independent_decode_gqa_f32.restype = None
    l.oracle_f32_to_f16_array.argtypes = [_F, _U16, _SZ]
    l.oracle_f32_to_f16_array.restype = None
    l.oracle_f16_to_f32_array.argtypes = [_U16, _F, _SZ]
    l.oracle_f16_to_f32_array.restype = None
    l.oracle_normal_f16.argtypes = [ctypes.c_uint64, ctypes.c_float, _U16, _SZ]
    l.oracle_normal_f16.restype = None
    l.oracle_normal_f32.argtypes = [ctypes.c_uint64, _F, _SZ]
    l.oracle_normal_f32.restype = None
    l.oracle_set_expf_overrides.argtypes = [_U32, _U32, _SZ]
    l.oracle_set_expf_overrides.restype = None
    l.oracle_blake3.argtypes = [_U8, _SZ, _U8]
    l.oracle_blake3.restype = None


def _f32(a) -> np.ndarray:
    return np.ascontiguousarray(a, dtype=np.float32)


def _ptr(a: np.ndarray, t):
    return a.ctypes.data_as(t)


def _check(rc: int) -> None:
    if rc != 0:
        raise OracleError(rc)


def decode_gqa_f32(query, key, value, cache_tokens, query_heads, key_value_heads, head_dim) -> np.ndarray:
    q, k, v = _f32(query).ravel(), _f32(key).ravel(), _f32(value).ravel()
    out = np.zeros(query_heads * head_dim, dtype=np.float32)
    _check(lib().oracle_decode_gqa_f32(_ptr(q, _F), q.size, _ptr(k, _F), k.size, _ptr(v, _F), v.size,
                                       cache_tokens, query_heads, key_value_heads, head_dim, _ptr(out, _F)))
    return out


def causal_gqa_f32(query, key, value, tokens, query_heads, key_value_heads, head_dim) -> np.ndarray:
    q, k, v = _f32(query).ravel(), _f32(key).ravel(), _f32(value).ravel()
    out = np.zeros(max(q.size, 1), dtype=np.float32)
    _check(lib().oracle_causal_gqa_f32(_ptr(q, _F), q.size, _ptr(k, _F), k.size, _ptr(v, _F), v.size,
                                       tokens, query_heads, key_value_heads, head_dim, _ptr(out, _F)))
    return out[: q.size]


def top1_f32(logits) -> tuple[int, int]:
    """decoder_logits_top1_f32 (decoder_stack_session.rs:308-366): (index, f32 bits of the logit)."""
    x = _f32(logits).ravel()
    index, bits = ctypes.c_uint32(), ctypes.c_uint32()
    _check(lib().oracle_top1_f32(_ptr(x, _F), x.size, ctypes.byref(index), ctypes.byref(bits)))
    return index.value, bits.value


def linear_f32(input, rows, input_width, weights, bias, output_width) -> np.ndarray:
    """linear_f32 (cpu-ref lib.rs:131-140 via patch_projection_f32 :88-128)."""
    x, w, b = _f32(input).ravel(), _f32(weights).ravel(), _f32(bias).ravel()
    out = np.zeros(max(rows * output_width, 1), dtype=np.float32)
    _check(lib().oracle_linear_f32(_ptr(x, _F), x.size, rows, input_width, _ptr(w, _F), w.size, _ptr(b, _F),
                                   b.size, output_width, _ptr(out, _F)))
    return out[: rows * output_width]


def append_kv_f32(prefix_keys, prefix_values, prefix_tokens, rotated_key, value, key_value_heads, head_dim):
    pk, pv = _f32(prefix_keys).ravel(), _f32(prefix_values).ravel()
    rk, v = _f32(rotated_key).ravel(), _f32(value).ravel()
    width = key_value_heads * head_dim
    ok = np.zeros((prefix_tokens + 1) * width, dtype=np.float32)
    ov = np.zeros_like(ok)
    _check(lib().oracle_append_kv_f32(_ptr(pk, _F), _ptr(pv, _F), prefix_tokens, _ptr(rk, _F), rk.size,
                                      _ptr(v, _F), v.size, key_value_heads, head_dim, _ptr(ok, _F),
                                      _ptr(ov, _F)))
    return ok, ov


def write_prefill_kv_f32(rotated_key, value, tokens, key_value_heads, head_dim):
    k, v = _f32(rotated_key).ravel(), _f32(value).ravel()
    ok, ov = np.zeros(max(k.size, 1), np.float32), np.zeros(max(v.size, 1), np.float32)
    _check(lib().oracle_write_prefill_kv_f32(_ptr(k, _F), k.size, _ptr(v, _F), v.size, tokens,
                                             key_value_heads, head_dim, _ptr(ok, _F), _ptr(ov, _F)))
    return ok[: k.size], ov[: v.size]


def rope_neox_f32(values, rows, width, rotary_dim, positions, base) -> np.ndarray:
    x = _f32(values).ravel().copy()
    pos = np.ascontiguousarray(positions, dtype=np.uint32)
    _check(lib().oracle_rope_neox_f32(_ptr(x, _F), x.size, rows, width, rotary_dim, _ptr(pos, _U32), pos.size,
                                      ctypes.c_float(base)))
    return x


def mrope_f32(query, key, tokens, query_heads, key_value_heads, head_dim, raw_cos, raw_sin, sections):
    q, k = _f32(query).ravel(), _f32(key).ravel()
    c, s = _f32(raw_cos).ravel(), _f32(raw_sin).ravel()
    if c.size != s.size:
        raise OracleError(1)
    sec = (ctypes.c_size_t * 3)(*sections)
    rq, rk = np.zeros(max(q.size, 1), np.float32), np.zeros(max(k.size, 1), np.float32)
    _check(lib().oracle_mrope_f32(_ptr(q, _F), q.size, _ptr(k, _F), k.size, tokens, query_heads, key_value_heads,
                                  head_dim, _ptr(c, _F), _ptr(s, _F), c.size, sec, _ptr(rq, _F), _ptr(rk, _F)))
    return rq[: q.size], rk[: k.size]


def independent_decode_gqa_f32(query, key, value, cache_tokens, query_heads, key_value_heads, head_dim,
                               scale=None, rotate_groups=False) -> np.ndarray:
    q, k, v = _f32(query).ravel(), _f32(key).ravel(), _f32(value).ravel()
    if scale is None:
        scale = np.float32(1.0) / np.sqrt(np.float32(head_dim))
    out = np.zeros(query_heads * head_dim, dtype=np.float32)
    lib().oracle_independent_decode_gqa_f32(_ptr(q, _F), _ptr(k, _F), _ptr(v, _F), cache_tokens, query_heads,
                                            key_value_heads, head_dim, ctypes.c_float(scale),
                                            int(rotate_groups), _ptr(out, _F))
    return out


_override_tables = None


def set_expf_overrides(pairs) -> None:
    """Install ``[(arg_bits, result_bits), ...]`` replacing glibc expf at exact
    arguments; an empty list restores glibc everywhere."""
    global _override_tables
    args = np.ascontiguousarray([a for a, _ in pairs] or [0], dtype=np.uint32)
    results = np.ascontiguousarray([r for _, r in pairs] or [0], dtype=np.uint32)
    _override_tables = (args, results)  # keep alive while installed
    lib().oracle_set_expf_overrides(_ptr(args, _U32), _ptr(results, _U32), len(pairs))


def f32_to_f16(values) -> np.ndarray:
    x = _f32(values)
    out = np.zeros(x.shape, dtype=np.uint16)
    lib().oracle_f32_to_f16_array(_ptr(x, _F), _ptr(out, _U16), x.size)
    return out


def f16_to_f32(bits) -> np.ndarray:
    b = np.ascontiguousarray(bits, dtype=np.uint16)
    out = np.zeros(b.shape, dtype=np.float32)
    lib().oracle_f16_to_f32_array(_ptr(b, _U16), _ptr(out, _F), b.size)
    return out


def normal_f16(seed: int, n: int, scale: float = 1.0) -> np.ndarray:
    """Seeded N(0,1)*scale drawn as fp16 bit patterns (uint16)."""
    out = np.zeros(n, dtype=np.uint16)
    lib().oracle_normal_f16(ctypes.c_uint64(seed), ctypes.c_float(scale), _ptr(out, _U16), n)
    return out


def normal_f32(seed: int, n: int) -> np.ndarray:
    out = np.zeros(n, dtype=np.float32)
    lib().oracle_normal_f32(ctypes.c_uint64(seed), _ptr(out, _F), n)
    return out


def blake3_hex(data: bytes) -> str:
    buf = np.frombuffer(bytes(data), dtype=np.uint8) if data else np.zeros(1, np.uint8)
    out = np.zeros(32, dtype=np.uint8)
    lib().oracle_blake3(_ptr(buf, _U8), len(data), _ptr(out, _U8))
    return out.tobytes().hex()


def stream_seed(config: int, tensor: int, index: int = 0) -> int:
    """Seed of one input stream, keyed by (config, tensor, layer/sequence)."""
    return ((config & 0xFFFF) << 48) | ((tensor & 0xFFFF) << 32) | (index & 0xFFFFFFFF)
