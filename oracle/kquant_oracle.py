"""ctypes front end of the CPU oracle -- TEST INFRASTRUCTURE ONLY.

Loads oracle/build/libkquant_oracle.so (built by `make -C oracle`), or the
library KQUANT_ORACLE_LIBRARY names (the ASan + UBSan build of
`make -C oracle asan`, for tests/test_sanitizers.py). Only tests/,
__graft_entry__.smoke() and bench.py's cpu_baseline leg may import this module;
the product package engine_amd never does.
"""
from __future__ import annotations

import ctypes
import os

import numpy as np

_HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.environ.get("KQUANT_ORACLE_LIBRARY") or os.path.join(_HERE, "build", "libkquant_oracle.so")

OK = 0
UNSUPPORTED_TYPE = 1
INVALID_BLOCK_LENGTH = 2
DIMENSION_MISMATCH = 3
BLOCK_MISMATCH = 4
OVERFLOW = 5
INVALID_DIMENSION_COUNT = 6
OUT_OF_SCOPE = 7
BAD_ARGUMENT = 8

BLOCK_BYTES = {12: 144, 13: 176, 14: 210}

_lib = None


def lib():
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            raise RuntimeError(f"oracle library missing: {LIB_PATH} (run `make -C oracle`)")
        l = ctypes.CDLL(LIB_PATH)
        u8p = ctypes.POINTER(ctypes.c_uint8)
        f32p = ctypes.POINTER(ctypes.c_float)
        u64p = ctypes.POINTER(ctypes.c_uint64)
        szp = ctypes.POINTER(ctypes.c_size_t)
        l.oracle_f16_to_f32.restype = ctypes.c_float
        l.oracle_f16_to_f32.argtypes = [ctypes.c_uint16]
        l.oracle_tensor_layout.argtypes = [ctypes.c_uint32, u64p, u64p]
        l.oracle_byte_len.argtypes = [u64p, ctypes.c_size_t, ctypes.c_uint32, u64p]
        l.oracle_q4_k_scales.argtypes = [u8p, u8p, u8p]
        l.oracle_q4_k_scales.restype = None
        l.oracle_dequantize_block.argtypes = [ctypes.c_uint32, u8p, ctypes.c_size_t, f32p,
                                              ctypes.c_size_t, szp]
        l.oracle_dequantize_tensor.argtypes = [ctypes.c_uint32, u8p, ctypes.c_size_t, f32p,
                                               ctypes.c_size_t]
        l.oracle_gguf_gemv.argtypes = [f32p, ctypes.c_size_t, ctypes.c_size_t, f32p, f32p]
        l.oracle_quant_gemv.argtypes = [ctypes.c_uint32, u8p, ctypes.c_size_t, ctypes.c_size_t,
                                        ctypes.c_size_t, f32p, f32p, ctypes.c_size_t]
        l.oracle_quant_gemv_threads.argtypes = [ctypes.c_uint32, u8p, ctypes.c_size_t,
                                                ctypes.c_size_t, ctypes.c_size_t, f32p, f32p,
                                                ctypes.c_int]
        l.oracle_rms_norm_raw.argtypes = [f32p, f32p, ctypes.c_size_t, ctypes.c_float, f32p]
        l.oracle_swiglu.argtypes = [f32p, f32p, ctypes.c_size_t, f32p]
        l.oracle_swiglu.restype = None
        u16p = ctypes.POINTER(ctypes.c_uint16)
        l.oracle_f32_to_f16_bits.restype = ctypes.c_uint16
        l.oracle_f32_to_f16_bits.argtypes = [ctypes.c_float]
        l.oracle_rope_neox.restype = None
        l.oracle_rope_neox.argtypes = [f32p, ctypes.c_size_t, ctypes.c_size_t, ctypes.c_size_t,
                                       ctypes.c_size_t, ctypes.c_float]
        l.oracle_qwen3_attention.argtypes = [f32p, f32p, f32p, f32p, f32p, ctypes.c_float, ctypes.c_float,
                                             ctypes.c_size_t, ctypes.c_size_t, ctypes.c_size_t,
                                             ctypes.c_size_t, u16p, u16p, ctypes.c_size_t, f32p]
        l.oracle_argmax.restype = ctypes.c_size_t
        l.oracle_argmax.argtypes = [f32p, ctypes.c_size_t]
        l.oracle_time_quant_gemv.argtypes = [ctypes.c_uint32, u8p, ctypes.c_size_t,
                                             ctypes.c_size_t, ctypes.c_size_t, f32p, f32p,
                                             ctypes.c_int, ctypes.c_int, ctypes.c_int,
                                             ctypes.POINTER(ctypes.c_double),
                                             ctypes.POINTER(ctypes.c_double)]
        _lib = l
    return _lib


def _u8(a):
    return a.ctypes.data_as(ctypes.POINTER(ctypes.c_uint8))


def _f32(a):
    return a.ctypes.data_as(ctypes.POINTER(ctypes.c_float))


class OracleError(Exception):
    def __init__(self, status, expected=None):
        super().__init__(f"oracle status {status}")
        self.status = status
        self.expected = expected


def f16_to_f32(bits: int) -> float:
    return lib().oracle_f16_to_f32(bits)


def tensor_layout(value_type: int):
    e = ctypes.c_uint64()
    b = ctypes.c_uint64()
    st = lib().oracle_tensor_layout(value_type, ctypes.byref(e), ctypes.byref(b))
    if st != OK:
        raise OracleError(st)
    return e.value, b.value


def byte_len(dims, value_type: int) -> int:
    arr = (ctypes.c_uint64 * max(1, len(dims)))(*dims)
    out = ctypes.c_uint64()
    st = lib().oracle_byte_len(arr, len(dims), value_type, ctypes.byref(out))
    if st != OK:
        raise OracleError(st)
    return out.value


def q4_k_scales(packed12: bytes):
    src = np.frombuffer(bytes(packed12), dtype=np.uint8).copy()
    sc = np.zeros(8, np.uint8)
    mn = np.zeros(8, np.uint8)
    lib().oracle_q4_k_scales(_u8(src), _u8(sc), _u8(mn))
    return sc, mn


def dequantize_block(value_type: int, encoded) -> np.ndarray:
    enc = np.ascontiguousarray(np.frombuffer(bytes(encoded), dtype=np.uint8))
    out = np.zeros(256, np.float32)
    expected = ctypes.c_size_t()
    st = lib().oracle_dequantize_block(value_type, _u8(enc), enc.size, _f32(out), out.size,
                                       ctypes.byref(expected))
    if st != OK:
        raise OracleError(st, expected.value)
    elems, _ = tensor_layout(value_type)
    return out[:elems].copy()


def dequantize_tensor(value_type: int, encoded: np.ndarray) -> np.ndarray:
    enc = np.ascontiguousarray(encoded, dtype=np.uint8).reshape(-1)
    elems, bb = tensor_layout(value_type)
    out = np.zeros((enc.size // bb) * elems, np.float32)
    st = lib().oracle_dequantize_tensor(value_type, _u8(enc), enc.size, _f32(out), out.size)
    if st != OK:
        raise OracleError(st)
    return out


def gguf_gemv(weight: np.ndarray, in_dim: int, x: np.ndarray) -> np.ndarray:
    w = np.ascontiguousarray(weight, dtype=np.float32).reshape(-1)
    xx = np.ascontiguousarray(x, dtype=np.float32)
    y = np.zeros(w.size // in_dim, np.float32)
    st = lib().oracle_gguf_gemv(_f32(w), w.size, in_dim, _f32(xx), _f32(y))
    if st != OK:
        raise OracleError(st)
    return y


def quant_gemv(value_type: int, encoded: np.ndarray, k: int, n: int, x: np.ndarray,
               members: int = 1, threads: int = 1) -> np.ndarray:
    enc = np.ascontiguousarray(encoded, dtype=np.uint8).reshape(-1)
    xx = np.ascontiguousarray(x, dtype=np.float32).reshape(-1)
    if xx.size != k * members:
        raise ValueError("x must hold members*k values")
    y = np.zeros(n * members, np.float32)
    if threads == 1:
        st = lib().oracle_quant_gemv(value_type, _u8(enc), enc.size, k, n, _f32(xx), _f32(y),
                                     members)
    else:
        if members != 1:
            raise ValueError("threaded oracle handles one member")
        st = lib().oracle_quant_gemv_threads(value_type, _u8(enc), enc.size, k, n, _f32(xx),
                                             _f32(y), threads)
    if st != OK:
        raise OracleError(st)
    return y.reshape(members, n) if members > 1 else y


def rms_norm_raw(x: np.ndarray, weight: np.ndarray, eps: float) -> np.ndarray:
    xx = np.ascontiguousarray(x, dtype=np.float32)
    ww = np.ascontiguousarray(weight, dtype=np.float32)
    out = np.zeros_like(xx)
    st = lib().oracle_rms_norm_raw(_f32(xx), _f32(ww), xx.size, eps, _f32(out))
    if st != OK:
        raise OracleError(st)
    return out


def swiglu(gate: np.ndarray, up: np.ndarray) -> np.ndarray:
    g = np.ascontiguousarray(gate, dtype=np.float32)
    u = np.ascontiguousarray(up, dtype=np.float32)
    out = np.zeros_like(g)
    lib().oracle_swiglu(_f32(g), _f32(u), g.size, _f32(out))
    return out


def time_quant_gemv(value_type, encoded, k, n, x, threads=1, warmup=3, iters=20):
    enc = np.ascontiguousarray(encoded, dtype=np.uint8).reshape(-1)
    xx = np.ascontiguousarray(x, dtype=np.float32)
    y = np.zeros(n, np.float32)
    med = ctypes.c_double()
    mn = ctypes.c_double()
    st = lib().oracle_time_quant_gemv(value_type, _u8(enc), enc.size, k, n, _f32(xx), _f32(y),
                                      threads, warmup, iters, ctypes.byref(med), ctypes.byref(mn))
    if st != OK:
        raise OracleError(st)
    return med.value, mn.value, y


def f32_to_f16_bits(value: float) -> int:
    return int(lib().oracle_f32_to_f16_bits(value))


def rope_neox(values: np.ndarray, heads: int, head_dim: int, rot_dims: int, pos: int,
              base: float) -> np.ndarray:
    out = np.ascontiguousarray(values, dtype=np.float32).copy()
    lib().oracle_rope_neox(_f32(out), heads, head_dim, rot_dims, pos, base)
    return out


def qwen3_attention(q, k, v, q_norm, k_norm, eps, rope_base, q_heads, kv_heads, head_dim, pos,
                    kv_keys: np.ndarray, kv_values: np.ndarray) -> np.ndarray:
    """One attention step; kv_keys / kv_values ([capacity][kv_heads][head_dim]
    uint16 binary16 bits) are updated in place at `pos`."""
    arrs = [np.ascontiguousarray(a, dtype=np.float32) for a in (q, k, v, q_norm, k_norm)]
    assert kv_keys.dtype == np.uint16 and kv_keys.flags.c_contiguous
    assert kv_values.dtype == np.uint16 and kv_values.flags.c_contiguous
    out = np.zeros(q_heads * head_dim, np.float32)
    u16 = ctypes.POINTER(ctypes.c_uint16)
    st = lib().oracle_qwen3_attention(*[_f32(a) for a in arrs], eps, rope_base, q_heads, kv_heads,
                                      head_dim, pos, kv_keys.ctypes.data_as(u16),
                                      kv_values.ctypes.data_as(u16), kv_keys.shape[0], _f32(out))
    if st != OK:
        raise OracleError(st)
    return out


def argmax(logits: np.ndarray) -> int:
    x = np.ascontiguousarray(logits, dtype=np.float32)
    return int(lib().oracle_argmax(_f32(x), x.size))
