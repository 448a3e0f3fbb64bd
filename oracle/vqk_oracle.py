"""TEST INFRASTRUCTURE ONLY - Python face of the CPU oracle.

Wraps oracle/liboracle.so (vqk_oracle.c, a CPU restatement of the reference plugin's
arithmetic) with numpy-level functions, plus the synthetic input generators of the
benchmark configurations.  Only tests/, __graft_entry__.smoke() and bench.py's
cpu_baseline leg import this module; the product (vllm_quant_kernels) never does.
"""
from __future__ import annotations

import ctypes
import os

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(HERE, "liboracle.so")

_P = ctypes.c_void_p
_L = ctypes.c_int64
_I = ctypes.c_int
_F = ctypes.c_float
_U64 = ctypes.c_uint64

_SIG = {
    "vqko_philox4x32_10": (None, [_P, _P, _P]),
    "vqko_uniform": (_F, [ctypes.c_uint32]),
    "vqko_rand": (_F, [_U64, ctypes.c_uint32]),
    "vqko_logf": (_F, [_F]),
    "vqko_gumbel": (_F, [_F]),
    "vqko_gumbel_max_over_all_words": (_F, []),
    "vqko_gumbel_upper": (_F, [_F]),
    "vqko_gumbel_upper_min_slack": (_F, []),
    "vqko_gumbel_scores": (None, [_P, _L, _L, _L, _P, _P, _P, _P]),
    "vqko_gumbel_argmax": (None, [_P, _L, _L, _L, _P, _P, _P, _P, _I]),
    "vqko_e4m3_to_f32": (_F, [ctypes.c_uint8]),
    "vqko_f32_to_e4m3": (ctypes.c_uint8, [_F]),
    "vqko_f32_to_e2m1": (ctypes.c_uint8, [_F]),
    "vqko_e2m1_to_f32": (_F, [ctypes.c_uint8]),
    "vqko_mx_exponent": (_I, [_F, _F]),
    "vqko_quant_rows_int8": (None, [_P, _L, _L, _P, _P]),
    "vqko_quant_rows_fp8": (None, [_P, _L, _L, _P, _P]),
    "vqko_quant_mx": (None, [_P, _L, _L, _I, _P, _P]),
    "vqko_act_quant_int8": (None, [_P, _L, _P, _P]),
    "vqko_lmhead_w8a16": (None, [_P, _P, _P, _L, _L, _L, _P]),
    "vqko_lmhead_w8a8": (None, [_P, _P, _P, _F, _L, _L, _L, _P, _P]),
    "vqko_lmhead_fp8": (None, [_P, _P, _P, _L, _L, _L, _P]),
    "vqko_lmhead_mx": (None, [_P, _P, _P, _P, _I, _L, _L, _L, _P]),
    "vqko_max_threads": (_I, []),
    "vqko_set_threads": (None, [_I]),
    "vqko_f32_to_e4m3_array": (None, [_P, _L, _P]),
    "vqko_f32_to_e2m1_array": (None, [_P, _L, _P]),
    "vqko_rand_array": (None, [_U64, _P, _L, _P]),
    "vqko_philox_array": (None, [_P, _P, _L, _P]),
    "vqko_logf_array": (None, [_P, _L, _P]),
    "vqko_gumbel_array": (None, [_P, _L, _P]),
    "vqko_mx_exponent_array": (None, [_P, _L, _F, _P]),
}

_lib = None


def lib():
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            from . import build as _b  # noqa: F401  (package-relative import when available)
        _lib = ctypes.CDLL(LIB_PATH)
        for n, (r, a) in _SIG.items():
            f = getattr(_lib, n)
            f.restype = r
            f.argtypes = a
    return _lib


def _p(a: np.ndarray):
    assert a.flags["C_CONTIGUOUS"]
    return a.ctypes.data_as(ctypes.c_void_p)


def _f32(a):
    return np.ascontiguousarray(a, dtype=np.float32)


# -- number formats -------------------------------------------------------------------

def e4m3_encode(x) -> np.ndarray:
    x = _f32(x)
    out = np.empty(x.shape, np.uint8)
    lib().vqko_f32_to_e4m3_array(_p(x), x.size, _p(out))
    return out


def e4m3_decode(b) -> np.ndarray:
    lut = np.array([lib().vqko_e4m3_to_f32(i) for i in range(256)], np.float32)
    return lut[np.asarray(b, np.uint8)]


def e2m1_encode(y) -> np.ndarray:
    y = _f32(y)
    out = np.empty(y.shape, np.uint8)
    lib().vqko_f32_to_e2m1_array(_p(y), y.size, _p(out))
    return out


def e2m1_decode(n) -> np.ndarray:
    lut = np.array([lib().vqko_e2m1_to_f32(i) for i in range(16)], np.float32)
    return lut[np.asarray(n, np.uint8)]


def mx_exponent(amax, qmax: float) -> np.ndarray:
    a = _f32(amax)
    out = np.empty(a.shape, np.int32)
    lib().vqko_mx_exponent_array(_p(a), a.size, qmax, _p(out))
    return out


def to_f16_bits(x) -> np.ndarray:
    """float32 -> fp16 bits, round to nearest even (numpy's conversion)."""
    return _f32(x).astype(np.float16).view(np.uint16)


# -- quantizers (inputs: exact float32 values of the source tensor) ----------------------

def quant_rows_int8(w):
    w = _f32(w)
    M, K = w.shape
    q = np.empty((M, K), np.int8)
    s = np.empty(M, np.float32)
    lib().vqko_quant_rows_int8(_p(w), M, K, _p(q), _p(s))
    return q, s


def quant_rows_fp8(w):
    w = _f32(w)
    M, K = w.shape
    q = np.empty((M, K), np.uint8)
    s = np.empty(M, np.float32)
    lib().vqko_quant_rows_fp8(_p(w), M, K, _p(q), _p(s))
    return q, s


def quant_mxfp8(t):
    t = _f32(t)
    R, K = t.shape
    q = np.empty((R, K), np.uint8)
    s = np.empty((R, K // 32), np.uint8)
    lib().vqko_quant_mx(_p(t), R, K, 0, _p(q), _p(s))
    return q, s


def quant_mxfp4(t):
    t = _f32(t)
    R, K = t.shape
    q = np.empty((R, K // 2), np.uint8)
    s = np.empty((R, K // 32), np.uint8)
    lib().vqko_quant_mx(_p(t), R, K, 1, _p(q), _p(s))
    return q, s


def act_quant_int8(x):
    x = _f32(x)
    xq = np.empty(x.shape, np.int8)
    xs = np.empty(1, np.float32)
    lib().vqko_act_quant_int8(_p(x), x.size, _p(xq), _p(xs))
    return xq, float(xs[0])


# -- lm_head references: fp32 values before the final fp16 cast ---------------------------

def lmhead_w8a16(q, s16, x):
    q = np.ascontiguousarray(q, np.int8)
    s = _f32(s16)
    x = _f32(x)
    M, K = q.shape
    B = x.shape[0]
    out = np.empty((B, M), np.float32)
    lib().vqko_lmhead_w8a16(_p(q), _p(s), _p(x), M, K, B, _p(out))
    return out


def lmhead_w8a8(q, ws, xq, xs):
    q = np.ascontiguousarray(q, np.int8)
    ws = _f32(ws)
    xq = np.ascontiguousarray(xq, np.int8)
    M, K = q.shape
    B = xq.shape[0]
    acc = np.empty((B, M), np.int32)
    out = np.empty((B, M), np.float32)
    lib().vqko_lmhead_w8a8(_p(q), _p(ws), _p(xq), float(xs), M, K, B, _p(acc), _p(out))
    return acc, out


def lmhead_fp8(q, s16, xq):
    q = np.ascontiguousarray(q, np.uint8)
    s = _f32(s16)
    xq = np.ascontiguousarray(xq, np.uint8)
    M, K = q.shape
    B = xq.shape[0]
    out = np.empty((B, M), np.float32)
    lib().vqko_lmhead_fp8(_p(q), _p(s), _p(xq), M, K, B, _p(out))
    return out


def lmhead_mx(w, ws, xq, xs, fp4: bool, K: int):
    w = np.ascontiguousarray(w, np.uint8)
    ws = np.ascontiguousarray(ws, np.uint8)
    xq = np.ascontiguousarray(xq, np.uint8)
    xs = np.ascontiguousarray(xs, np.uint8)
    M = w.shape[0]
    B = xq.shape[0]
    out = np.empty((B, M), np.float32)
    lib().vqko_lmhead_mx(_p(w), _p(ws), _p(xq), _p(xs), 1 if fp4 else 0, M, K, B, _p(out))
    return out


# -- sampler -------------------------------------------------------------------------

def philox(ctr, key) -> np.ndarray:
    ctr = np.ascontiguousarray(ctr, np.uint32).reshape(-1, 4)
    key = np.ascontiguousarray(key, np.uint32).reshape(-1, 2)
    out = np.empty_like(ctr)
    lib().vqko_philox_array(_p(ctr), _p(key), ctr.shape[0], _p(out))
    return out


def rand(seed: int, offsets) -> np.ndarray:
    off = np.ascontiguousarray(offsets, np.uint32)
    out = np.empty(off.shape, np.float32)
    lib().vqko_rand_array(int(seed) & (2**64 - 1), _p(off), off.size, _p(out))
    return out


def logf(x) -> np.ndarray:
    x = _f32(x)
    out = np.empty(x.shape, np.float32)
    lib().vqko_logf_array(_p(x), x.size, _p(out))
    return out


def gumbel(u) -> np.ndarray:
    u = _f32(u)
    out = np.empty(u.shape, np.float32)
    lib().vqko_gumbel_array(_p(u), u.size, _p(out))
    return out


def seeds_u64(seeds) -> np.ndarray:
    """int32 seeds sign-extend to 64 bits (Triton casts the int32 seed to uint64)."""
    s = np.asarray(seeds)
    return s.astype(np.int64).view(np.uint64) if s.dtype != np.uint64 else s


def gumbel_scores(logits, temp, seeds, thr=None) -> np.ndarray:
    x = _f32(logits)
    B, V = x.shape
    sd = np.ascontiguousarray(seeds_u64(seeds), np.uint64)
    t = _f32(temp) if temp is not None else None
    th = _f32(thr) if thr is not None else None
    out = np.empty((B, V), np.float32)
    lib().vqko_gumbel_scores(_p(x), B, V, V, _p(t) if t is not None else None, _p(sd),
                             _p(th) if th is not None else None, _p(out))
    return out


def gumbel_argmax(logits, temp, seeds, thr=None, nthreads: int = 0) -> np.ndarray:
    x = _f32(logits)
    B, V = x.shape
    sd = np.ascontiguousarray(seeds_u64(seeds), np.uint64)
    t = _f32(temp) if temp is not None else None
    th = _f32(thr) if thr is not None else None
    out = np.empty(B, np.int64)
    lib().vqko_gumbel_argmax(_p(x), B, V, V, _p(t) if t is not None else None, _p(sd),
                             _p(th) if th is not None else None, _p(out), int(nthreads))
    return out


def gumbel_max_over_all_words() -> float:
    return float(lib().vqko_gumbel_max_over_all_words())


def gumbel_upper(u) -> np.ndarray:
    u = _f32(u)
    return np.array([lib().vqko_gumbel_upper(float(x)) for x in u.ravel()], np.float32).reshape(u.shape)


def gumbel_upper_min_slack() -> float:
    return float(lib().vqko_gumbel_upper_min_slack())
