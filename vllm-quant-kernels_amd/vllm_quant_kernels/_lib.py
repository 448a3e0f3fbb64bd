"""ctypes binding of libvqk_hip.so (the gfx950 kernels behind this plugin).

The library is built in-tree by ``csrc/build.py`` (``__graft_entry__.build()``) and lives
next to this file.  There is no fallback: if the library or a gfx950 device is missing,
every entry point raises, so a run that produces numbers has run the HIP kernels.

Error mapping (mirrors the reference's contract, src/vllm_quant_kernels/_sampler_kernels.py:
148-156 and _quant.py:47, 78-79): argument problems detected before launch raise
``ValueError`` (``AssertionError`` is used by the Python wrappers for the reference's own
asserts); launch failures raise ``RuntimeError``.
"""
from __future__ import annotations

import ctypes
import os
import threading

_HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.environ.get("VQK_LIB", os.path.join(_HERE, "libvqk_hip.so"))

VQK_OK = 0
VQK_EINVAL = -1
VQK_EUNSUPPORTED = -2
VQK_ENODEVICE = -3
VQK_EWORKSPACE = -4

VQK_F32, VQK_F16, VQK_BF16 = 0, 1, 2

_P = ctypes.c_void_p
_I = ctypes.c_int
_L = ctypes.c_int64

# name -> (restype, argtypes); the order follows include/vqk.h
SIGNATURES = {
    "vqk_abi_version": (_I, []),
    "vqk_device_check": (_I, []),
    "vqk_strerror": (ctypes.c_char_p, [_I]),
    "vqk_quant_rows_int8": (_I, [_P, _I, _L, _L, _L, _P, _P, _I, _P]),
    "vqk_quant_rows_fp8": (_I, [_P, _I, _L, _L, _L, _P, _P, _P]),
    "vqk_quant_mxfp8": (_I, [_P, _I, _L, _L, _L, _P, _P, _P]),
    "vqk_quant_mxfp4": (_I, [_P, _I, _L, _L, _L, _P, _P, _P]),
    "vqk_act_quant_int8": (_I, [_P, _I, _L, _L, _L, _P, _P, _P]),
    "vqk_act_cast_e4m3": (_I, [_P, _I, _L, _L, _L, _P, _P]),
    "vqk_lmhead_w8a16": (_I, [_P, _P, _P, _L, _P, _L, _L, _L, _L, _P]),
    "vqk_lmhead_w8a8": (_I, [_P, _P, _P, _I, _L, _P, _L, _P, _L, _L, _L, _P]),
    "vqk_lmhead_fp8": (_I, [_P, _P, _P, _I, _L, _P, _L, _L, _L, _L, _P]),
    "vqk_lmhead_mxfp8": (_I, [_P, _P, _P, _I, _L, _P, _L, _L, _L, _L, _P]),
    "vqk_lmhead_mxfp4": (_I, [_P, _P, _P, _I, _L, _P, _L, _L, _L, _L, _P]),
    "vqk_gemm_fp8": (_I, [_P, _P, _P, _P, _L, _L, _L, _L, _P]),
    "vqk_gemm_w8a8": (_I, [_P, _P, _P, ctypes.c_float, _P, _L, _P, _L, _L, _L, _P]),
    "vqk_gemm_w8a8_devscale": (_I, [_P, _P, _P, _P, _P, _L, _P, _L, _L, _L, _P]),
    "vqk_lmhead_sample_workspace_size": (_L, [_L]),
    "vqk_topk_threshold_workspace_size": (_L, [_L, _L]),
    "vqk_topk_threshold": (_I, [_P, _L, _L, _L, _P, _I, _P, _P, _L, _P]),
    "vqk_lmhead_sample": (_I, [_I, _P, _P, _P, _I, _L, _P, _L, _L, _L, _L, _P, _P, _I, _P, _P, _L, _P]),
    "vqk_gemm_mxfp8": (_I, [_P, _P, _P, _P, _P, _L, _L, _L, _L, _P]),
    "vqk_gemm_mxfp4": (_I, [_P, _P, _P, _P, _P, _L, _L, _L, _L, _P]),
    "vqk_gumbel_workspace_size": (_L, [_L, _L]),
    "vqk_gumbel_argmax": (_I, [_P, _L, _L, _L, _P, _P, _I, _P, _P, _P, _L, _P]),
    "vqk_gumbel_scores": (_I, [_P, _L, _L, _L, _P, _P, _I, _P, _P, _P]),
    "vqk_gumbel_noalloc_max_bytes": (_L, []),
    "vqk_gumbel_argmax_noalloc": (_I, [_P, _L, _L, _L, _P, _P, _I, _P, _P, _P]),
    "vqk_debug_e4m3_hw_check": (_I, [ctypes.c_uint32, ctypes.c_uint32, _I, _P, _P, _P]),
    "vqk_hash128": (_I, [_P, _L, _P, _P]),
}

_lib = None
_lock = threading.Lock()


class VqkLibraryMissing(RuntimeError):
    pass


def load(path: str | None = None):
    """Load (once) and return the ctypes handle; raises VqkLibraryMissing if absent."""
    global _lib
    if _lib is not None and path is None:
        return _lib
    with _lock:
        if _lib is not None and path is None:
            return _lib
        p = path or LIB_PATH
        if not os.path.exists(p):
            raise VqkLibraryMissing(
                f"[vllm-quant-kernels] {p} is missing: build it with "
                f"`python vllm-quant-kernels_amd/csrc/build.py` (or __graft_entry__.build())")
        lib = ctypes.CDLL(p)
        for name, (res, args) in SIGNATURES.items():
            fn = getattr(lib, name)
            fn.restype = res
            fn.argtypes = args
        if path is None:
            _lib = lib
        return lib


def strerror(code: int) -> str:
    return load().vqk_strerror(code).decode()


def check(rc: int, what: str) -> None:
    if rc == VQK_OK:
        return
    msg = f"{what}: {strerror(rc)} (code {rc})"
    if rc < 0:
        raise ValueError(msg)
    raise RuntimeError(msg)


def call(name: str, *args) -> None:
    check(getattr(load(), name)(*args), name)


def device_ok() -> bool:
    """True when the library loads and the current HIP device is a gfx950."""
    try:
        return load().vqk_device_check() == VQK_OK
    except (OSError, VqkLibraryMissing):
        return False
