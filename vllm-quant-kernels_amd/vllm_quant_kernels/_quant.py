"""Quantized lm_head: the OOT ``LogitsProcessor`` replacement and the weight quantizers.

Host-side counterpart of the reference's src/vllm_quant_kernels/_quant.py with the same
public surface:

* ``QuantizedLogitsProcessor`` is registered with ``PluggableLayer.register_oot(name=
  "LogitsProcessor")``; on the first ``_get_logits`` it quantizes ``lm_head.weight`` once
  (mode chosen by the VLLM_USE_*_LMHEAD env vars, same priority and gates) and stores the
  result under the reference's attribute names, which are also the dispatch keys;
* ``_quantize_to_mxfp8`` / ``_quantize_to_mxfp4`` / ``MXFP4_GROUP_SIZE`` stay importable.

What changes is underneath: every quantizer and every projection is a gfx950 HIP kernel
(libvqk_hip.so via ctypes), the runtime activation quantization is fused into the
projection launch (no torch op chain, no ``.item()`` sync), and one kernel family serves
every batch size.  The device gate is "gfx950" instead of the reference's Thor check.

vLLM is imported when present.  Without it the module still imports (for benchmarks and
kernel-level use) with a minimal stand-in base class whose upstream path raises.
"""
from __future__ import annotations

import os
import sys
from typing import Optional

import torch

from . import _kernels as K_
from . import _checkpoint as _ckpt
from . import _lib
from ._kernels import MXFP4_GROUP_SIZE, MXFP8_GROUP_SIZE  # noqa: F401  (reference re-export)

try:  # pragma: no cover - exercised through the fake-vllm tests and on real vLLM
    from vllm.model_executor.custom_op import PluggableLayer
    from vllm.model_executor.layers.logits_processor import LogitsProcessor
    from vllm.model_executor.layers.vocab_parallel_embedding import VocabParallelEmbedding
    HAVE_VLLM = True
except ImportError:
    HAVE_VLLM = False
    PluggableLayer = None
    VocabParallelEmbedding = object

    class LogitsProcessor:  # minimal stand-in so the quantized path works without vLLM
        def __init__(self, vocab_size, org_vocab_size=None, scale=1.0, logits_as_input=False,
                     soft_cap=None):
            self.vocab_size = vocab_size
            self.org_vocab_size = org_vocab_size or vocab_size
            self.scale = scale
            self.logits_as_input = logits_as_input
            self.soft_cap = soft_cap
            self.use_all_gather = False

        def _get_logits(self, hidden_states, lm_head, embedding_bias, skip_gather=False):
            raise RuntimeError("upstream LogitsProcessor path needs vLLM, which is not installed")


_TAG = "[vllm-quant-kernels]"

# E2M1 grid midpoints (reference src/vllm_quant_kernels/_quant.py:27-31); the HIP quantizer
# implements the same bucketize with ties to the lower magnitude.
_E2M1_MIDPOINTS = (0.25, 0.75, 1.25, 1.75, 2.5, 3.5, 5.0)
_E2M1_MAX = 6.0


def _quantize_to_mxfp8(t: torch.Tensor, group_size: int = MXFP8_GROUP_SIZE):
    """(R, K) float -> (e4m3 values as uint8 (R, K), E8M0 scales uint8 (R, K/32)).
    Same contract as the reference (src/vllm_quant_kernels/_quant.py:34-61)."""
    assert group_size == MXFP8_GROUP_SIZE, "MX group size is 32"
    R, K = t.shape
    assert K % group_size == 0, f"K={K} must be divisible by group_size={group_size}"
    return K_.quant_mxfp8(t.detach())


def _quantize_to_mxfp4(t: torch.Tensor, group_size: int = MXFP4_GROUP_SIZE):
    """(R, K) float -> (packed E2M1 uint8 (R, K/2), low nibble = even k; E8M0 uint8 (R, K/32)).
    Same contract as the reference (src/vllm_quant_kernels/_quant.py:64-105)."""
    assert group_size == MXFP4_GROUP_SIZE, "MX group size is 32"
    R, K = t.shape
    assert K % group_size == 0, f"K={K} must be divisible by group_size={group_size}"
    assert K % 2 == 0, f"K={K} must be even (FP4 packing)"
    return K_.quant_mxfp4(t.detach())


def _env_bool(name: str) -> bool:
    return os.environ.get(name, "").lower() in ("1", "true", "yes", "on")


def _device_supported(device: torch.device) -> bool:
    """True on a gfx950 device with libvqk_hip.so loadable (replaces `cap[0] >= 10`)."""
    if device.type != "cuda" or getattr(torch.version, "hip", None) is None:
        return False
    try:
        arch = getattr(torch.cuda.get_device_properties(device), "gcnArchName", "")
    except Exception:
        return False
    if not arch.startswith("gfx950"):
        return False
    with torch.cuda.device(device):
        return _lib.device_ok()


def _kernel_k_ok(mode: str, K: int) -> bool:
    """Shapes the HIP projections handle: K % 128 == 0 (K % 256 for MXFP4)."""
    return K % (256 if mode == "mxfp4" else 128) == 0


class QuantizedLogitsProcessor(LogitsProcessor):
    """vLLM LogitsProcessor whose lm_head matmul runs on quantized weights (gfx950 HIP).

    Quantizes lm_head.weight on the first call and keeps the fp16/bf16 original (it may
    be tied to the embedding).  Falls back to the upstream implementation when the weight
    is not fp16/bf16, the vocabulary is small, or the device is not a gfx950.
    """

    _VOCAB_THRESHOLD = 100_000

    def _get_logits(
        self,
        hidden_states: torch.Tensor,
        lm_head: "VocabParallelEmbedding",
        embedding_bias: Optional[torch.Tensor],
        skip_gather: bool = False,
    ) -> Optional[torch.Tensor]:
        if not hasattr(self, "_int8_initialized"):
            self._int8_initialized = True
            self._init_int8(lm_head)
        if not any(hasattr(lm_head, a) for a in ("_int8_w", "_fp8_w", "_w8a8_w", "_mxfp8_w", "_mxfp4_w")):
            return super()._get_logits(hidden_states, lm_head, embedding_bias, skip_gather)
        return self._quantized_forward(hidden_states, lm_head, embedding_bias)

    # -- one-time quantization ---------------------------------------------------------

    def _init_int8(self, lm_head) -> None:
        """Quantize lm_head.weight per the env vars (priority MXFP4 > MXFP8 > FP8 > W8A8 >
        INT8), with the reference's gates and fallbacks
        (src/vllm_quant_kernels/_quant.py:143-243)."""
        w = lm_head.weight.data
        if w.dtype not in (torch.bfloat16, torch.float16):
            return
        if w.shape[0] <= self._VOCAB_THRESHOLD:
            return
        _sys = sys
        ok = _device_supported(w.device)
        Kdim = int(w.shape[1])

        if _env_bool("VLLM_USE_MXFP4_LMHEAD"):
            if not ok:
                print(f"{_TAG} VLLM_USE_MXFP4_LMHEAD requires gfx950 (MI355X), falling back to int8",
                      file=_sys.stderr, flush=True)
            elif Kdim % MXFP4_GROUP_SIZE != 0:
                print(f"{_TAG} VLLM_USE_MXFP4_LMHEAD requires K divisible by {MXFP4_GROUP_SIZE} "
                      f"(got K={Kdim}), falling back to int8", file=_sys.stderr, flush=True)
            elif Kdim % 2 != 0:
                print(f"{_TAG} VLLM_USE_MXFP4_LMHEAD requires even K (got K={Kdim}), falling back to int8",
                      file=_sys.stderr, flush=True)
            elif not _kernel_k_ok("mxfp4", Kdim):
                print(f"{_TAG} VLLM_USE_MXFP4_LMHEAD: the gfx950 kernel needs K % 256 == 0 "
                      f"(got K={Kdim}), falling back to int8", file=_sys.stderr, flush=True)
            else:
                self._init_cached("mxfp4", lm_head, w, _sys, lambda: self._init_mxfp4(lm_head, w, _sys))
                return

        if _env_bool("VLLM_USE_MXFP8_LMHEAD"):
            if not ok:
                print(f"{_TAG} VLLM_USE_MXFP8_LMHEAD requires gfx950 (MI355X), falling back to int8",
                      file=_sys.stderr, flush=True)
            elif Kdim % MXFP8_GROUP_SIZE != 0:
                print(f"{_TAG} VLLM_USE_MXFP8_LMHEAD requires K divisible by {MXFP8_GROUP_SIZE} "
                      f"(got K={Kdim}), falling back to int8", file=_sys.stderr, flush=True)
            elif not _kernel_k_ok("mxfp8", Kdim):
                print(f"{_TAG} VLLM_USE_MXFP8_LMHEAD: the gfx950 kernel needs K % 128 == 0 "
                      f"(got K={Kdim}), falling back to int8", file=_sys.stderr, flush=True)
            else:
                self._init_cached("mxfp8", lm_head, w, _sys, lambda: self._init_mxfp8(lm_head, w, _sys))
                return

        if _env_bool("VLLM_USE_FP8_LMHEAD"):
            if not ok or not _kernel_k_ok("fp8", Kdim):
                print(f"{_TAG} VLLM_USE_FP8_LMHEAD requires gfx950 (MI355X), falling back to int8",
                      file=_sys.stderr, flush=True)
            else:
                self._init_cached("fp8", lm_head, w, _sys, lambda: self._init_fp8(lm_head, w, _sys))
                return

        if _env_bool("VLLM_USE_W8A8_LMHEAD"):
            if not ok or not _kernel_k_ok("w8a8", Kdim):
                print(f"{_TAG} VLLM_USE_W8A8_LMHEAD requires gfx950 (MI355X), falling back to w8a16 int8",
                      file=_sys.stderr, flush=True)
            else:
                self._init_cached("w8a8", lm_head, w, _sys, lambda: self._init_w8a8(lm_head, w, _sys))
                return

        if not ok or not _kernel_k_ok("int8", Kdim):
            # The reference's INT8 kernel runs anywhere; this build's kernels are gfx950-only,
            # so elsewhere the lm_head stays on the upstream (unquantized) path.
            print(f"{_TAG} lm_head left unquantized: the int8 kernel needs a gfx950 (MI355X) "
                  f"device and K % 128 == 0 (got K={Kdim})", file=_sys.stderr, flush=True)
            return
        self._init_cached("int8", lm_head, w, _sys, lambda: self._init_int8_weights(lm_head, w, _sys, ok))

    def _init_cached(self, mode, lm_head, w, _sys, quantize) -> None:
        """Quantize, or, with VQK_LMHEAD_CACHE_DIR set (an extension; the reference always
        quantizes at load), load the packed weight from that directory when a file made
        from this very weight exists, and write one after quantizing otherwise."""
        d = os.environ.get("VQK_LMHEAD_CACHE_DIR", "")
        path = _ckpt.cache_path(d, mode, int(w.shape[0]), int(w.shape[1])) if d else ""
        if d:
            try:
                if _ckpt.load_quantized(lm_head, path, mode=mode, source=w) == mode:
                    self._install_handles(mode, lm_head)
                    print(f"{_TAG} lm_head {mode} weights loaded from {path}", file=_sys.stderr, flush=True)
                    return
            except Exception as e:  # an unreadable cache file: quantize as usual
                print(f"{_TAG} lm_head cache {path} not used ({e})", file=_sys.stderr, flush=True)
        quantize()
        if d:
            try:
                _ckpt.save_quantized(lm_head, path, source=w)
                print(f"{_TAG} lm_head {mode} weights written to {path}", file=_sys.stderr, flush=True)
            except Exception as e:
                print(f"{_TAG} lm_head cache {path} not written ({e})", file=_sys.stderr, flush=True)

    @staticmethod
    def _install_handles(mode, lm_head) -> None:
        """The non-tensor attributes each mode's init leaves on lm_head."""
        if mode == "int8":
            lm_head._int8_use_thor = True
            lm_head._int8_block_m = 128
            lm_head._int8_block_k = 256
            lm_head._int8_gemm_kernel, lm_head._int8_n_bucket = K_._make_thor_gemm_kernel()
        elif mode == "w8a8":
            lm_head._w8a8_gemm_kernel, lm_head._w8a8_n_bucket = K_._make_thor_w8a8_gemm_kernel()
        elif mode == "fp8":
            lm_head._fp8_gemm_kernel, lm_head._fp8_n_bucket = K_._make_thor_fp8_gemm_kernel()
        elif mode == "mxfp8":
            lm_head._mxfp8_gemm_kernel, lm_head._mxfp8_n_bucket = K_._make_thor_mxfp8_gemm_kernel()
        elif mode == "mxfp4":
            lm_head._mxfp4_gemm_kernel, lm_head._mxfp4_n_bucket = K_._make_thor_mxfp4_gemm_kernel()

    def _init_int8_weights(self, lm_head, w, _sys, is_thor: bool) -> None:
        """Per-row INT8 weight-only (reference _quant.py:245-276)."""
        lm_head._int8_use_thor = is_thor
        q, s = K_.quant_rows_int8(w, torch.float16)
        lm_head._int8_w = q
        lm_head._int8_scales = s
        saved_mb = w.numel() * w.element_size() // 1024 // 1024
        print(f"{_TAG} lm_head quantized: fp16 {q.shape[0]}×{q.shape[1]} → int8 "
              f"(saved {saved_mb} MB, kernel=gfx950/int8)", file=_sys.stderr, flush=True)
        lm_head._int8_block_m = 128
        lm_head._int8_block_k = 256
        lm_head._int8_gemm_kernel, lm_head._int8_n_bucket = K_._make_thor_gemm_kernel()

    def _init_w8a8(self, lm_head, w, _sys) -> None:
        """Per-row INT8 weights, fp32 scales; per-tensor INT8 activations at runtime
        (reference _quant.py:278-302)."""
        q, s = K_.quant_rows_int8(w, torch.float32)
        lm_head._w8a8_w = q
        lm_head._w8a8_scales = s
        lm_head._w8a8_gemm_kernel, lm_head._w8a8_n_bucket = K_._make_thor_w8a8_gemm_kernel()
        saved_mb = w.numel() * w.element_size() // 1024 // 1024
        print(f"{_TAG} lm_head quantized: fp16 {q.shape[0]}×{q.shape[1]} → int8 w8a8 "
              f"(saved {saved_mb} MB, kernel=gfx950/w8a8)", file=_sys.stderr, flush=True)

    def _init_fp8(self, lm_head, w, _sys) -> None:
        """Per-row FP8 e4m3, fp16 scales; stored as an int8 view (reference _quant.py:304-325)."""
        q, s = K_.quant_rows_fp8(w)
        lm_head._fp8_w = q.view(torch.int8)
        lm_head._fp8_scales = s
        saved_mb = w.numel() * w.element_size() // 1024 // 1024
        print(f"{_TAG} lm_head quantized: fp16 {q.shape[0]}×{q.shape[1]} → fp8e4m3 "
              f"(saved {saved_mb} MB, kernel=gfx950/fp8)", file=_sys.stderr, flush=True)
        lm_head._fp8_gemm_kernel, lm_head._fp8_n_bucket = K_._make_thor_fp8_gemm_kernel()

    def _init_mxfp8(self, lm_head, w, _sys) -> None:
        """MXFP8 e4m3 + per-32 E8M0 (reference _quant.py:327-348)."""
        q, s = _quantize_to_mxfp8(w)
        lm_head._mxfp8_w = q
        lm_head._mxfp8_w_scales = s
        saved_mb = w.numel() * w.element_size() // 1024 // 1024
        scale_mb = s.numel() // 1024 // 1024
        print(f"{_TAG} lm_head quantized: fp16 {q.shape[0]}×{q.shape[1]} → mxfp8 e4m3 "
              f"(saved {saved_mb} MB, scales {scale_mb} MB, kernel=gfx950/mxfp8)",
              file=_sys.stderr, flush=True)
        lm_head._mxfp8_gemm_kernel, lm_head._mxfp8_n_bucket = K_._make_thor_mxfp8_gemm_kernel()

    def _init_mxfp4(self, lm_head, w, _sys) -> None:
        """MXFP4 E2M1 + per-32 E8M0; activations MXFP8 at runtime (reference _quant.py:350-380)."""
        q, s = _quantize_to_mxfp4(w)
        lm_head._mxfp4_w = q
        lm_head._mxfp4_w_scales = s
        lm_head._mxfp4_K = int(w.shape[1])
        orig_mb = w.numel() * w.element_size() // 1024 // 1024
        new_mb = (q.numel() + s.numel()) // 1024 // 1024
        print(f"{_TAG} lm_head quantized: fp16 {w.shape[0]}×{w.shape[1]} → mxfp4 e2m1 "
              f"({orig_mb} MB → {new_mb} MB, kernel=gfx950/mxfp4 [EXPERIMENTAL])",
              file=_sys.stderr, flush=True)
        lm_head._mxfp4_gemm_kernel, lm_head._mxfp4_n_bucket = K_._make_thor_mxfp4_gemm_kernel()

    # -- per-step forward ----------------------------------------------------------------

    def _quantized_forward(self, hidden_states, lm_head, embedding_bias):
        """Dispatch on which packed weight exists (reference _quant.py:382-397)."""
        if hasattr(lm_head, "_mxfp4_w"):
            return self._mxfp4_forward(hidden_states, lm_head, embedding_bias)
        if hasattr(lm_head, "_mxfp8_w"):
            return self._mxfp8_forward(hidden_states, lm_head, embedding_bias)
        if hasattr(lm_head, "_fp8_w"):
            return self._fp8_forward(hidden_states, lm_head, embedding_bias)
        if hasattr(lm_head, "_w8a8_w"):
            return self._w8a8_forward(hidden_states, lm_head, embedding_bias)
        return self._int8_forward(hidden_states, lm_head, embedding_bias)

    @staticmethod
    def _finish(out, hidden_states, M, embedding_bias):
        logits = out.view(hidden_states.shape[:-1] + (M,))
        if embedding_bias is not None:
            logits = logits + embedding_bias
        return logits

    def _fp8_forward(self, hidden_states, lm_head, embedding_bias):
        M, K = lm_head._fp8_w.shape
        x = hidden_states.reshape(-1, K)
        out = K_.lmhead_fp8(x, lm_head._fp8_w, lm_head._fp8_scales)
        return self._finish(out, hidden_states, M, embedding_bias)

    def _mxfp8_forward(self, hidden_states, lm_head, embedding_bias):
        M, K = lm_head._mxfp8_w.shape
        x = hidden_states.reshape(-1, K)
        out = K_.lmhead_mxfp8(x, lm_head._mxfp8_w, lm_head._mxfp8_w_scales)
        return self._finish(out, hidden_states, M, embedding_bias)

    def _mxfp4_forward(self, hidden_states, lm_head, embedding_bias=None):
        K = lm_head._mxfp4_K
        M = lm_head._mxfp4_w.shape[0]
        x = hidden_states.reshape(-1, K)
        out = K_.lmhead_mxfp4(x, lm_head._mxfp4_w, lm_head._mxfp4_w_scales, K)
        return self._finish(out, hidden_states, M, embedding_bias)

    def _w8a8_forward(self, hidden_states, lm_head, embedding_bias):
        M, K = lm_head._w8a8_w.shape
        x = hidden_states.reshape(-1, K)
        out = K_.lmhead_w8a8(x, lm_head._w8a8_w, lm_head._w8a8_scales)
        return self._finish(out, hidden_states, M, embedding_bias)

    def _int8_forward(self, hidden_states, lm_head, embedding_bias):
        M, K = lm_head._int8_w.shape
        x = hidden_states.reshape(-1, K)
        out = K_.lmhead_w8a16(x.to(torch.float16), lm_head._int8_w, lm_head._int8_scales)
        return self._finish(out, hidden_states, M, embedding_bias)


if HAVE_VLLM:  # pragma: no cover - depends on the environment
    QuantizedLogitsProcessor = PluggableLayer.register_oot(name="LogitsProcessor")(QuantizedLogitsProcessor)
