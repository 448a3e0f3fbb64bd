"""On-disk format of a quantized lm_head (safetensors), so a model load can skip the
load-time quantization.

The reference quantizes `lm_head.weight` on the first `_get_logits` call every time the
model loads (src/vllm_quant_kernels/_quant.py:245-380).  This module persists exactly the
attributes that quantization leaves on `lm_head` (the packing contract of that file:
`_int8_w`/`_int8_scales`, `_w8a8_w`/`_w8a8_scales`, `_fp8_w`/`_fp8_scales`,
`_mxfp8_w`/`_mxfp8_w_scales`, `_mxfp4_w`/`_mxfp4_w_scales` + `_mxfp4_K`) in one
safetensors file, with metadata naming the mode, the shape and a fingerprint of the whole
source weight, and loads it back onto the weight's device.  Nothing is executed from the file
(safetensors holds raw tensors and string metadata only).

File layout (safetensors; tensor names are the attribute names without the leading
underscore):
  int8 : int8_w int8 [M,K],            int8_scales fp16 [M]
  w8a8 : w8a8_w int8 [M,K],            w8a8_scales fp32 [M]
  fp8  : fp8_w int8 [M,K] (e4m3 bytes), fp8_scales fp16 [M]
  mxfp8: mxfp8_w uint8 [M,K] (e4m3),   mxfp8_w_scales uint8 [M,K/32] (E8M0)
  mxfp4: mxfp4_w uint8 [M,K/2] (E2M1 pairs, low nibble = even k), mxfp4_w_scales uint8 [M,K/32]
metadata: format="vqk-lmhead", version="1", mode, M, K, source_dtype, fingerprint.
"""
from __future__ import annotations

import hashlib
import os

import torch

FORMAT = "vqk-lmhead"
VERSION = "1"

MODE_TENSORS = {
    "int8": ("_int8_w", "_int8_scales"),
    "w8a8": ("_w8a8_w", "_w8a8_scales"),
    "fp8": ("_fp8_w", "_fp8_scales"),
    "mxfp8": ("_mxfp8_w", "_mxfp8_w_scales"),
    "mxfp4": ("_mxfp4_w", "_mxfp4_w_scales"),
}
# expected dtype of each stored tensor
_DTYPES = {
    "_int8_w": torch.int8, "_int8_scales": torch.float16,
    "_w8a8_w": torch.int8, "_w8a8_scales": torch.float32,
    "_fp8_w": torch.int8, "_fp8_scales": torch.float16,
    "_mxfp8_w": torch.uint8, "_mxfp8_w_scales": torch.uint8,
    "_mxfp4_w": torch.uint8, "_mxfp4_w_scales": torch.uint8,
}


def fingerprint(w: torch.Tensor) -> str:
    """Identity of a weight's whole content: SHA-256 over its shape, dtype and either every
    byte (host tensors) or the device's 128-bit content hash of every byte (``vqk_hash128``,
    one pass over the weight, about 0.2 ms for a 763 MB lm_head), so two weights that
    differ in any element get different fingerprints.  The device kind is part of the
    digest: a fingerprint taken on the GPU is compared with another taken on the GPU."""
    h = hashlib.sha256()
    h.update(f"{tuple(w.shape)}|{w.dtype}|{w.device.type}".encode())
    t = w.detach().contiguous()
    if t.is_cuda:
        from . import _lib
        out = torch.zeros(2, dtype=torch.int64, device=t.device)
        if t.numel():
            _lib.call("vqk_hash128", t.data_ptr(), t.numel() * t.element_size(), out.data_ptr(),
                      torch.cuda.current_stream(t.device).cuda_stream)
        h.update(out.cpu().numpy().tobytes())
    else:
        h.update(t.view(torch.uint8).numpy().tobytes() if t.numel() else b"")
    return h.hexdigest()


def mode_of(lm_head) -> str | None:
    for mode, (wname, _) in MODE_TENSORS.items():
        if hasattr(lm_head, wname):
            return mode
    return None


def cache_path(directory: str, mode: str, M: int, K: int) -> str:
    return os.path.join(directory, f"lm_head_{mode}_{M}x{K}.safetensors")


def save_quantized(lm_head, path: str, source: torch.Tensor | None = None) -> str:
    """Write the quantized attributes on `lm_head` to `path`; returns the mode.
    `source` (default lm_head.weight) is the weight the fingerprint is taken of."""
    from safetensors.torch import save_file

    mode = mode_of(lm_head)
    if mode is None:
        raise ValueError("lm_head carries no quantized weight")
    src = source if source is not None else lm_head.weight.data
    M, K = int(src.shape[0]), int(src.shape[1])
    tensors = {}
    for name in MODE_TENSORS[mode]:
        t = getattr(lm_head, name)
        tensors[name.lstrip("_")] = t.detach().contiguous().cpu()
    meta = {"format": FORMAT, "version": VERSION, "mode": mode, "M": str(M), "K": str(K),
            "source_dtype": str(src.dtype).replace("torch.", ""), "fingerprint": fingerprint(src)}
    os.makedirs(os.path.dirname(os.path.abspath(path)), exist_ok=True)
    tmp = path + ".tmp"
    save_file(tensors, tmp, metadata=meta)
    os.replace(tmp, path)  # readers never see a half-written file
    return mode


def load_quantized(lm_head, path: str, mode: str | None = None, source: torch.Tensor | None = None) -> str | None:
    """Install the quantized attributes stored in `path` on `lm_head`, on the device of its
    weight.  Returns the mode, or None (nothing installed) when the file is missing, of
    another format or mode, or was made from a different weight."""
    from safetensors import safe_open

    if not os.path.exists(path):
        return None
    src = source if source is not None else lm_head.weight.data
    with safe_open(path, framework="pt", device="cpu") as f:
        meta = f.metadata() or {}
        if meta.get("format") != FORMAT or meta.get("version") != VERSION:
            return None
        fmode = meta.get("mode")
        if fmode not in MODE_TENSORS or (mode is not None and fmode != mode):
            return None
        M, K = int(src.shape[0]), int(src.shape[1])
        if meta.get("M") != str(M) or meta.get("K") != str(K):
            return None
        if meta.get("fingerprint") != fingerprint(src):
            return None
        loaded = {}
        for name in MODE_TENSORS[fmode]:
            t = f.get_tensor(name.lstrip("_"))
            if t.dtype != _DTYPES[name]:
                return None
            loaded[name] = t
    kb = K // 2 if fmode == "mxfp4" else K
    wname, sname = MODE_TENSORS[fmode]
    if tuple(loaded[wname].shape) != (M, kb):
        return None
    want_s = (M, K // 32) if fmode.startswith("mx") else (M,)
    if tuple(loaded[sname].shape) != want_s:
        return None
    for name, t in loaded.items():
        setattr(lm_head, name, t.to(src.device, non_blocking=False).contiguous())
    if fmode == "mxfp4":
        lm_head._mxfp4_K = K
    return fmode
