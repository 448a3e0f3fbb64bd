"""Fused Gumbel-argmax sampling over [B, V] fp32 logits (two or three short HIP launches).

Replaces the reference's Triton block-argmax kernel plus its two-op host tail
(src/vllm_quant_kernels/_sampler_kernels.py:38-182) with ``vqk_gumbel_argmax``: the
temperature scaling, Philox noise, top-k masking, per-slice argmax and the cross-slice
reduction all happen on the device without a host synchronisation.  Up to ~2M logits one
launch scores each workgroup's slice against its own best candidate and a second reduces
the workgroups' keys to the tokens; larger batches stream the logits once to find every
row's candidates and block maxima, re-read only the slices that can still hold the winner
(mostly from the last-level cache) and then reduce.

Per row b and vocab index v the kernel takes the argmax (smallest index on ties) of
  y = x                                  if temperature is None or temperature[b] < 1e-5,
  y = x / temperature[b] + G(seed_b, v)  otherwise,
with y = -inf where topk_threshold is given and x < topk_threshold[b] (raw logits).
G = -log(-log(max(u, 2^-126))) and u is Triton's tl.rand(seed, v) (Philox4x32-10, word 0
of counter (v,0,0,0), key = the seed widened to 64 bits), so a given (seed, v) draws the
same uniform as the reference.
"""
from __future__ import annotations

import threading

import torch

from . import _lib

_GREEDY_EPS = 1e-5
_ws_lock = threading.Lock()
_workspaces: dict = {}


def _workspace(device: torch.device, stream: int, B: int, V: int) -> torch.Tensor:
    """Per (device, stream) workspace, grown as needed.  The kernels write every value
    before reading it, so it needs no initialisation.  Launches on one stream are ordered,
    so sharing it among them is safe; different streams get different workspaces.  A
    workspace outgrown by a larger batch is kept alive rather than freed: a HIP graph
    captured earlier on that stream may still replay into it."""
    need = int(_lib.load().vqk_gumbel_workspace_size(B, V))
    key = (device.index, stream)
    with _ws_lock:
        held = _workspaces.setdefault(key, [])
        if not held or held[-1].numel() < need:
            held.append(torch.empty(max(need, 4096), dtype=torch.uint8, device=device))
        return held[-1]


def fused_gumbel_sample(
    logits: torch.Tensor,                         # [B, V] fp32
    temperature: torch.Tensor | None,             # [B] fp32 (None => plain argmax)
    seeds: torch.Tensor,                          # [B] int32 (or int64)
    topk_threshold: torch.Tensor | None = None,   # [B] fp32 or None
    block_size: int = 1024,
) -> torch.Tensor:
    """Fused Gumbel-argmax sampling; returns [B] int64 token ids.

    Same contract as the reference function (src/vllm_quant_kernels/_sampler_kernels.py:123-182);
    ``block_size`` is accepted for signature compatibility and does not change the result
    (the noise depends only on (seed, v)).  int64 seeds are accepted as an extension: the
    full 64 bits key the Philox stream.
    """
    B, V = logits.shape
    assert logits.dtype == torch.float32, f"Fused sampler requires fp32 logits, got {logits.dtype}"
    assert logits.is_contiguous(), "Fused sampler requires contiguous logits"
    assert seeds.shape == (B,) and seeds.dtype in (torch.int32, torch.int64)
    if temperature is not None:
        assert temperature.shape == (B,) and temperature.dtype == torch.float32
    if topk_threshold is not None:
        assert topk_threshold.shape == (B,) and topk_threshold.dtype == torch.float32
    if not logits.is_cuda:
        raise ValueError("fused_gumbel_sample: logits must live on the ROCm device")
    seeds = seeds.contiguous()
    temperature = temperature.contiguous() if temperature is not None else None
    topk_threshold = topk_threshold.contiguous() if topk_threshold is not None else None
    out = torch.empty(B, dtype=torch.int64, device=logits.device)
    if B == 0:
        return out
    stream = torch.cuda.current_stream(logits.device).cuda_stream
    ws = _workspace(logits.device, stream, B, V)
    _lib.call(
        "vqk_gumbel_argmax",
        logits.data_ptr(), logits.stride(0), B, V,
        temperature.data_ptr() if temperature is not None else None,
        seeds.data_ptr(), 1 if seeds.dtype == torch.int64 else 0,
        topk_threshold.data_ptr() if topk_threshold is not None else None,
        out.data_ptr(), ws.data_ptr(), ws.numel(), stream,
    )
    return out


def gumbel_scores(logits, temperature, seeds, topk_threshold=None) -> torch.Tensor:
    """Debug: the [B, V] fp32 values the sampler takes its argmax over."""
    B, V = logits.shape
    assert logits.dtype == torch.float32 and logits.is_contiguous()
    seeds = seeds.contiguous()
    scores = torch.empty(B, V, dtype=torch.float32, device=logits.device)
    stream = torch.cuda.current_stream(logits.device).cuda_stream
    _lib.call(
        "vqk_gumbel_scores",
        logits.data_ptr(), logits.stride(0), B, V,
        temperature.data_ptr() if temperature is not None else None,
        seeds.data_ptr(), 1 if seeds.dtype == torch.int64 else 0,
        topk_threshold.data_ptr() if topk_threshold is not None else None,
        scores.data_ptr(), stream,
    )
    return scores


def topk_threshold(logits: torch.Tensor, top_k: torch.Tensor) -> torch.Tensor:
    """Per-row top-k threshold computed on the device (two short launches, no host sync):
    thr[b] = the max(top_k[b], 1)-th largest raw logit of row b, or -inf for every row
    when max(top_k) >= V, where the reference returns None (-inf masks nothing, so the
    sampler's result is the same).  Replaces the reference's _compute_topk_threshold
    (src/vllm_quant_kernels/_sampler.py:62-93: .item(), torch.topk, gather)."""
    B, V = logits.shape
    assert logits.dtype == torch.float32 and logits.is_contiguous()
    assert top_k.shape == (B,) and top_k.dtype in (torch.int32, torch.int64)
    if not logits.is_cuda:
        raise ValueError("topk_threshold: logits must live on the ROCm device")
    top_k = top_k.to(logits.device).contiguous()
    thr = torch.empty(B, dtype=torch.float32, device=logits.device)
    if B == 0:
        return thr
    need = int(_lib.load().vqk_topk_threshold_workspace_size(B, V))
    ws = torch.empty(max(need, 16), dtype=torch.uint8, device=logits.device)
    _lib.call("vqk_topk_threshold", logits.data_ptr(), logits.stride(0), B, V, top_k.data_ptr(),
              1 if top_k.dtype == torch.int64 else 0, thr.data_ptr(), ws.data_ptr(), ws.numel(),
              torch.cuda.current_stream(logits.device).cuda_stream)
    return thr
