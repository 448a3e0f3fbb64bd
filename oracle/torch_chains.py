"""TEST INFRASTRUCTURE ONLY - the reference's own torch op chains, restated.

Where the reference computes a step with a short chain of torch operators rather than a
kernel, the chain is restated here with the same operators so the device implementations
can be checked against it.  Only tests/ import this module; the product never does.
"""
from __future__ import annotations

import torch


def compute_topk_threshold(logits: torch.Tensor, top_k: torch.Tensor, vocab_size: int):
    """Per-row k-th largest raw logit, or None when top-k is off for every row
    (reference src/vllm_quant_kernels/_sampler.py:62-93): max_k = top_k.max().item();
    None if max_k >= V; else torch.topk(logits, max_k, sorted=True) and a gather at
    column clamp(top_k, max=max_k) - 1 (clamped at 0)."""
    max_k = int(top_k.max().item())
    if max_k >= vocab_size:
        return None
    vals, _ = torch.topk(logits, max_k, dim=-1, sorted=True)
    col = (top_k.clamp(max=max_k) - 1).clamp(min=0).to(torch.int64).unsqueeze(-1)
    return vals.gather(dim=-1, index=col).squeeze(-1).contiguous()
