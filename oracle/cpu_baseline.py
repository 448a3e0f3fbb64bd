"""TEST INFRASTRUCTURE / BASELINE ONLY - the reference's CPU dequantize-then-matmul.

The reference's lm_head math (src/vllm_quant_kernels/_kernels.py:49-84, with the same
quantized weights) restated as plain torch CPU fp32 ops: each call dequantizes the int8
weight in 16384-row chunks and runs F.linear in fp32 (the dequantize-then-matmul of
tests/test_mxfp4_kernel.py:57-77).  bench.py times it as the CPU baseline; nothing in the product uses it.
"""
from __future__ import annotations

import time

import torch
import torch.nn.functional as F

CHUNK = 16384


def w8a16_dequant_matmul(q: torch.Tensor, s16: torch.Tensor, x16: torch.Tensor) -> torch.Tensor:
    """fp16( (x_f32 @ (q_f32 * s16_f32[:, None]).T) ) on the CPU."""
    M = q.shape[0]
    x = x16.float()
    out = torch.empty(x.shape[0], M, dtype=torch.float32)
    s = s16.float()
    for i in range(0, M, CHUNK):
        j = min(i + CHUNK, M)
        wd = q[i:j].float() * s[i:j, None]
        out[:, i:j] = F.linear(x, wd)
    return out.to(torch.float16)


def w8a16_dequant_matmul_us(q_dev, s_dev, x_dev, threads: int, reps: int = 3) -> float:
    """Median wall time (us) of one CPU call on `threads` host threads."""
    torch.set_num_threads(max(1, int(threads)))
    q = q_dev.cpu()
    s = s_dev.cpu()
    x = x_dev.cpu()
    w8a16_dequant_matmul(q, s, x)  # warmup
    ts = []
    for _ in range(reps):
        t = time.perf_counter()
        w8a16_dequant_matmul(q, s, x)
        ts.append((time.perf_counter() - t) * 1e6)
    ts.sort()
    return ts[len(ts) // 2]
