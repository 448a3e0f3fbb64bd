"""TEST INFRASTRUCTURE / BASELINE ONLY - the reference's CPU dequantize-then-matmul.

The reference's lm_head math (src/vllm_quant_kernels/_kernels.py:49-84, with the same
quantized weights) restated as plain torch CPU fp32 ops: each call dequantizes the int8
weight in 16384-row chunks and runs F.linear in fp32 (the dequantize-then-matmul of
tests/test_mxfp4_kernel.py:57-77).  bench.py times it as the CPU baseline; nothing in the product uses it.
Also the sampler's host restatement with numpy (below), the sampler's CPU baseline.
"""
from __future__ import annotations

import time

import numpy as np
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


def w8a16_dequant_matmul_us(q_dev, s_dev, x_dev, threads: int, reps: int = 5) -> float:
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


# ---------------------------------------------------------------------------------------
# Sampler: the reference's fused_gumbel_sample (src/vllm_quant_kernels/_sampler_kernels.py:
# 38-182) restated with numpy array operations on the host: Philox4x32-10 word 0 of counter
# (v, 0, 0, 0) under the row's 64-bit seed (Triton's tl.rand), u = int31(word) * 2^-31 in
# float32, G = -log(-log(max(u, 2^-126))), y = x / T + G (greedy rows: y = x), y = -inf
# below the top-k threshold, argmax with the first index on ties.  np.log is the host libm
# float32 logarithm (within an ulp of the device's), so this is the timing baseline, not
# the checker; its tokens are compared with the C oracle's in tests/test_oracle.py.

_MA, _MB, _WA, _WB = 0xD2511F53, 0xCD9E8D57, 0x9E3779B9, 0xBB67AE85
_M32 = np.uint64(0xFFFFFFFF)


def _philox_word0_np(v: np.ndarray, k0: int, k1: int) -> np.ndarray:
    c0 = v.astype(np.uint64)
    c1 = np.zeros_like(c0)
    c2 = np.zeros_like(c0)
    c3 = np.zeros_like(c0)
    for _ in range(10):
        pa = c0 * np.uint64(_MA)          # < 2^64: exact 32 x 32 -> 64-bit product
        pb = c2 * np.uint64(_MB)
        n0 = (pb >> np.uint64(32)) ^ c1 ^ np.uint64(k0)
        n2 = (pa >> np.uint64(32)) ^ c3 ^ np.uint64(k1)
        c1 = pb & _M32
        c3 = pa & _M32
        c0, c2 = n0, n2
        k0 = (k0 + _WA) & 0xFFFFFFFF
        k1 = (k1 + _WB) & 0xFFFFFFFF
    return c0.astype(np.uint32)


def gumbel_argmax_numpy(logits: np.ndarray, temp, seeds, thr=None) -> np.ndarray:
    """Token ids [B] (int64) of the fused sampler, computed row by row with numpy."""
    x = np.ascontiguousarray(logits, np.float32)
    B, V = x.shape
    sd = np.asarray(seeds).astype(np.int64).view(np.uint64)
    v = np.arange(V, dtype=np.uint32)
    out = np.empty(B, np.int64)
    tiny = np.float32(2.0 ** -126)
    for b in range(B):
        y = x[b]
        t = None if temp is None else np.float32(temp[b])
        if t is not None and not (t < np.float32(1e-5)):
            key = int(sd[b])
            w = _philox_word0_np(v, key & 0xFFFFFFFF, key >> 32).view(np.int32)
            w = np.where(w < 0, -w - 1, w)
            u = w.astype(np.float32) * np.float32(4.6566127342e-10)
            g = -np.log(-np.log(np.maximum(u, tiny)))
            y = y / t + g
        if thr is not None:
            y = np.where(x[b] < np.float32(thr[b]), np.float32(-np.inf), y)
        out[b] = int(np.argmax(y))
    return out


def sampler_numpy_us(logits, temp, seeds, reps: int = 5) -> float:
    """Median wall time (us) of gumbel_argmax_numpy on host copies of the inputs (1 warmup)."""
    x = logits.detach().cpu().numpy() if hasattr(logits, "detach") else logits
    t = temp.detach().cpu().numpy() if hasattr(temp, "detach") else temp
    s = seeds.detach().cpu().numpy() if hasattr(seeds, "detach") else seeds
    gumbel_argmax_numpy(x, t, s)
    ts = []
    for _ in range(reps):
        t0 = time.perf_counter()
        gumbel_argmax_numpy(x, t, s)
        ts.append((time.perf_counter() - t0) * 1e6)
    ts.sort()
    return ts[len(ts) // 2]
