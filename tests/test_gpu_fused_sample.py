"""Fused lm_head + Gumbel-argmax sampling (vqk_lmhead_sample): the tokens must equal the
unfused path's (lm_head -> fp16 logits -> fp32 -> sampler) bit for bit, and the logits it
writes must equal the plain lm_head's."""
import numpy as np
import pytest
import torch

from oracle import vqk_oracle as O
from vllm_quant_kernels import _kernels as K_
from vllm_quant_kernels import _sampler_kernels as S_

pytestmark = pytest.mark.gpu


def _weights(M, K, seed=7):
    g = torch.Generator(device="cuda").manual_seed(seed)
    w = torch.randn(M, K, generator=g, device="cuda") * 0.02
    f = torch.exp(torch.rand(M, 1, generator=g, device="cuda") * np.log(6.0))
    return (w * f).clamp(-0.19, 0.19)


def _quantized(mode, w):
    if mode == "w8a16":
        return K_.quant_rows_int8(w, torch.float16)
    if mode == "w8a8":
        return K_.quant_rows_int8(w, torch.float32)
    if mode == "fp8":
        return K_.quant_rows_fp8(w)
    if mode == "mxfp8":
        return K_.quant_mxfp8(w)
    return K_.quant_mxfp4(w)


def _plain(mode, x, q, s, K):
    if mode == "mxfp4":
        return K_.lmhead_mxfp4(x, q, s, K)
    return getattr(K_, "lmhead_" + mode)(x, q, s)


@pytest.mark.parametrize("mode,B", [(m, b) for m in ("w8a16", "w8a8", "fp8", "mxfp8", "mxfp4")
                                    for b in (1, 4, 13, 16, 32) if not (m == "w8a16" and b > 16)])
def test_fused_sample_matches_unfused(mode, B):
    M, K = 20_011, 1024   # ragged M: the last tile is partial
    w = _weights(M, K)
    q, s = _quantized(mode, w)
    g = torch.Generator(device="cuda").manual_seed(100 + B)
    x = (torch.randn(B, K, generator=g, device="cuda") * 2.0).half()
    temp = torch.rand(B, generator=g, device="cuda") * 1.2 + 0.3
    temp[::3] = 0.0                                   # greedy rows mixed in
    seeds = torch.randint(0, 2**62, (B,), generator=g, device="cuda", dtype=torch.int64)
    tok, logits = K_.lmhead_sample(mode, x, q, s, temp, seeds, K=K)
    ref_logits = _plain(mode, x, q, s, K)
    assert torch.equal(logits, ref_logits)
    ref_tok = S_.fused_gumbel_sample(ref_logits.float().contiguous(), temp, seeds)
    assert torch.equal(tok, ref_tok)
    o = O.gumbel_argmax(ref_logits.float().cpu().numpy(), temp.cpu().numpy(), seeds.cpu().numpy())
    assert np.array_equal(tok.cpu().numpy(), o)


def test_fused_sample_plain_argmax_and_int32_seeds():
    M, K, B = 8192, 2048, 6
    w = _weights(M, K, seed=9)
    q, s = _quantized("fp8", w)
    x = torch.randn(B, K, device="cuda").half()
    seeds = torch.randint(0, 2**31 - 1, (B,), device="cuda", dtype=torch.int32)
    tok, logits = K_.lmhead_sample("fp8", x, q, s, None, seeds)
    assert torch.equal(tok, logits.float().argmax(dim=-1))
    temp = torch.full((B,), 0.7, device="cuda")
    tok, logits = K_.lmhead_sample("fp8", x, q, s, temp, seeds)
    assert torch.equal(tok, S_.fused_gumbel_sample(logits.float().contiguous(), temp, seeds))


@pytest.mark.parametrize("mode,B", [("w8a16", 17), ("w8a16", 33), ("fp8", 33), ("mxfp4", 33)])
def test_fused_sample_rejects_large_batches(mode, B):
    """One batch group only: 16 rows for W8A16 (fp16 activations take twice the LDS per
    row), 32 for the other modes."""
    M, K = 4096, 1024
    w = _weights(M, K)
    q, s = _quantized(mode, w)
    x = torch.randn(B, K, device="cuda").half()
    seeds = torch.zeros(B, dtype=torch.int32, device="cuda")
    with pytest.raises(ValueError):
        K_.lmhead_sample(mode, x, q, s, None, seeds, K=K)
