"""HIP-graph capture of the hot path: every replay must equal the eager result.

The lm_head and sampler launches allocate nothing and issue no memset (every sampler
launch writes each workspace value before reading it), so both are capturable.  As a guard
against replay-dependent state, each graph is replayed several times with unrelated eager
work and synchronizations in between, and every replay is compared with eager execution.
"""
import numpy as np
import pytest
import torch
from oracle import vqk_oracle as O
from vllm_quant_kernels import _kernels as K_
from vllm_quant_kernels import _sampler_kernels as S_
from vllm_quant_kernels import _synthetic as syn

pytestmark = pytest.mark.gpu


def _capture(fn, warm):
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        for _ in range(warm):
            fn()
    torch.cuda.current_stream().wait_stream(s)
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g, stream=s):
        out = fn()
    return g, out


@pytest.mark.parametrize("B", [4, 32])  # single-pass and two-pass forms
def test_sampler_graph_replays_match_eager(B):
    logits, temp, seeds = syn.sampler_inputs(B)
    eager = S_.fused_gumbel_sample(logits, temp, seeds).clone()
    g, out = _capture(lambda: S_.fused_gumbel_sample(logits, temp, seeds), 2)
    for r in range(5):
        g.replay()
        torch.cuda.synchronize()
        assert torch.equal(out, eager), f"replay {r}"
        junk = torch.randn(1000, 1000, device="cuda") @ torch.randn(1000, 1000, device="cuda")
        assert torch.equal(S_.fused_gumbel_sample(logits, temp, seeds), eager)
        del junk
    # new inputs written in place are picked up by the next replay
    logits.mul_(-1.0)
    eager2 = S_.fused_gumbel_sample(logits, temp, seeds).clone()
    g.replay()
    torch.cuda.synchronize()
    assert torch.equal(out, eager2)


def test_sampler_graph_survives_larger_call_on_capture_stream():
    """A larger batch sampled on the capture stream after capture needs a larger workspace;
    the one the graph captured must stay allocated (and zero at rest) for its replays."""
    logits, temp, seeds = syn.sampler_inputs(4, 50_000)
    eager = S_.fused_gumbel_sample(logits, temp, seeds).clone()
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        S_.fused_gumbel_sample(logits, temp, seeds)
    torch.cuda.current_stream().wait_stream(s)
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g, stream=s):
        out = S_.fused_gumbel_sample(logits, temp, seeds)
    big, btemp, bseeds = syn.sampler_inputs(64)
    with torch.cuda.stream(s):
        tok_big = S_.fused_gumbel_sample(big, btemp, bseeds)
        junk = torch.full((1 << 22,), 7, dtype=torch.uint8, device="cuda")  # reuses freed blocks
    torch.cuda.synchronize()
    ref_big = O.gumbel_argmax(big.cpu().numpy(), btemp.cpu().numpy(), bseeds.cpu().numpy())
    assert np.array_equal(tok_big.cpu().numpy(), ref_big)
    for r in range(3):
        g.replay()
        torch.cuda.synchronize()
        assert torch.equal(out, eager), f"replay {r}"
    del junk


@pytest.mark.parametrize("mode,B", [("w8a16", 4), ("w8a8", 4), ("fp8", 4), ("mxfp8", 4), ("mxfp4", 4),
                                    ("w8a16", 64), ("fp8", 128), ("mxfp4", 48)])
def test_lmhead_graph_replays_match_eager(mode, B):
    """Batch 4: one group, fused activation prologue, held logits; W8A16 64 / FP8 128: four
    XCD-grouped batch groups in one launch (FP8 after a separate activation cast, 32-row
    groups flushing held logits); MXFP4 48: two groups of 24."""
    M, K = 16384, 3072
    g0 = torch.Generator(device="cuda").manual_seed(3)
    w = (torch.randn(M, K, generator=g0, device="cuda") * 0.02).half()
    x = torch.randn(B, K, generator=g0, device="cuda").half()
    if mode == "w8a16":
        q, s = K_.quant_rows_int8(w, torch.float16)
        f = lambda: K_.lmhead_w8a16(x, q, s)  # noqa: E731
    elif mode == "w8a8":
        q, s = K_.quant_rows_int8(w, torch.float32)
        f = lambda: K_.lmhead_w8a8(x, q, s)  # noqa: E731
    elif mode == "fp8":
        q, s = K_.quant_rows_fp8(w)
        f = lambda: K_.lmhead_fp8(x, q, s)  # noqa: E731
    elif mode == "mxfp8":
        q, s = K_.quant_mxfp8(w)
        f = lambda: K_.lmhead_mxfp8(x, q, s)  # noqa: E731
    else:
        q, s = K_.quant_mxfp4(w)
        f = lambda: K_.lmhead_mxfp4(x, q, s, K)  # noqa: E731
    eager = f().clone()
    g, out = _capture(f, 2)
    for r in range(4):
        g.replay()
        torch.cuda.synchronize()
        assert torch.equal(out, eager), f"{mode} replay {r}"
        assert torch.equal(f(), eager)
