"""vqk_gumbel_argmax_noalloc: the sampler with its workspace in the library's own static
device array.  Called through the C ABI and compared with vqk_gumbel_argmax (caller
workspace) on two calls in a row, the second smaller, so stale contents of the shared
array from the first call must not leak into the second."""
import numpy as np
import pytest
import torch
from oracle import vqk_oracle as O
from vllm_quant_kernels import _lib
from vllm_quant_kernels import _synthetic as syn

pytestmark = pytest.mark.gpu


def _with_workspace(logits, temp, seeds, thr=None):
    B, V = logits.shape
    need = int(_lib.load().vqk_gumbel_workspace_size(B, V))
    ws = torch.empty(need, dtype=torch.uint8, device="cuda")
    out = torch.empty(B, dtype=torch.int64, device="cuda")
    _lib.call("vqk_gumbel_argmax", logits.data_ptr(), logits.stride(0), B, V, temp.data_ptr(), seeds.data_ptr(),
              1 if seeds.dtype == torch.int64 else 0, None if thr is None else thr.data_ptr(), out.data_ptr(),
              ws.data_ptr(), need, torch.cuda.current_stream().cuda_stream)
    return out


def _noalloc(logits, temp, seeds, thr=None):
    B, V = logits.shape
    out = torch.empty(B, dtype=torch.int64, device="cuda")
    _lib.call("vqk_gumbel_argmax_noalloc", logits.data_ptr(), logits.stride(0), B, V, temp.data_ptr(),
              seeds.data_ptr(), 1 if seeds.dtype == torch.int64 else 0, None if thr is None else thr.data_ptr(),
              out.data_ptr(), torch.cuda.current_stream().cuda_stream)
    return out


def test_noalloc_matches_workspace_form_twice():
    # a large call (three-launch form, B * V > 2M), then a small one (two-launch form)
    for B, V, topk in ((32, 248_320, False), (4, 50_000, True)):
        logits, temp, seeds = syn.sampler_inputs(B, V)
        thr = torch.topk(logits, 50, dim=-1).values[:, -1].contiguous() if topk else None
        ref = _with_workspace(logits, temp, seeds, thr)
        got = _noalloc(logits, temp, seeds, thr)
        torch.cuda.synchronize()
        assert torch.equal(got, ref), (B, V)
        o = O.gumbel_argmax(logits.cpu().numpy(), temp.cpu().numpy(), seeds.cpu().numpy(),
                            None if thr is None else thr.cpu().numpy())
        assert np.array_equal(got.cpu().numpy(), o), (B, V)


def test_noalloc_rejects_batches_beyond_its_array():
    lib = _lib.load()
    cap = int(lib.vqk_gumbel_noalloc_max_bytes())
    V = 248_320
    B = 1
    while lib.vqk_gumbel_workspace_size(B + 1, V) <= cap:
        B += 1
    assert int(lib.vqk_gumbel_workspace_size(B, V)) <= cap < int(lib.vqk_gumbel_workspace_size(B + 1, V))
    logits, temp, seeds = syn.sampler_inputs(B + 1, V)
    with pytest.raises(ValueError):
        _noalloc(logits, temp, seeds)
    # the largest batch that fits still runs, and matches the workspace form
    got = _noalloc(logits[:B].contiguous(), temp[:B].contiguous(), seeds[:B].contiguous())
    ref = _with_workspace(logits[:B].contiguous(), temp[:B].contiguous(), seeds[:B].contiguous())
    assert torch.equal(got, ref)
