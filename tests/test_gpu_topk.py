"""Device top-k threshold (vqk_topk_threshold) against the reference's torch chain
(_compute_topk_threshold: max_k with .item(), torch.topk sorted, gather; NaN ranked
largest), and the sampler fed with it against the oracle."""
import numpy as np
import pytest
import torch

from oracle import vqk_oracle as O
from vllm_quant_kernels import _sampler_kernels as S_
from vllm_quant_kernels import _synthetic as syn
from oracle.torch_chains import compute_topk_threshold as _compute_topk_threshold

pytestmark = pytest.mark.gpu


def _ref_thr(logits, top_k):
    """The reference chain on the host; None (all rows disabled) becomes -inf."""
    B, V = logits.shape
    t = _compute_topk_threshold(logits.cpu(), top_k.cpu(), V)
    return torch.full((B,), float("-inf")) if t is None else t


def _same(a, b):
    a, b = a.cpu().numpy(), b.cpu().numpy()
    both_nan = np.isnan(a) & np.isnan(b)
    return bool(np.all(both_nan | (a == b)))   # -0.0 == +0.0 as the mask compares


@pytest.mark.parametrize("B,V", [(8, 152_064), (5, 248_320), (3, 1000), (4, 4099)])
def test_topk_threshold_matches_torch(B, V):
    g = torch.Generator(device="cuda").manual_seed(B * 1000 + V % 997)
    logits = torch.randn(B, V, generator=g, device="cuda") * 3.0
    for ks in ([1, 5, 50, 100, 200, 7, 13, 64][:B], [max(V // 3, 1)] * B, [V - 1] * B):
        top_k = torch.tensor((ks * B)[:B], dtype=torch.int32, device="cuda")
        assert _same(S_.topk_threshold(logits, top_k), _ref_thr(logits, top_k)), ks


def test_topk_threshold_ties_nan_zeros_and_disabled():
    B, V = 6, 20_000
    g = torch.Generator(device="cuda").manual_seed(3)
    logits = torch.randint(-20, 20, (B, V), generator=g, device="cuda").float()  # heavy ties
    logits[1, ::7] = float("nan")                  # more NaNs than k: threshold NaN
    logits[2, 100] = float("nan")                  # one NaN, ranked first
    logits[3] = 0.0
    logits[3, ::2] = -0.0                          # signed zeros tie
    logits[4, 5000:] = float("-inf")
    top_k = torch.tensor([3, 10, 4, 17, 19_000, 0], dtype=torch.int32, device="cuda")  # k=0 -> 1
    assert _same(S_.topk_threshold(logits, top_k), _ref_thr(logits, top_k))
    t64 = top_k.to(torch.int64)
    assert _same(S_.topk_threshold(logits, t64), _ref_thr(logits, t64))
    top_k[5] = V                                   # one row disabled -> the reference passes None
    thr = S_.topk_threshold(logits, top_k)
    assert bool(torch.all(thr == float("-inf")))


@pytest.mark.parametrize("B", [4, 32])
def test_sampler_with_device_topk_threshold(B):
    logits, temp, seeds = syn.sampler_inputs(B)
    g = torch.Generator(device="cuda").manual_seed(B)
    top_k = torch.randint(1, 120, (B,), generator=g, device="cuda", dtype=torch.int32)
    thr = S_.topk_threshold(logits, top_k)
    assert _same(thr, _ref_thr(logits, top_k))
    out = S_.fused_gumbel_sample(logits, temp, seeds, topk_threshold=thr)
    ref = O.gumbel_argmax(logits.cpu().numpy(), temp.cpu().numpy(), seeds.cpu().numpy(), thr.cpu().numpy())
    assert np.array_equal(out.cpu().numpy(), ref)
    # every sampled token is inside its row's top-k
    vals, _ = torch.topk(logits, int(top_k.max()), dim=-1)
    kth = vals.gather(1, (top_k.long() - 1).unsqueeze(1)).squeeze(1)
    assert bool(torch.all(logits.gather(1, out.unsqueeze(1)).squeeze(1) >= kth))
