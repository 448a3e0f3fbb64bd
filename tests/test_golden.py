"""Committed known-answer vectors (tests/golden/golden.npz, made by make_golden.py).

CPU: the oracle still reproduces every stored vector (guards the checker itself).
GPU: the HIP kernels reproduce them - quantized bytes, int32 accumulators, fp16 logits
(bit-exact for W8A8; within 1e-3 relative for the float-accumulating modes) and tokens.
"""
import os

import numpy as np
import pytest

from oracle import vqk_oracle as O

G = np.load(os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden", "golden.npz"))


def test_oracle_reproduces_golden():
    for i, s in enumerate(G["rand_seeds"]):
        assert np.array_equal(O.rand(int(s), G["rand_offsets"]), G["rand_u"][i])
    assert np.array_equal(O.gumbel(G["rand_u"]), G["rand_g"])
    wf = G["w"].astype(np.float32)
    q, s = O.quant_rows_int8(wf)
    assert np.array_equal(q, G["int8_q"]) and np.array_equal(s, G["int8_s32"])
    q, _ = O.quant_rows_fp8(wf)
    assert np.array_equal(q, G["fp8_q"])
    for fn, kq, ks in ((O.quant_mxfp8, "mxfp8_q", "mxfp8_s"), (O.quant_mxfp4, "mxfp4_q", "mxfp4_s")):
        q, s = fn(wf)
        assert np.array_equal(q, G[kq]) and np.array_equal(s, G[ks])
    xf = G["x"].astype(np.float32)
    assert np.array_equal(O.to_f16_bits(O.lmhead_w8a16(G["int8_q"], G["int8_s16"].astype(np.float32), xf)),
                          G["out_w8a16"])
    xq, xs = O.act_quant_int8(xf)
    acc, o = O.lmhead_w8a8(G["int8_q"], G["int8_s32"], xq, xs)
    assert np.array_equal(acc, G["w8a8_acc"]) and np.array_equal(O.to_f16_bits(o), G["out_w8a8"])
    assert np.array_equal(O.gumbel_argmax(G["smp_logits"], G["smp_temp"], G["smp_seeds"]), G["smp_tokens"])
    assert np.array_equal(O.gumbel_argmax(G["smp_logits"], G["smp_temp"], G["smp_seeds"], G["smp_thr"]),
                          G["smp_tokens_topk"])


def _rel(out_bits, ref_bits):
    o = out_bits.view(np.float16).astype(np.float64)
    r = ref_bits.view(np.float16).astype(np.float64)
    return np.linalg.norm(o - r) / np.linalg.norm(r)


@pytest.mark.gpu
def test_kernels_reproduce_golden():
    import torch
    from vllm_quant_kernels import _kernels as K_
    from vllm_quant_kernels import _sampler_kernels as S_
    d = "cuda"
    w = torch.from_numpy(G["w"]).to(d)
    x = torch.from_numpy(G["x"]).to(d)
    q, s = K_.quant_rows_int8(w, torch.float16)
    assert np.array_equal(q.cpu().numpy(), G["int8_q"])
    assert np.array_equal(s.cpu().numpy(), G["int8_s16"])
    o = K_.lmhead_w8a16(x, q, s).cpu().numpy().view(np.uint16)
    assert _rel(o, G["out_w8a16"]) <= 1e-3
    qa, sa = K_.quant_rows_int8(w, torch.float32)
    acc = torch.empty(3, 48, dtype=torch.int32, device=d)
    o = K_.lmhead_w8a8(x, qa, sa, acc=acc).cpu().numpy().view(np.uint16)
    assert np.array_equal(acc.cpu().numpy(), G["w8a8_acc"]) and np.array_equal(o, G["out_w8a8"])
    qf, sf = K_.quant_rows_fp8(w)
    assert np.array_equal(qf.cpu().numpy(), G["fp8_q"])
    assert _rel(K_.lmhead_fp8(x, qf, sf).cpu().numpy().view(np.uint16), G["out_fp8"]) <= 1e-3
    qm, sm = K_.quant_mxfp8(w)
    assert np.array_equal(qm.cpu().numpy(), G["mxfp8_q"]) and np.array_equal(sm.cpu().numpy(), G["mxfp8_s"])
    assert _rel(K_.lmhead_mxfp8(x, qm, sm).cpu().numpy().view(np.uint16), G["out_mxfp8"]) <= 1e-3
    q4, s4 = K_.quant_mxfp4(w)
    assert np.array_equal(q4.cpu().numpy(), G["mxfp4_q"]) and np.array_equal(s4.cpu().numpy(), G["mxfp4_s"])
    assert _rel(K_.lmhead_mxfp4(x, q4, s4, 256).cpu().numpy().view(np.uint16), G["out_mxfp4"]) <= 1e-3
    lg = torch.from_numpy(G["smp_logits"]).to(d)
    t = torch.from_numpy(G["smp_temp"]).to(d)
    sd = torch.from_numpy(G["smp_seeds"]).to(d)
    thr = torch.from_numpy(G["smp_thr"]).to(d)
    assert np.array_equal(S_.fused_gumbel_sample(lg, t, sd).cpu().numpy(), G["smp_tokens"])
    assert np.array_equal(S_.fused_gumbel_sample(lg, t, sd, thr).cpu().numpy(), G["smp_tokens_topk"])
    sc = S_.gumbel_scores(lg, t, sd).cpu().numpy()[3]
    assert np.array_equal(sc.view(np.uint32), G["smp_scores_row3"].view(np.uint32))
