"""Writes tests/golden/golden.npz: small known-answer vectors for every hot-path function,
produced by the CPU oracle (oracle/vqk_oracle.c, itself pinned by tests/test_oracle.py).

The reference (himikk/vllm-quant-kernels) ships no golden vectors and cannot run here
(it needs vLLM and a Triton GPU backend), so these fixtures freeze this build's oracle:
tests/test_golden.py checks the oracle still reproduces them (CPU) and the HIP kernels
reproduce them (GPU).  Inputs are generated from fixed numpy seeds and stored too.

Usage: python tests/golden/make_golden.py
"""
import os
import sys

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.dirname(os.path.dirname(HERE)))
from oracle import vqk_oracle as O  # noqa: E402


def main():
    rng = np.random.default_rng(20261201)
    g = {}
    # Philox / uniform / Gumbel
    seeds = np.array([0, 1, 12345, 2**31 - 2, 2**63 + 77], np.uint64)
    offs = np.array([0, 1, 2, 4095, 4096, 248319, 2**31 - 1], np.uint32)
    g["rand_seeds"] = seeds
    g["rand_offsets"] = offs
    g["rand_u"] = np.stack([O.rand(int(s), offs) for s in seeds])
    g["rand_g"] = O.gumbel(g["rand_u"])
    # weights: fp16 [48, 256] with a 6x row-absmax spread, adversarial rows
    w = (rng.standard_normal((48, 256)) * 0.02 * np.exp(rng.uniform(0, np.log(6), (48, 1)))).clip(-0.19, 0.19)
    w = w.astype(np.float16)
    w[0] = 0
    w[1, :32] = np.float16(2.0) ** np.arange(-16, 16)
    w[2, :32] = np.tile(np.array([0.25, 0.75, 1.25, 1.75, 2.5, 3.5, 5.0, 6.0], np.float16), 4) * np.float16(0.01)
    g["w"] = w
    wf = w.astype(np.float32)
    g["int8_q"], g["int8_s32"] = O.quant_rows_int8(wf)
    g["int8_s16"] = g["int8_s32"].astype(np.float16)
    g["fp8_q"], s = O.quant_rows_fp8(wf)
    g["fp8_s16"] = s.astype(np.float16)
    g["mxfp8_q"], g["mxfp8_s"] = O.quant_mxfp8(wf)
    g["mxfp4_q"], g["mxfp4_s"] = O.quant_mxfp4(wf)
    # activations fp16 [3, 256]
    x = rng.standard_normal((3, 256)).astype(np.float16)
    g["x"] = x
    xf = x.astype(np.float32)
    g["out_w8a16"] = O.to_f16_bits(O.lmhead_w8a16(g["int8_q"], g["int8_s16"].astype(np.float32), xf))
    xq, xs = O.act_quant_int8(xf)
    acc, o8 = O.lmhead_w8a8(g["int8_q"], g["int8_s32"], xq, xs)
    g["w8a8_acc"], g["out_w8a8"] = acc, O.to_f16_bits(o8)
    g["out_fp8"] = O.to_f16_bits(O.lmhead_fp8(g["fp8_q"], g["fp8_s16"].astype(np.float32), O.e4m3_encode(xf)))
    xq8, xs8 = O.quant_mxfp8(xf)
    g["out_mxfp8"] = O.to_f16_bits(O.lmhead_mx(g["mxfp8_q"], g["mxfp8_s"], xq8, xs8, False, 256))
    g["out_mxfp4"] = O.to_f16_bits(O.lmhead_mx(g["mxfp4_q"], g["mxfp4_s"], xq8, xs8, True, 256))
    # sampler: logits [6, 5000], mixed greedy / temperatures, 64-bit seeds, top-k thresholds
    lg = (rng.standard_normal((6, 5000)) * 3).astype(np.float32)
    lg[:, rng.integers(0, 5000, 6)] += 15
    t = np.array([0.0, 0.3, 0.7, 1.0, 1.5, 0.9], np.float32)
    sd = rng.integers(0, 2**63, 6, dtype=np.int64)
    thr = np.sort(lg, axis=1)[:, -7].copy()
    g["smp_logits"], g["smp_temp"], g["smp_seeds"], g["smp_thr"] = lg, t, sd, thr
    g["smp_tokens"] = O.gumbel_argmax(lg, t, sd)
    g["smp_tokens_topk"] = O.gumbel_argmax(lg, t, sd, thr)
    g["smp_scores_row3"] = O.gumbel_scores(lg, t, sd)[3]
    np.savez_compressed(os.path.join(HERE, "golden.npz"), **g)
    print("wrote", os.path.join(HERE, "golden.npz"), sorted(g))


if __name__ == "__main__":
    main()
