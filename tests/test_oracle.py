"""Pins the CPU oracle (oracle/vqk_oracle.c) before it is trusted as the checker.

Each function is checked against something independent of its own formula:
  Philox4x32-10   Random123 known-answer vectors + torch's own header-only engine
                  (ATen/core/PhiloxRNGEngine.h) compiled with g++;
  uniform         the exact rational value of Triton's conversion, and its range ends;
  log / Gumbel    the libm double log (<= 1.5 ulp) and the exhaustive bound used by the
                  sampler's pruning;
  e4m3 encode     torch's float8_e4m3fn cast, exhaustively over all fp16 inputs and over
                  fp32 boundary sweeps;
  E2M1 encode     torch.bucketize with the reference's midpoints (ties, -0, clamp);
  MX exponent     torch's fp32 ceil(log2()) on every positive fp16 (exact agreement is
                  proved for fp16 inputs) plus the closed form on powers of two;
  quantizers      the reference's torch op chains run by torch on the CPU, and invariants;
  lm_head refs    integer/float64 numpy matmuls and one-hot closed forms;
  sampler         greedy == argmax, tie rules, and the reference's statistical tests.
A planted mistake (wrong rounding, dropped term, swapped word) fails at least one of these.
"""
import os
import subprocess
import sysconfig

import numpy as np
import pytest
import torch

from oracle import vqk_oracle as O

TORCH_INC = os.path.join(os.path.dirname(torch.__file__), "include")


# ---------------------------------------------------------------------------------------
# Philox

KAT = [  # Random123 kat_vectors, philox4x32 10 rounds: ctr, key, expected
    ([0, 0, 0, 0], [0, 0], [0x6627E8D5, 0xE169C58D, 0xBC57AC4C, 0x9B00DBD8]),
    ([0xFFFFFFFF] * 4, [0xFFFFFFFF] * 2, [0x408F276D, 0x41C83B0E, 0xA20BC7C6, 0x6D5451FD]),
    ([0x243F6A88, 0x85A308D3, 0x13198A2E, 0x03707344], [0xA4093822, 0x299F31D0],
     [0xD16CFE09, 0x94FDCCEB, 0x5001E420, 0x24126EA1]),
]


@pytest.mark.parametrize("ctr,key,exp", KAT)
def test_philox_known_answers(ctr, key, exp):
    assert O.philox(ctr, key)[0].tolist() == exp


def test_philox_matches_torch_engine(tmp_path):
    src = tmp_path / "p.cpp"
    src.write_text(r'''
#include <ATen/core/PhiloxRNGEngine.h>
#include <cstdio>
#include <cstdlib>
int main(int argc, char** argv) {
  unsigned long long seeds[4] = {0ull, 1234567ull, 0xFFFFFFFFull, 0xDEADBEEF12345678ull};
  unsigned offs[5] = {0u, 1u, 77u, 248319u, 4000000000u};
  for (auto s : seeds) for (auto o : offs) {
    at::philox_engine e(s, 0, 0);
    e.set_offset(o);   // counter = (o, 0, 0, 0), key = (seed lo, seed hi)
    std::printf("%llu %u %u\n", s, o, e());
  }
  return 0;
}''')
    exe = tmp_path / "p"
    r = subprocess.run(["g++", "-std=c++17", "-O1", f"-I{TORCH_INC}", str(src), "-o", str(exe)],
                       capture_output=True, text=True)
    if r.returncode != 0:
        pytest.skip("torch Philox header did not compile here: " + r.stderr[-300:])
    lines = subprocess.run([str(exe)], capture_output=True, text=True, check=True).stdout.split("\n")
    n = 0
    for ln in lines:
        if not ln.strip():
            continue
        s, o, w = (int(v) for v in ln.split())
        got = O.philox([o, 0, 0, 0], [s & 0xFFFFFFFF, s >> 32])[0, 0]
        assert got == w, (s, o)
        n += 1
    assert n == 20


def test_uniform_conversion():
    lib = O.lib()
    c = np.float32(4.6566127342e-10)
    assert c.view(np.uint32) == 0x2FFFFFFF
    # exact value for sampled words: fold negatives with -x-1, RNE int->float, one multiply
    rng = np.random.default_rng(0)
    words = np.concatenate([rng.integers(0, 2**32, 20000, dtype=np.uint64),
                            np.array([0, 1, 2**31 - 1, 2**31, 2**32 - 1, 2**24, 2**24 + 1], np.uint64)])
    for w in words.tolist():
        x = w - 2**32 if w >= 2**31 else w
        x = -x - 1 if x < 0 else x
        ref = np.float32(np.float32(x) * c)
        assert lib.vqko_uniform(w) == ref
    assert lib.vqko_uniform(0) == 0.0
    assert lib.vqko_uniform(2**31 - 1) == np.float32(1 - 2.0**-24)   # never reaches 1
    assert lib.vqko_uniform(2**31) == np.float32(1 - 2.0**-24)       # -2^31 folds to 2^31-1


def test_rand_is_philox_word0():
    for seed in (0, 42, 2**31 - 2, -5, 2**40 + 3):
        s = seed & (2**64 - 1)
        offs = np.array([0, 1, 2, 1000, 248319], np.uint32)
        u = O.rand(s, offs)
        for o, uu in zip(offs.tolist(), u.tolist()):
            w = O.philox([o, 0, 0, 0], [s & 0xFFFFFFFF, s >> 32])[0, 0]
            assert uu == O.lib().vqko_uniform(int(w))


# ---------------------------------------------------------------------------------------
# log / Gumbel

def test_logf_accuracy():
    rng = np.random.default_rng(1)
    xs = np.concatenate([
        np.geomspace(1e-37, 3e38, 400_000).astype(np.float32),
        rng.uniform(0.5, 2.0, 400_000).astype(np.float32),
        (1.0 - np.arange(1, 5000) * 2.0 ** -24).astype(np.float32),
        (1.0 + np.arange(1, 5000) * 2.0 ** -23).astype(np.float32),
        np.array([2.0 ** k for k in range(-126, 128)], np.float32),
    ])
    y = O.logf(xs).astype(np.float64)
    ref = np.log(xs.astype(np.float64))
    ulp = np.spacing(np.abs(ref).astype(np.float32)).astype(np.float64)
    err = np.abs(y - ref) / np.maximum(ulp, np.spacing(np.float32(0)))
    assert err.max() <= 1.5, f"max {err.max()} ulp"
    assert O.logf(np.array([1.0], np.float32))[0] == 0.0


def test_gumbel_range_and_pruning_bound():
    gmax = O.gumbel_max_over_all_words()
    assert abs(gmax - 16.635532) < 1e-5          # -log(-log(1 - 2^-24))
    assert gmax <= 16.6356                        # GUMBEL_MAX in csrc/vqk_math.h
    g = O.gumbel(np.array([0.0, 2.0 ** -126, 0.5, 1 - 2.0 ** -24], np.float32))
    assert g[0] == g[1]                           # clamp of u = 0 to 2^-126
    assert abs(g[1] - (-np.log(-np.log(2.0 ** -126)))) < 1e-5
    assert abs(g[2] - (-np.log(np.log(2.0)))) < 1e-6


def test_gumbel_upper_bound_holds_for_every_word():
    """The GPU sampler skips the exact score of a logit when x*RN(1/T) + gumbel_upper(u)
    (+ margins) is below a real element's score; that is exact only if gumbel_upper(u)
    bounds the computed noise for every Philox word.  Walk every distinct uniform."""
    slack = O.gumbel_upper_min_slack()
    assert slack > 0.005, slack               # margin 0.01 minus rounding, never negative
    u = np.array([0.0, 0.5, 0.75, 1 - 2.0 ** -24, 1 - 2.0 ** -10], np.float32)
    ub = O.gumbel_upper(u)
    g = O.gumbel(u)
    assert np.all(ub >= g)
    # the bound is tight near u = 1 (where the skip decisions are close calls) and loose
    # by at most ln 2 + 0.01 + (-log(-log u) vs -log(1-u)) elsewhere
    assert ub[3] - g[3] < 0.02 and ub[4] - g[4] < 0.7


# ---------------------------------------------------------------------------------------
# number formats

def test_e4m3_exhaustive_fp16_vs_torch():
    h = np.arange(65536, dtype=np.uint32).astype(np.uint16).view(np.float16)
    ref = torch.from_numpy(h.copy()).to(torch.float8_e4m3fn).view(torch.uint8).numpy()
    got = O.e4m3_encode(h.astype(np.float32))
    nan = np.isnan(h)
    assert np.array_equal(got[~nan], ref[~nan])
    assert np.all((got[nan] & 0x7F) == 0x7F)


def test_e4m3_fp32_sweeps_vs_torch():
    rng = np.random.default_rng(2)
    x = np.concatenate([
        rng.standard_normal(300_000).astype(np.float32) * 100,
        rng.standard_normal(300_000).astype(np.float32) * 1e-3,
        np.linspace(440, 500, 20001, dtype=np.float32), -np.linspace(440, 500, 20001, dtype=np.float32),
        np.linspace(0, 2.0 ** -5, 20001, dtype=np.float32),
        np.array([464.0, 464.00003, 463.99997, 480.0, np.inf, -np.inf, 2.0 ** -10, 3 * 2.0 ** -11,
                  1.5 * 2.0 ** -9, 0.0, -0.0], np.float32),
    ])
    ref = torch.from_numpy(x).to(torch.float8_e4m3fn).view(torch.uint8).numpy()
    got = O.e4m3_encode(x)
    assert np.array_equal(got, ref)


def test_e4m3_decode_roundtrip():
    codes = np.array([c for c in range(256) if (c & 0x7F) != 0x7F], np.uint8)
    vals = O.e4m3_decode(codes)
    ref = torch.from_numpy(codes).view(torch.float8_e4m3fn).float().numpy()
    assert np.array_equal(vals, ref)
    assert np.array_equal(O.e4m3_encode(vals), codes)


def test_e2m1_vs_bucketize():
    mids = torch.tensor([0.25, 0.75, 1.25, 1.75, 2.5, 3.5, 5.0])
    rng = np.random.default_rng(3)
    y = np.concatenate([rng.uniform(-7, 7, 200_000).astype(np.float32),
                        np.array([0, -0.0, .25, .2501, .75, 1.25, 1.75, 2.5, 3.5, 5.0, 5.01, 6, 7, -1e-9,
                                  -.75, -5.0], np.float32)])
    t = torch.from_numpy(y)
    ref = (((t < 0).to(torch.uint8) << 3) | torch.bucketize(t.abs().clamp(max=6.0), mids).to(torch.uint8)).numpy()
    assert np.array_equal(O.e2m1_encode(y), ref)
    # values exactly on a midpoint round down (bucketize with right=False): 0.25 -> 0,
    # 0.75 -> 0.5, 5.0 -> 4, while just above a midpoint rounds up
    assert O.e2m1_encode(np.array([0, .25, .2501, .75, 1.25, 1.75, 2.5, 3.5, 5.0, 5.01, 6], np.float32)).tolist() \
        == [0, 0, 1, 1, 2, 3, 4, 5, 6, 7, 7]
    assert O.e2m1_encode(np.array([-0.0, -1e-6], np.float32)).tolist() == [0, 8]
    dec = O.e2m1_decode(np.arange(16, dtype=np.uint8))
    assert dec.tolist() == [0, .5, 1, 1.5, 2, 3, 4, 6, -0.0, -.5, -1, -1.5, -2, -3, -4, -6]


def test_mx_exponent_vs_torch_all_fp16():
    h = np.arange(1, 0x7C00, dtype=np.uint16).view(np.float16).astype(np.float32)  # every positive finite fp16
    for qmax in (448.0, 6.0):
        t = torch.from_numpy(h).clamp(min=1e-30)
        ref = torch.ceil(torch.log2(t / qmax)).clamp(-127, 127).to(torch.int32).numpy()
        assert np.array_equal(O.mx_exponent(h, qmax), ref)
    # powers of two: q = 2^e exactly -> k = e
    for e in range(-40, 40):
        assert O.mx_exponent(np.array([448.0 * 2.0 ** e], np.float32), 448.0)[0] == e
        assert O.mx_exponent(np.array([6.0 * 2.0 ** e * 1.0000001], np.float32), 6.0)[0] == e + 1
    assert O.mx_exponent(np.array([0.0], np.float32), 448.0)[0] == int(np.ceil(np.log2(1e-30 / 448)))


# ---------------------------------------------------------------------------------------
# quantizers vs the reference's torch chains (run by torch on the CPU)

def _ref_int8(w):  # src/vllm_quant_kernels/_quant.py:248-252
    s = (w.float().abs().amax(dim=1) / 127.0).clamp(min=1e-12)
    q = (w.float() / s.unsqueeze(1)).round().clamp(-127, 127).to(torch.int8)
    return q, s


def _ref_fp8(w):  # src/vllm_quant_kernels/_quant.py:306-310
    s = (w.float().abs().amax(dim=1) / 448.0).clamp(min=1e-12)
    q = (w.float() / s.unsqueeze(1)).clamp(-448, 448).to(torch.float8_e4m3fn)
    return q.view(torch.uint8), s


def _ref_mx(t, fp4):  # src/vllm_quant_kernels/_quant.py:46-61 / :77-105
    R, K = t.shape
    g = t.float().view(R, K // 32, 32)
    gmax = g.abs().amax(dim=-1).clamp(min=1e-30)
    k = torch.ceil(torch.log2(gmax / (6.0 if fp4 else 448.0))).clamp(-127, 127)
    sc = torch.pow(2.0, k).unsqueeze(-1)
    if not fp4:
        q = (g / sc).clamp(-448, 448).to(torch.float8_e4m3fn).view(R, K).view(torch.uint8)
    else:
        y = (g / sc).view(R, K)
        nib = ((y < 0).to(torch.uint8) << 3) | torch.bucketize(
            y.abs().clamp(max=6.0), torch.tensor([0.25, 0.75, 1.25, 1.75, 2.5, 3.5, 5.0])).to(torch.uint8)
        q = (nib[:, 1::2] << 4) | nib[:, 0::2]
    return q, (k + 127).to(torch.uint8)


def _w(M, K, dtype, seed=0):
    g = torch.Generator().manual_seed(seed)
    w = torch.randn(M, K, generator=g) * 0.02 * torch.exp(torch.rand(M, 1, generator=g) * 1.79)
    return w.clamp(-0.19, 0.19).to(dtype)


@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16])
def test_quantizers_match_reference_chains(dtype):
    w = _w(512, 768, dtype)
    w[3] = 0.0  # all-zero row
    wf = w.float().numpy()
    q, s = O.quant_rows_int8(wf)
    rq, rs = _ref_int8(w)
    assert np.array_equal(q, rq.numpy()) and np.array_equal(s, rs.numpy())
    assert np.abs(q).max() <= 127 and all(np.abs(q[i]).max() == 127 for i in range(512) if i != 3)
    q, s = O.quant_rows_fp8(wf)
    rq, rs = _ref_fp8(w)
    assert np.array_equal(q, rq.numpy()) and np.array_equal(s, rs.numpy())
    for fp4 in (False, True):
        q, s = (O.quant_mxfp4 if fp4 else O.quant_mxfp8)(wf)
        rq, rs = _ref_mx(w, fp4)
        assert np.array_equal(s, rs.numpy()) and np.array_equal(q, rq.numpy())


def test_act_quant_int8_matches_reference_chain():
    x = torch.randn(4, 3072, generator=torch.Generator().manual_seed(5)).to(torch.float16)
    xq, xs = O.act_quant_int8(x.float().numpy())
    s = (x.float().abs().amax() / 127.0).clamp(min=1e-12)     # _quant.py:536-539
    rq = (x.float() / s).round().clamp(-127, 127).to(torch.int8)
    assert xs == float(s) and np.array_equal(xq, rq.numpy())


# ---------------------------------------------------------------------------------------
# lm_head references

def test_lmhead_refs_vs_numpy():
    rng = np.random.default_rng(7)
    M, K, B = 300, 256, 3
    q = rng.integers(-127, 128, (M, K)).astype(np.int8)
    s = rng.uniform(1e-4, 2e-3, M).astype(np.float32)
    x = rng.standard_normal((B, K)).astype(np.float16).astype(np.float32)
    out = O.lmhead_w8a16(q, s, x)
    ref = (x.astype(np.float64) @ q.astype(np.float64).T).astype(np.float32) * s
    assert np.array_equal(out, ref)
    xq = rng.integers(-127, 128, (B, K)).astype(np.int8)
    acc, o8 = O.lmhead_w8a8(q, s, xq, 0.0123)
    iacc = xq.astype(np.int64) @ q.astype(np.int64).T
    assert np.array_equal(acc, iacc)
    assert np.array_equal(o8, (iacc.astype(np.float32) * s) * np.float32(0.0123))
    # one-hot activations pick out a dequantized column (closed form)
    wq = O.e4m3_encode(rng.standard_normal((M, K)).astype(np.float32) * 50)
    wq[wq & 0x7F == 0x7F] = 0
    xo = np.zeros((1, K), np.uint8)
    xo[0, 17] = O.e4m3_encode(np.array([2.0], np.float32))[0]
    o = O.lmhead_fp8(wq, s, xo)
    assert np.array_equal(o[0], (O.e4m3_decode(wq[:, 17]) * 2.0).astype(np.float32) * s)
    ws = rng.integers(110, 140, (M, K // 32)).astype(np.uint8)
    xs = np.full((1, K // 32), 127, np.uint8)
    om = O.lmhead_mx(wq, ws, xo, xs, False, K)
    assert np.allclose(om[0], O.e4m3_decode(wq[:, 17]) * 2.0 * 2.0 ** (ws[:, 0].astype(np.float64) - 127), rtol=0)
    p4 = rng.integers(0, 256, (M, K // 2)).astype(np.uint8)
    o4 = O.lmhead_mx(p4, ws, xo, xs, True, K)
    col = O.e2m1_decode((p4[:, 8] >> 4) & 15)  # k = 17 -> byte 8, high nibble
    assert np.allclose(o4[0], col * 2.0 * 2.0 ** (ws[:, 0].astype(np.float64) - 127), rtol=0)


# ---------------------------------------------------------------------------------------
# sampler semantics

def test_sampler_greedy_and_ties():
    rng = np.random.default_rng(9)
    x = rng.standard_normal((6, 5000)).astype(np.float32)
    x[0, 10] = x[0, 20] = 9.0             # tie: smallest index
    x[1, :] = -np.inf                     # all -inf -> 0
    x[2, 3] = -0.0
    out = O.gumbel_argmax(x, None, np.zeros(6, np.int32))
    assert out.tolist() == np.argmax(x, axis=1).tolist() and out[0] == 10 and out[1] == 0
    t = np.zeros(6, np.float32)
    assert O.gumbel_argmax(x, t, np.arange(6, dtype=np.int32)).tolist() == out.tolist()


def test_sampler_scores_formula():
    rng = np.random.default_rng(10)
    x = rng.standard_normal((2, 100)).astype(np.float32)
    t = np.array([0.7, 1.3], np.float32)
    seeds = np.array([5, -3], np.int64)
    sc = O.gumbel_scores(x, t, seeds)
    for b in range(2):
        s = int(seeds[b]) & (2**64 - 1)
        u = O.rand(s, np.arange(100, dtype=np.uint32))
        g = O.gumbel(u)
        assert np.array_equal(sc[b], (x[b] / t[b]).astype(np.float32) + g)
    thr = np.array([0.5, -10.0], np.float32)
    sc2 = O.gumbel_scores(x, t, seeds, thr)
    assert np.all(np.isneginf(sc2[0][x[0] < 0.5])) and np.array_equal(sc2[1], sc[1])


def test_sampler_distribution_chi_square():
    """Reference statistical test (tests/test_fused_sampler_kernel.py:74-104) on the oracle."""
    V, N = 32, 8000
    logits = torch.randn(V, generator=torch.Generator().manual_seed(7)).numpy().astype(np.float32)
    p = torch.softmax(torch.from_numpy(logits), 0).numpy()
    x = np.ascontiguousarray(np.broadcast_to(logits, (N, V)))
    seeds = np.random.default_rng(11).integers(0, 2**31 - 1, N).astype(np.int32)
    out = O.gumbel_argmax(x, np.ones(N, np.float32), seeds)
    counts = np.bincount(out, minlength=V)
    chi = np.sum((counts - p * N) ** 2 / (p * N))
    assert chi < 60.0, chi


@pytest.mark.parametrize("T", [0.1, 1.0, 5.0])
def test_sampler_temperature_scaling(T):
    """Reference statistical test (tests/test_fused_sampler_kernel.py:106-137) on the oracle."""
    V, N = 16, 4000
    logits = torch.randn(V, generator=torch.Generator().manual_seed(11)).numpy().astype(np.float32)
    x = np.ascontiguousarray(np.broadcast_to(logits, (N, V)))
    seeds = np.random.default_rng(int(T * 10)).integers(0, 2**31 - 1, N).astype(np.int32)
    out = O.gumbel_argmax(x, np.full(N, T, np.float32), seeds)
    emp = np.mean(out == np.argmax(logits))
    theo = float(torch.softmax(torch.from_numpy(logits) / T, 0).max())
    assert abs(emp - theo) < 3 * np.sqrt(theo * (1 - theo) / N) + 0.01


def test_numpy_sampler_baseline_matches_oracle():
    """The host timing baseline of the sampler (numpy) gives the C oracle's tokens on
    config-5 style rows: greedy rows, temperatures 0.3-1.5, spikes, a top-k threshold."""
    from oracle import cpu_baseline as CB
    rng = np.random.default_rng(3)
    B, V = 12, 20_000
    x = (rng.standard_normal((B, V)) * 3).astype(np.float32)
    for b in range(B):
        x[b, rng.choice(V, 5, replace=False)] += 10 + 10 * rng.random(5).astype(np.float32)
    t = (0.3 + 1.2 * rng.random(B)).astype(np.float32)
    t[[1, 6]] = 0.0
    seeds = rng.integers(-(2 ** 63), 2 ** 63 - 1, B, dtype=np.int64)
    assert np.array_equal(CB.gumbel_argmax_numpy(x, t, seeds), O.gumbel_argmax(x, t, seeds))
    thr = np.sort(x, axis=1)[:, -50].copy()
    assert np.array_equal(CB.gumbel_argmax_numpy(x, t, seeds, thr), O.gumbel_argmax(x, t, seeds, thr))
