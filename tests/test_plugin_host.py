"""Host-side behaviour of the plugin boundary (CPU only, test-only vLLM stand-in).

Mirrors the reference's host tests and contracts:
  env var names / truthy set / priority     src/vllm_quant_kernels/_registration.py:7-81
  OOT registration + gates + fallbacks      src/vllm_quant_kernels/_quant.py:108-243
  Sampler patch + fast-path predicate       src/vllm_quant_kernels/_sampler.py:28-214
  tests/test_int8_logits.py:81-136, tests/test_fused_sampler_predicate.py:65-172
and checks that libvqk_hip.so exports every symbol include/vqk.h declares.
"""
import ctypes
import os
import re
import subprocess
import sys
from types import SimpleNamespace

import pytest
import torch

REPO = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HEADER = os.path.join(REPO, "include", "vqk.h")
ENVS = ["VLLM_USE_INT8_LMHEAD", "VLLM_USE_W8A8_LMHEAD", "VLLM_USE_FP8_LMHEAD",
        "VLLM_USE_MXFP8_LMHEAD", "VLLM_USE_MXFP4_LMHEAD", "VLLM_USE_FUSED_SAMPLER"]


@pytest.fixture
def clean_env(monkeypatch):
    for e in ENVS:
        monkeypatch.delenv(e, raising=False)
    return monkeypatch


# ---------------------------------------------------------------------------------------
# registration and env vars

def test_entry_point_declared():
    txt = open(os.path.join(REPO, "vllm-quant-kernels_amd", "pyproject.toml")).read()
    assert '[project.entry-points."vllm.general_plugins"]' in txt
    assert 'quant_kernels = "vllm_quant_kernels:register"' in txt


@pytest.mark.parametrize("val,exp", [("1", True), ("true", True), ("TRUE", True), ("yes", True), ("On", True),
                                     ("0", False), ("false", False), ("", False), ("2", False), ("y", False)])
def test_truthy_set(clean_env, val, exp):
    from vllm_quant_kernels import _registration as R
    clean_env.setenv("VLLM_USE_INT8_LMHEAD", val)
    assert R._env_bool("VLLM_USE_INT8_LMHEAD") is exp


def test_priority_order(clean_env):
    from vllm_quant_kernels import _registration as R
    assert R.selected_lmhead_mode() is None
    order = [("VLLM_USE_INT8_LMHEAD", "int8"), ("VLLM_USE_W8A8_LMHEAD", "w8a8"), ("VLLM_USE_FP8_LMHEAD", "fp8"),
             ("VLLM_USE_MXFP8_LMHEAD", "mxfp8"), ("VLLM_USE_MXFP4_LMHEAD", "mxfp4")]
    for var, mode in order:   # each higher-priority var overrides everything set before it
        clean_env.setenv(var, "1")
        assert R.selected_lmhead_mode() == mode


def test_register_disabled_message(clean_env, capsys):
    import vllm_quant_kernels
    vllm_quant_kernels.register()
    err = capsys.readouterr().err
    assert "Plugin loaded but disabled" in err


def test_register_oot_and_idempotent(clean_env, capsys):
    from vllm.model_executor.custom_op import PluggableLayer
    from vllm_quant_kernels import _registration as R
    clean_env.setenv("VLLM_USE_FP8_LMHEAD", "1")
    R.register_all()
    R.register_all()
    from vllm_quant_kernels._quant import QuantizedLogitsProcessor
    assert PluggableLayer.oot_registry["LogitsProcessor"] is QuantizedLogitsProcessor
    err = capsys.readouterr().err
    assert "Registered QuantizedLogitsProcessor" in err and "dtype=fp8" in err
    import vllm.envs as envs
    for v in ENVS:
        assert v in envs.environment_variables
    clean_env.setenv("VLLM_USE_MXFP4_LMHEAD", "yes")
    assert envs.environment_variables["VLLM_USE_MXFP4_LMHEAD"]() == "yes"  # each lambda reads its own var


def test_class_is_logits_processor():
    from vllm.model_executor.layers.logits_processor import LogitsProcessor
    from vllm_quant_kernels._quant import QuantizedLogitsProcessor
    assert issubclass(QuantizedLogitsProcessor, LogitsProcessor)
    assert QuantizedLogitsProcessor(32000)._VOCAB_THRESHOLD == 100_000


# ---------------------------------------------------------------------------------------
# gates and fallbacks of _init_int8 (no gfx950 here: the quantized path must not engage)

def _lm_head(w):
    return SimpleNamespace(weight=SimpleNamespace(data=w, dtype=w.dtype, shape=w.shape, device=w.device))


def test_gate_non_fp_weight(clean_env):
    from vllm_quant_kernels._quant import QuantizedLogitsProcessor
    clean_env.setenv("VLLM_USE_INT8_LMHEAD", "1")
    h = _lm_head(torch.tensor([[1, 2], [3, 4]], dtype=torch.int8))
    QuantizedLogitsProcessor(32000)._init_int8(h)
    assert not hasattr(h, "_int8_w")


def test_gate_small_vocab(clean_env):
    from vllm_quant_kernels._quant import QuantizedLogitsProcessor
    clean_env.setenv("VLLM_USE_INT8_LMHEAD", "1")
    h = _lm_head(torch.zeros(1000, 64, dtype=torch.float16))
    QuantizedLogitsProcessor(1000)._init_int8(h)
    assert not hasattr(h, "_int8_w")


def test_unsupported_device_falls_back_to_upstream(clean_env, capsys):
    """On a device that is not a gfx950 every requested mode degrades like the reference's
    non-Thor path; with no gfx950 INT8 kernel either, the lm_head stays on the upstream path."""
    from vllm_quant_kernels._quant import QuantizedLogitsProcessor
    clean_env.setenv("VLLM_USE_MXFP4_LMHEAD", "1")
    clean_env.setenv("VLLM_USE_W8A8_LMHEAD", "1")
    M, K = 100_352, 64
    w = (torch.randn(M, K) * 0.02).to(torch.float16)
    proc = QuantizedLogitsProcessor(M)
    h = SimpleNamespace(weight=torch.nn.Parameter(w, requires_grad=False))
    x = torch.randn(2, K, dtype=torch.float16)
    out = proc._get_logits(x, h, None)
    err = capsys.readouterr().err
    assert "requires gfx950 (MI355X), falling back to int8" in err
    assert "lm_head left unquantized" in err
    for a in ("_int8_w", "_w8a8_w", "_fp8_w", "_mxfp8_w", "_mxfp4_w"):
        assert not hasattr(h, a)
    assert torch.equal(out, torch.nn.functional.linear(x, w))
    assert proc._int8_initialized


def test_mx_gate_messages(clean_env, capsys, monkeypatch):
    """K % 32 gates run before quantization (reference _quant.py:188-216)."""
    from vllm_quant_kernels import _quant as Q
    monkeypatch.setattr(Q, "_device_supported", lambda dev: True)
    called = []
    monkeypatch.setattr(Q.QuantizedLogitsProcessor, "_init_int8_weights",
                        lambda self, h, w, s, t: called.append("int8"))
    clean_env.setenv("VLLM_USE_MXFP4_LMHEAD", "1")
    clean_env.setenv("VLLM_USE_MXFP8_LMHEAD", "1")
    h = _lm_head(torch.zeros(100_001, 48, dtype=torch.bfloat16))
    Q.QuantizedLogitsProcessor(100_001)._init_int8(h)
    err = capsys.readouterr().err
    assert "VLLM_USE_MXFP4_LMHEAD requires K divisible by 32 (got K=48)" in err
    assert "VLLM_USE_MXFP8_LMHEAD requires K divisible by 32 (got K=48)" in err
    assert "lm_head left unquantized" in err and called == []  # K=48: no int8 kernel shape either


def test_dispatch_order(monkeypatch):
    from vllm_quant_kernels._quant import QuantizedLogitsProcessor
    proc = QuantizedLogitsProcessor(10)
    seen = []
    for name in ("_mxfp4_forward", "_mxfp8_forward", "_fp8_forward", "_w8a8_forward", "_int8_forward"):
        monkeypatch.setattr(QuantizedLogitsProcessor, name, lambda self, hs, h, b, n=name: seen.append(n))
    h = SimpleNamespace(_int8_w=1, _w8a8_w=1, _fp8_w=1, _mxfp8_w=1, _mxfp4_w=1)
    for attr in ("_mxfp4_w", "_mxfp8_w", "_fp8_w", "_w8a8_w", "_int8_w"):
        proc._quantized_forward(None, h, None)
        delattr(h, attr)
    assert seen == ["_mxfp4_forward", "_mxfp8_forward", "_fp8_forward", "_w8a8_forward", "_int8_forward"]


def test_wrappers_reject_cpu_tensors():
    from vllm_quant_kernels import _kernels as K_
    w = torch.zeros(256, 128, dtype=torch.float16)
    with pytest.raises(ValueError, match="no CPU path"):
        K_.quant_rows_int8(w)
    from vllm_quant_kernels._sampler_kernels import fused_gumbel_sample
    with pytest.raises(AssertionError):
        fused_gumbel_sample(torch.zeros(2, 8, dtype=torch.float16), None, torch.zeros(2, dtype=torch.int32))
    with pytest.raises(AssertionError):
        fused_gumbel_sample(torch.zeros(2, 8), None, torch.zeros(3, dtype=torch.int32))
    with pytest.raises(ValueError):
        fused_gumbel_sample(torch.zeros(2, 8), None, torch.zeros(2, dtype=torch.int32))


def test_reference_kernel_level_names():
    from vllm_quant_kernels import _kernels as K_
    from vllm_quant_kernels._quant import MXFP4_GROUP_SIZE, _quantize_to_mxfp4, _quantize_to_mxfp8  # noqa: F401
    assert MXFP4_GROUP_SIZE == 32 and K_.MXFP8_GROUP_SIZE == 32
    assert [K_._n_bucket(n) for n in (1, 3, 4, 7, 8, 31, 32, 64)] == [0, 0, 1, 1, 2, 2, 3, 3]
    for f in (K_._make_thor_gemm_kernel, K_._make_thor_fp8_gemm_kernel, K_._make_thor_w8a8_gemm_kernel,
              K_._make_thor_mxfp8_gemm_kernel, K_._make_thor_mxfp4_gemm_kernel):
        kern, nb = f()
        assert nb is K_._n_bucket and callable(kern[lambda meta: (1,)])
    assert callable(K_.int8_gmv[(1,)])


# ---------------------------------------------------------------------------------------
# fused sampler hook

def _sm(B, V, *, all_greedy=False, top_p=None, top_k=None, generators=None, max_num_logprobs=None,
        allowed=None, bad_words=None, procs=None, temp=1.0):
    from vllm.v1.sample.logits_processor.state import LogitsProcessors
    from vllm.v1.sample.metadata import SamplingMetadata
    t = torch.zeros(B) if all_greedy else torch.full((B,), temp)
    return SamplingMetadata(
        temperature=t, all_greedy=all_greedy, all_random=not all_greedy, top_p=top_p, top_k=top_k,
        generators=generators or {}, max_num_logprobs=max_num_logprobs, no_penalties=True,
        prompt_token_ids=None, frequency_penalties=torch.zeros(B), presence_penalties=torch.zeros(B),
        repetition_penalties=torch.ones(B), output_token_ids=[[] for _ in range(B)],
        allowed_token_ids_mask=allowed, bad_words_token_ids=bad_words or {},
        logitsprocs=procs or LogitsProcessors(), logprob_token_ids=None, spec_token_ids=None,
        thinking_budget_state_holder=None)


@pytest.fixture
def fused_cls():
    import vllm.v1.sample.sampler as up
    from vllm_quant_kernels._sampler import install_fused_sampler
    orig = up.Sampler
    install_fused_sampler()
    yield up.Sampler
    up.Sampler = orig


def test_install_patches_subclass(fused_cls):
    import vllm.v1.sample.sampler as up
    assert up.Sampler is fused_cls and fused_cls.__name__ == "FusedSampler"
    s = fused_cls()
    for m in ("compute_logprobs", "gather_logprobs", "apply_temperature"):
        assert hasattr(s, m)


def test_registration_installs_sampler(clean_env):
    import vllm.v1.sample.sampler as up
    from vllm_quant_kernels import _registration as R
    orig = up.Sampler
    try:
        clean_env.setenv("VLLM_USE_FUSED_SAMPLER", "on")
        R.register_all()
        assert up.Sampler.__name__ == "FusedSampler"
    finally:
        up.Sampler = orig


def test_fast_path_predicate():
    from vllm.v1.sample.logits_processor.state import LogitsProcessors
    from vllm_quant_kernels._sampler import _fast_path_ok
    B, V = 2, 16
    assert _fast_path_ok(_sm(B, V))
    assert not _fast_path_ok(_sm(B, V, top_p=torch.full((B,), 0.9)))
    assert not _fast_path_ok(_sm(B, V, allowed=torch.zeros(B, V, dtype=torch.bool)))
    assert not _fast_path_ok(_sm(B, V, bad_words={0: [[1]]}))
    assert not _fast_path_ok(_sm(B, V, procs=LogitsProcessors(argmax_invariant=[object()])))
    assert not _fast_path_ok(_sm(B, V, procs=LogitsProcessors(non_argmax_invariant=[object()])))
    assert not _fast_path_ok(_sm(B, V, generators={0: torch.Generator()}))
    holder = SimpleNamespace(has_tracked_requests=lambda: True)
    sm = _sm(B, V)
    sm.thinking_budget_state_holder = holder
    assert not _fast_path_ok(sm)


def test_greedy_and_fallbacks_on_host(fused_cls):
    """Paths that never reach the kernel: all-greedy argmax and every upstream fallback."""
    B, V = 4, 4096
    torch.manual_seed(303)
    logits = torch.randn(B, V)
    s = fused_cls()
    out, _ = s.sample(logits.clone(), _sm(B, V, all_greedy=True))
    assert torch.equal(out, logits.argmax(dim=-1))
    out, _ = s.sample(logits.clone(), _sm(B, V, top_p=torch.full((B,), 0.9)))
    assert out.shape == (B,) and bool(((out >= 0) & (out < V)).all())
    out, _ = s.sample(logits.clone(), _sm(B, V, generators={0: torch.Generator().manual_seed(42)}))
    assert out.shape == (B,)
    sp = fused_cls(logprobs_mode="processed_logprobs")
    out, processed = sp.sample(logits.clone(), _sm(B, V, max_num_logprobs=5))
    assert out.shape == (B,) and processed is not None


def test_topk_threshold_host():
    from oracle.torch_chains import compute_topk_threshold as _compute_topk_threshold
    torch.manual_seed(0)
    logits = torch.randn(3, 50)
    k = torch.tensor([1, 5, 50], dtype=torch.int32)
    assert _compute_topk_threshold(logits, torch.full((3,), 50, dtype=torch.int32), 50) is None
    thr = _compute_topk_threshold(logits, torch.tensor([1, 5, 7], dtype=torch.int32), 50)
    srt = logits.sort(dim=-1, descending=True).values
    assert torch.equal(thr, torch.stack([srt[0, 0], srt[1, 4], srt[2, 6]]))
    # max_k >= V means every row is effectively unrestricted (reference _sampler.py:81-83)
    assert _compute_topk_threshold(logits, torch.tensor([1, 5, 50], dtype=torch.int32), 50) is None
    del k


# ---------------------------------------------------------------------------------------
# C ABI

def test_library_exports_header_symbols():
    from vllm_quant_kernels import _lib
    decls = set(re.findall(r"\b(vqk_[a-z0-9_]+)\s*\(", open(HEADER).read()))
    assert len(decls) >= 20
    lib = _lib.load()
    missing = [d for d in decls if not hasattr(lib, d)]
    assert not missing, missing
    assert set(_lib.SIGNATURES) == decls, set(_lib.SIGNATURES) ^ decls
    assert lib.vqk_abi_version() == 2
    assert _lib.strerror(-1) == "invalid argument" and _lib.strerror(-3) == "no gfx950 HIP device"
    nm = subprocess.run(["nm", "-D", "--defined-only", _lib.LIB_PATH], capture_output=True, text=True).stdout
    exported = set(re.findall(r" T (vqk_[a-z0-9_]+)$", nm, re.M))
    assert decls <= exported


def _bundle_targets(path):
    """Target triples of every clang offload bundle embedded in a file built here: each
    bundle is the magic string, an entry count and (offset, size, triple length, triple)
    records (all little-endian u64)."""
    import struct
    data = open(path, "rb").read()
    magic = b"__CLANG_OFFLOAD_BUNDLE__"
    targets, i = [], data.find(magic)
    while i >= 0:
        n = struct.unpack_from("<Q", data, i + len(magic))[0]
        p = i + len(magic) + 8
        for _ in range(n):
            _off, _size, tl = struct.unpack_from("<QQQ", data, p)
            targets.append(data[p + 24:p + 24 + tl].decode())
            p += 24 + tl
        i = data.find(magic, p)
    return targets


def test_library_has_gfx950_code_only():
    from vllm_quant_kernels import _lib
    targets = [t for t in _bundle_targets(_lib.LIB_PATH) if "amdgcn" in t]
    assert targets and all(t.endswith("gfx950") for t in targets), targets


# ---------------------------------------------------------------------------------------
# on-disk quantized lm_head (safetensors)

def _fake_head(M, K, seed=0):
    from types import SimpleNamespace
    g = torch.Generator().manual_seed(seed)
    w = torch.randn(M, K, generator=g).half()
    return SimpleNamespace(weight=SimpleNamespace(data=w, dtype=w.dtype, shape=w.shape, device=w.device)), g


@pytest.mark.parametrize("mode", ["int8", "w8a8", "fp8", "mxfp8", "mxfp4"])
def test_quantized_checkpoint_round_trip(tmp_path, mode):
    from vllm_quant_kernels import _checkpoint as C
    M, K = 300, 128
    head, g = _fake_head(M, K)
    kb = K // 2 if mode == "mxfp4" else K
    wname, sname = C.MODE_TENSORS[mode]
    wt = C._DTYPES[wname]
    q = torch.randint(-128 if wt == torch.int8 else 0, 128 if wt == torch.int8 else 256, (M, kb),
                      generator=g, dtype=torch.int32).to(wt)
    st = C._DTYPES[sname]
    s = (torch.randint(100, 150, (M, K // 32), generator=g, dtype=torch.int32).to(st) if mode.startswith("mx")
         else torch.rand(M, generator=g).to(st))
    setattr(head, wname, q)
    setattr(head, sname, s)
    path = str(tmp_path / "lm.safetensors")
    assert C.save_quantized(head, path) == mode
    fresh, _ = _fake_head(M, K)                       # same weight (same seed)
    assert C.load_quantized(fresh, path) == mode
    assert torch.equal(getattr(fresh, wname), q) and torch.equal(getattr(fresh, sname), s)
    if mode == "mxfp4":
        assert fresh._mxfp4_K == K
    other, _ = _fake_head(M, K, seed=1)               # another weight: refused
    assert C.load_quantized(other, path) is None and not hasattr(other, wname)
    wrong = "int8" if mode != "int8" else "fp8"
    assert C.load_quantized(fresh, path, mode=wrong) is None
    assert C.load_quantized(fresh, str(tmp_path / "missing.safetensors")) is None


def test_quantized_checkpoint_fingerprint_covers_every_row(tmp_path):
    """A weight that differs from the cached one in a single element of any row (here rows
    a sampling fingerprint would skip: 1 and M // 2 + 1) must not load the stale file."""
    from vllm_quant_kernels import _checkpoint as C
    M, K = 1000, 64
    head, _ = _fake_head(M, K)
    head._int8_w = torch.zeros(M, K, dtype=torch.int8)
    head._int8_scales = torch.ones(M, dtype=torch.float16)
    path = str(tmp_path / "lm.safetensors")
    C.save_quantized(head, path)
    for row in (1, M // 2 + 1, M - 2):
        other, _ = _fake_head(M, K)
        other.weight.data[row, 7] += 1.0
        assert C.fingerprint(other.weight.data) != C.fingerprint(head.weight.data)
        assert C.load_quantized(other, path) is None, row
    same, _ = _fake_head(M, K)
    assert C.load_quantized(same, path) == "int8"


def test_quantized_checkpoint_rejects_foreign_files(tmp_path):
    from safetensors.torch import save_file
    from vllm_quant_kernels import _checkpoint as C
    head, _ = _fake_head(64, 32)
    p = str(tmp_path / "x.safetensors")
    save_file({"int8_w": torch.zeros(64, 32, dtype=torch.int8)}, p, metadata={"format": "other"})
    assert C.load_quantized(head, p) is None
    meta = {"format": C.FORMAT, "version": C.VERSION, "mode": "int8", "M": "64", "K": "32",
            "source_dtype": "float16", "fingerprint": C.fingerprint(head.weight.data)}
    save_file({"int8_w": torch.zeros(64, 32, dtype=torch.uint8),              # wrong dtype
               "int8_scales": torch.zeros(64, dtype=torch.float16)}, p, metadata=meta)
    assert C.load_quantized(head, p) is None
    save_file({"int8_w": torch.zeros(64, 16, dtype=torch.int8),               # wrong shape
               "int8_scales": torch.zeros(64, dtype=torch.float16)}, p, metadata=meta)
    assert C.load_quantized(head, p) is None


def test_init_cached_writes_then_loads(tmp_path, monkeypatch, capsys):
    from vllm_quant_kernels._quant import QuantizedLogitsProcessor
    M, K = 200, 64
    head, _ = _fake_head(M, K)
    monkeypatch.setenv("VQK_LMHEAD_CACHE_DIR", str(tmp_path))
    calls = []

    def quantize():
        calls.append(1)
        head._w8a8_w = torch.ones(M, K, dtype=torch.int8)
        head._w8a8_scales = torch.full((M,), 0.5)

    proc = QuantizedLogitsProcessor.__new__(QuantizedLogitsProcessor)
    proc._init_cached("w8a8", head, head.weight.data, sys, quantize)
    assert calls == [1] and (tmp_path / f"lm_head_w8a8_{M}x{K}.safetensors").exists()
    head2, _ = _fake_head(M, K)
    proc._init_cached("w8a8", head2, head2.weight.data, sys, quantize)
    assert calls == [1]                                # loaded, not re-quantized
    assert torch.equal(head2._w8a8_w, head._w8a8_w) and hasattr(head2, "_w8a8_gemm_kernel")
    assert "loaded from" in capsys.readouterr().err
