"""Tensor-level wrappers over the gfx950 kernels in libvqk_hip.so.

Two layers live here:

* plain functions taking torch device tensors (``lmhead_w8a16``, ``quant_mxfp4``, ...),
  used by ``QuantizedLogitsProcessor`` and the sampler;
* the reference's kernel-level names (``int8_gmv``, ``_make_thor_*_gemm_kernel``,
  ``_n_bucket``, ``MXFP*_GROUP_SIZE``) with the same argument meaning, so code written
  against src/vllm_quant_kernels/_kernels.py keeps working.  The Triton launch syntax
  ``kernel[grid](...)`` is accepted; the grid is ignored because every HIP launch here
  sizes its own persistent grid.

All work is enqueued on torch's current stream of the tensors' device.  Nothing falls
back to the CPU or to torch: non-device tensors are rejected.
"""
from __future__ import annotations

import torch

from . import _lib

MXFP8_GROUP_SIZE = 32   # reference: src/vllm_quant_kernels/_kernels.py:488
MXFP4_GROUP_SIZE = 32   # reference: src/vllm_quant_kernels/_kernels.py:646

_DT = {torch.float32: _lib.VQK_F32, torch.float16: _lib.VQK_F16, torch.bfloat16: _lib.VQK_BF16}


def _stream(t: torch.Tensor) -> int:
    return torch.cuda.current_stream(t.device).cuda_stream


def _dev(*ts: torch.Tensor) -> None:
    for t in ts:
        if t is not None and not t.is_cuda:
            raise ValueError("vllm_quant_kernels: tensors must live on the ROCm device "
                             f"(got a {t.device} tensor); there is no CPU path")


def _rowmajor(t: torch.Tensor, name: str) -> None:
    if t.dim() != 2 or t.stride(1) != 1:
        raise ValueError(f"{name} must be a 2-D tensor with unit stride along its last dim")


def _contig(t: torch.Tensor, name: str) -> None:
    if not t.is_contiguous():
        raise ValueError(f"{name} must be contiguous")


# ---------------------------------------------------------------------------------------
# Weight quantizers

def quant_rows_int8(w: torch.Tensor, scale_dtype: torch.dtype = torch.float16):
    """Per-row symmetric INT8 (reference _quant.py:245-302): returns (q int8 [M,K], s [M])."""
    _dev(w)
    _rowmajor(w, "w")
    M, K = w.shape
    q = torch.empty(M, K, dtype=torch.int8, device=w.device)
    s = torch.empty(M, dtype=scale_dtype, device=w.device)
    if scale_dtype not in (torch.float16, torch.float32):
        raise ValueError("scale_dtype must be float16 or float32")
    _lib.call("vqk_quant_rows_int8", w.data_ptr(), _DT[w.dtype], M, K, w.stride(0), q.data_ptr(),
              s.data_ptr(), 1 if scale_dtype == torch.float32 else 0, _stream(w))
    return q, s


def quant_rows_fp8(w: torch.Tensor):
    """Per-row FP8 e4m3 (reference _quant.py:304-325): returns (q uint8 [M,K], s fp16 [M])."""
    _dev(w)
    _rowmajor(w, "w")
    M, K = w.shape
    q = torch.empty(M, K, dtype=torch.uint8, device=w.device)
    s = torch.empty(M, dtype=torch.float16, device=w.device)
    _lib.call("vqk_quant_rows_fp8", w.data_ptr(), _DT[w.dtype], M, K, w.stride(0), q.data_ptr(),
              s.data_ptr(), _stream(w))
    return q, s


def quant_mxfp8(t: torch.Tensor):
    """MXFP8 (reference _quant.py:34-61): returns (e4m3 bytes uint8 [R,K], E8M0 uint8 [R,K/32])."""
    _dev(t)
    _rowmajor(t, "t")
    R, K = t.shape
    assert K % MXFP8_GROUP_SIZE == 0, f"K={K} must be divisible by group_size={MXFP8_GROUP_SIZE}"
    q = torch.empty(R, K, dtype=torch.uint8, device=t.device)
    s = torch.empty(R, K // 32, dtype=torch.uint8, device=t.device)
    _lib.call("vqk_quant_mxfp8", t.data_ptr(), _DT[t.dtype], R, K, t.stride(0), q.data_ptr(),
              s.data_ptr(), _stream(t))
    return q, s


def quant_mxfp4(t: torch.Tensor):
    """MXFP4 (reference _quant.py:64-105): returns (packed uint8 [R,K/2], E8M0 uint8 [R,K/32])."""
    _dev(t)
    _rowmajor(t, "t")
    R, K = t.shape
    assert K % MXFP4_GROUP_SIZE == 0, f"K={K} must be divisible by group_size={MXFP4_GROUP_SIZE}"
    assert K % 2 == 0, f"K={K} must be even (FP4 packing)"
    q = torch.empty(R, K // 2, dtype=torch.uint8, device=t.device)
    s = torch.empty(R, K // 32, dtype=torch.uint8, device=t.device)
    _lib.call("vqk_quant_mxfp4", t.data_ptr(), _DT[t.dtype], R, K, t.stride(0), q.data_ptr(),
              s.data_ptr(), _stream(t))
    return q, s


# ---------------------------------------------------------------------------------------
# Runtime activation quantizers (standalone; the lm_head wrappers fuse them)

def act_quant_int8(x: torch.Tensor):
    """Per-tensor INT8 (reference _quant.py:535-540): returns (xq int8 [B,K], xs fp32 [1])."""
    _dev(x)
    _rowmajor(x, "x")
    B, K = x.shape
    xq = torch.empty(B, K, dtype=torch.int8, device=x.device)
    xs = torch.empty(1, dtype=torch.float32, device=x.device)
    _lib.call("vqk_act_quant_int8", x.data_ptr(), _DT[x.dtype], x.stride(0), B, K, xq.data_ptr(),
              xs.data_ptr(), _stream(x))
    return xq, xs


def act_cast_e4m3(x: torch.Tensor):
    """x.to(float8_e4m3fn) as raw bytes (reference _quant.py:413)."""
    _dev(x)
    _rowmajor(x, "x")
    B, K = x.shape
    xq = torch.empty(B, K, dtype=torch.uint8, device=x.device)
    _lib.call("vqk_act_cast_e4m3", x.data_ptr(), _DT[x.dtype], x.stride(0), B, K, xq.data_ptr(),
              _stream(x))
    return xq


# ---------------------------------------------------------------------------------------
# lm_head projections: x [B,K] -> out fp16 [B,M]

def _out(out, B, M, device):
    if out is None:
        return torch.empty(B, M, dtype=torch.float16, device=device)
    if out.dtype != torch.float16 or out.dim() != 2 or out.shape != (B, M) or out.stride(1) != 1:
        raise ValueError(f"out must be fp16 [{B},{M}] with unit inner stride")
    return out


def _x_for(x, K):
    _rowmajor(x, "x")
    if x.shape[1] != K:
        raise ValueError(f"activation width {x.shape[1]} != K={K}")
    if x.dtype not in _DT:
        raise ValueError(f"unsupported activation dtype {x.dtype}")
    return x


# From these batch sizes on, the W8A8, e4m3 and MX lm_head wrappers quantize the activations
# once in a separate launch and run the pre-quantized kernel: the fused form re-quantizes
# the activations in every workgroup's prologue, which costs more than a launch once the
# batch is large.  Crossovers measured on MI355X at 248320 x 3072 (median us per call,
# fused / separate): W8A8 B=8 123.3 / 121.2; FP8 B=12 121.7 / 123.3, B=16 124.0 / 124.4,
# B=32 134.1 / 131.5; MXFP8 B=8 118.5 / 119.7, B=12 124.5 / 124.3, B=16 126.5 / 125.5;
# MXFP4 B=8 66.0 / 67.2, B=12 71.0 / 71.0, B=16 74.0 / 72.2.  Both forms give identical
# logits.
SEPARATE_ACT_QUANT_MIN_B = {"w8a8": 8, "fp8": 16, "mxfp8": 12, "mxfp4": 12}


def lmhead_w8a16(x, w, s, out=None):
    """out = fp16(s16[m] * sum_k f32(w[m,k]) * f32(x[b,k])) (reference int8_gmv / int8_gemm)."""
    _dev(x, w, s)
    _contig(w, "w")
    M, K = w.shape
    x = _x_for(x, K)
    if x.dtype != torch.float16:
        x = x.to(torch.float16)
    B = x.shape[0]
    out = _out(out, B, M, x.device)
    _lib.call("vqk_lmhead_w8a16", w.data_ptr(), s.data_ptr(), x.data_ptr(), x.stride(0),
              out.data_ptr(), out.stride(0), M, K, B, _stream(x))
    return out


def lmhead_w8a8(x, w, ws, out=None, acc=None):
    """Per-tensor INT8 activations quantized in-kernel; int32 accumulate (reference
    _w8a8_forward + int8_w8a8_gemm).  ``acc`` (int32 [B,M]) optionally receives the raw sums."""
    _dev(x, w, ws, acc)
    _contig(w, "w")
    M, K = w.shape
    x = _x_for(x, K)
    B = x.shape[0]
    if acc is not None:
        assert acc.dtype == torch.int32 and acc.shape == (B, M) and acc.is_contiguous()
    if B >= SEPARATE_ACT_QUANT_MIN_B["w8a8"]:
        xq, xs = act_quant_int8(x)
        return gemm_w8a8_devscale(xq, xs, w, ws, out=out, acc=acc)
    out = _out(out, B, M, x.device)
    _lib.call("vqk_lmhead_w8a8", w.data_ptr(), ws.data_ptr(), x.data_ptr(), _DT[x.dtype], x.stride(0),
              out.data_ptr(), out.stride(0), acc.data_ptr() if acc is not None else None, M, K, B,
              _stream(x))
    return out


def lmhead_fp8(x, w, s, out=None):
    """e4m3 activation cast in-kernel (reference _fp8_forward + fp8_gemm)."""
    _dev(x, w, s)
    _contig(w, "w")
    M, K = w.shape
    x = _x_for(x, K)
    B = x.shape[0]
    if B >= SEPARATE_ACT_QUANT_MIN_B["fp8"]:
        return gemm_fp8(act_cast_e4m3(x), w, s, out=out)
    out = _out(out, B, M, x.device)
    _lib.call("vqk_lmhead_fp8", w.data_ptr(), s.data_ptr(), x.data_ptr(), _DT[x.dtype], x.stride(0),
              out.data_ptr(), out.stride(0), M, K, B, _stream(x))
    return out


def lmhead_mxfp8(x, w, ws, out=None):
    """MXFP8 activation quantization in-kernel (reference _mxfp8_forward + mxfp8_gemm)."""
    _dev(x, w, ws)
    _contig(w, "w")
    _contig(ws, "ws")
    M, K = w.shape
    x = _x_for(x, K)
    B = x.shape[0]
    if B >= SEPARATE_ACT_QUANT_MIN_B["mxfp8"]:
        xq, xs = quant_mxfp8(x)
        return gemm_mxfp8(xq, xs, w, ws, out=out)
    out = _out(out, B, M, x.device)
    _lib.call("vqk_lmhead_mxfp8", w.data_ptr(), ws.data_ptr(), x.data_ptr(), _DT[x.dtype], x.stride(0),
              out.data_ptr(), out.stride(0), M, K, B, _stream(x))
    return out


def lmhead_mxfp4(x, w_packed, ws, K=None, out=None):
    """W4A8: E2M1 weights, MXFP8 activations quantized in-kernel (reference _mxfp4_forward +
    mxfp4_gemm)."""
    _dev(x, w_packed, ws)
    _contig(w_packed, "w_packed")
    _contig(ws, "ws")
    M = w_packed.shape[0]
    K = int(K) if K is not None else 2 * w_packed.shape[1]
    x = _x_for(x, K)
    B = x.shape[0]
    if B >= SEPARATE_ACT_QUANT_MIN_B["mxfp4"]:
        xq, xs = quant_mxfp8(x)
        return gemm_mxfp4(xq, xs, w_packed, ws, K, out=out)
    out = _out(out, B, M, x.device)
    _lib.call("vqk_lmhead_mxfp4", w_packed.data_ptr(), ws.data_ptr(), x.data_ptr(), _DT[x.dtype],
              x.stride(0), out.data_ptr(), out.stride(0), M, K, B, _stream(x))
    return out



_SAMPLE_MODES = {"w8a16": 0, "w8a8": 1, "fp8": 2, "mxfp8": 3, "mxfp4": 4}


def lmhead_sample(mode: str, x, w, ws, temperature, seeds, K=None, out=None):
    """Fused lm_head + Gumbel-argmax sampling (opt-in, one batch group: B <= 32, and
    B <= 16 for W8A16; larger batches raise ValueError): returns (tokens int64 [B],
    logits fp16 [B,M]).  The tokens equal those of lmhead_<mode> followed by
    fused_gumbel_sample(logits.float(), temperature, seeds) bit for bit; the sampling runs
    in the projection's epilogue, so the logits are not re-read.  No top-k."""
    code = _SAMPLE_MODES[mode]
    _dev(x, w, ws, seeds)
    _contig(w, "w")
    M = w.shape[0]
    K = int(K) if K is not None else (2 * w.shape[1] if mode == "mxfp4" else w.shape[1])
    x = _x_for(x, K)
    if mode == "w8a16" and x.dtype != torch.float16:
        x = x.to(torch.float16)
    B = x.shape[0]
    if B > (16 if mode == "w8a16" else 32):
        raise ValueError(f"lmhead_sample: batch {B} exceeds one batch group of the {mode} kernel "
                         f"({16 if mode == 'w8a16' else 32} rows)")
    assert seeds.shape == (B,) and seeds.dtype in (torch.int32, torch.int64)
    seeds = seeds.contiguous()
    if temperature is not None:
        assert temperature.shape == (B,) and temperature.dtype == torch.float32
        temperature = temperature.contiguous()
    out = _out(out, B, M, x.device)
    tokens = torch.empty(B, dtype=torch.int64, device=x.device)
    need = int(_lib.load().vqk_lmhead_sample_workspace_size(B))
    wsp = torch.empty(max(need, 8), dtype=torch.uint8, device=x.device)
    _lib.call("vqk_lmhead_sample", code, w.data_ptr(), ws.data_ptr(), x.data_ptr(), _DT[x.dtype], x.stride(0),
              out.data_ptr(), out.stride(0), M, K, B,
              temperature.data_ptr() if temperature is not None else None,
              seeds.data_ptr(), 1 if seeds.dtype == torch.int64 else 0, tokens.data_ptr(),
              wsp.data_ptr(), wsp.numel(), _stream(x))
    return tokens, out

def gemm_fp8(xq, w, s, out=None):
    _dev(xq, w, s)
    M, K = w.shape
    B = xq.shape[0]
    xq = xq.contiguous()
    out = _out(out, B, M, xq.device)
    _lib.call("vqk_gemm_fp8", w.data_ptr(), s.data_ptr(), xq.data_ptr(), out.data_ptr(), out.stride(0),
              M, K, B, _stream(xq))
    return out


def gemm_w8a8(xq, xs: float, w, ws, out=None, acc=None):
    _dev(xq, w, ws, acc)
    M, K = w.shape
    B = xq.shape[0]
    xq = xq.contiguous()
    out = _out(out, B, M, xq.device)
    _lib.call("vqk_gemm_w8a8", w.data_ptr(), ws.data_ptr(), xq.data_ptr(), float(xs), out.data_ptr(),
              out.stride(0), acc.data_ptr() if acc is not None else None, M, K, B, _stream(xq))
    return out


def gemm_w8a8_devscale(xq, xs, w, ws, out=None, acc=None):
    """gemm_w8a8 with the per-tensor scale xs (fp32 [1]) read on the device: no host sync."""
    _dev(xq, xs, w, ws, acc)
    M, K = w.shape
    B = xq.shape[0]
    xq = xq.contiguous()
    assert xs.dtype == torch.float32 and xs.numel() == 1
    out = _out(out, B, M, xq.device)
    _lib.call("vqk_gemm_w8a8_devscale", w.data_ptr(), ws.data_ptr(), xq.data_ptr(), xs.data_ptr(),
              out.data_ptr(), out.stride(0), acc.data_ptr() if acc is not None else None, M, K, B,
              _stream(xq))
    return out


def gemm_mxfp8(xq, xs, w, ws, out=None):
    _dev(xq, xs, w, ws)
    M, K = w.shape
    B = xq.shape[0]
    xq, xs = xq.contiguous(), xs.contiguous()
    out = _out(out, B, M, xq.device)
    _lib.call("vqk_gemm_mxfp8", w.data_ptr(), ws.data_ptr(), xq.data_ptr(), xs.data_ptr(),
              out.data_ptr(), out.stride(0), M, K, B, _stream(xq))
    return out


def gemm_mxfp4(xq, xs, w_packed, ws, K=None, out=None):
    _dev(xq, xs, w_packed, ws)
    M = w_packed.shape[0]
    K = int(K) if K is not None else 2 * w_packed.shape[1]
    B = xq.shape[0]
    xq, xs = xq.contiguous(), xs.contiguous()
    out = _out(out, B, M, xq.device)
    _lib.call("vqk_gemm_mxfp4", w_packed.data_ptr(), ws.data_ptr(), xq.data_ptr(), xs.data_ptr(),
              out.data_ptr(), out.stride(0), M, K, B, _stream(xq))
    return out


# ---------------------------------------------------------------------------------------
# Reference kernel-level names (src/vllm_quant_kernels/_kernels.py)

class _Launch:
    """Accepts Triton's ``kernel[grid](...)`` launch syntax; the grid is ignored."""

    def __init__(self, fn, name):
        self._fn = fn
        self.__name__ = name

    def __getitem__(self, grid):
        return self._fn

    def __call__(self, *a, **k):
        return self._fn(*a, **k)


def _n_bucket(n: int) -> int:
    """Batch bucket of the reference's autotune key (src/vllm_quant_kernels/_kernels.py:87-98).
    Kept for API compatibility; the HIP dispatcher does not autotune."""
    if n < 4:
        return 0
    if n < 8:
        return 1
    if n < 32:
        return 2
    return 3


def _view(ptr_t, rows, cols, stride_r):
    return ptr_t.as_strided((rows, cols), (stride_r, 1))


def _int8_gmv(out, w, x, s, M, K, stride_ob, stride_xb, NUM_BATCH=1, **_):
    """int8_gmv (src/vllm_quant_kernels/_kernels.py:8-84): out[b, :M] for b < NUM_BATCH.
    The reference kernel loads x in whatever float dtype it has; the HIP kernel reads fp16,
    so bf16/fp32 activations are converted first (as _int8_gemm does).  out must be fp16."""
    B = int(NUM_BATCH)
    xv = _view(x, B, K, stride_xb)
    ov = _view(out, B, M, stride_ob)
    _dev(xv, w, s, ov)
    if out.dtype != torch.float16:
        raise ValueError(f"int8_gmv: out must be float16, got {out.dtype}")
    if xv.dtype not in _DT:
        raise ValueError(f"int8_gmv: unsupported activation dtype {xv.dtype}")
    if xv.dtype != torch.float16:
        xv = xv.to(torch.float16)
    _lib.call("vqk_lmhead_w8a16", w.data_ptr(), s.data_ptr(), xv.data_ptr(), xv.stride(0), ov.data_ptr(),
              stride_ob, M, K, B, _stream(w))


int8_gmv = _Launch(_int8_gmv, "int8_gmv")


def _check_strides(stride_om, stride_wk, stride_xk, w, stride_wm, K):
    if stride_om != 1 or stride_wk != 1 or stride_xk != 1 or stride_wm != K:
        raise ValueError("the HIP kernels take row-major, contiguous-row operands "
                         "(stride_om == stride_wk == stride_xk == 1, stride_wm == K)")


def _int8_gemm(out, w, x, s, M, N, K, N_BUCKET, stride_om, stride_on, stride_wm, stride_wk,
               stride_xn, stride_xk, **_):
    _check_strides(stride_om, stride_wk, stride_xk, w, stride_wm, K)
    xv = _view(x, N, K, stride_xn)
    if xv.dtype != torch.float16:
        xv = xv.to(torch.float16)
    _lib.call("vqk_lmhead_w8a16", w.data_ptr(), s.data_ptr(), xv.data_ptr(), xv.stride(0), out.data_ptr(),
              stride_on, M, K, N, _stream(w))


def _fp8_gemm(out, w, x, s, M, N, K, N_BUCKET, stride_om, stride_on, stride_wm, stride_wk,
              stride_xn, stride_xk, **_):
    _check_strides(stride_om, stride_wk, stride_xk, w, stride_wm, K)
    xv = _view(x, N, K, stride_xn).contiguous()
    _lib.call("vqk_gemm_fp8", w.data_ptr(), s.data_ptr(), xv.data_ptr(), out.data_ptr(), stride_on,
              M, K, N, _stream(w))


def _w8a8_gemm(out, w, x, ws, xs, M, N, K, N_BUCKET, stride_om, stride_on, stride_wm, stride_wk,
               stride_xn, stride_xk, **_):
    _check_strides(stride_om, stride_wk, stride_xk, w, stride_wm, K)
    xv = _view(x, N, K, stride_xn).contiguous()
    _lib.call("vqk_gemm_w8a8", w.data_ptr(), ws.data_ptr(), xv.data_ptr(), float(xs), out.data_ptr(),
              stride_on, None, M, K, N, _stream(w))


def _mx_gemm(fp4):
    def run(out, w, x, ws, xs, M, N, K, N_BUCKET, stride_om, stride_on, stride_wm, stride_wk,
            stride_xn, stride_xk, stride_wsm, stride_wsg, stride_xsn, stride_xsg, GROUP_SIZE=32, **_):
        if GROUP_SIZE != 32:
            raise ValueError("MX group size must be 32")
        kb = K // 2 if fp4 else K
        if stride_om != 1 or stride_wk != 1 or stride_xk != 1 or stride_wm != kb:
            raise ValueError("the HIP kernels take row-major, contiguous-row operands")
        if stride_wsg != 1 or stride_wsm != K // 32 or stride_xsg != 1:
            raise ValueError("MX scales must be row-major [rows, K/32]")
        xv = _view(x, N, K, stride_xn).contiguous()
        xsv = _view(xs, N, K // 32, stride_xsn).contiguous()
        name = "vqk_gemm_mxfp4" if fp4 else "vqk_gemm_mxfp8"
        _lib.call(name, w.data_ptr(), ws.data_ptr(), xv.data_ptr(), xsv.data_ptr(), out.data_ptr(),
                  stride_on, M, K, N, _stream(w))
    return run


def _make_thor_gemm_kernel():
    """W8A16 GEMM (reference _kernels.py:148-250); returns (kernel, _n_bucket)."""
    return _Launch(_int8_gemm, "int8_gemm"), _n_bucket


def _make_thor_fp8_gemm_kernel():
    """FP8 GEMM (reference _kernels.py:258-360); returns (kernel, _n_bucket)."""
    return _Launch(_fp8_gemm, "fp8_gemm"), _n_bucket


def _make_thor_w8a8_gemm_kernel():
    """W8A8 GEMM (reference _kernels.py:369-479); returns (kernel, _n_bucket)."""
    return _Launch(_w8a8_gemm, "int8_w8a8_gemm"), _n_bucket


def _make_thor_mxfp8_gemm_kernel():
    """MXFP8 GEMM (reference _kernels.py:491-634); returns (kernel, _n_bucket)."""
    return _Launch(_mx_gemm(False), "mxfp8_gemm"), _n_bucket


def _make_thor_mxfp4_gemm_kernel():
    """MXFP4 W4A8 GEMM (reference _kernels.py:649-804); returns (kernel, _n_bucket)."""
    return _Launch(_mx_gemm(True), "mxfp4_gemm"), _n_bucket
