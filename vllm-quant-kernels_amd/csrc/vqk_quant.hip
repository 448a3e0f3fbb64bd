// vqk_quant.hip - weight quantizers (run once per lm_head) and standalone activation
// quantizers for gfx950.  Each reproduces the reference's torch op chain bit for bit:
//   per-row INT8   src/vllm_quant_kernels/_quant.py:245-302
//   per-row FP8    src/vllm_quant_kernels/_quant.py:304-325
//   MXFP8          src/vllm_quant_kernels/_quant.py:34-61
//   MXFP4          src/vllm_quant_kernels/_quant.py:64-105
//   W8A8 act quant src/vllm_quant_kernels/_quant.py:535-540
//   FP8 act cast   src/vllm_quant_kernels/_quant.py:413
// Per-row kernels use one 256-thread workgroup per row (amax, then quantize); the MX
// kernels use one thread per 32-element group.  These are byte-streaming kernels bound by
// HBM, so they use plain coalesced loads and no LDS staging beyond the row reduction.
#include <hip/hip_runtime.h>
#include <stdint.h>

#include "vqk.h"
#include "vqk_internal.h"
#include "vqk_math.h"

namespace vqk {

constexpr int QT = 256;

__device__ __forceinline__ float block_max(float m, float* red) {
  for (int off = 32; off > 0; off >>= 1) m = fmaxf(m, __shfl_xor(m, off));
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  if (lane == 0) red[wave] = m;
  __syncthreads();
  float r = red[0];
  for (int w = 1; w < (int)(blockDim.x >> 6); ++w) r = fmaxf(r, red[w]);
  __syncthreads();
  return r;
}

__global__ void __launch_bounds__(QT) quant_rows_int8_kernel(const void* w, int dt, int64_t K, int64_t ldw,
                                                              int8_t* q, void* sout, int s_f32) {
  __shared__ float red[QT / 64];
  const int64_t row = blockIdx.x;
  const int64_t off = row * ldw;
  float m = 0.f;
  for (int64_t k = threadIdx.x; k < K; k += QT) m = fmaxf(m, fabsf(load_as_f32(w, dt, off + k)));
  m = block_max(m, red);
  const float s = fmaxf(m / 127.0f, 1e-12f);
  for (int64_t k = threadIdx.x; k < K; k += QT) {
    float v = __builtin_rintf(load_as_f32(w, dt, off + k) / s);
    v = fminf(fmaxf(v, -127.f), 127.f);
    q[row * K + k] = (int8_t)(int)v;
  }
  if (threadIdx.x == 0) {
    if (s_f32) ((float*)sout)[row] = s;
    else ((uint16_t*)sout)[row] = f2h(s);
  }
}

__global__ void __launch_bounds__(QT) quant_rows_fp8_kernel(const void* w, int dt, int64_t K, int64_t ldw,
                                                             uint8_t* q, uint16_t* sout) {
  __shared__ float red[QT / 64];
  const int64_t row = blockIdx.x;
  const int64_t off = row * ldw;
  float m = 0.f;
  for (int64_t k = threadIdx.x; k < K; k += QT) m = fmaxf(m, fabsf(load_as_f32(w, dt, off + k)));
  m = block_max(m, red);
  const float s = fmaxf(m / 448.0f, 1e-12f);
  for (int64_t k = threadIdx.x; k < K; k += QT) {
    float v = load_as_f32(w, dt, off + k) / s;
    v = fminf(fmaxf(v, -448.f), 448.f);
    q[row * K + k] = f32_to_e4m3(v);
  }
  if (threadIdx.x == 0) sout[row] = f2h(s);
}

// One thread per 32-element group; the group's 32 elements come in with 16-byte loads when
// rows are 16-byte aligned (vec).
template <int DT>
__global__ void quant_mx_kernel(const void* t, int64_t R, int64_t K, int64_t ldt, uint8_t* q,
                                uint8_t* scales, int fp4, int vec) {
  // Four lanes per 32-element group, 8 elements each: the group's amax takes two lane
  // exchanges, then every lane encodes its own 8 elements (short per-lane chains: at
  // activation sizes the launch is latency-bound).
  const int64_t G = K / 32;
  const int64_t tid = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  const int64_t gid = tid >> 2;
  const int part = (int)(tid & 3);
  const bool live = gid < R * G;
  const int64_t g = live ? gid : 0;  // idle lanes mirror group 0 so the exchanges see 4 lanes
  const int64_t row = g / G, grp = g - row * G;
  float v[8];
  load_run<DT, 8>(t, row * ldt + grp * 32 + part * 8, vec != 0, v);
  float amax = 0.f;
#pragma unroll
  for (int e = 0; e < 8; ++e) amax = fmaxf(amax, fabsf(v[e]));
  amax = fmaxf(amax, __shfl_xor(amax, 1));
  amax = fmaxf(amax, __shfl_xor(amax, 2));
  const int k = mx_exponent(amax, fp4 ? 6.0f : 448.0f);
  const float isc = exp2i(-k);  // x / 2^k as x * 2^-k: the same correctly rounded value
  if (!live) return;
  if (part == 0) scales[row * G + grp] = (uint8_t)(k + 127);
  if (!fp4) {
    float y[8];
#pragma unroll
    for (int e = 0; e < 8; ++e) y[e] = fminf(fmaxf(v[e] * isc, -448.f), 448.f);
    const uint32_t w[2] = {e4m3x4_clamped(y[0], y[1], y[2], y[3]), e4m3x4_clamped(y[4], y[5], y[6], y[7])};
    uint32_t* dst = (uint32_t*)(q + row * K + grp * 32 + part * 8);
    dst[0] = w[0];
    dst[1] = w[1];
  } else {
    uint32_t w = 0;
#pragma unroll
    for (int e = 0; e < 8; ++e) w |= f32_to_e2m1(v[e] * isc) << (4 * e);
    *(uint32_t*)(q + row * (K / 2) + grp * 16 + part * 4) = w;
  }
}

// Per-tensor INT8 activation quantization.  The activation is small (B x K of a decode
// step), so every workgroup computes the whole tensor's amax itself (the re-reads come from
// L2) and then quantizes its own share: one launch, no cross-workgroup exchange, and as
// many CUs as shares.  8 consecutive elements per thread and step when rows allow 16-byte
// loads.  Codes are rint(x / s) exactly (rint_div_i8), clamped to +-127.
template <int DT>
__global__ void __launch_bounds__(1024) act_quant_int8_kernel(const void* x, int64_t ldx, int64_t B, int64_t K,
                                                              int vec, int8_t* xq, float* xs) {
  __shared__ float red[16];
  // 32-bit indices (B * K / 8 < 2^31 on the vector path): a 64-bit division per step
  // would cost more than the loads
  const int per_row = (int)(K / 8), total = (int)B * per_row;
  const bool contig = ldx == K;
  float m = 0.f;
  if (vec) {
    // The whole tensor in rounds of AQ_LOADS 8-element chunks per thread, every load of a
    // round issued before any is used (each round costs one L2 latency).  Chunks past the
    // end re-read the thread's first chunk of the round, which changes no maximum.  Rows
    // stored back to back (ldx == K) address chunk c at 8c: the division by the row length
    // (a ~40-instruction sequence per chunk) was most of the launch.
    constexpr int AQ_LOADS = (DT == VQK_F16) ? 16 : 8;  // (bf16 at 16 spills)
    for (int c0 = threadIdx.x; c0 < total; c0 += AQ_LOADS * (int)blockDim.x) {
      float v[AQ_LOADS][8];
      if (contig) {
#pragma unroll
        for (int u = 0; u < AQ_LOADS; ++u) {
          const int c = c0 + u * (int)blockDim.x;
          load_run<DT, 8>(x, (int64_t)8 * (c < total ? c : c0), true, v[u]);
        }
      } else {
#pragma unroll
        for (int u = 0; u < AQ_LOADS; ++u) {
          int c = c0 + u * (int)blockDim.x;
          c = c < total ? c : c0;
          const int b = c / per_row, k8 = c - b * per_row;
          load_run<DT, 8>(x, (int64_t)b * ldx + 8 * k8, true, v[u]);
        }
      }
#pragma unroll
      for (int u = 0; u < AQ_LOADS; ++u)
#pragma unroll
        for (int e = 0; e < 8; ++e) m = fmaxf(m, fabsf(v[u][e]));
    }
  } else {
    for (int64_t b = 0; b < B; ++b)
      for (int64_t k = threadIdx.x; k < K; k += blockDim.x) m = fmaxf(m, fabsf(load_dt<DT>(x, b * ldx + k)));
  }
  m = block_max(m, red);
  const float s = fmaxf(m / 127.0f, 1e-12f);
  const float r = 1.0f / s;
  if (vec) {
    // this workgroup's share of the 8-element chunks
    const int share = (total + gridDim.x - 1) / gridDim.x;
    const int c0 = blockIdx.x * share, c1 = min(total, c0 + share);
#pragma unroll 2
    for (int c = c0 + threadIdx.x; c < c1; c += blockDim.x) {
      int64_t off = (int64_t)8 * c;
      if (!contig) {
        const int b = c / per_row, k8 = c - b * per_row;
        off = (int64_t)b * ldx + 8 * k8;
      }
      float v[8];
      load_run<DT, 8>(x, off, true, v);
      uint32_t w[2] = {0u, 0u};
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        const float q = fminf(fmaxf(rint_div_i8(v[e], s, r), -127.f), 127.f);
        w[e >> 2] |= ((uint32_t)(int)q & 0xFFu) << (8 * (e & 3));
      }
      *(uint2*)(xq + (int64_t)8 * c) = make_uint2(w[0], w[1]);  // xq rows are K apart
    }
  } else if (blockIdx.x == 0) {
    for (int64_t b = 0; b < B; ++b)
      for (int64_t k = threadIdx.x; k < K; k += blockDim.x) {
        const float q = fminf(fmaxf(rint_div_i8(load_dt<DT>(x, b * ldx + k), s, r), -127.f), 127.f);
        xq[b * K + k] = (int8_t)(int)q;
      }
  }
  if (blockIdx.x == 0 && threadIdx.x == 0) *xs = s;
}

__global__ void act_cast_e4m3_kernel(const void* x, int dt, int64_t ldx, int64_t B, int64_t K, uint8_t* xq) {
  const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= B * K) return;
  const int64_t b = i / K, k = i - b * K;
  xq[i] = f32_to_e4m3(load_as_f32(x, dt, b * ldx + k));
}

// The same cast, 8 consecutive elements per thread: one 16-byte load (fp16/bf16; two for
// fp32), the hardware conversion with torch's NaN and overflow semantics (e4m3x4_torch,
// equal to f32_to_e4m3 on every float32) and one 8-byte store, with 32-bit indices.  At
// activation sizes the launch is a few latencies long, so the per-element form's 64-bit
// division and byte stores were most of it.
template <int DT>
__global__ void __launch_bounds__(256) act_cast_e4m3_vec_kernel(const void* x, int64_t ldx, int per_row, int total,
                                                                uint8_t* xq) {
  const int c = blockIdx.x * 256 + threadIdx.x;
  if (c >= total) return;
  const int b = c / per_row, k8 = c - b * per_row;
  float v[8];
  load_run<DT, 8>(x, (int64_t)b * ldx + 8 * k8, true, v);
  *(uint2*)(xq + (int64_t)b * per_row * 8 + 8 * k8) =
      make_uint2(e4m3x4_torch(v[0], v[1], v[2], v[3]), e4m3x4_torch(v[4], v[5], v[6], v[7]));
}

static int dt_ok(int dt) { return dt == VQK_F32 || dt == VQK_F16 || dt == VQK_BF16; }

static int finish() {
  hipError_t e = hipGetLastError();
  return e == hipSuccess ? VQK_OK : (int)e;
}

}  // namespace vqk

using namespace vqk;

extern "C" int vqk_quant_rows_int8(const void* w, int w_dtype, int64_t M, int64_t K, int64_t ldw, int8_t* q,
                                   void* scale_out, int scale_is_f32, vqk_stream_t stream) {
  int rc = vqk_device_check();
  if (rc) return rc;
  if (!w || !q || !scale_out || !dt_ok(w_dtype) || M < 0 || K < 1 || ldw < K) return VQK_EINVAL;
  if (M == 0) return VQK_OK;
  if (M > INT32_MAX) return VQK_EUNSUPPORTED;
  hipLaunchKernelGGL(quant_rows_int8_kernel, dim3((unsigned)M), dim3(QT), 0, (hipStream_t)stream, w, w_dtype,
                     K, ldw, q, scale_out, scale_is_f32 ? 1 : 0);
  return finish();
}

extern "C" int vqk_quant_rows_fp8(const void* w, int w_dtype, int64_t M, int64_t K, int64_t ldw, uint8_t* q,
                                  uint16_t* scale_f16, vqk_stream_t stream) {
  int rc = vqk_device_check();
  if (rc) return rc;
  if (!w || !q || !scale_f16 || !dt_ok(w_dtype) || M < 0 || K < 1 || ldw < K) return VQK_EINVAL;
  if (M == 0) return VQK_OK;
  if (M > INT32_MAX) return VQK_EUNSUPPORTED;
  hipLaunchKernelGGL(quant_rows_fp8_kernel, dim3((unsigned)M), dim3(QT), 0, (hipStream_t)stream, w, w_dtype, K,
                     ldw, q, scale_f16);
  return finish();
}

static int quant_mx(const void* t, int dt, int64_t R, int64_t K, int64_t ldt, uint8_t* q, uint8_t* s, int fp4,
                    hipStream_t st) {
  int rc = vqk_device_check();
  if (rc) return rc;
  if (!t || !q || !s || !dt_ok(dt) || R < 0 || K < 1 || ldt < K) return VQK_EINVAL;
  if (K % 32 != 0) return VQK_EINVAL;
  if (R == 0) return VQK_OK;
  const int64_t n = 4 * R * (K / 32);  // four lanes per 32-element group
  const int th = 256;
  const int64_t nb = (n + th - 1) / th;
  if (nb > INT32_MAX) return VQK_EUNSUPPORTED;
  const int es = (dt == VQK_F32) ? 4 : 2;
  const int vec = (((uintptr_t)t & 15) == 0 && (ldt * es) % 16 == 0) ? 1 : 0;
  if (dt == VQK_F32)
    hipLaunchKernelGGL(quant_mx_kernel<VQK_F32>, dim3((unsigned)nb), dim3(th), 0, st, t, R, K, ldt, q, s, fp4, vec);
  else if (dt == VQK_F16)
    hipLaunchKernelGGL(quant_mx_kernel<VQK_F16>, dim3((unsigned)nb), dim3(th), 0, st, t, R, K, ldt, q, s, fp4, vec);
  else
    hipLaunchKernelGGL(quant_mx_kernel<VQK_BF16>, dim3((unsigned)nb), dim3(th), 0, st, t, R, K, ldt, q, s, fp4, vec);
  return finish();
}

extern "C" int vqk_quant_mxfp8(const void* t, int t_dtype, int64_t R, int64_t K, int64_t ldt, uint8_t* q,
                               uint8_t* scales, vqk_stream_t stream) {
  return quant_mx(t, t_dtype, R, K, ldt, q, scales, 0, (hipStream_t)stream);
}

extern "C" int vqk_quant_mxfp4(const void* t, int t_dtype, int64_t R, int64_t K, int64_t ldt, uint8_t* packed,
                               uint8_t* scales, vqk_stream_t stream) {
  return quant_mx(t, t_dtype, R, K, ldt, packed, scales, 1, (hipStream_t)stream);
}

extern "C" int vqk_act_quant_int8(const void* x, int x_dtype, int64_t ldx, int64_t B, int64_t K, int8_t* xq,
                                  float* xs, vqk_stream_t stream) {
  int rc = vqk_device_check();
  if (rc) return rc;
  if (!x || !xq || !xs || !dt_ok(x_dtype) || B < 0 || K < 1 || ldx < K) return VQK_EINVAL;
  if (B == 0) return VQK_OK;
  const int es = (x_dtype == VQK_F32) ? 4 : 2;
  const int vec = (K % 8 == 0 && ((uintptr_t)x & 15) == 0 && (ldx * es) % 16 == 0 && ((uintptr_t)xq & 7) == 0 &&
                   B * (K / 8) < (int64_t)INT32_MAX) ? 1 : 0;
  // one share per ~8192 elements, at most 32 (each workgroup re-reads the whole tensor for
  // the amax, so large activations take fewer shares)
  const int64_t n = B * K;
  int grid = (int)((n + 8191) / 8192);
  if (grid > 32) grid = 32;
  if (n > ((int64_t)1 << 22)) grid = 4;
  if (!vec || grid < 1) grid = 1;
  if (x_dtype == VQK_F32)
    hipLaunchKernelGGL(act_quant_int8_kernel<VQK_F32>, dim3(grid), dim3(1024), 0, (hipStream_t)stream, x, ldx, B, K, vec, xq, xs);
  else if (x_dtype == VQK_F16)
    hipLaunchKernelGGL(act_quant_int8_kernel<VQK_F16>, dim3(grid), dim3(1024), 0, (hipStream_t)stream, x, ldx, B, K, vec, xq, xs);
  else
    hipLaunchKernelGGL(act_quant_int8_kernel<VQK_BF16>, dim3(grid), dim3(1024), 0, (hipStream_t)stream, x, ldx, B, K, vec, xq, xs);
  return finish();
}

extern "C" int vqk_act_cast_e4m3(const void* x, int x_dtype, int64_t ldx, int64_t B, int64_t K, uint8_t* xq,
                                 vqk_stream_t stream) {
  int rc = vqk_device_check();
  if (rc) return rc;
  if (!x || !xq || !dt_ok(x_dtype) || B < 0 || K < 1 || ldx < K) return VQK_EINVAL;
  if (B == 0) return VQK_OK;
  const int64_t n = B * K;
  const int es = (x_dtype == VQK_F32) ? 4 : 2;
  const bool vec = K % 8 == 0 && ((uintptr_t)x & 15) == 0 && (ldx * es) % 16 == 0 && ((uintptr_t)xq & 7) == 0 &&
                   n / 8 < (int64_t)INT32_MAX - 256;
  if (vec) {
    const int per_row = (int)(K / 8), total = (int)(n / 8);
    const dim3 grid((unsigned)((total + 255) / 256));
    const hipStream_t st = (hipStream_t)stream;
    if (x_dtype == VQK_F32) hipLaunchKernelGGL(act_cast_e4m3_vec_kernel<VQK_F32>, grid, dim3(256), 0, st, x, ldx, per_row, total, xq);
    else if (x_dtype == VQK_F16) hipLaunchKernelGGL(act_cast_e4m3_vec_kernel<VQK_F16>, grid, dim3(256), 0, st, x, ldx, per_row, total, xq);
    else hipLaunchKernelGGL(act_cast_e4m3_vec_kernel<VQK_BF16>, grid, dim3(256), 0, st, x, ldx, per_row, total, xq);
    return finish();
  }
  hipLaunchKernelGGL(act_cast_e4m3_kernel, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, (hipStream_t)stream,
                     x, x_dtype, ldx, B, K, xq);
  return finish();
}

// ---------------------------------------------------------------------------------------
// Debug: compare the hardware e4m3 conversions with this library's encoder (f32_to_e4m3,
// torch's cast semantics) on every float32 bit pattern of [lo, hi): e4m3x4_clamped on the
// magnitudes up to 448 it is used for, or, with full set, e4m3x4_torch on every pattern
// (infinities, NaNs and overflow included).
// Counts mismatches and keeps the smallest mismatching pattern (UINT32_MAX: none).
__global__ void __launch_bounds__(256) e4m3_hw_check_kernel(uint32_t lo, uint32_t hi, int full,
                                                            unsigned int* count, unsigned int* first) {
  unsigned int n = 0, f = 0xFFFFFFFFu;
  const uint32_t stride = gridDim.x * blockDim.x;
  for (uint64_t b = (uint64_t)lo + blockIdx.x * blockDim.x + threadIdx.x; b < hi; b += stride) {
    const uint32_t u = (uint32_t)b;
    if (!full && (u & 0x7FFFFFFFu) > 0x43E00000u) continue;  // |x| > 448 or NaN
    const float x = __uint_as_float(u);
    const uint32_t hw = (full ? e4m3x4_torch(x, x, x, x) : e4m3x4_clamped(x, x, x, x)) & 0xFFu;
    if (hw != f32_to_e4m3(x)) {
      ++n;
      f = u < f ? u : f;
    }
  }
  for (int off = 32; off > 0; off >>= 1) {
    n += __shfl_xor(n, off);
    const unsigned int o = __shfl_xor(f, off);
    f = o < f ? o : f;
  }
  if ((threadIdx.x & 63) == 0 && n) {
    atomicAdd(count, n);
    atomicMin(first, f);
  }
}

extern "C" int vqk_debug_e4m3_hw_check(uint32_t lo, uint32_t hi, int full, unsigned int* count,
                                       unsigned int* first, vqk_stream_t stream) {
  int rc = vqk_device_check();
  if (rc) return rc;
  if (!count || !first || hi < lo) return VQK_EINVAL;
  hipLaunchKernelGGL(e4m3_hw_check_kernel, dim3(4096), dim3(256), 0, (hipStream_t)stream, lo, hi, full, count,
                     first);
  return finish();
}
