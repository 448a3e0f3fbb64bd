// vqk_device.hip - device checks and small ABI helpers of libvqk_hip.so.
#include <hip/hip_runtime.h>
#include <string.h>

#include <mutex>

#include "vqk.h"
#include "vqk_internal.h"

namespace {
constexpr int kMaxDev = 64;
int g_state[kMaxDev];  // 0 unknown, 1 ok (gfx950), -1 rejected
int g_cus[kMaxDev];
std::mutex g_mu;
}  // namespace

extern "C" int vqk_abi_version(void) { return 2; }

extern "C" int vqk_device_check(void) {
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= kMaxDev) return VQK_ENODEVICE;
  if (g_state[dev] == 1) return VQK_OK;
  if (g_state[dev] == -1) return VQK_ENODEVICE;
  std::lock_guard<std::mutex> lk(g_mu);
  hipDeviceProp_t p;
  if (hipGetDeviceProperties(&p, dev) != hipSuccess) return VQK_ENODEVICE;
  const bool ok = strncmp(p.gcnArchName, "gfx950", 6) == 0;
  g_cus[dev] = p.multiProcessorCount;
  g_state[dev] = ok ? 1 : -1;
  return ok ? VQK_OK : VQK_ENODEVICE;
}

int vqk_cu_count() {
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= kMaxDev) return 256;
  return g_cus[dev] > 0 ? g_cus[dev] : 256;
}

extern "C" const char* vqk_strerror(int code) {
  switch (code) {
    case VQK_OK: return "ok";
    case VQK_EINVAL: return "invalid argument";
    case VQK_EUNSUPPORTED: return "unsupported shape";
    case VQK_ENODEVICE: return "no gfx950 HIP device";
    case VQK_EWORKSPACE: return "workspace too small";
    default: break;
  }
  if (code > 0) return hipGetErrorString((hipError_t)code);
  return "unknown error";
}

// ---------------------------------------------------------------------------------------
// Content hash of a device buffer (the identity of a source weight in the on-disk
// quantized-lm_head cache).  Chunk i (16 bytes: words lo, hi; a partial last chunk is
// zero-padded) contributes f(lo, i) and g(lo, hi, i), each a splitmix64 finalisation of
// the words keyed by i, to two 64-bit sums; a changed byte anywhere, or two chunks
// exchanged, moves both sums by pseudo-random amounts.  Each workgroup adds its partial
// sums to out[0], out[1] with one atomic each.
namespace {
__device__ __forceinline__ unsigned long long smix(unsigned long long z) {
  z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ull;
  z = (z ^ (z >> 27)) * 0x94D049BB133111EBull;
  return z ^ (z >> 31);
}

__global__ void __launch_bounds__(256) hash128_kernel(const unsigned char* p, int64_t nbytes,
                                                      unsigned long long* out) {
  const int64_t nfull = nbytes >> 4;
  const int64_t nchunk = (nbytes + 15) >> 4;
  unsigned long long a = 0, b = 0;
  for (int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x; i < nchunk; i += (int64_t)gridDim.x * 256) {
    unsigned long long lo = 0, hi = 0;
    if (i < nfull) {
      const ulonglong2 t = ((const ulonglong2*)p)[i];
      lo = t.x;
      hi = t.y;
    } else {
      for (int64_t k = i * 16; k < nbytes; ++k) {
        const unsigned long long by = p[k];
        const int sh = (int)(k - i * 16);
        if (sh < 8) lo |= by << (8 * sh);
        else hi |= by << (8 * (sh - 8));
      }
    }
    const unsigned long long key = (unsigned long long)i * 0x9E3779B97F4A7C15ull;
    const unsigned long long f = smix(lo ^ key);
    a += f;
    b += smix(hi ^ (f + 0xD6E8FEB86659FD93ull));
  }
  __shared__ unsigned long long ra[256], rb[256];
  ra[threadIdx.x] = a;
  rb[threadIdx.x] = b;
  __syncthreads();
  for (int off = 128; off > 0; off >>= 1) {
    if ((int)threadIdx.x < off) {
      ra[threadIdx.x] += ra[threadIdx.x + off];
      rb[threadIdx.x] += rb[threadIdx.x + off];
    }
    __syncthreads();
  }
  if (threadIdx.x == 0) {
    atomicAdd(&out[0], ra[0]);
    atomicAdd(&out[1], rb[0]);
  }
}
}  // namespace

extern "C" int vqk_hash128(const void* p, int64_t nbytes, uint64_t* out, vqk_stream_t stream) {
  int rc = vqk_device_check();
  if (rc) return rc;
  if (!p || !out || nbytes < 0 || ((uintptr_t)p & 15) != 0 || ((uintptr_t)out & 7) != 0) return VQK_EINVAL;
  if (nbytes == 0) return VQK_OK;
  const int64_t nchunk = (nbytes + 15) >> 4;
  int64_t grid = (nchunk + 255) / 256;
  const int64_t cap = (int64_t)vqk_cu_count() * 8;
  if (grid > cap) grid = cap;
  hipLaunchKernelGGL(hash128_kernel, dim3((unsigned)grid), dim3(256), 0, (hipStream_t)stream,
                     (const unsigned char*)p, nbytes, (unsigned long long*)out);
  hipError_t e = hipGetLastError();
  return e == hipSuccess ? VQK_OK : (int)e;
}
