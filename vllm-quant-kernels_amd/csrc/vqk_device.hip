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
