// vqk_sampler.hip - single-launch Gumbel-argmax sampler over [B, V] fp32 logits (gfx950).
//
// Semantics follow the reference's _gumbel_block_argmax_kernel + host tail
// (src/vllm_quant_kernels/_sampler_kernels.py:38-182):
//   y[b,v] = x                                    (no temperature, or T[b] < 1e-5: greedy)
//   y[b,v] = x / T[b] + G(seed_b, v)              (otherwise; IEEE division)
//   y[b,v] = -inf   where x < thr[b]              (optional top-k threshold on raw logits)
//   out[b] = argmax_v y[b,v], smallest index on ties.
// G = -log(-log(max(u, 2^-126))) with u = Triton's tl.rand(seed, v): Philox4x32-10 word 0
// of counter (v, 0, 0, 0) under key (seed lo32, seed hi32).
//
// Design (MI355X): one workgroup of 256 threads per 8192-element slice of a row; each
// thread holds 32 logits from eight coalesced 16-byte loads, so the logits are read from
// HBM exactly once.  The Philox/log work is the expensive part (~150 VALU ops per element),
// so the kernel prunes exactly instead of computing noise everywhere:
//   * every thread first scores its own largest raw logit (one Philox each, in parallel);
//     each slice publishes the best of those with a 64-bit atomicMax and waits (bounded
//     in time, so it can never deadlock) until all slices of its row have published; the
//     row's best candidate L is then a value the row's winner is >= to;
//   * since G <= GUMBEL_MAX for every possible u, an element with
//     fl(fl(x/T) + GUMBEL_MAX) < L can never win (rounding is monotone), and that test
//     reduces to one compare of the raw logit against a per-row cutoff;
//   * the surviving elements are compacted per wave through LDS and scored 64 at a time.
// The per-row winner is merged with atomicMax on the key (orderable(y) << 32 | ~v), which
// gives the largest y and, among equal y, the smallest v; the last slice of a row (an
// atomic counter) writes out[b] and resets the row's workspace for the next launch.
#include <hip/hip_runtime.h>
#include <stdint.h>

#include "vqk.h"
#include "vqk_internal.h"
#include "vqk_math.h"

namespace vqk {

typedef float v4f __attribute__((ext_vector_type(4)));

constexpr int SMP_THREADS = 256;
constexpr int SMP_EPT = 32;                               // elements per thread
constexpr int SMP_CHUNK = SMP_THREADS * SMP_EPT;          // elements per workgroup
constexpr float GREEDY_EPS = 1e-5f;

struct SmpArgs {
  const float* logits;
  int64_t ld;
  int B, V;
  const float* temp;
  const void* seeds;
  int seed64;
  const float* thr;
  int64_t* out;
  unsigned long long* keys;  // [B] row best key
  unsigned int* arrive;      // [B] slices that published their candidates
  unsigned int* done;        // [B] slices finished
  int nchunks;
  int vec;                   // 16-byte loads allowed
  uint64_t wait_ticks;       // bound of the wait for the row's other slices (wall clock)
  float* scores;             // debug: write y for every element (scores kernel only)
};

struct RowParams {
  bool greedy;
  float T;
  uint32_t k0, k1;
  bool has_thr;
  float thr;
};

__device__ __forceinline__ RowParams row_params(const SmpArgs& a, int row) {
  RowParams p;
  p.T = 1.0f;
  p.greedy = true;
  if (a.temp) {
    p.T = a.temp[row];
    p.greedy = p.T < GREEDY_EPS;
  }
  uint64_t s;
  if (a.seed64) {
    s = ((const uint64_t*)a.seeds)[row];
  } else {
    s = (uint64_t)(int64_t)((const int32_t*)a.seeds)[row];  // int32 -> uint64 sign-extends
  }
  p.k0 = (uint32_t)s;
  p.k1 = (uint32_t)(s >> 32);
  p.has_thr = a.thr != nullptr;
  p.thr = p.has_thr ? a.thr[row] : 0.f;
  return p;
}

// The value the argmax is taken over, for a valid element.
__device__ __forceinline__ float score(const RowParams& p, float x, uint32_t v) {
  if (p.has_thr && !(x >= p.thr)) return -__builtin_inff();
  if (p.greedy) return x;
  float a = x / p.T;
  float u = philox_uniform(philox_word0(v, p.k0, p.k1));
  return a + gumbel_from_uniform(u);
}

__device__ __forceinline__ unsigned long long make_key(float y, uint32_t v) {
  return ((unsigned long long)orderable(y) << 32) | (unsigned long long)(~v);
}

__device__ __forceinline__ unsigned long long wave_max_u64(unsigned long long k) {
#pragma unroll
  for (int off = 32; off > 0; off >>= 1) {
    unsigned long long o = __shfl_xor(k, off);
    k = (o > k) ? o : k;
  }
  return k;
}

// Cross-workgroup protocol.  Only device-scope atomics on the workspace are used, relaxed:
// acquire/release fences would write back and invalidate the L2 of the issuing XCD
// (buffer_wbl2 / buffer_inv), which costs far more than the whole reduction.  Ordering that
// matters is enforced by waiting for an atomic's return (s_waitcnt) before the next one:
//  * a slice's key max is performed before its arrive/done increment is issued;
//  * the last slice (the one whose done increment returns nchunks-1) reads the key after
//    that increment returned, so it sees every slice's max.
// Any key value read earlier is a real candidate's key, hence always a valid pruning bound.
__device__ __forceinline__ unsigned long long ld_relaxed_u64(unsigned long long* p) {
  return __hip_atomic_load(p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ unsigned int ld_relaxed_u32(unsigned int* p) {
  return __hip_atomic_load(p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ unsigned long long amax_u64(unsigned long long* p, unsigned long long v) {
  return __hip_atomic_fetch_max(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ unsigned int aadd_u32(unsigned int* p, unsigned int v) {
  return __hip_atomic_fetch_add(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ void wait_vmem() { asm volatile("s_waitcnt vmcnt(0)" ::: "memory"); }

constexpr int QCAP = 128;  // per-wave survivor queue (entries)

__global__ void __launch_bounds__(SMP_THREADS) gumbel_argmax_kernel(SmpArgs a) {
  __shared__ unsigned long long red[SMP_THREADS / 64];
  __shared__ float qx[SMP_THREADS / 64][QCAP];
  __shared__ uint32_t qv[SMP_THREADS / 64][QCAP];
  __shared__ unsigned long long row_best;

  const int row = blockIdx.y;
  const int chunk = blockIdx.x;
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const float* rowp = a.logits + (int64_t)row * a.ld;
  const int base = chunk * SMP_CHUNK;
  const RowParams p = row_params(a, row);
  const float NEG_INF = -__builtin_inff();

  // ---- load 32 logits per thread (element e of load i sits at base + (i*256 + tid)*4 + e)
  float x[SMP_EPT];
  if (a.vec && base + SMP_CHUNK <= a.V) {
#pragma unroll
    for (int i = 0; i < SMP_EPT / 4; ++i) {
      v4f t = __builtin_nontemporal_load((const v4f*)(rowp + base + (i * SMP_THREADS + tid) * 4));
      x[4 * i + 0] = t.x;
      x[4 * i + 1] = t.y;
      x[4 * i + 2] = t.z;
      x[4 * i + 3] = t.w;
    }
  } else {
#pragma unroll
    for (int i = 0; i < SMP_EPT / 4; ++i)
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        int v = base + (i * SMP_THREADS + tid) * 4 + e;
        x[4 * i + e] = (v < a.V) ? rowp[v] : NEG_INF;
      }
  }
  auto vidx = [&](int q) -> uint32_t { return (uint32_t)(base + ((q >> 2) * SMP_THREADS + tid) * 4 + (q & 3)); };
  auto valid = [&](int q) -> bool { return (int)vidx(q) < a.V; };
  auto admissible = [&](int q) -> bool { return !(p.has_thr && !(x[q] >= p.thr)); };

  unsigned long long best = 0ull;  // below every real key
  if (p.greedy) {
#pragma unroll
    for (int q = 0; q < SMP_EPT; ++q) {
      if (!valid(q)) continue;
      float y = admissible(q) ? x[q] : NEG_INF;
      unsigned long long k = make_key(y, vidx(q));
      best = (k > best) ? k : best;
    }
  } else {
    // 1) each thread scores its largest admissible raw logit (ties -> smallest index);
    //    inadmissible elements still compete as -inf, as in the reference's masking
    int qm = -1;
    float xm = NEG_INF;
#pragma unroll
    for (int q = 0; q < SMP_EPT; ++q) {
      if (!valid(q)) continue;
      if (!admissible(q)) {
        unsigned long long k = make_key(NEG_INF, vidx(q));
        best = (k > best) ? k : best;
      } else if (qm < 0 || x[q] > xm) {
        qm = q;
        xm = x[q];
      }
    }
    if (qm >= 0) {
      unsigned long long k = make_key(score(p, xm, vidx(qm)), vidx(qm));
      best = (k > best) ? k : best;
    }
    // 2) publish this slice's best to the row; wait (bounded) until every slice of the
    //    row has published, so the pruning bound below is the row-wide one.  The wait
    //    only affects speed: the pruning is exact with whatever bound is visible.
    unsigned long long wb = wave_max_u64(best);
    if (lane == 0) red[wave] = wb;
    __syncthreads();
    if (tid == 0) {
      unsigned long long gb = red[0];
#pragma unroll
      for (int w = 1; w < SMP_THREADS / 64; ++w) gb = (red[w] > gb) ? red[w] : gb;
      amax_u64(&a.keys[row], gb);
      wait_vmem();
      aadd_u32(&a.arrive[row], 1u);
      const uint64_t t0 = wall_clock64();
      while (ld_relaxed_u32(&a.arrive[row]) < (unsigned int)a.nchunks && wall_clock64() - t0 < a.wait_ticks)
        __builtin_amdgcn_s_sleep(8);
      row_best = ld_relaxed_u64(&a.keys[row]);
    }
    __syncthreads();
    const unsigned long long lk = row_best;
    const float L = from_orderable((uint32_t)(lk >> 32));
    // 3) raw-logit cutoff xc with fl(fl(xc/T) + GUMBEL_MAX) < L; elements with x <= xc
    //    cannot reach L (G <= GUMBEL_MAX for every Philox word; rounding is monotone)
    float xc = NEG_INF;
    if (L > NEG_INF && L == L) {
      float c = (L - GUMBEL_MAX) * p.T;
      for (int it = 0; it < 16; ++it) {
        if ((c / p.T) + GUMBEL_MAX < L) {
          xc = c;
          break;
        }
        c = c - fmaxf(fabsf(c) * 4.76837158e-7f, 1e-30f);
      }
    }
    // 4) score the survivors through a per-wave queue: full 64-lane batches of Philox work
    //    instead of mostly-masked lanes
    int qn = 0;
#pragma unroll
    for (int q = 0; q < SMP_EPT; ++q) {
      const bool s = valid(q) && q != qm && admissible(q) && !(x[q] <= xc);
      const unsigned long long m = __ballot(s);
      if (m == 0ull) continue;
      const int pos = qn + __popcll(m & ((1ull << lane) - 1ull));
      if (s) {
        qx[wave][pos] = x[q];
        qv[wave][pos] = vidx(q);
      }
      qn += __popcll(m);
      __builtin_amdgcn_wave_barrier();
      if (qn >= 64) {
        const float xv = qx[wave][lane];
        const uint32_t v = qv[wave][lane];
        const float xr = (qn - 64 > lane) ? qx[wave][64 + lane] : 0.f;
        const uint32_t vr = (qn - 64 > lane) ? qv[wave][64 + lane] : 0u;
        __builtin_amdgcn_wave_barrier();
        if (qn - 64 > lane) {
          qx[wave][lane] = xr;
          qv[wave][lane] = vr;
        }
        qn -= 64;
        const unsigned long long k = make_key(score(p, xv, v), v);
        best = (k > best) ? k : best;
        __builtin_amdgcn_wave_barrier();
      }
    }
    if (lane < qn) {
      const float xv = qx[wave][lane];
      const uint32_t v = qv[wave][lane];
      const unsigned long long k = make_key(score(p, xv, v), v);
      best = (k > best) ? k : best;
    }
  }

  // ---- workgroup reduce, merge into the row, last slice writes the token and resets
  unsigned long long wb = wave_max_u64(best);
  if (lane == 0) red[wave] = wb;
  __syncthreads();
  if (tid == 0) {
    unsigned long long gb = red[0];
#pragma unroll
    for (int w = 1; w < SMP_THREADS / 64; ++w) gb = (red[w] > gb) ? red[w] : gb;
    amax_u64(&a.keys[row], gb);
    wait_vmem();
    unsigned int d = aadd_u32(&a.done[row], 1u);
    if (d == (unsigned int)(a.nchunks - 1)) {
      // every other slice's max was performed before its done increment
      unsigned long long k = amax_u64(&a.keys[row], 0ull);
      a.out[row] = (int64_t)(~(uint32_t)(k & 0xFFFFFFFFull));
      __hip_atomic_store(&a.keys[row], 0ull, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      __hip_atomic_store(&a.arrive[row], 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      __hip_atomic_store(&a.done[row], 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    }
  }
}

// Debug kernel: y for every element.
__global__ void gumbel_scores_kernel(SmpArgs a) {
  const int row = blockIdx.y;
  const RowParams p = row_params(a, row);
  const float* rowp = a.logits + (int64_t)row * a.ld;
  for (int v = blockIdx.x * blockDim.x + threadIdx.x; v < a.V; v += gridDim.x * blockDim.x)
    a.scores[(int64_t)row * a.V + v] = score(p, rowp[v], (uint32_t)v);
}

}  // namespace vqk

using namespace vqk;

extern "C" int64_t vqk_gumbel_workspace_size(int64_t B) {
  if (B < 0) return 0;
  return B * (int64_t)(sizeof(unsigned long long) + 2 * sizeof(unsigned int)) + 16;
}

// Wall-clock ticks per microsecond of the current device (the counter wall_clock64 reads).
static uint64_t ticks_per_us() {
  static thread_local int dev_cached = -1;
  static thread_local uint64_t tpu = 100;
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess) return tpu;
  if (dev != dev_cached) {
    int khz = 0;
    if (hipDeviceGetAttribute(&khz, hipDeviceAttributeWallClockRate, dev) == hipSuccess && khz > 0)
      tpu = (uint64_t)khz / 1000u;
    if (tpu == 0) tpu = 1;
    dev_cached = dev;
  }
  return tpu;
}

static int smp_check(const float* logits, int64_t ld, int64_t B, int64_t V, const void* seeds) {
  if (!logits || B < 0 || V < 1 || ld < V) return VQK_EINVAL;
  if (B > 65535 || V > (int64_t)INT32_MAX - SMP_CHUNK) return VQK_EUNSUPPORTED;
  if (!seeds) return VQK_EINVAL;
  return VQK_OK;
}

extern "C" int vqk_gumbel_argmax(const float* logits, int64_t ld, int64_t B, int64_t V, const float* temp,
                                 const void* seeds, int seed_is_64bit, const float* topk_thr, int64_t* out,
                                 void* workspace, int64_t ws_bytes, vqk_stream_t stream) {
  int rc = vqk_device_check();
  if (rc) return rc;
  rc = smp_check(logits, ld, B, V, seeds);
  if (rc) return rc;
  if (!out || !workspace) return VQK_EINVAL;
  if (B == 0) return VQK_OK;
  if (ws_bytes < vqk_gumbel_workspace_size(B)) return VQK_EWORKSPACE;
  if (((uintptr_t)workspace & 7) != 0) return VQK_EINVAL;
  SmpArgs a = {};
  a.logits = logits;
  a.ld = ld;
  a.B = (int)B;
  a.V = (int)V;
  a.temp = temp;
  a.seeds = seeds;
  a.seed64 = seed_is_64bit ? 1 : 0;
  a.thr = topk_thr;
  a.out = out;
  a.keys = (unsigned long long*)workspace;
  a.arrive = (unsigned int*)((char*)workspace + B * sizeof(unsigned long long));
  a.done = a.arrive + B;
  a.wait_ticks = 8 * ticks_per_us();
  a.nchunks = (int)((V + SMP_CHUNK - 1) / SMP_CHUNK);
  a.vec = (((uintptr_t)logits & 15) == 0 && (ld % 4) == 0) ? 1 : 0;
  hipLaunchKernelGGL(gumbel_argmax_kernel, dim3(a.nchunks, (unsigned)B), dim3(SMP_THREADS), 0,
                     (hipStream_t)stream, a);
  hipError_t e = hipGetLastError();
  return e == hipSuccess ? VQK_OK : (int)e;
}

extern "C" int vqk_gumbel_scores(const float* logits, int64_t ld, int64_t B, int64_t V, const float* temp,
                                 const void* seeds, int seed_is_64bit, const float* topk_thr, float* scores,
                                 vqk_stream_t stream) {
  int rc = vqk_device_check();
  if (rc) return rc;
  rc = smp_check(logits, ld, B, V, seeds);
  if (rc) return rc;
  if (!scores) return VQK_EINVAL;
  if (B == 0) return VQK_OK;
  SmpArgs a = {};
  a.logits = logits;
  a.ld = ld;
  a.B = (int)B;
  a.V = (int)V;
  a.temp = temp;
  a.seeds = seeds;
  a.seed64 = seed_is_64bit ? 1 : 0;
  a.thr = topk_thr;
  a.scores = scores;
  int gx = (int)((V + 255) / 256);
  if (gx > 1024) gx = 1024;
  hipLaunchKernelGGL(gumbel_scores_kernel, dim3(gx, (unsigned)B), dim3(256), 0, (hipStream_t)stream, a);
  hipError_t e = hipGetLastError();
  return e == hipSuccess ? VQK_OK : (int)e;
}
