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
// Design (MI355X).  The Philox + two logs cost ~140 VALU instructions per element, so
// scoring every element of a [32, 248320] batch is ALU-bound (~30 us).  The kernel prunes
// exactly instead: the noise is bounded (G <= GUMBEL_MAX for every Philox word), so once a
// row's winner is known to be >= L, every element with fl(fl(x/T) + GUMBEL_MAX) < L is out.
// A good L needs the whole row, so the work is three launches with no spinning or
// cross-workgroup waits:
//   1. gumbel_cand_kernel streams the logits (256 threads x 64 floats per workgroup,
//      coalesced 16-byte loads); greedy rows take their argmax here; sampled rows score
//      one candidate per thread (its largest raw logit); each workgroup publishes its best
//      with one 64-bit atomicMax on (orderable(y) << 32 | ~v) - largest y, then smallest v;
//   2. gumbel_surv_kernel re-reads the sampled rows (recently streamed, so mostly served by
//      the 256 MB last-level cache) in small slices, drops everything under the row's
//      cutoff with one compare and scores the survivors through a per-workgroup LDS
//      queue, 64 per wave-step;
//   3. gumbel_finish_kernel turns each row key into the token and clears it.
// On the BASELINE logits about 19% of the sampled elements of a B=32 batch survive, almost
// all of them in the rows with the highest temperatures.
#include <hip/hip_runtime.h>
#include <stdint.h>

#include "vqk.h"
#include "vqk_internal.h"
#include "vqk_math.h"

namespace vqk {

typedef float v4f __attribute__((ext_vector_type(4)));

constexpr int SMP_THREADS = 256;
constexpr int SMP_EPT = 64;                               // elements per thread
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
  uint32_t* bkeys;           // [B, nblk] orderable key of each 1024-logit block's largest
                             // admissible logit (0: none)
  int nblk;
  int nchunks;
  int vec;                   // 16-byte loads allowed
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
// (buffer_wbl2 / buffer_inv), which costs far more than the whole reduction.  The ordering
// that matters is the one between launches, which the launch boundaries give: every atomic
// of a launch is performed before the next launch reads the keys.
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


__device__ __forceinline__ unsigned long long block_max_u64(unsigned long long k, unsigned long long* red) {
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  k = wave_max_u64(k);
  if (lane == 0) red[wave] = k;
  __syncthreads();
  unsigned long long r = red[0];
#pragma unroll
  for (int w = 1; w < SMP_THREADS / 64; ++w) r = (red[w] > r) ? red[w] : r;
  return r;
}

// Branch-free running maximum on the order-preserving key (so NaN is the largest and
// -0.0 == +0.0); a strict compare keeps the first, i.e. smallest, index.
__device__ __forceinline__ void take_max(uint32_t k, int q, uint32_t& km, int& qm) {
  const bool b = k > km;
  km = b ? k : km;
  qm = b ? q : qm;
}

// One thread's 64 logits of a slice, all loads issued before any is used.  Full slices
// (16-byte aligned rows) take sixteen 16-byte loads; the row's last, ragged slice (or an
// unaligned row) takes clamped scalar loads, always in bounds, masked by the caller.  The
// two forms sit in separate branches around the whole batch of loads: a data-dependent
// choice per load would make the compiler wait for each load before issuing the next.
__device__ __forceinline__ int slice_v(int base, int tid, int q) {
  return base + ((q >> 2) * SMP_THREADS + tid) * 4 + (q & 3);
}
__device__ __forceinline__ void load_slice(const float* rowp, int base, int tid, int V, bool full,
                                           float (&xv)[SMP_EPT]) {
  if (full) {
#pragma unroll
    for (int i = 0; i < SMP_EPT / 4; ++i) {
      const v4f t = *(const v4f*)(rowp + base + (i * SMP_THREADS + tid) * 4);
      xv[4 * i] = t.x;
      xv[4 * i + 1] = t.y;
      xv[4 * i + 2] = t.z;
      xv[4 * i + 3] = t.w;
    }
  } else {
#pragma unroll
    for (int q = 0; q < SMP_EPT; ++q) {
      const int v = slice_v(base, tid, q);
      xv[q] = rowp[v < V ? v : V - 1];
    }
  }
}

// Launch 1 (streams every logit once): 256 threads x 64 floats per workgroup.  Greedy rows:
// each thread keeps its argmax of y = (admissible ? x : -inf).  Sampled rows: each thread
// keeps its largest admissible raw logit and scores it (one Philox per 64 elements); a thread
// with no admissible element offers its first element as -inf.  The workgroup's best key goes
// to the row with one fire-and-forget 64-bit atomicMax.
__global__ void __launch_bounds__(SMP_THREADS) gumbel_cand_kernel(SmpArgs a) {
  __shared__ unsigned long long red[SMP_THREADS / 64];
  __shared__ uint32_t bred[SMP_THREADS / 64][16];
  const int row = blockIdx.y, tid = threadIdx.x, lane = tid & 63;
  const float* rowp = a.logits + (int64_t)row * a.ld;
  const int base = blockIdx.x * SMP_CHUNK;
  const bool full = a.vec && base + SMP_CHUNK <= a.V;
  float xv[SMP_EPT];
  load_slice(rowp, base, tid, a.V, full, xv);
  const RowParams p = row_params(a, row);
  const float NEG_INF = -__builtin_inff();
  const float thr = p.has_thr ? p.thr : NEG_INF;  // x < thr is masked (NaN is not)
  // One pass: the thread's best key (greedy: y itself; sampled: the raw logit, which ranks
  // the candidates) and the best key of each of its 16 element groups (group i of every
  // thread is 1024-logit block i of the slice).  Inadmissible elements count as -inf, out
  // of range ones as key 0, below every real key.
  uint32_t km = 0u;
  int qm = -1;
  uint32_t mb[16];
  bool slow = !full;
  if (full) {
    // Fast form in float compares: strict > keeps the first index and treats -0 == +0;
    // NaN (which must rank above everything) only raises a flag that sends the thread to
    // the key form below.
    float m = NEG_INF, mf[16];
    int qf = 0;
    bool nan = false;
#pragma unroll
    for (int i = 0; i < 16; ++i) mf[i] = NEG_INF;
#pragma unroll
    for (int q = 0; q < SMP_EPT; ++q) {
      const float x = xv[q] < thr ? NEG_INF : xv[q];
      nan = nan || (x != x);
      const bool b = x > m;
      m = b ? x : m;
      qf = b ? q : qf;
      mf[q >> 2] = fmaxf(mf[q >> 2], x);
    }
    if (!nan) {
      km = orderable(m);
      qm = qf;
#pragma unroll
      for (int i = 0; i < 16; ++i) mb[i] = orderable(mf[i]);
    }
    slow = nan;
  }
  if (slow) {
    // Key form: orderable keys (NaN on top); out-of-range elements are key 0.
    km = 0u;
    qm = -1;
#pragma unroll
    for (int i = 0; i < 16; ++i) mb[i] = 0u;
#pragma unroll
    for (int q = 0; q < SMP_EPT; ++q) {
      const uint32_t k = slice_v(base, tid, q) < a.V ? orderable(xv[q] < thr ? NEG_INF : xv[q]) : 0u;
      take_max(k, q, km, qm);
      mb[q >> 2] = k > mb[q >> 2] ? k : mb[q >> 2];
    }
  }
  unsigned long long best = 0ull;
  if (qm >= 0) {
    const uint32_t v = (uint32_t)slice_v(base, tid, qm);
    float y = from_orderable(km);
    if (!p.greedy && y > NEG_INF) y = score(p, y, v);
    best = make_key(y, v);
  }
  if (!p.greedy) {
    // Block maxima for the survivor pass.  A butterfly that halves the values at each of
    // its first four steps leaves lane l with the wave's maximum of block (l >> 2) & 15.
#pragma unroll
    for (int step = 0; step < 4; ++step) {
      const int half = 8 >> step, bit = 32 >> step;
      const bool up = (lane & bit) != 0;
#pragma unroll
      for (int j = 0; j < half; ++j) {
        const uint32_t send = up ? mb[j] : mb[j + half];
        const uint32_t keep = up ? mb[j + half] : mb[j];
        const uint32_t got = (uint32_t)__shfl_xor((int)send, bit);
        mb[j] = got > keep ? got : keep;
      }
    }
#pragma unroll
    for (int bit = 2; bit >= 1; bit >>= 1) {
      const uint32_t got = (uint32_t)__shfl_xor((int)mb[0], bit);
      mb[0] = got > mb[0] ? got : mb[0];
    }
    if ((lane & 3) == 0) bred[tid >> 6][lane >> 2] = mb[0];
    __syncthreads();
    const int blk = blockIdx.x * 16 + tid;
    if (tid < 16 && blk < a.nblk) {
      uint32_t k = bred[0][tid];
#pragma unroll
      for (int w = 1; w < SMP_THREADS / 64; ++w) k = bred[w][tid] > k ? bred[w][tid] : k;
      a.bkeys[(int64_t)row * a.nblk + blk] = k;
    }
  }
  const unsigned long long gb = block_max_u64(best, red);
  if (tid == 0) amax_u64(&a.keys[row], gb);
}

// Launch 2 (sampled rows only; greedy rows return at once).  The row key holds every
// candidate, a score L the winner is >= to.  Since G <= GUMBEL_MAX for every Philox word
// and rounding is monotone, x with fl(fl(x/T) + GUMBEL_MAX) < L cannot win; the test is
// one compare against a per-row raw-logit cutoff; whole 1024-logit blocks whose largest
// admissible logit is under the cutoff are skipped unread.  Survivors cluster in the rows
// with high temperature, so this pass uses small slices (EPT elements per thread): many
// short workgroups let the dispatcher spread one hot row over every CU.  A workgroup
// touches the row key only if it found a better score than L, which is rare.

template <int EPT>
__global__ void __launch_bounds__(SMP_THREADS) gumbel_surv_kernel(SmpArgs a) {
  constexpr int CAP = SMP_THREADS * EPT;  // every element of the slice may survive
  __shared__ unsigned long long red[SMP_THREADS / 64];
  __shared__ float qx[CAP];
  __shared__ uint32_t qv[CAP];
  __shared__ int qn;
  const int row = blockIdx.y, tid = threadIdx.x, lane = tid & 63;
  // every per-row and per-block value this workgroup needs is loaded at once, so the
  // decision to skip costs one memory latency
  constexpr int NB = EPT / 4;  // 1024-logit blocks per slice
  const unsigned long long lk = ld_relaxed_u64(&a.keys[row]);
  uint32_t bk[NB];
#pragma unroll
  for (int i = 0; i < NB; ++i) {
    const int blk = blockIdx.x * NB + i;
    bk[i] = blk < a.nblk ? a.bkeys[(int64_t)row * a.nblk + blk] : 0u;
  }
  const RowParams p = row_params(a, row);
  if (p.greedy) return;
  const float NEG_INF = -__builtin_inff();
  const float L = from_orderable((uint32_t)(lk >> 32));
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
  // skip the slice without reading it when no block of it has an admissible logit > xc
  // (wave-uniform: every thread reads the same keys)
  {
    bool any = false;
#pragma unroll
    for (int i = 0; i < NB; ++i) any = any || (bk[i] != 0u && !(from_orderable(bk[i]) <= xc));
    if (!any) return;
  }
  const float* rowp = a.logits + (int64_t)row * a.ld;
  const int base = blockIdx.x * (SMP_THREADS * EPT);
  const bool full = a.vec && base + SMP_THREADS * EPT <= a.V;
  float xv[EPT];
  if (full) {
#pragma unroll
    for (int i = 0; i < EPT / 4; ++i) {
      const v4f t = *(const v4f*)(rowp + base + (i * SMP_THREADS + tid) * 4);
      xv[4 * i] = t.x;
      xv[4 * i + 1] = t.y;
      xv[4 * i + 2] = t.z;
      xv[4 * i + 3] = t.w;
    }
  } else {
#pragma unroll
    for (int q = 0; q < EPT; ++q) {
      const int v = base + ((q >> 2) * SMP_THREADS + tid) * 4 + (q & 3);
      xv[q] = rowp[v < a.V ? v : a.V - 1];
    }
  }
  // Survivors of the whole workgroup go to one LDS queue (one LDS atomic per wave and
  // element step reserves the wave's run), then every thread scores queue entries tid,
  // tid + 256, ...: n survivors cost ceil(n / 64) wave-scores however they are spread.
  if (tid == 0) qn = 0;
  __syncthreads();
#pragma unroll
  for (int q = 0; q < EPT; ++q) {
    const int v = base + ((q >> 2) * SMP_THREADS + tid) * 4 + (q & 3);
    const bool s = v < a.V && !(p.has_thr && !(xv[q] >= p.thr)) && !(xv[q] <= xc);
    const unsigned long long m = __ballot(s);
    if (m) {
      int wbase = 0;
      if (lane == 0)
        wbase = __hip_atomic_fetch_add(&qn, (int)__popcll(m), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
      wbase = __shfl(wbase, 0);
      if (s) {
        const int pos = wbase + (int)__popcll(m & ((1ull << lane) - 1ull));
        qx[pos] = xv[q];
        qv[pos] = (uint32_t)v;
      }
    }
  }
  __syncthreads();
  const int n = qn;
  unsigned long long best = 0ull;
  for (int i = tid; i < n; i += SMP_THREADS) {
    const float x = qx[i];
    const uint32_t v = qv[i];
    const unsigned long long k = make_key(score(p, x, v), v);
    best = (k > best) ? k : best;
  }
  const unsigned long long gb = block_max_u64(best, red);
  if (tid == 0 && gb > lk) amax_u64(&a.keys[row], gb);
}

// Launch 3: the token of each row from its key; the whole workspace (keys and block keys)
// is cleared for the next call, whatever its batch size.
__global__ void gumbel_finish_kernel(SmpArgs a) {
  const int i = blockIdx.x * blockDim.x + threadIdx.x;
  if (i < a.B) {
    const unsigned long long k = ld_relaxed_u64(&a.keys[i]);
    a.out[i] = (int64_t)(~(uint32_t)(k & 0xFFFFFFFFull));
    __hip_atomic_store(&a.keys[i], 0ull, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  }
  if (i < a.B * a.nblk) a.bkeys[i] = 0u;
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

static int64_t gumbel_nblk(int64_t V) { return (V + 1023) / 1024; }

extern "C" int64_t vqk_gumbel_workspace_size(int64_t B, int64_t V) {
  if (B < 0 || V < 0) return 0;
  return B * (int64_t)sizeof(unsigned long long) + B * gumbel_nblk(V) * (int64_t)sizeof(uint32_t) + 16;
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
  if (ws_bytes < vqk_gumbel_workspace_size(B, V)) return VQK_EWORKSPACE;
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
  a.bkeys = (uint32_t*)((char*)workspace + B * sizeof(unsigned long long));
  a.nblk = (int)gumbel_nblk(V);
  a.nchunks = (int)((V + SMP_CHUNK - 1) / SMP_CHUNK);
  a.vec = (((uintptr_t)logits & 15) == 0 && (ld % 4) == 0) ? 1 : 0;
  hipLaunchKernelGGL(gumbel_cand_kernel, dim3(a.nchunks, (unsigned)B), dim3(SMP_THREADS), 0,
                     (hipStream_t)stream, a);
  // survivor pass: 1024 logits per workgroup for up to ~8M elements, else 4096
  // survivor slices: 1024 logits per workgroup for small batches (more workgroups to spread
  // a hot row over), 2048 beyond ~2M elements (measured best at B = 32 and 128)
  if (B * V <= ((int64_t)2 << 20)) {
    const int ns = (int)((V + SMP_THREADS * 4 - 1) / (SMP_THREADS * 4));
    hipLaunchKernelGGL(gumbel_surv_kernel<4>, dim3(ns, (unsigned)B), dim3(SMP_THREADS), 0, (hipStream_t)stream, a);
  } else {
    const int ns = (int)((V + SMP_THREADS * 8 - 1) / (SMP_THREADS * 8));
    hipLaunchKernelGGL(gumbel_surv_kernel<8>, dim3(ns, (unsigned)B), dim3(SMP_THREADS), 0, (hipStream_t)stream, a);
  }
  const int64_t nfin = B * (int64_t)a.nblk;
  hipLaunchKernelGGL(gumbel_finish_kernel, dim3((unsigned)((nfin + 255) / 256)), dim3(256), 0, (hipStream_t)stream, a);
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
