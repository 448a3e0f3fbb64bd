// vqk_topk.hip - per-row top-k threshold of [B, V] fp32 logits on the device (gfx950).
//
// Semantics of the reference's _compute_topk_threshold (src/vllm_quant_kernels/_sampler.py:
// 62-93): with max_k = max_b top_k[b], if max_k >= V there is no threshold; otherwise
// thr[b] = the k-th largest raw logit of row b, k = max(top_k[b], 1) (the reference takes
// column clamp(top_k[b], max=max_k) - 1, clamped at 0, of torch.topk(logits, max_k), sorted
// descending, NaN ranked largest).  "No threshold" is written as thr[b] = -inf, which masks
// nothing (the sampler masks x < thr), so the same array always feeds the sampler and no
// host synchronisation is needed (the reference reads max_k with .item()).
//
// Design: selection, not sorting, on order-preserving 32-bit keys (NaN on top, -0 folded
// into +0: both compare equal, so either is the same threshold).
//   1. topk_blockmax_kernel streams the logits once and stores the largest key of every
//      block of bs logits (bs = 64 up to V = 256K, 256 up to 1M), so a row has at most 4096
//      block maxima, which fit LDS.
//   2. topk_select_kernel, one workgroup per row: t0 = the k-th largest block maximum (for
//      k <= 256 the lower edge of its 16-bit key bin) is a lower bound of the answer (k
//      distinct logits are >= that maximum) and every logit >= the answer lies in a block
//      whose maximum is >= t0.  A 4-pass MSB-first 8-bit radix
//      select then runs over the keys >= t0 of those blocks only (collected into LDS on the
//      first pass when they fit, else re-read from memory each pass, 16 loads in flight per
//      thread).  For k up to the number of blocks that is a few times k keys per row;
//      larger k (or rows of more than 4096 blocks) fall back to t0 = the smallest key,
//      i.e. four passes over the whole row.
#include <hip/hip_runtime.h>
#include <stdint.h>

#include "vqk.h"
#include "vqk_internal.h"
#include "vqk_math.h"

namespace vqk {

constexpr int TK_THREADS = 256;
constexpr int TK_EPW = 4096;         // logits per workgroup in the streaming pass
constexpr int TK_MAX_NBLK = 4096;    // block maxima per row the select kernel keeps in LDS
constexpr int TK_CAP = 6144;         // candidate keys collected in LDS
constexpr int TK_U = 16;             // loads in flight per thread in the candidate scan
constexpr int TS_THREADS = 1024;     // threads of the per-row select workgroup

__device__ __forceinline__ uint32_t key_at(const float* rowp, int v) { return orderable(rowp[v]); }

// Pass 1: bmax[row][blk] = largest key of logits [blk*BS, blk*BS+BS) of the row.  Each
// thread takes 4 consecutive logits per step; the BS/4 lanes of a block reduce by xor
// exchanges (BS = 64 or 256, so a block never straddles waves).
template <int BS>
__global__ void __launch_bounds__(TK_THREADS) topk_blockmax_kernel(const float* logits, int64_t ld, int V,
                                                                   int nblk, int vec, uint32_t* bmax) {
  const int row = blockIdx.y, tid = threadIdx.x;
  const float* rowp = logits + (int64_t)row * ld;
#pragma unroll
  for (int it = 0; it < TK_EPW / (4 * TK_THREADS); ++it) {
    const int base = blockIdx.x * TK_EPW + it * 4 * TK_THREADS + 4 * tid;
    uint32_t k = 0u;
    if (vec && base + 4 <= V) {
      const float4 t = *(const float4*)(rowp + base);
      k = max(max(orderable(t.x), orderable(t.y)), max(orderable(t.z), orderable(t.w)));
    } else {
#pragma unroll
      for (int e = 0; e < 4; ++e)
        if (base + e < V) k = max(k, key_at(rowp, base + e));
    }
#pragma unroll
    for (int off = 1; off < BS / 4; off <<= 1) k = max(k, (uint32_t)__shfl_xor((int)k, off));
    const int blk = base / BS;
    if ((tid & (BS / 4 - 1)) == 0 && blk < nblk) bmax[(int64_t)row * nblk + blk] = k;
  }
}

// Digit selection of one radix pass (the caller has synchronised after filling hist):
// hist[0..255] holds the counts of the remaining candidates by digit; sets sh[0] to the
// digit d holding the rem-th largest and sh[1] to the count of candidates with a larger
// digit.  Wave 0 alone scans (lane l owns digits 4l..4l+3): one barrier, not a
// workgroup-wide scan.
__device__ __forceinline__ void pick_digit(const int* hist, int rem, int* sh) {
  const int l = threadIdx.x;
  if (l < 64) {
    const int h0 = hist[4 * l], h1 = hist[4 * l + 1], h2 = hist[4 * l + 2], h3 = hist[4 * l + 3];
    const int mine = h0 + h1 + h2 + h3;
    int incl = mine;  // inclusive suffix sum over lanes >= l
#pragma unroll
    for (int off = 1; off < 64; off <<= 1) {
      const int o = __shfl_down(incl, off);
      if (l + off < 64) incl += o;
    }
    const int s4 = incl - mine;  // candidates with a digit above 4l+3
    const int s3 = s4 + h3, s2 = s3 + h2, s1 = s2 + h1, s0 = s1 + h0;
    if (s4 < rem && s3 >= rem) { sh[0] = 4 * l + 3; sh[1] = s4; }
    if (s3 < rem && s2 >= rem) { sh[0] = 4 * l + 2; sh[1] = s3; }
    if (s2 < rem && s1 >= rem) { sh[0] = 4 * l + 1; sh[1] = s2; }
    if (s1 < rem && s0 >= rem) { sh[0] = 4 * l; sh[1] = s1; }
  }
  __syncthreads();
}

// Pass 2: one workgroup per row.
__global__ void __launch_bounds__(TS_THREADS) topk_select_kernel(const float* logits, int64_t ld, int B, int V,
                                                                 int nblk, int bs, const void* top_k,
                                                                 int topk64, const uint32_t* bmax, float* thr) {
  __shared__ uint32_t sb[TK_MAX_NBLK];     // block maxima of the row
  __shared__ int cblk[TK_MAX_NBLK];        // blocks whose maximum is >= t0
  __shared__ uint32_t ckey[TK_CAP];        // candidate keys (when they fit)
  __shared__ int hist[256];
  __shared__ int sh[4];
  __shared__ long long smk[TS_THREADS / 64];
  const int row = blockIdx.x, tid = threadIdx.x;
  auto topk_at = [&](int b) -> int64_t {
    return topk64 ? ((const int64_t*)top_k)[b] : (int64_t)((const int32_t*)top_k)[b];
  };
  // the reference's "all rows disabled" test, max over the whole batch
  int64_t mk = INT64_MIN;
  for (int b = tid; b < B; b += TS_THREADS) {
    const int64_t t = topk_at(b);
    mk = t > mk ? t : mk;
  }
#pragma unroll
  for (int off = 32; off > 0; off >>= 1) {
    const int64_t o = __shfl_xor(mk, off);
    mk = o > mk ? o : mk;
  }
  if ((tid & 63) == 0) smk[tid >> 6] = mk;
  __syncthreads();
  mk = smk[0];
  for (int w = 1; w < TS_THREADS / 64; ++w) mk = mk > smk[w] ? mk : smk[w];
  if (mk >= (int64_t)V) {
    if (tid == 0) thr[row] = -__builtin_inff();
    return;
  }
  const int64_t kk = topk_at(row);
  const int k = (int)(kk < 1 ? 1 : kk);  // k < V here
  const float* rowp = logits + (int64_t)row * ld;

  // t0: the k-th largest block maximum or the 16-bit bin edge below it (0, the smallest
  // key, when k exceeds the blocks or the row has more blocks than LDS holds)
  uint32_t t0 = 0u;
  int nb = nblk;
  const bool fit = nblk <= TK_MAX_NBLK;
  if (fit) {
    {
      // every load issued before any is stored (one memory latency, not one per step)
      uint32_t t[TK_MAX_NBLK / TS_THREADS];
#pragma unroll
      for (int r = 0; r < TK_MAX_NBLK / TS_THREADS; ++r) {
        const int i = r * TS_THREADS + tid;
        t[r] = bmax[(int64_t)row * nblk + (i < nblk ? i : nblk - 1)];
      }
#pragma unroll
      for (int r = 0; r < TK_MAX_NBLK / TS_THREADS; ++r)
        if (r * TS_THREADS + tid < nblk) sb[r * TS_THREADS + tid] = t[r];
    }
    __syncthreads();
    if (k <= nblk) {
      uint32_t prefix = 0u, mask = 0u;
      int rem = k;
      // t0 only has to be a lower bound of the answer: for k <= 256 the lower edge of the
      // 16-bit key bin that holds the k-th largest block maximum serves (the bin spans 2^-7
      // of the value, so it adds a few candidate blocks and saves two passes: k = 50
      // 23.4 -> 21.8 us); larger k, whose candidates are re-read from memory each pass,
      // take the exact maximum (four passes).
      const int last = k <= 256 ? 16 : 0;
      for (int shift = 24; shift >= last; shift -= 8) {
        if (tid < 256) hist[tid] = 0;
        __syncthreads();
        for (int i = tid; i < nblk; i += TS_THREADS) {
          const uint32_t key = sb[i];
          if ((key & mask) == prefix) atomicAdd(&hist[(key >> shift) & 255], 1);
        }
        __syncthreads();
        pick_digit(hist, rem, sh);
        prefix |= (uint32_t)sh[0] << shift;
        mask |= 0xFFu << shift;
        rem -= sh[1];
        __syncthreads();
      }
      t0 = prefix;
    }
    // the candidate blocks (any order)
    if (tid == 0) sh[2] = 0;
    __syncthreads();
    for (int i = tid; i < nblk; i += TS_THREADS)
      if (sb[i] >= t0) cblk[atomicAdd(&sh[2], 1)] = i;
    __syncthreads();
    nb = sh[2];
  }
  const int64_t total = (int64_t)nb * bs;

  // radix select over the keys >= t0 of the candidate blocks
  uint32_t prefix = 0u, mask = 0u;
  int rem = k;
  bool in_lds = false;
  int nkey = 0;
  for (int shift = 24; shift >= 0; shift -= 8) {
    if (tid < 256) hist[tid] = 0;
    if (tid == 0) sh[3] = 0;
    __syncthreads();
    if (in_lds) {
      for (int i = tid; i < nkey; i += TS_THREADS) {
        const uint32_t key = ckey[i];
        if ((key & mask) == prefix) atomicAdd(&hist[(key >> shift) & 255], 1);
      }
    } else {
      const bool collect = shift == 24;
      for (int64_t i0 = 0; i0 < total; i0 += (int64_t)TK_U * TS_THREADS) {
        // all loads of the step first, then their use
        uint32_t kv[TK_U];
#pragma unroll
        for (int u = 0; u < TK_U; ++u) {
          const int64_t i = i0 + u * TS_THREADS + tid;
          int v = V;
          if (i < total) {
            const int j = (int)(i / bs), e = (int)(i - (int64_t)j * bs);
            v = (fit ? cblk[j] : j) * bs + e;
          }
          const uint32_t key = key_at(rowp, v < V ? v : V - 1);  // unconditional load
          kv[u] = v < V ? key : 0u;
        }
#pragma unroll
        for (int u = 0; u < TK_U; ++u) {
          const int64_t i = i0 + u * TS_THREADS + tid;
          const uint32_t key = kv[u];
          const bool c = i < total && key >= t0 && (key & mask) == prefix;
          if (c) atomicAdd(&hist[(key >> shift) & 255], 1);
          if (collect) {
            // one LDS atomic per wave reserves the run of its candidates
            const unsigned long long m = __ballot(c);
            if (m) {
              int base = 0;
              if ((tid & 63) == 0) base = atomicAdd(&sh[3], (int)__popcll(m));
              base = __shfl(base, 0);
              const int p = base + (int)__popcll(m & ((1ull << (tid & 63)) - 1ull));
              if (c && p < TK_CAP) ckey[p] = key;
            }
          }
        }
      }
    }
    __syncthreads();
    if (shift == 24) {
      nkey = sh[3];
      in_lds = nkey <= TK_CAP;
    }
    pick_digit(hist, rem, sh);
    prefix |= (uint32_t)sh[0] << shift;
    mask |= 0xFFu << shift;
    rem -= sh[1];
    __syncthreads();
  }
  if (tid == 0) thr[row] = from_orderable(prefix);
}

}  // namespace vqk

using namespace vqk;

// block size of the maxima: 64 logits while the row has at most 4096 such blocks, else 256
static int topk_bs(int64_t V) { return V <= (int64_t)TK_MAX_NBLK * 64 ? 64 : 256; }

extern "C" int64_t vqk_topk_threshold_workspace_size(int64_t B, int64_t V) {
  if (B < 0 || V < 0) return 0;
  const int bs = topk_bs(V);
  return B * ((V + bs - 1) / bs) * (int64_t)sizeof(uint32_t) + 16;
}

extern "C" int vqk_topk_threshold(const float* logits, int64_t ld, int64_t B, int64_t V, const void* top_k,
                                  int top_k_is_64bit, float* thr, void* workspace, int64_t ws_bytes,
                                  vqk_stream_t stream) {
  int rc = vqk_device_check();
  if (rc) return rc;
  if (!logits || !top_k || !thr || !workspace || B < 0 || V < 1 || ld < V) return VQK_EINVAL;
  if (B == 0) return VQK_OK;
  if (B > 65535 || V > (int64_t)INT32_MAX - TK_EPW) return VQK_EUNSUPPORTED;
  if (ws_bytes < vqk_topk_threshold_workspace_size(B, V)) return VQK_EWORKSPACE;
  if (((uintptr_t)workspace & 3) != 0) return VQK_EINVAL;
  const int bs = topk_bs(V);
  const int nblk = (int)((V + bs - 1) / bs);
  const int vec = (((uintptr_t)logits & 15) == 0 && (ld % 4) == 0) ? 1 : 0;
  uint32_t* bmax = (uint32_t*)workspace;
  const dim3 g1((unsigned)((V + TK_EPW - 1) / TK_EPW), (unsigned)B);
  if (bs == 64)
    hipLaunchKernelGGL(topk_blockmax_kernel<64>, g1, dim3(TK_THREADS), 0, (hipStream_t)stream, logits, ld, (int)V,
                       nblk, vec, bmax);
  else
    hipLaunchKernelGGL(topk_blockmax_kernel<256>, g1, dim3(TK_THREADS), 0, (hipStream_t)stream, logits, ld, (int)V,
                       nblk, vec, bmax);
  hipLaunchKernelGGL(topk_select_kernel, dim3((unsigned)B), dim3(TS_THREADS), 0, (hipStream_t)stream, logits, ld,
                     (int)B, (int)V, nblk, bs, top_k, top_k_is_64bit ? 1 : 0, bmax, thr);
  hipError_t e = hipGetLastError();
  return e == hipSuccess ? VQK_OK : (int)e;
}
