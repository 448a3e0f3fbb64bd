// vqk_sampler.hip - Gumbel-argmax sampler over [B, V] fp32 logits (gfx950), in two or three
// launches without workspace initialisation.
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
// Design (MI355X).  The Philox + two logs + division cost over a hundred VALU instructions
// per element, so scoring every element of a [32, 248320] batch is ALU-bound (~30 us).
// The kernels prune exactly instead: the noise is bounded (G <= GUMBEL_MAX for every
// Philox word), so once a row's winner is known to be >= L, every element with
// fl(fl(x/T) + GUMBEL_MAX) < L is out.
// A good L needs the whole row, so batches of more than ~2M logits take three launches
// with no spinning, no cross-workgroup waits and no workspace initialisation:
//   1. gumbel_cand_kernel streams the logits (256 threads x 64 floats per workgroup,
//      coalesced 16-byte loads, about three instructions per element); greedy rows take
//      their argmax here; sampled rows score one candidate per thread (its largest raw
//      logit); each workgroup stores its best key (orderable(y) << 32 | ~v: largest y,
//      then smallest v) and its blocks' largest admissible logits;
//   2. gumbel_surv_kernel re-reads the surviving slices of the sampled rows (recently
//      streamed, so mostly served by the 256 MB last-level cache), skips slices whose blocks
//      all lie under the row's cutoff, drops everything else under it with one compare and
//      scores the survivors through a per-workgroup LDS queue, 64 per wave-step, skipping
//      the logarithms and the division of those whose Philox word alone bounds them below
//      a real score (score_fold);
//   3. gumbel_finish_kernel reduces each row's keys to the token.
// Smaller batches are a few workgroup latencies long, so launches dominate there: they
// take gumbel_local_kernel (one pass, each wave pruned against its own best candidate)
// and the finish.  On the BASELINE logits about a fifth of the sampled elements of a B=32
// batch survive, almost all of them in the rows with the highest temperatures.
#include <hip/hip_runtime.h>
#include <stdint.h>

#include <mutex>

#include "vqk.h"
#include "vqk_internal.h"
#include "vqk_math.h"

namespace vqk {

typedef float v4f __attribute__((ext_vector_type(4)));

// candidate pass: logits per thread (a power of two >= 8; 32 measured within noise, 128 does
// not fit the block-max butterfly's registers); survivor pass: logits per thread (4 and 16
// measured 0.7-6 us slower)
constexpr int SMP_CAND_EPT = 64;
constexpr int SMP_SURV_EPT = 8;
constexpr int SMP_THREADS = 256;
// candidate pass: 64 elements per thread (16 for small batches, which gives more, shorter
// workgroups); its smallest chunk bounds the number of candidate slots per row
constexpr int SMP_MIN_CHUNK = SMP_THREADS * 4;
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
  unsigned long long* ckeys;  // [B, nchunks] best key of each candidate workgroup
  unsigned long long* rkeys;  // [B] survivor pass's row key (cleared by the candidate pass)
  uint32_t* bkeys;            // [B, nblk] orderable key of each 1024-logit block's largest
                              // admissible logit (-inf: none)
  int nblk;
  int nchunks;
  int vec;                   // 16-byte loads allowed
  float* scores;             // debug: write y for every element (scores kernel only)
};

struct RowParams {
  bool greedy;
  float T;
  float rT;  // RN(1/T), for the prune bound only
  uint32_t k0, k1;
  bool has_thr;
  float thr;
};

// Every load is unconditional (an absent operand reads the first logit instead and the
// value is then replaced), so the compiler issues them together behind one wait rather than
// one wait per optional operand.
__device__ __forceinline__ RowParams row_params(const SmpArgs& a, int row) {
  const float* any = a.logits;
  const float t = *(a.temp ? a.temp + row : any);
  const float h = *(a.thr ? a.thr + row : any);
  const uint32_t* sp = (const uint32_t*)a.seeds;
  const uint32_t lo = sp[a.seed64 ? 2 * row : row];
  const uint32_t hi = sp[a.seed64 ? 2 * row + 1 : row];
  RowParams p;
  p.T = a.temp ? t : 1.0f;
  p.rT = 1.0f / p.T;
  p.greedy = a.temp ? (t < GREEDY_EPS) : true;
  p.k0 = lo;
  p.k1 = a.seed64 ? hi : (uint32_t)((int32_t)lo >> 31);  // int32 -> uint64 sign-extends
  p.has_thr = a.thr != nullptr;
  p.thr = p.has_thr ? h : 0.f;
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

// Score of an admissible, non-NaN logit of a sampled row: score() without the masks.
__device__ __forceinline__ float score_sampled(const RowParams& p, float x, uint32_t v) {
  const float a = x / p.T;
  return a + gumbel_from_uniform(philox_uniform(philox_word0(v, p.k0, p.k1)));
}

// Fold an admissible, non-NaN logit of a sampled row into a running (best score, index)
// pair, skipping the exact score when it provably falls below floor or the running best
// (both scores of real elements, so such a logit cannot be the argmax).  The bound needs
// only the Philox word: y = x/T + G(u) <= x*RN(1/T) + gumbel_upper(u) + 1e-5*|x*RN(1/T)|
// (x*RN(1/T) is within 2^-22 relative of x/T; the exact path rounds twice more, each
// well inside the margins).  Survivors of hot rows sit ~10 below the row's best, where
// fewer than 1 in 10^4 Philox words come close, so most skip both logarithms and the
// division.
__device__ __forceinline__ void score_fold(const RowParams& p, float x, uint32_t v, float floor, float& by,
                                           uint32_t& bv) {
  const float u = philox_uniform(philox_word0(v, p.k0, p.k1));
  const float aq = x * p.rT;
  const float yub = aq + gumbel_upper(u) + 1e-5f * fabsf(aq);
  if (yub < fmaxf(floor, by)) return;
  const float y = x / p.T + gumbel_from_uniform(u);
  const bool b = (y > by) || (y == by && v < bv);
  by = b ? y : by;
  bv = b ? v : bv;
}


__device__ __forceinline__ uint32_t wave_max_u32(uint32_t k) {
#pragma unroll
  for (int off = 32; off > 0; off >>= 1) {
    const uint32_t o = (uint32_t)__shfl_xor((int)k, off);
    k = o > k ? o : k;
  }
  return k;
}

__device__ __forceinline__ unsigned long long wave_max_u64(unsigned long long k) {
#pragma unroll
  for (int off = 32; off > 0; off >>= 1) {
    unsigned long long o = __shfl_xor(k, off);
    k = (o > k) ? o : k;
  }
  return k;
}

// Cross-workgroup protocol.  Candidate workgroups store to slots of their own; survivor
// workgroups that beat the candidates use one relaxed device-scope atomicMax on the row
// key (acquire/release fences would write back and invalidate the L2 of the issuing XCD,
// which costs far more than the whole reduction).  The ordering that matters is the one
// between launches, which the launch boundaries give: every store and atomic of a launch
// is performed before the next launch reads them.
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
template <int EPT>
__device__ __forceinline__ void load_slice(const float* rowp, int base, int tid, int V, bool full,
                                           float (&xv)[EPT]) {
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
      const int v = slice_v(base, tid, q);
      xv[q] = rowp[v < V ? v : V - 1];
    }
  }
}

// v_max3_f32 / v_max_f32 as written: fmaxf would first quiet each operand (one more
// instruction per element) for IEEE NaN semantics.  Only NaN-free lanes use these; a lane
// holding a NaN takes the key form.
__device__ __forceinline__ float max3_nn(float a, float b, float c) {
  float r;
  asm("v_max3_f32 %0, %1, %2, %3" : "=v"(r) : "v"(a), "v"(b), "v"(c));
  return r;
}
__device__ __forceinline__ float max_nn(float a, float b) {
  float r;
  asm("v_max_f32 %0, %1, %2" : "=v"(r) : "v"(a), "v"(b));
  return r;
}
// Order-preserving key of a NaN-free float (-0.0 ranks just below +0.0, which no consumer
// of these keys distinguishes).
__device__ __forceinline__ uint32_t orderable_nn(float y) {
  const uint32_t b = bits_f32(y);
  return b ^ ((uint32_t)((int32_t)b >> 31) | 0x80000000u);
}

// Launch 1 (streams every logit once): 256 threads x 64 floats per workgroup.  Each
// thread masks its inadmissible elements (below the top-k threshold, past the row end) to
// -inf and takes, in float arithmetic, the maximum of each 4-element group (its share of
// one 1024-logit block) and of all 64, then the first index holding that maximum: about
// three instructions per element.  A lane with a NaN (which must rank above everything)
// redoes its slice on order-preserving keys instead.  Greedy rows: the thread's best is
// (max, first index).  Sampled rows: the thread scores its largest admissible logit (one
// Philox per 64 elements) and the workgroup also stores the largest admissible logit of
// each of its 16 blocks for the survivor pass.  The workgroup's best key
// (orderable(y) << 32 | ~v: largest y, then smallest v) goes to its own slot: no atomics.
template <int EPT>
__global__ void __launch_bounds__(SMP_THREADS) gumbel_cand_kernel(SmpArgs a) {
  constexpr int CHUNK = SMP_THREADS * EPT;
  constexpr int NB = EPT / 4;                      // 1024-logit blocks per chunk
  constexpr int LOGNB = NB == 16 ? 4 : (NB == 8 ? 3 : (NB == 4 ? 2 : (NB == 2 ? 1 : 0)));
  static_assert((1 << LOGNB) == NB, "EPT / 4 must be a power of two");
  __shared__ unsigned long long red[SMP_THREADS / 64];
  __shared__ uint32_t bred[SMP_THREADS / 64][NB];
  const int row = blockIdx.y, tid = threadIdx.x, lane = tid & 63;
  const float* rowp = a.logits + (int64_t)row * a.ld;
  const int base = blockIdx.x * CHUNK;
  const bool inrange = base + CHUNK <= a.V;
  float xv[EPT];
  load_slice<EPT>(rowp, base, tid, a.V, a.vec && inrange, xv);
  const RowParams p = row_params(a, row);
  // the survivor pass accumulates into the row key; cleared here, one launch ahead of it
  if (blockIdx.x == 0 && tid == 0) a.rkeys[row] = 0ull;
  const float NEG_INF = -__builtin_inff();
  if (p.has_thr) {
#pragma unroll
    for (int q = 0; q < EPT; ++q) xv[q] = xv[q] < p.thr ? NEG_INF : xv[q];  // NaN stays
  }
  if (!inrange) {
#pragma unroll
    for (int q = 0; q < EPT; ++q) xv[q] = slice_v(base, tid, q) < a.V ? xv[q] : NEG_INF;
  }
  // group maxima and the NaN test in load order, so each group waits only for its own load
  bool nan = false;
  float mf[NB];
#pragma unroll
  for (int i = 0; i < NB; ++i) {
    nan |= __builtin_isunordered(xv[4 * i], xv[4 * i + 1]) | __builtin_isunordered(xv[4 * i + 2], xv[4 * i + 3]);
    mf[i] = max_nn(max3_nn(xv[4 * i], xv[4 * i + 1], xv[4 * i + 2]), xv[4 * i + 3]);
  }
  uint32_t km, mb[NB];
  int qm;
  if (!nan) {
    float m = mf[0];
#pragma unroll
    for (int i = 1; i + 1 < NB; i += 2) m = max3_nn(m, mf[i], mf[i + 1]);
    if ((NB & 1) == 0 && NB > 1) m = max_nn(m, mf[NB - 1]);
    int qf = 0;
#pragma unroll
    for (int q = EPT - 1; q >= 0; --q) qf = (xv[q] == m) ? q : qf;
    km = orderable_nn(m);
    qm = qf;
#pragma unroll
    for (int i = 0; i < NB; ++i) mb[i] = orderable_nn(mf[i]);
  } else {
    km = 0u;
    qm = 0;
#pragma unroll
    for (int i = 0; i < NB; ++i) mb[i] = 0u;
#pragma unroll
    for (int q = 0; q < EPT; ++q) {
      const uint32_t k = orderable(xv[q]);
      take_max(k, q, km, qm);
      mb[q >> 2] = k > mb[q >> 2] ? k : mb[q >> 2];
    }
  }
  // a thread whose first element is past the row end has none in range
  unsigned long long best = 0ull;
  if (slice_v(base, tid, 0) < a.V) {
    const uint32_t v = (uint32_t)slice_v(base, tid, qm);
    float y = from_orderable(km);
    if (!p.greedy && y > NEG_INF) y = score(p, y, v);
    best = make_key(y, v);
  }
  if (!p.greedy) {
    // Block maxima for the survivor pass.  A butterfly that halves the values at each of
    // its first LOGNB steps leaves lane l with the wave's maximum over the lanes sharing
    // bits 5..SH of l of block (l >> SH) & (NB - 1); the remaining steps reduce over the
    // low SH bits.  At each halving exchange the lanes with `bit` set swap the pair (a
    // masked xor swap, which the compiler cannot turn into a dynamically indexed register
    // select), so that every lane keeps mb[j] and sends mb[j + half].
    constexpr int SH = 6 - LOGNB;
#pragma unroll
    for (int step = 0; step < LOGNB; ++step) {
      const int half = NB >> (step + 1), bit = 32 >> step;
      const uint32_t upm = (lane & bit) ? 0xFFFFFFFFu : 0u;
#pragma unroll
      for (int j = 0; j < half; ++j) {
        const uint32_t t = (mb[j] ^ mb[j + half]) & upm;
        mb[j] ^= t;
        mb[j + half] ^= t;
        const uint32_t got = (uint32_t)__shfl_xor((int)mb[j + half], bit);
        mb[j] = got > mb[j] ? got : mb[j];
      }
    }
#pragma unroll
    for (int bit = 1 << (SH - 1); bit >= 1; bit >>= 1) {
      const uint32_t got = (uint32_t)__shfl_xor((int)mb[0], bit);
      mb[0] = got > mb[0] ? got : mb[0];
    }
    if ((lane & ((1 << SH) - 1)) == 0) bred[tid >> 6][lane >> SH] = mb[0];
    __syncthreads();
    const int blk = blockIdx.x * NB + tid;
    if (tid < NB && blk < a.nblk) {
      uint32_t k = bred[0][tid];
#pragma unroll
      for (int w = 1; w < SMP_THREADS / 64; ++w) k = bred[w][tid] > k ? bred[w][tid] : k;
      a.bkeys[(int64_t)row * a.nblk + blk] = k;
    }
  }
  const unsigned long long gb = block_max_u64(best, red);
  if (tid == 0) a.ckeys[(int64_t)row * a.nchunks + blockIdx.x] = gb;
}

// The raw-logit cutoff of a sampled row whose winner scores >= L: every x <= xc has
// fl(fl(x/T) + GUMBEL_MAX) < L, so its score (x/T + G with G <= GUMBEL_MAX, rounding
// monotone) is < L and it cannot win.  Starts from the real-arithmetic bound and steps
// down until the rounded test holds; -inf (nothing pruned) when L is -inf or NaN.
__device__ __forceinline__ float raw_cutoff(float L, float T) {
  float xc = -__builtin_inff();
  if (L > xc && L == L) {
    float c = (L - GUMBEL_MAX) * T;
    for (int it = 0; it < 16; ++it) {
      if ((c / T) + GUMBEL_MAX < L) {
        xc = c;
        break;
      }
      c = c - fmaxf(fabsf(c) * 4.76837158e-7f, 1e-30f);
    }
  }
  return xc;
}

// The score part (high word) of the row's candidate keys: lane l reads slot l (and l + 64,
// ... past 64 slots); reduce with wave_max_u32.
__device__ __forceinline__ uint32_t row_cand_score(const SmpArgs& a, int row, int lane) {
  const uint32_t* s = (const uint32_t*)(a.ckeys + (int64_t)row * a.nchunks) + 1;
  uint32_t k = lane < a.nchunks ? s[2 * lane] : 0u;  // no wait here unless V > 1M
  for (int c = lane + 64; c < a.nchunks; c += 64) k = s[2 * c] > k ? s[2 * c] : k;
  return k;
}

// The row's best candidate key: the maximum of the candidate pass's slots, reduced over
// one wave (every lane returns it).
__device__ __forceinline__ unsigned long long row_cand_key(const SmpArgs& a, int row, int lane) {
  const unsigned long long* s = a.ckeys + (int64_t)row * a.nchunks;
  unsigned long long k = lane < a.nchunks ? s[lane] : 0ull;  // no wait here unless V > 1M
  for (int c = lane + 64; c < a.nchunks; c += 64) k = s[c] > k ? s[c] : k;
  return k;
}

// Launch 2 (sampled rows only; greedy rows return at once).  The candidates give a score L
// the winner is >= to.  Since G <= GUMBEL_MAX for every Philox word and rounding is
// monotone, x with fl(fl(x/T) + GUMBEL_MAX) < L cannot win; the test is one compare
// against a per-row raw-logit cutoff; whole 1024-logit blocks whose largest admissible
// logit is under the cutoff are skipped unread.  Survivors cluster in the rows with high
// temperature, so this pass uses small slices (EPT elements per thread): many short
// workgroups let the dispatcher spread one hot row over every CU.  A workgroup touches the
// row key only if it found a better score than L, which is rare.

template <int EPT>
__global__ void __launch_bounds__(SMP_THREADS) gumbel_surv_kernel(SmpArgs a) {
  constexpr int CAP = SMP_THREADS * EPT;  // every element of the slice may survive
  constexpr int NB = EPT / 4;             // 1024-logit blocks per slice
  __shared__ float qx[CAP];
  __shared__ uint32_t qv[CAP];
  __shared__ int qn, sgo;
  __shared__ float sxc, sL;
  const int row = blockIdx.y, tid = threadIdx.x, lane = tid & 63;
  const float* rowp = a.logits + (int64_t)row * a.ld;
  const int base = blockIdx.x * CAP;
  const bool ragged = !(base + CAP <= a.V);
  // The row's candidate keys (wave 0, which alone derives the row's cutoff), the slice's
  // block keys and the row's parameters are requested together; the slice's logits (a
  // re-read mostly served by the last-level cache) only once the slice is known to survive.
  uint32_t lh = 0u;
  if (tid < 64) lh = row_cand_score(a, row, lane);
  uint32_t bk[NB];
#pragma unroll
  for (int i = 0; i < NB; ++i) {
    const int blk = blockIdx.x * NB + i;
    bk[i] = blk < a.nblk ? a.bkeys[(int64_t)row * a.nblk + blk] : 0x007FFFFFu;  // -inf: none
  }
  float xv[EPT];
  auto load_logits = [&]() {
    if (a.vec && !ragged) {
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
      for (int q = 0; q < EPT; ++q) xv[q] = rowp[min(slice_v(base, tid, q), a.V - 1)];
    }
  };
  const RowParams p = row_params(a, row);
  if (p.greedy) return;
  const float NEG_INF = -__builtin_inff();
  if (tid < 64) {
    // L: the best candidate score of the row.  A NaN there means the row holds a NaN,
    // whose first occurrence the candidates already hold and nothing can beat.
    const float L = from_orderable(wave_max_u32(lh));
    const float xc = raw_cutoff(L, p.T);
    // the slice is needed only if some block of it has an admissible logit > xc
    bool any = false;
#pragma unroll
    for (int i = 0; i < NB; ++i) any = any || !(from_orderable(bk[i]) <= xc);
    if (lane == 0) {
      sxc = xc;
      sL = L;
      qn = 0;
      sgo = (any && L == L) ? 1 : 0;
    }
  }
  __syncthreads();
  if (!sgo) return;
  // the logits only now: greedy rows and skipped slices never read them (B=32 24.3 ->
  // 23.8 us, all-greedy B=128 45.7 -> 32.3 us against requesting them with the keys)
  load_logits();
  const float xc = sxc, L = sL;
  // Survivors of the whole workgroup go to one LDS queue: each wave counts its survivors
  // of every step (ballots), reserves its run with one LDS atomic and writes them in
  // order; then every thread scores entries tid, tid + 256, ...: n survivors cost
  // ceil(n / 64) wave-scores however they are spread over the slice.
  unsigned long long bm[EPT];
  int cnt = 0;
#pragma unroll
  for (int q = 0; q < EPT; ++q) {
    bool s = !(xv[q] <= xc);
    if (p.has_thr) s = s && xv[q] >= p.thr;
    if (ragged) s = s && slice_v(base, tid, q) < a.V;
    bm[q] = __ballot(s);
    cnt += (int)__popcll(bm[q]);
  }
  if (cnt) {
    int wbase = 0;
    if (lane == 0) wbase = __hip_atomic_fetch_add(&qn, cnt, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
    wbase = __builtin_amdgcn_readfirstlane(wbase);
    const unsigned long long below = (1ull << lane) - 1ull;
#pragma unroll
    for (int q = 0; q < EPT; ++q) {
      if ((bm[q] >> lane) & 1ull) {
        const int pos = wbase + (int)__popcll(bm[q] & below);
        qx[pos] = xv[q];
        qv[pos] = (uint32_t)slice_v(base, tid, q);
      }
      wbase += (int)__popcll(bm[q]);
    }
  }
  __syncthreads();
  const int n = qn;
  // Running maximum in float with the smallest index on ties (no survivor is NaN: NaN rows
  // stopped above; -0.0 == +0.0 as the order-preserving key has it).
  float by = NEG_INF;
  uint32_t bv = 0xFFFFFFFFu;  // none yet
  for (int i = tid; i < n; i += SMP_THREADS) score_fold(p, qx[i], qv[i], L, by, bv);
  // beating the candidates (score >= L) is rare: only then a wave reduction and an atomic
  if (__ballot(bv != 0xFFFFFFFFu && by >= L)) {
    const unsigned long long gb = wave_max_u64(bv != 0xFFFFFFFFu ? make_key(by, bv) : 0ull);
    if (lane == 0) amax_u64(&a.rkeys[row], gb);
  }
}

// Single pass for small batches (up to ~2M logits), where three launches of a few
// latencies each would dominate: 256 threads x 4 logits per workgroup; each wave takes its
// largest admissible logit (first index) as its candidate, scores it (L), prunes its other
// logits with raw_cutoff(L) and scores the rest through a per-wave LDS queue.  Exact for
// the same reason as the two-pass form: a pruned logit scores < L <= the row's best.
// Greedy rows keep the wave's argmax; a NaN (ranked above everything) wins at its first
// occurrence and needs no scoring.  Each workgroup stores its best key in its slot.
__global__ void __launch_bounds__(SMP_THREADS) gumbel_local_kernel(SmpArgs a) {
  constexpr int EPT = 4, CHUNK = SMP_THREADS * EPT;
  __shared__ float qx[SMP_THREADS * EPT];
  __shared__ uint32_t qv[SMP_THREADS * EPT];
  __shared__ unsigned long long red[SMP_THREADS / 64];
  const int row = blockIdx.y, tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const float* rowp = a.logits + (int64_t)row * a.ld;
  const int base = blockIdx.x * CHUNK;
  const bool inrange = base + CHUNK <= a.V;
  float xv[EPT];
  load_slice<EPT>(rowp, base, tid, a.V, a.vec && inrange, xv);
  const RowParams p = row_params(a, row);
  if (blockIdx.x == 0 && tid == 0) a.rkeys[row] = 0ull;  // unused by this path: finish reads 0
  const float NEG_INF = -__builtin_inff();
  // the thread's largest admissible logit on order-preserving keys (NaN on top)
  uint32_t km = 0u;
  int qm = -1;
#pragma unroll
  for (int q = 0; q < EPT; ++q) {
    if (p.has_thr) xv[q] = xv[q] < p.thr ? NEG_INF : xv[q];  // NaN stays
    if (slice_v(base, tid, q) < a.V) take_max(orderable(xv[q]), q, km, qm);
  }
  const unsigned long long tk =
      qm >= 0 ? (((unsigned long long)km << 32) | (unsigned long long)(~(uint32_t)slice_v(base, tid, qm))) : 0ull;
  unsigned long long best = wave_max_u64(tk);  // greedy rows: the wave's argmax
  const float xm = from_orderable((uint32_t)(best >> 32));
  if (!p.greedy && best != 0ull && xm == xm) {
    const uint32_t vm = ~(uint32_t)best;
    const float L = xm > NEG_INF ? score_sampled(p, xm, vm) : NEG_INF;
    best = make_key(L, vm);
    const float xc = raw_cutoff(L, p.T);
    // survivors: in range, admissible (masked ones are -inf <= xc), above the cutoff, not
    // the candidate itself; compacted into this wave's quarter of the queue
    float* wx = qx + wave * 64 * EPT;
    uint32_t* wv = qv + wave * 64 * EPT;
    const unsigned long long below = (1ull << lane) - 1ull;
    int n = 0;
#pragma unroll
    for (int q = 0; q < EPT; ++q) {
      const uint32_t v = (uint32_t)slice_v(base, tid, q);
      const bool s = (int)v < a.V && !(xv[q] <= xc) && v != vm;
      const unsigned long long m = __ballot(s);
      if (s) {
        const int pos = n + (int)__popcll(m & below);
        wx[pos] = xv[q];
        wv[pos] = v;
      }
      n += (int)__popcll(m);
    }
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    float by = NEG_INF;
    uint32_t bv = 0xFFFFFFFFu;
    // exact scores throughout: a wave's own candidate is a weak floor, so the bound of
    // score_fold rarely rules a logit out here (measured slower at B = 1 and 4)
    for (int i = lane; i < n; i += 64) {
      const float x = wx[i];
      const uint32_t v = wv[i];
      const float y = score_sampled(p, x, v);
      const bool b = (y > by) || (y == by && v < bv);
      by = b ? y : by;
      bv = b ? v : bv;
    }
    const unsigned long long k = bv != 0xFFFFFFFFu ? make_key(by, bv) : 0ull;
    const unsigned long long wk = wave_max_u64(k);
    best = wk > best ? wk : best;
  }
  const unsigned long long gb = block_max_u64(best, red);
  if (tid == 0) a.ckeys[(int64_t)row * a.nchunks + blockIdx.x] = gb;
}

// Launch 3: one wave per row reduces the candidate slots and the survivor pass's row key
// to the token.
__global__ void __launch_bounds__(256) gumbel_finish_kernel(SmpArgs a) {
  const int row = blockIdx.x * 4 + (threadIdx.x >> 6), lane = threadIdx.x & 63;
  if (row >= a.B) return;
  unsigned long long k = row_cand_key(a, row, lane);
  if (lane == 0) {
    const unsigned long long r = ld_relaxed_u64(&a.rkeys[row]);
    k = r > k ? r : k;
  }
  k = wave_max_u64(k);
  if (lane == 0) a.out[row] = (int64_t)(~(uint32_t)(k & 0xFFFFFFFFull));
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
static int64_t gumbel_nchunks(int64_t V, int64_t chunk) { return (V + chunk - 1) / chunk; }

// ckeys [B, nchunks] u64, rkeys [B] u64, bkeys [B, nblk] u32: every launch writes each
// value before reading it, so the workspace needs no initialisation.
extern "C" int64_t vqk_gumbel_workspace_size(int64_t B, int64_t V) {
  if (B < 0 || V < 0) return 0;
  return B * (gumbel_nchunks(V, SMP_MIN_CHUNK) + 1) * (int64_t)sizeof(unsigned long long) +
         B * gumbel_nblk(V) * (int64_t)sizeof(uint32_t) + 16;
}

static int smp_check(const float* logits, int64_t ld, int64_t B, int64_t V, const void* seeds) {
  if (!logits || B < 0 || V < 1 || ld < V) return VQK_EINVAL;
  if (B > 65535 || V > (int64_t)INT32_MAX - SMP_THREADS * 64) return VQK_EUNSUPPORTED;
  if (!seeds) return VQK_EINVAL;
  return VQK_OK;
}

// Enqueues the sampler's launches with `workspace` (checked by the callers: at least
// vqk_gumbel_workspace_size(B, V) bytes, 8-byte aligned, device memory).
static int gumbel_launch(const float* logits, int64_t ld, int64_t B, int64_t V, const float* temp,
                         const void* seeds, int seed_is_64bit, const float* topk_thr, int64_t* out,
                         void* workspace, vqk_stream_t stream) {
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
  a.nblk = (int)gumbel_nblk(V);
  // Small batches (up to ~2M logits) take the single-pass form: the whole call is then a
  // few workgroup latencies long, and three launches would cost more than the extra
  // scoring.  Larger ones take the candidate and survivor passes.
  const bool small = B * V <= ((int64_t)2 << 20);
  const int64_t max_chunks = gumbel_nchunks(V, SMP_MIN_CHUNK);
  a.nchunks = (int)gumbel_nchunks(V, small ? SMP_THREADS * 4 : SMP_THREADS * SMP_CAND_EPT);
  a.ckeys = (unsigned long long*)workspace;
  a.rkeys = a.ckeys + B * max_chunks;
  a.bkeys = (uint32_t*)(a.rkeys + B);
  a.vec = (((uintptr_t)logits & 15) == 0 && (ld % 4) == 0) ? 1 : 0;
  if (small) {
    hipLaunchKernelGGL(gumbel_local_kernel, dim3(a.nchunks, (unsigned)B), dim3(SMP_THREADS), 0,
                       (hipStream_t)stream, a);
  } else {
    hipLaunchKernelGGL(gumbel_cand_kernel<SMP_CAND_EPT>, dim3(a.nchunks, (unsigned)B), dim3(SMP_THREADS), 0,
                       (hipStream_t)stream, a);
    const int ns = (int)((V + SMP_THREADS * SMP_SURV_EPT - 1) / (SMP_THREADS * SMP_SURV_EPT));
    hipLaunchKernelGGL(gumbel_surv_kernel<SMP_SURV_EPT>, dim3(ns, (unsigned)B), dim3(SMP_THREADS), 0, (hipStream_t)stream, a);
  }
  hipLaunchKernelGGL(gumbel_finish_kernel, dim3((unsigned)((B + 3) / 4)), dim3(256), 0, (hipStream_t)stream, a);
  hipError_t e = hipGetLastError();
  return e == hipSuccess ? VQK_OK : (int)e;
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
  return gumbel_launch(logits, ld, B, V, temp, seeds, seed_is_64bit, topk_thr, out, workspace, stream);
}

// ---------------------------------------------------------------------------------------
// Allocation-free form: the workspace is this file's own device array.  Every GPU the
// library runs on holds one copy until the process ends; host code must use the address
// hipGetSymbolAddress returns for the current device (the array's name on the host is
// only a stand-in), resolved once per device on the first call there.  The sampler writes
// every workspace value before reading it, so nothing needs clearing between calls; calls
// that overlap on one GPU (two streams at once) share the array and race.
constexpr int64_t SMP_STATIC_BYTES = 1 << 20;
static __device__ __align__(256) unsigned char scratch[SMP_STATIC_BYTES];

namespace {
constexpr int kMaxScratchDev = 64;
void* g_scratch[kMaxScratchDev];
std::mutex g_scratch_mu;
}  // namespace

static int scratch_ptr(void** out) {
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= kMaxScratchDev) return VQK_ENODEVICE;
  std::lock_guard<std::mutex> lk(g_scratch_mu);
  if (!g_scratch[dev]) {
    void* p = nullptr;
    const hipError_t e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    if (e != hipSuccess) return (int)e;
    if (!p) return VQK_ENODEVICE;
    g_scratch[dev] = p;
  }
  *out = g_scratch[dev];
  return VQK_OK;
}

extern "C" int64_t vqk_gumbel_noalloc_max_bytes(void) { return SMP_STATIC_BYTES; }

extern "C" int vqk_gumbel_argmax_noalloc(const float* logits, int64_t ld, int64_t B, int64_t V, const float* temp,
                                         const void* seeds, int seed_is_64bit, const float* topk_thr,
                                         int64_t* out, vqk_stream_t stream) {
  int rc = vqk_device_check();
  if (rc) return rc;
  rc = smp_check(logits, ld, B, V, seeds);
  if (rc) return rc;
  if (!out) return VQK_EINVAL;
  if (B == 0) return VQK_OK;
  if (vqk_gumbel_workspace_size(B, V) > SMP_STATIC_BYTES) return VQK_EWORKSPACE;
  void* ws = nullptr;
  rc = scratch_ptr(&ws);
  if (rc) return rc;
  return gumbel_launch(logits, ld, B, V, temp, seeds, seed_is_64bit, topk_thr, out, ws, stream);
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
