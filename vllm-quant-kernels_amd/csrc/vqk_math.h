// vqk_math.h - scalar device helpers shared by the gfx950 kernels: number formats
// (fp16/bf16 bits, OCP e4m3fn, E2M1, E8M0), the MX group exponent, Philox4x32-10,
// the Gumbel noise and an order-preserving float key.
//
// Every function here is a pure function of its arguments built only from IEEE-754
// float32 operations with a single rounding each (add, mul, fma, div, int<->float
// conversion), so the CPU oracle (oracle/vqk_oracle.c) reproduces its results bit for bit.
// The translation unit must be compiled with -ffp-contract=off.
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

namespace vqk {

__device__ __forceinline__ float f32_bits(uint32_t u) { return __uint_as_float(u); }
__device__ __forceinline__ uint32_t bits_f32(float f) { return __float_as_uint(f); }

// fp16 bits -> float (exact).
__device__ __forceinline__ float h2f(uint16_t h) {
  _Float16 v = __builtin_bit_cast(_Float16, h);
  return (float)v;
}
// float -> fp16 bits, round to nearest even (hardware v_cvt_f16_f32).  The empty asm
// pins f as a float32 register value first: otherwise the backend may fold a preceding
// multiply into v_fma_mix (one rounding straight to fp16), while the reference rounds the
// product to float32 and then to fp16.
__device__ __forceinline__ uint16_t f2h(float f) {
  asm volatile("" : "+v"(f));
  _Float16 v = (_Float16)f;
  return __builtin_bit_cast(uint16_t, v);
}
// bf16 bits -> float (exact).
__device__ __forceinline__ float bf2f(uint16_t b) { return __uint_as_float((uint32_t)b << 16); }

// Load element i of a weight/activation row of dtype code dt (0 f32, 1 f16, 2 bf16) as float.
__device__ __forceinline__ float load_as_f32(const void* p, int dt, int64_t i) {
  if (dt == 0) return ((const float*)p)[i];
  if (dt == 1) return h2f(((const uint16_t*)p)[i]);
  return bf2f(((const uint16_t*)p)[i]);
}
// The same with the dtype fixed at compile time: unrolled runs of these loads carry no
// per-element branch, so they issue back to back instead of one memory latency each.
template <int DT>
__device__ __forceinline__ float load_dt(const void* p, int64_t i) {
  if constexpr (DT == 0) return ((const float*)p)[i];
  else if constexpr (DT == 1) return h2f(((const uint16_t*)p)[i]);
  else return bf2f(((const uint16_t*)p)[i]);
}

// N contiguous elements (dtype code DT) from element offset off as float (N % 8 == 0), with
// 16-byte loads when the host found the rows aligned.  All loads are issued before any
// conversion.
template <int DT, int N>
__device__ __forceinline__ void load_run(const void* x, int64_t off, bool vec, float (&out)[N]) {
  if (vec) {
    if constexpr (DT == VQK_F32) {
      float4 t[N / 4];
#pragma unroll
      for (int i = 0; i < N / 4; ++i) t[i] = ((const float4*)((const float*)x + off))[i];
#pragma unroll
      for (int i = 0; i < N / 4; ++i) {
        out[4 * i] = t[i].x;
        out[4 * i + 1] = t[i].y;
        out[4 * i + 2] = t[i].z;
        out[4 * i + 3] = t[i].w;
      }
    } else {
      uint4 t[N / 8];
#pragma unroll
      for (int i = 0; i < N / 8; ++i) t[i] = ((const uint4*)((const uint16_t*)x + off))[i];
#pragma unroll
      for (int i = 0; i < N / 8; ++i) {
        const uint32_t w[4] = {t[i].x, t[i].y, t[i].z, t[i].w};
#pragma unroll
        for (int j = 0; j < 4; ++j) {
          const uint16_t lo = (uint16_t)(w[j] & 0xFFFFu), hi = (uint16_t)(w[j] >> 16);
          out[8 * i + 2 * j] = (DT == VQK_F16) ? h2f(lo) : bf2f(lo);
          out[8 * i + 2 * j + 1] = (DT == VQK_F16) ? h2f(hi) : bf2f(hi);
        }
      }
    }
  } else {
#pragma unroll
    for (int e = 0; e < N; ++e) out[e] = load_dt<DT>(x, off + e);
  }
}

// rint(fl(x / s)) for |x / s| <= 128 (int8 quantization) with one multiply in the common
// case.  r = fl(1/s); t = x*r differs from x/s by at most 2^-23 * 128 = 2^-16, and fl(x/s)
// from x/s by at most 2^-17, so t and fl(x/s) are within 2^-15 of each other: unless a
// half-integer lies that close to t, both round to the same integer.  Otherwise (rare) the
// IEEE division decides, ties included.
__device__ __forceinline__ float rint_div_i8(float x, float s, float r) {
  float t = x * r;
  const float h = floorf(t) + 0.5f;
  if (fabsf(t - h) < 3.0517578125e-05f) t = x / s;  // 2^-15
  return __builtin_rintf(t);
}

// ---------------------------------------------------------------------------------------
// OCP float8_e4m3fn encoding with torch's cast semantics (Appendix of the plugin notes):
// round to nearest even; no saturation: anything that rounds above 448 is NaN (0x7F),
// i.e. |x| > 464; NaN keeps its sign bit; -0.0 -> 0x80.
// Method: split off the sign, then
//   |x| < 2^-6 (subnormal range, quantum 2^-9): code = rint(|x| * 2^9) (exact scaling),
//   otherwise: round the fp32 mantissa to 3 bits with the usual add-half-minus-one-plus-odd
//   trick and re-bias the exponent from 127 to 7.  Codes above 0x7E mean "rounded past
//   448", which is NaN in this format.
__device__ __forceinline__ uint8_t f32_to_e4m3(float x) {
  // Both cases are computed and one is selected (no branches: this runs per element in
  // unrolled loops).  The normal-range code saturates at 0x7F, which covers NaN, +-inf and
  // everything that rounds past 448 (|x| > 464 or NaN give codes >= 0x7F).
  const uint32_t b = bits_f32(x);
  const uint32_t sign = (b >> 24) & 0x80u;
  const uint32_t a = b & 0x7FFFFFFFu;
  const uint32_t odd = (a >> 20) & 1u;
  const uint32_t cn = min(((a + 0x7FFFFu + odd) >> 20) - ((127u - 7u) << 3), 0x7Fu);
  // |x| < 2^-6: rint(|x| * 2^9) in [0, 8] (the operand is clamped so the conversion
  // stays in range whichever case is selected)
  const uint32_t cs = (uint32_t)__builtin_rintf(fminf(__uint_as_float(a), 0.015625f) * 512.0f);
  const uint32_t code = (a < 0x3C800000u) ? cs : cn;
  return (uint8_t)(code | sign);
}

// Four floats of magnitude at most 448 -> their e4m3fn bytes (a in the low byte), by the
// hardware conversion: on that range it equals f32_to_e4m3 for every float32 (checked
// exhaustively on the GPU by vqk_debug_e4m3_hw_check).  Callers clamp first.
__device__ __forceinline__ uint32_t e4m3x4_clamped(float a, float b, float c, float d) {
  int w = __builtin_amdgcn_cvt_pk_fp8_f32(a, b, 0, false);
  w = __builtin_amdgcn_cvt_pk_fp8_f32(c, d, w, true);
  return (uint32_t)w;
}

// The same for any floats with torch's float8_e4m3fn cast semantics (no clamp: overflow
// and infinities give NaN 0x7F | sign).  The hardware conversion agrees with
// f32_to_e4m3 on every float32 except positive NaNs, which are set here (checked
// exhaustively by vqk_debug_e4m3_hw_check with full set).
__device__ __forceinline__ uint32_t e4m3x4_torch(float a, float b, float c, float d) {
  uint32_t w = (uint32_t)__builtin_amdgcn_cvt_pk_fp8_f32(a, b, 0, false);
  w = (uint32_t)__builtin_amdgcn_cvt_pk_fp8_f32(c, d, (int)w, true);
  const float v[4] = {a, b, c, d};
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const uint32_t bi = bits_f32(v[i]);
    const uint32_t code = ((bi >> 24) & 0x80u) | 0x7Fu;
    if ((bi & 0x7FFFFFFFu) > 0x7F800000u) w = (w & ~(0xFFu << (8 * i))) | (code << (8 * i));
  }
  return w;
}

// e4m3fn byte -> float (exact).
__device__ __forceinline__ float e4m3_to_f32(uint8_t v) {
  uint32_t s = (v & 0x80u) << 24;
  uint32_t e = (v >> 3) & 0xFu, m = v & 7u;
  if (e == 0xF && m == 7) return __uint_as_float(s | 0x7FC00000u);
  float mag = (e == 0) ? (float)m * (1.0f / 512.0f)
                       : __uint_as_float(((e + 120u) << 23) | (m << 20));
  return __uint_as_float(__float_as_uint(mag) | s);
}

// E2M1 nibble of an already-scaled value y with the plugin's bucketize semantics:
// sign bit = (y < 0) (so -0.0 gives 0 and a tiny negative gives 0x8), magnitude index =
// number of midpoints {.25,.75,1.25,1.75,2.5,3.5,5} strictly below min(|y|, 6): a value
// exactly on a midpoint goes to the lower grid point.
__device__ __forceinline__ uint32_t f32_to_e2m1(float y) {
  float m = fminf(fabsf(y), 6.0f);
  uint32_t idx = (m > 0.25f) + (m > 0.75f) + (m > 1.25f) + (m > 1.75f) + (m > 2.5f) +
                 (m > 3.5f) + (m > 5.0f);
  return ((y < 0.0f) ? 8u : 0u) | idx;
}

// MX group exponent k = clamp(ceil(log2(max(amax, 1e-30) / qmax)), -127, 127), computed
// exactly: q = gmax/qmax (one IEEE division, as the reference does), then ceil(log2 q) is
// the binary exponent of q, minus one when q is an exact power of two.
__device__ __forceinline__ int mx_exponent(float amax, float qmax) {
  float gmax = fmaxf(amax, 1e-30f);
  float q = gmax / qmax;
  uint32_t qb = bits_f32(q);
  int e = (int)((qb >> 23) & 0xFF) - 127;  // q = 1.m * 2^e  (q is normal: q >= 1e-30/448)
  int k = ((qb & 0x7FFFFFu) == 0u) ? e : e + 1;
  return k < -127 ? -127 : (k > 127 ? 127 : k);
}
// 2^k as float for k in [-127, 127] (exact; 2^-127 is subnormal).
__device__ __forceinline__ float exp2i(int k) {
  return (k >= -126) ? __uint_as_float((uint32_t)(k + 127) << 23) : __uint_as_float(0x00400000u);
}

// ---------------------------------------------------------------------------------------
// Philox4x32-10 (Salmon et al., SC'11).  Counter (c0,c1,c2,c3), key (k0,k1); a round is
//   c0' = hi(Mb*c2) ^ c1 ^ k0,  c1' = lo(Mb*c2),  c2' = hi(Ma*c0) ^ c3 ^ k1,  c3' = lo(Ma*c0)
// followed by the Weyl key bump.  Word 0 of the output is the only one the sampler uses
// (the reference draws u from tl.rand(seed, v): counter (v,0,0,0), key = the 64-bit seed).
constexpr uint32_t PHILOX_MA = 0xD2511F53u, PHILOX_MB = 0xCD9E8D57u;
constexpr uint32_t PHILOX_WA = 0x9E3779B9u, PHILOX_WB = 0xBB67AE85u;

// a ^ b ^ k as one v_bitop3_b32 (truth table 0x96: odd parity); k must be wave-uniform.
__device__ __forceinline__ uint32_t xor3_vvs(uint32_t a, uint32_t b, uint32_t k) {
  uint32_t r;
  asm("v_bitop3_b32 %0, %1, %2, %3 bitop3:0x96" : "=v"(r) : "v"(a), "v"(b), "s"(k));
  return r;
}

// The key (k0, k1) must be wave-uniform (every caller keys a whole row with one seed).
__device__ __forceinline__ uint32_t philox_word0(uint32_t v, uint32_t k0, uint32_t k1) {
  uint32_t c0 = v, c1 = 0u, c2 = 0u, c3 = 0u;
  // Rounds 0 and 1 in plain C, which the compiler folds: c1 = c2 = c3 = 0 at first, and
  // word 0 after round 0 is the key itself, so round 1's Ma product is uniform.
#pragma unroll
  for (int r = 0; r < 2; ++r) {
    const uint64_t pa = (uint64_t)PHILOX_MA * c0;
    const uint64_t pb = (uint64_t)PHILOX_MB * c2;
    const uint32_t n0 = (uint32_t)(pb >> 32) ^ c1 ^ k0;
    const uint32_t n2 = (uint32_t)(pa >> 32) ^ c3 ^ k1;
    c1 = (uint32_t)pb;
    c3 = (uint32_t)pa;
    c0 = n0;
    c2 = n2;
    k0 += PHILOX_WA;
    k1 += PHILOX_WB;
  }
  // Rounds 2-9: both words per round are one 3-input xor each.
#pragma unroll
  for (int r = 2; r < 10; ++r) {
    const uint64_t pa = (uint64_t)PHILOX_MA * c0;
    const uint64_t pb = (uint64_t)PHILOX_MB * c2;
    const uint32_t n0 = xor3_vvs((uint32_t)(pb >> 32), c1, k0);
    const uint32_t n2 = xor3_vvs((uint32_t)(pa >> 32), c3, k1);
    c1 = (uint32_t)pb;
    c3 = (uint32_t)pa;
    c0 = n0;
    c2 = n2;
    k0 += PHILOX_WA;
    k1 += PHILOX_WB;
  }
  return c0;
}

// philox_word0 for a key that differs between lanes (plain xors, no uniform operand).
__device__ __forceinline__ uint32_t philox_word0_vk(uint32_t v, uint32_t k0, uint32_t k1) {
  uint32_t c0 = v, c1 = 0u, c2 = 0u, c3 = 0u;
#pragma unroll
  for (int r = 0; r < 10; ++r) {
    const uint64_t pa = (uint64_t)PHILOX_MA * c0;
    const uint64_t pb = (uint64_t)PHILOX_MB * c2;
    const uint32_t n0 = (uint32_t)(pb >> 32) ^ c1 ^ k0;
    const uint32_t n2 = (uint32_t)(pa >> 32) ^ c3 ^ k1;
    c1 = (uint32_t)pb;
    c3 = (uint32_t)pa;
    c0 = n0;
    c2 = n2;
    k0 += PHILOX_WA;
    k1 += PHILOX_WB;
  }
  return c0;
}

// Triton's uint_to_uniform_float for a 32-bit word: reinterpret as int32, fold negatives
// with -x-1, convert to float (RNE) and multiply by float(4.6566127342e-10) = 0x2FFFFFFF.
__device__ __forceinline__ float philox_uniform(uint32_t w) {
  int32_t x = (int32_t)w;
  x = (x < 0) ? (-x - 1) : x;
  return (float)x * __uint_as_float(0x2FFFFFFFu);
}

// Natural log of a positive normal float: x = 2^e * m with m in [sqrt(1/2), sqrt(2)),
// f = m - 1, log(1+f) = f - f^2/2 + f^3 * P(f) with this project's degree-7 least-squares
// fit P (csrc/fit_logf.py), plus e*ln2 in two parts.  Error <= about 1 ulp.
__device__ __forceinline__ float vqk_logf(float x) {
  uint32_t b = bits_f32(x);
  int e = (int)((b >> 23) & 0xFF) - 127;
  uint32_t mb = b & 0x7FFFFFu;
  float m;
  if (mb > 0x3504F3u) {
    m = __uint_as_float(mb | 0x3F000000u);
    e += 1;
  } else {
    m = __uint_as_float(mb | 0x3F800000u);
  }
  float f = m - 1.0f;
  float p = __uint_as_float(0xBDA5F323u);
  p = __builtin_fmaf(p, f, __uint_as_float(0x3E022E8Bu));
  p = __builtin_fmaf(p, f, __uint_as_float(0xBE04D571u));
  p = __builtin_fmaf(p, f, __uint_as_float(0x3E116DD4u));
  p = __builtin_fmaf(p, f, __uint_as_float(0xBE2A6AACu));
  p = __builtin_fmaf(p, f, __uint_as_float(0x3E4CD0AAu));
  p = __builtin_fmaf(p, f, __uint_as_float(0xBE800063u));
  p = __builtin_fmaf(p, f, __uint_as_float(0x3EAAAAA9u));
  float f2 = f * f;
  float f3 = f2 * f;
  float t = __builtin_fmaf(f3, p, -0.5f * f2);
  float y = f + t;
  float ef = (float)e;
  y = __builtin_fmaf(ef, __uint_as_float(0x35BFBE8Eu), y);  // ln2 low part
  y = __builtin_fmaf(ef, __uint_as_float(0x3F317200u), y);  // ln2 high part (exact products)
  return y;
}

// Gumbel noise of uniform u: -log(-log(max(u, 2^-126))).  For u in [0, 1-2^-24] the
// result lies in [GUMBEL_MIN, GUMBEL_MAX] (checked exhaustively over the top of the
// range by the oracle tests).
constexpr float GUMBEL_MAX = 16.6356f;
__device__ __forceinline__ float gumbel_from_uniform(float u) {
  u = fmaxf(u, __uint_as_float(0x00800000u));
  float l1 = vqk_logf(u);
  return -vqk_logf(-l1);
}

// An upper bound of gumbel_from_uniform(u) for a Philox uniform u <= 1 - 2^-24 from the
// exponent of 1 - u alone: -log(-log u) <= -log(1 - u) (as -log u >= 1 - u), and
// -log t <= -e*ln2 for t = m*2^e, m in [1, 2).  The 0.01 margin covers the rounding of
// 1 - u and of the exact path (both below 1e-5 here).
__device__ __forceinline__ float gumbel_upper(float u) {
  const float t = 1.0f - u;
  const int e = (int)((bits_f32(t) >> 23) & 0xFFu) - 127;
  return (float)(-e) * 0.693147182f + 0.01f;
}

// Order-preserving map float -> uint32 (larger float -> larger key); -0.0 is folded into
// +0.0 and every NaN into the positive quiet NaN, which orders above +inf (torch.argmax
// treats NaN as the maximum).
__device__ __forceinline__ uint32_t orderable(float y) {
  uint32_t b = bits_f32(y);
  if ((b & 0x7FFFFFFFu) > 0x7F800000u) b = 0x7FC00000u;
  if (b == 0x80000000u) b = 0u;
  return (b & 0x80000000u) ? ~b : (b | 0x80000000u);
}
__device__ __forceinline__ float from_orderable(uint32_t k) {
  uint32_t b = (k & 0x80000000u) ? (k & 0x7FFFFFFFu) : ~k;
  return __uint_as_float(b);
}

// Argmax key of score y at vocabulary index v: larger y first, then smaller v.
__device__ __forceinline__ unsigned long long make_key(float y, uint32_t v) {
  return ((unsigned long long)orderable(y) << 32) | (unsigned long long)(~v);
}

}  // namespace vqk
