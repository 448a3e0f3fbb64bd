/*
 * vqk_oracle.c - TEST INFRASTRUCTURE ONLY.  CPU restatement of the reference plugin's
 * arithmetic (himikk/vllm-quant-kernels), used by tests/, __graft_entry__.smoke() and
 * bench.py's cpu_baseline leg as the checker.  Nothing in the product links or calls it.
 *
 * It is written independently of the HIP kernels (different methods where a choice
 * exists: nearest-value search instead of bit tricks for e4m3, frexp instead of exponent
 * extraction, double-precision dot products) so that a shared mistake is unlikely; the
 * tests pin it against torch's own casts, closed forms and known-answer vectors.
 *
 * Reference file:line for each function is given in its comment.  Build: oracle/build.py
 * (gcc -O2 -fopenmp -ffp-contract=off).
 */
#include <math.h>
#include <stdint.h>
#include <stdlib.h>
#include <string.h>

#ifdef _OPENMP
#include <omp.h>
#endif

/* ---------------------------------------------------------------------------------- */
/* Philox4x32-10 (Salmon, Moraes, Dror, Shaw, SC'11), as used by Triton's tl.rand
 * (triton/language/random.py:12-110, third-party, Triton 3.6.0): per round
 *   (c0,c1,c2,c3) <- (hi(B*c2)^c1^k0, lo(B*c2), hi(A*c0)^c3^k1, lo(A*c0)),
 * A = 0xD2511F53, B = 0xCD9E8D57, then k0 += 0x9E3779B9, k1 += 0xBB67AE85. */
void vqko_philox4x32_10(const uint32_t ctr[4], const uint32_t key[2], uint32_t out[4]) {
  uint32_t x0 = ctr[0], x1 = ctr[1], x2 = ctr[2], x3 = ctr[3];
  uint32_t k0 = key[0], k1 = key[1];
  for (int r = 0; r < 10; ++r) {
    uint64_t p0 = (uint64_t)0xD2511F53u * (uint64_t)x0;
    uint64_t p1 = (uint64_t)0xCD9E8D57u * (uint64_t)x2;
    uint32_t y0 = (uint32_t)(p1 >> 32) ^ x1 ^ k0;
    uint32_t y1 = (uint32_t)p1;
    uint32_t y2 = (uint32_t)(p0 >> 32) ^ x3 ^ k1;
    uint32_t y3 = (uint32_t)p0;
    x0 = y0; x1 = y1; x2 = y2; x3 = y3;
    k0 += 0x9E3779B9u;
    k1 += 0xBB67AE85u;
  }
  out[0] = x0; out[1] = x1; out[2] = x2; out[3] = x3;
}

/* Triton uint_to_uniform_float for 32-bit words (triton/language/random.py:126-143). */
float vqko_uniform(uint32_t w) {
  int32_t x;
  memcpy(&x, &w, 4);
  if (x < 0) x = -x - 1;
  const float scale = 4.6566127342e-10f;
  return (float)x * scale;
}

/* tl.rand(seed, offset) word for the sampler (src/vllm_quant_kernels/_sampler_kernels.py:104):
 * counter (offset, 0, 0, 0), key (seed lo32, seed hi32). */
float vqko_rand(uint64_t seed, uint32_t offset) {
  uint32_t c[4] = {offset, 0u, 0u, 0u};
  uint32_t k[2] = {(uint32_t)seed, (uint32_t)(seed >> 32)};
  uint32_t o[4];
  vqko_philox4x32_10(c, k, o);
  return vqko_uniform(o[0]);
}

/* Natural log used for the Gumbel noise.  The reference calls tl.log, whose bits depend
 * on the backend; this build defines the noise with one fixed float32 log so that the
 * HIP kernel and this oracle agree bit for bit: x = 2^e * m, m in [sqrt(1/2), sqrt(2)),
 * f = m - 1, log(1+f) = f - f^2/2 + f^3 P(f) (degree-7 least-squares fit, csrc/fit_logf.py),
 * + e*ln2 split in two.  Accuracy ~1 ulp (pinned against the libm double log). */
static float f32_from_bits(uint32_t u) { float f; memcpy(&f, &u, 4); return f; }
static uint32_t bits_from_f32(float f) { uint32_t u; memcpy(&u, &f, 4); return u; }

float vqko_logf(float x) {
  static const uint32_t C[8] = {0x3EAAAAA9u, 0xBE800063u, 0x3E4CD0AAu, 0xBE2A6AACu,
                                0x3E116DD4u, 0xBE04D571u, 0x3E022E8Bu, 0xBDA5F323u};
  uint32_t b = bits_from_f32(x);
  int e = (int)((b >> 23) & 0xFFu) - 127;
  uint32_t mb = b & 0x7FFFFFu;
  float m;
  if (mb > 0x3504F3u) { m = f32_from_bits(mb | 0x3F000000u); e += 1; }
  else { m = f32_from_bits(mb | 0x3F800000u); }
  float f = m - 1.0f;
  float p = f32_from_bits(C[7]);
  for (int i = 6; i >= 0; --i) p = fmaf(p, f, f32_from_bits(C[i]));
  float f2 = f * f;
  float f3 = f2 * f;
  float t = fmaf(f3, p, -0.5f * f2);
  float y = f + t;
  float ef = (float)e;
  y = fmaf(ef, f32_from_bits(0x35BFBE8Eu), y);
  y = fmaf(ef, f32_from_bits(0x3F317200u), y);
  return y;
}

/* -log(-log(max(u, 2^-126))) (src/vllm_quant_kernels/_sampler_kernels.py:101-106). */
float vqko_gumbel(float u) {
  const float tiny = f32_from_bits(0x00800000u);
  if (u < tiny) u = tiny;
  float l1 = vqko_logf(u);
  return -vqko_logf(-l1);
}

/* Largest noise value any 32-bit Philox word can produce, by exhaustion over the distinct
 * uniforms (every float (float)n * scale for n in [0, 2^31)).  Used to validate the
 * pruning bound of the GPU sampler. */
float vqko_gumbel_max_over_all_words(void) {
  float best = -INFINITY;
  /* (float)x for x in [0, 2^31 - 1] takes every integer value below 2^24 and every float
   * of [2^24, 2^31] (2^31 included: large x round up to it); walk exactly those values */
  const float top = 2147483648.0f;
  float f = 0.0f;
  for (;;) {
    float g = vqko_gumbel(f * 4.6566127342e-10f);
    if (g > best) best = g;
    if (f >= top) break;
    f = (f < 16777216.0f) ? f + 1.0f : nextafterf(f, INFINITY);
  }
  return best;
}

/* The GPU sampler's cheap upper bound of the noise from the exponent of 1 - u (no
 * counterpart in the reference: it only decides which exact scores the GPU may skip), and
 * the smallest slack bound - noise over every distinct uniform, walked as above.  A
 * positive result proves the bound for every Philox word. */
float vqko_gumbel_upper(float u) {
  const float t = 1.0f - u;
  const int e = (int)((bits_from_f32(t) >> 23) & 0xFFu) - 127;
  return (float)(-e) * 0.693147182f + 0.01f;
}
float vqko_gumbel_upper_min_slack(void) {
  float worst = INFINITY;
  const float top = 2147483648.0f;
  float f = 0.0f;
  for (;;) {
    const float u = f * 4.6566127342e-10f;
    const float slack = vqko_gumbel_upper(u) - vqko_gumbel(u);
    if (slack < worst) worst = slack;
    if (f >= top) break;
    f = (f < 16777216.0f) ? f + 1.0f : nextafterf(f, INFINITY);
  }
  return worst;
}

/* Score y of element v (src/vllm_quant_kernels/_sampler_kernels.py:68-113). */
static float score(float x, int has_t, float T, uint64_t seed, int has_thr, float thr, uint32_t v) {
  if (has_thr && !(x >= thr)) return -INFINITY;
  if (!has_t || T < 1e-5f) return x;
  float a = x / T;
  return a + vqko_gumbel(vqko_rand(seed, v));
}

void vqko_gumbel_scores(const float *logits, int64_t B, int64_t V, int64_t ld, const float *temp,
                        const uint64_t *seeds, const float *thr, float *scores) {
#pragma omp parallel for schedule(static)
  for (int64_t b = 0; b < B; ++b) {
    const float *row = logits + b * ld;
    for (int64_t v = 0; v < V; ++v)
      scores[b * V + v] = score(row[v], temp != 0, temp ? temp[b] : 1.0f, seeds[b], thr != 0,
                                thr ? thr[b] : 0.f, (uint32_t)v);
  }
}

/* argmax with the smallest index on ties; NaN counts as the maximum (torch.argmax);
 * -0.0 == +0.0.  (Cross-block rule: torch argmax first occurrence,
 * src/vllm_quant_kernels/_sampler_kernels.py:180-181; in-block: tie_break_left.) */
static int64_t argmax_row(const float *y, int64_t V) {
  int64_t best = 0;
  float bv = y[0];
  for (int64_t v = 1; v < V; ++v) {
    float c = y[v];
    if (bv != bv) break;          /* first NaN already found */
    if (c != c) { best = v; bv = c; break; }
    if (c > bv) { best = v; bv = c; }
  }
  return best;
}

void vqko_gumbel_argmax(const float *logits, int64_t B, int64_t V, int64_t ld, const float *temp,
                        const uint64_t *seeds, const float *thr, int64_t *out, int nthreads) {
#ifdef _OPENMP
  if (nthreads > 0) omp_set_num_threads(nthreads);
#else
  (void)nthreads;
#endif
#pragma omp parallel
  {
    float *buf = 0;
    int64_t cap = 0;
#pragma omp for schedule(dynamic, 1)
    for (int64_t b = 0; b < B; ++b) {
      if (cap < V) {
        buf = (float *)realloc(buf, sizeof(float) * (size_t)V);
        cap = V;
      }
      const float *row = logits + b * ld;
      for (int64_t v = 0; v < V; ++v)
        buf[v] = score(row[v], temp != 0, temp ? temp[b] : 1.0f, seeds[b], thr != 0, thr ? thr[b] : 0.f,
                       (uint32_t)v);
      out[b] = argmax_row(buf, V);
    }
    free(buf);
  }
}

/* ---------------------------------------------------------------------------------- */
/* Number formats. */

/* e4m3fn value of code c (0..255); NaN for 0x7F/0xFF. */
float vqko_e4m3_to_f32(uint8_t c) {
  int s = c >> 7, e = (c >> 3) & 15, m = c & 7;
  if (e == 15 && m == 7) return NAN;
  double v = (e == 0) ? ldexp((double)m, -9) : ldexp(1.0 + m / 8.0, e - 7);
  return (float)(s ? -v : v);
}

/* float -> e4m3fn with torch's semantics (dependency behaviour of
 * tensor.to(torch.float8_e4m3fn), used at src/vllm_quant_kernels/_quant.py:60, :309, :413):
 * nearest of the 127 finite magnitudes, ties to the even code; magnitudes above 464 (the
 * midpoint between 448 and the first unrepresentable step, 480) give NaN; sign kept. */
static float g_e4m3_mags[127];
__attribute__((constructor)) static void init_e4m3_mags(void) {
  for (int c = 0; c < 127; ++c) g_e4m3_mags[c] = vqko_e4m3_to_f32((uint8_t)c);
}

uint8_t vqko_f32_to_e4m3(float x) {
  const float *mags = g_e4m3_mags;
  uint8_t s = signbit(x) ? 0x80 : 0x00;
  if (x != x) return (uint8_t)(0x7F | s);
  double a = fabs((double)x);
  if (a > 464.0) return (uint8_t)(0x7F | s);
  int lo = 0, hi = 126;  /* largest code with mags[code] <= a */
  while (lo < hi) {
    int mid = (lo + hi + 1) / 2;
    if ((double)mags[mid] <= a) lo = mid; else hi = mid - 1;
  }
  int c = lo;
  if (c < 126) {
    double d0 = a - mags[c], d1 = (double)mags[c + 1] - a;
    if (d1 < d0 || (d1 == d0 && (c & 1))) c = c + 1;
  } else if (a > 448.0) {
    /* between 448 and 464: 448 is nearest (464 itself ties to the even code 0x7E) */
    c = 126;
  }
  return (uint8_t)(c | s);
}

/* E2M1 nibble by the reference's bucketize semantics (src/vllm_quant_kernels/_quant.py:91-99):
 * sign = (y < 0); idx = #{midpoints < min(|y|, 6)} with midpoints .25 .75 1.25 1.75 2.5 3.5 5. */
uint8_t vqko_f32_to_e2m1(float y) {
  static const float mid[7] = {0.25f, 0.75f, 1.25f, 1.75f, 2.5f, 3.5f, 5.0f};
  float m = fabsf(y);
  if (m > 6.0f) m = 6.0f;
  int idx = 0;
  for (int i = 0; i < 7; ++i) idx += (mid[i] < m);
  return (uint8_t)(((y < 0.0f) ? 8 : 0) | idx);
}

float vqko_e2m1_to_f32(uint8_t n) {
  static const float mag[8] = {0.f, 0.5f, 1.f, 1.5f, 2.f, 3.f, 4.f, 6.f};
  float v = mag[n & 7];
  return (n & 8) ? -v : v;
}

/* MX exponent k = clamp(ceil(log2(max(amax,1e-30)/qmax)), -127, 127)
 * (src/vllm_quant_kernels/_quant.py:50-55, :83-87), exactly, via frexp. */
int vqko_mx_exponent(float amax, float qmax) {
  float g = amax > 1e-30f ? amax : 1e-30f;
  float q = g / qmax;
  if (isinf(q)) return 127;
  int e;
  float m = frexpf(q, &e); /* q = m 2^e, m in [0.5, 1) */
  int k = (m == 0.5f) ? e - 1 : e;
  if (k < -127) k = -127;
  if (k > 127) k = 127;
  return k;
}

/* ---------------------------------------------------------------------------------- */
/* Quantizers (inputs are the exact float32 values of the fp16/bf16/fp32 tensors). */

/* Per-row INT8 (src/vllm_quant_kernels/_quant.py:245-302): s = max(amax/127, 1e-12);
 * q = clamp(rint(w/s), -127, 127).  s_out is the fp32 scale. */
void vqko_quant_rows_int8(const float *w, int64_t M, int64_t K, int8_t *q, float *s_out) {
#pragma omp parallel for schedule(static)
  for (int64_t m = 0; m < M; ++m) {
    const float *row = w + m * K;
    float a = 0.f;
    for (int64_t k = 0; k < K; ++k) { float v = fabsf(row[k]); if (v > a) a = v; }
    float s = a / 127.0f;
    if (s < 1e-12f) s = 1e-12f;
    for (int64_t k = 0; k < K; ++k) {
      float v = rintf(row[k] / s);
      if (v < -127.f) v = -127.f;
      if (v > 127.f) v = 127.f;
      q[m * K + k] = (int8_t)v;
    }
    s_out[m] = s;
  }
}

/* Per-row FP8 (src/vllm_quant_kernels/_quant.py:304-325). */
void vqko_quant_rows_fp8(const float *w, int64_t M, int64_t K, uint8_t *q, float *s_out) {
#pragma omp parallel for schedule(static)
  for (int64_t m = 0; m < M; ++m) {
    const float *row = w + m * K;
    float a = 0.f;
    for (int64_t k = 0; k < K; ++k) { float v = fabsf(row[k]); if (v > a) a = v; }
    float s = a / 448.0f;
    if (s < 1e-12f) s = 1e-12f;
    for (int64_t k = 0; k < K; ++k) {
      float v = row[k] / s;
      if (v < -448.f) v = -448.f;
      if (v > 448.f) v = 448.f;
      q[m * K + k] = vqko_f32_to_e4m3(v);
    }
    s_out[m] = s;
  }
}

/* MXFP8 / MXFP4 (src/vllm_quant_kernels/_quant.py:34-105).  fp4: q is [R, K/2] packed,
 * low nibble = even k. */
void vqko_quant_mx(const float *t, int64_t R, int64_t K, int fp4, uint8_t *q, uint8_t *scales) {
  const int64_t G = K / 32;
#pragma omp parallel for schedule(static)
  for (int64_t r = 0; r < R; ++r) {
    for (int64_t g = 0; g < G; ++g) {
      const float *v = t + r * K + g * 32;
      float a = 0.f;
      for (int i = 0; i < 32; ++i) { float x = fabsf(v[i]); if (x > a) a = x; }
      int k = vqko_mx_exponent(a, fp4 ? 6.0f : 448.0f);
      float sc = ldexpf(1.0f, k);
      scales[r * G + g] = (uint8_t)(k + 127);
      if (!fp4) {
        for (int i = 0; i < 32; ++i) {
          float y = v[i] / sc;
          if (y < -448.f) y = -448.f;
          if (y > 448.f) y = 448.f;
          q[r * K + g * 32 + i] = vqko_f32_to_e4m3(y);
        }
      } else {
        for (int i = 0; i < 32; i += 2) {
          uint8_t lo = vqko_f32_to_e2m1(v[i] / sc), hi = vqko_f32_to_e2m1(v[i + 1] / sc);
          q[r * (K / 2) + g * 16 + i / 2] = (uint8_t)(lo | (hi << 4));
        }
      }
    }
  }
}

/* Per-tensor INT8 activations (src/vllm_quant_kernels/_quant.py:535-540). */
void vqko_act_quant_int8(const float *x, int64_t n, int8_t *xq, float *xs) {
  float a = 0.f;
  for (int64_t i = 0; i < n; ++i) { float v = fabsf(x[i]); if (v > a) a = v; }
  float s = a / 127.0f;
  if (s < 1e-12f) s = 1e-12f;
  for (int64_t i = 0; i < n; ++i) {
    float v = rintf(x[i] / s);
    if (v < -127.f) v = -127.f;
    if (v > 127.f) v = 127.f;
    xq[i] = (int8_t)v;
  }
  *xs = s;
}

/* ---------------------------------------------------------------------------------- */
/* lm_head references: dequantize-then-matmul with double accumulation, returning the
 * fp32 value right before the final fp16 cast (the caller rounds it to fp16).
 * x is [B,K] float32 (the exact activation values the kernel consumes). */

/* W8A16 (src/vllm_quant_kernels/_kernels.py:49-84): fp32(acc) * s16. */
void vqko_lmhead_w8a16(const int8_t *w, const float *s16, const float *x, int64_t M, int64_t K, int64_t B,
                       float *out) {
#pragma omp parallel for schedule(static)
  for (int64_t m = 0; m < M; ++m) {
    const int8_t *row = w + m * K;
    for (int64_t b = 0; b < B; ++b) {
      double acc = 0.0;
      const float *xb = x + b * K;
      for (int64_t k = 0; k < K; ++k) acc += (double)row[k] * (double)xb[k];
      out[b * M + m] = (float)acc * s16[m];
    }
  }
}

/* W8A8 (src/vllm_quant_kernels/_kernels.py:453-476): exact int acc; fp32(acc)*ws*xs. */
void vqko_lmhead_w8a8(const int8_t *w, const float *ws, const int8_t *xq, float xs, int64_t M, int64_t K,
                      int64_t B, int32_t *acc_out, float *out) {
#pragma omp parallel for schedule(static)
  for (int64_t m = 0; m < M; ++m) {
    const int8_t *row = w + m * K;
    for (int64_t b = 0; b < B; ++b) {
      int64_t acc = 0;
      const int8_t *xb = xq + b * K;
      for (int64_t k = 0; k < K; ++k) acc += (int64_t)row[k] * (int64_t)xb[k];
      acc_out[b * M + m] = (int32_t)acc;
      out[b * M + m] = ((float)acc * ws[m]) * xs;
    }
  }
}

/* FP8 per-row (src/vllm_quant_kernels/_kernels.py:332-352): fp32(sum e4m3*e4m3) * s16. */
void vqko_lmhead_fp8(const uint8_t *w, const float *s16, const uint8_t *xq, int64_t M, int64_t K, int64_t B,
                     float *out) {
  float lut[256];
  for (int i = 0; i < 256; ++i) lut[i] = vqko_e4m3_to_f32((uint8_t)i);
#pragma omp parallel for schedule(static)
  for (int64_t m = 0; m < M; ++m) {
    const uint8_t *row = w + m * K;
    for (int64_t b = 0; b < B; ++b) {
      double acc = 0.0;
      const uint8_t *xb = xq + b * K;
      for (int64_t k = 0; k < K; ++k) acc += (double)lut[row[k]] * (double)lut[xb[k]];
      out[b * M + m] = (float)acc * s16[m];
    }
  }
}

/* MXFP8 / MXFP4 (src/vllm_quant_kernels/_kernels.py:588-632, :757-802):
 * sum_g 2^(ws-127) 2^(xs-127) sum_{k in g} w*x, fp32 result. */
void vqko_lmhead_mx(const uint8_t *w, const uint8_t *ws, const uint8_t *xq, const uint8_t *xs, int fp4,
                    int64_t M, int64_t K, int64_t B, float *out) {
  float lut8[256], lut4[16];
  for (int i = 0; i < 256; ++i) lut8[i] = vqko_e4m3_to_f32((uint8_t)i);
  for (int i = 0; i < 16; ++i) lut4[i] = vqko_e2m1_to_f32((uint8_t)i);
  const int64_t G = K / 32;
#pragma omp parallel for schedule(static)
  for (int64_t m = 0; m < M; ++m) {
    for (int64_t b = 0; b < B; ++b) {
      double acc = 0.0;
      for (int64_t g = 0; g < G; ++g) {
        double part = 0.0;
        for (int i = 0; i < 32; ++i) {
          int64_t k = g * 32 + i;
          double wv;
          if (fp4) {
            uint8_t byte = w[m * (K / 2) + k / 2];
            wv = lut4[(k & 1) ? (byte >> 4) : (byte & 15)];
          } else {
            wv = lut8[w[m * K + k]];
          }
          part += wv * (double)lut8[xq[b * K + k]];
        }
        acc += part * ldexp(1.0, (int)ws[m * G + g] - 127) * ldexp(1.0, (int)xs[b * G + g] - 127);
      }
      out[b * M + m] = (float)acc;
    }
  }
}

int vqko_max_threads(void) {
#ifdef _OPENMP
  return omp_get_max_threads();
#else
  return 1;
#endif
}

void vqko_set_threads(int n) {
#ifdef _OPENMP
  if (n > 0) omp_set_num_threads(n);
#else
  (void)n;
#endif
}

/* ---------------------------------------------------------------------------------- */
/* Array helpers for the Python side of the oracle. */
void vqko_f32_to_e4m3_array(const float *x, int64_t n, uint8_t *out) {
#pragma omp parallel for schedule(static)
  for (int64_t i = 0; i < n; ++i) out[i] = vqko_f32_to_e4m3(x[i]);
}
void vqko_f32_to_e2m1_array(const float *x, int64_t n, uint8_t *out) {
  for (int64_t i = 0; i < n; ++i) out[i] = vqko_f32_to_e2m1(x[i]);
}
void vqko_rand_array(uint64_t seed, const uint32_t *offsets, int64_t n, float *out) {
#pragma omp parallel for schedule(static)
  for (int64_t i = 0; i < n; ++i) out[i] = vqko_rand(seed, offsets[i]);
}
void vqko_philox_array(const uint32_t *ctr4, const uint32_t *key2, int64_t n, uint32_t *out4) {
  for (int64_t i = 0; i < n; ++i) vqko_philox4x32_10(ctr4 + 4 * i, key2 + 2 * i, out4 + 4 * i);
}
void vqko_logf_array(const float *x, int64_t n, float *out) {
#pragma omp parallel for schedule(static)
  for (int64_t i = 0; i < n; ++i) out[i] = vqko_logf(x[i]);
}
void vqko_gumbel_array(const float *u, int64_t n, float *out) {
#pragma omp parallel for schedule(static)
  for (int64_t i = 0; i < n; ++i) out[i] = vqko_gumbel(u[i]);
}
void vqko_mx_exponent_array(const float *amax, int64_t n, float qmax, int32_t *out) {
  for (int64_t i = 0; i < n; ++i) out[i] = vqko_mx_exponent(amax[i], qmax);
}
