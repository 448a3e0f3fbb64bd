// vqk_lmhead.hip - quantized lm_head projections for gfx950 (MI355X), all five modes.
//
// out[b, m] = epilogue_m( sum_k W[m, k] * X[b, k] ) for a [M, K] quantized weight that is
// streamed from HBM exactly once per launch (per launch of up to four batch groups).  One
// kernel template serves every mode and batch size; the work is shaped for CDNA4 rather
// than for a warp-GEMV:
//
//  * Hot path, lmhead_lds_kernel: persistent 256-thread workgroups (one per CU, two for
//    W8A16 at small batches).  Each wave owns 16-row tiles and streams them through a
//    ring of 2-4 LDS stages per wave: a stage is 256 bytes of each of the tile's 16 rows,
//    fetched by global_load_lds DMA (16 lanes x 16 bytes per row, contiguous, rotated by
//    16 bytes per row so the MFMA-layout ds_read_b128s that follow are conflict-free),
//    with the stage's MX scale bytes riding the same DMA.  One s_waitcnt covers a stage.
//  * MFMA per mode, A = 16 weight rows, B = 16 batch columns (zero-padded; one column
//    tile per 16 batch rows): W8A16 v_mfma_f32_16x16x32_f16 after an exact int8 -> fp16
//    byte permute; W8A8 v_mfma_i32_16x16x64_i8; FP8 and MXFP8
//    v_mfma_scale_f32_16x16x128_f8f6f4 (e4m3, E8M0 scales per 32-k group straight into
//    the instruction; 127 = 1.0 for FP8); MXFP4 the same instruction with E2M1 weights.
//    A lane's 32 k values of the scaled forms are exactly one MX group.
//  * Activations are staged once per workgroup in LDS in MFMA-fragment order by the
//    prologue, fused with the runtime activation quantization (per-tensor INT8, e4m3
//    cast, MXFP8), so every B operand is an immediate-offset ds_read_b128; large batches
//    quantize once in a separate launch instead.
//  * The epilogue applies the reference's per-row scale order and either stores each
//    tile's fp16 logits (batch 1) or holds them in registers until the weight stream ends
//    (a store burst then, instead of stores queued behind the weight loads).
//  * Batches beyond one group's LDS budget run up to four XCD-grouped batch groups in one
//    launch, so the later readers of each weight line find it in L2 or the last-level cache.
//  * Batch rows 17-64 at K = 3072 (9-32 per launch for W8A16), lmhead_wide_kernel: the
//    waves of a workgroup split K instead of rows (three compute waves, six for W8A16),
//    keep their slice of every row's activation fragments in VGPRs, pass the partial
//    accumulators from wave to wave through LDS, and a writer wave holds the logits until
//    the weight stream ends.
//  * Fallback, lmhead_kernel: when K or the scale alignment rules out 256-byte stages, a
//    512-thread kernel keeps a D-deep ring of 128-byte chunks per lane in registers; same
//    prologue, MFMA and epilogue code.
//
// Reference semantics: src/vllm_quant_kernels/_kernels.py (int8_gmv :8-84, int8_gemm
// :148-250, fp8_gemm :258-360, int8_w8a8_gemm :369-479, mxfp8_gemm :491-634, mxfp4_gemm
// :649-804) and the activation quantization in src/vllm_quant_kernels/_quant.py (:34-61,
// :413, :535-540).
#include <hip/hip_runtime.h>
#include <stdint.h>

#include "vqk.h"
#include "vqk_internal.h"
#include "vqk_math.h"

namespace vqk {

// Measured choices (MI355X, 248320 x 3072):
// - activation prologue: 8-element items per thread and round;
constexpr int LM_XU = 4;
// - logits held in registers for up to this many tiles per wave before a store burst
//   (32 slows batch 1 by ~1 us);
constexpr int LM_HOLD_TILES = 16;
// - register-ring kernel: up to two persistent workgroups per CU;
constexpr int LM_RING_WG_PER_CU = 2;
// - batch groups up to this size shrink the grid so every wave streams the same number
//   of tiles;
constexpr int LM_BALANCE_MAX_B = 8;
// - batch groups per launch of XCD-grouped workgroups;
constexpr int LM_MAX_GROUPS = 4;
// - cache policy of the weight DMA: non-temporal (one reader per line);
constexpr int LM_W_POLICY = 2;
// - cache policy of the MX scale pieces: temporal.  A stage reads 8-16 bytes of each row's
//   scale line and the following stages read the rest of that line, so the line must stay
//   in L2 (non-temporal pieces re-fetched it: 5.5% extra HBM reads, 3 us at MXFP4 batch 1).
constexpr int LM_S_POLICY = 0;
// - wide-batch kernel: weight ring stages per wave, and the smallest batch it serves;
constexpr int LM_WIDE_STAGES = 4;
// - wide-batch kernel: tiles of logits its writer wave holds in registers beyond those
//   that wait in LDS;
constexpr int LM_WIDE_HOLD_REGS = 24;
// (W8A16 at 248320 x 3072, us per call, row-tiled / wide: B=8 116.2-117.6 / 121.4-121.7
// (two column tiles), B=9 ~125 / 120.7-120.9 and B=16 123.5-126.1 / 120.3-120.9 (one
// tile), B=17 205-207 / 124-127)
constexpr int LM_WIDE_MIN_B_W8A16 = 9;
// (the other modes on one column tile, row-tiled / wide: FP8 B=16 123.5-124.9 /
// 122.2-123.8, B=12 121.3-122.7 / 121.1-122.5, B=9 120.4-121.0 / 121.1-121.5; MXFP8 B=16
// 124.8-125.6 / 124.4-124.7, B=12 equal, B=9 121.5-122.1 / 122.9-123.1; W8A8 B=16
// 125.9-127.9 / 124.9-126.1, B=13 125.9-126.5 / 124.2-124.7; MXFP4 B=16 70.8-71.5 /
// 69.5-70.0, B=13 70.1-70.8 / 69.2-69.6, B=9 68.6 / 70.1)
constexpr int LM_WIDE_MIN_B = 13;
// (batches above 64 rows, us per call, grouped row-tiled / balanced wide launches: FP8 80
// 240 / 252, 96 257 / 256, 128 315 / 268, 256 625 / 527; MXFP8 96 278 / 261, 128 342 / 271;
// W8A8 96 272 / 264, 128 335 / 278; MXFP4 80 176 / 166, 128 214 / 189)
constexpr int LM_WIDE_SPLIT_MIN_B = 96;

}  // namespace vqk

namespace vqk {

typedef int v4i __attribute__((ext_vector_type(4)));
typedef int v8i __attribute__((ext_vector_type(8)));
typedef float v4f __attribute__((ext_vector_type(4)));
typedef _Float16 v8h __attribute__((ext_vector_type(8)));
typedef _Float16 v2h __attribute__((ext_vector_type(2)));

enum Mode { M_W8A16 = 0, M_W8A8 = 1, M_FP8 = 2, M_MXFP8 = 3, M_MXFP4 = 4 };

template <int MODE>
struct ModeTraits;
// MPC: MFMAs per 128-byte chunk of a row; FB: bytes of one lane's B fragment;
// XB: LDS bytes per activation element; KPM: k values per MFMA (per row);
// MX: has E8M0 group scales; ACC_INT: int32 accumulator; ROWSCALE: per-row output scale.
template <> struct ModeTraits<M_W8A16> { enum { MPC = 4, FB = 16, XB = 2, KPM = 32, MX = 0, ACC_INT = 0, ROWSCALE = 1 }; };
template <> struct ModeTraits<M_W8A8>  { enum { MPC = 2, FB = 16, XB = 1, KPM = 64, MX = 0, ACC_INT = 1, ROWSCALE = 1 }; };
template <> struct ModeTraits<M_FP8>   { enum { MPC = 1, FB = 32, XB = 1, KPM = 128, MX = 0, ACC_INT = 0, ROWSCALE = 1 }; };
template <> struct ModeTraits<M_MXFP8> { enum { MPC = 1, FB = 32, XB = 1, KPM = 128, MX = 1, ACC_INT = 0, ROWSCALE = 0 }; };
template <> struct ModeTraits<M_MXFP4> { enum { MPC = 2, FB = 32, XB = 1, KPM = 128, MX = 1, ACC_INT = 0, ROWSCALE = 0 }; };

// Memory k of the activation element feeding byte/element p of lane k-block g's B fragment
// for the mi-th MFMA of a row.  It must pair with the weight addressing in load_chunk():
//  * W8A16 (16x16x32 f16, 8 elements per lane): mi = 4c + 2h + q, lane bytes
//    [128c + 64h + 16g, +16) of the row, q-th 8-byte half -> k = 128c + 64h + 16g + 8q + p;
//  * W8A8 (16x16x64 i8, 16 per lane): mi = 2c + h -> k = 128c + 64h + 16g + p;
//  * FP8 / MXFP8 / MXFP4 activations (16x16x128 f8f6f4, 32 per lane): the matrix core
//    reads a lane's 32 values as two halves, value p <-> k = 64*(p/16) + 16g + p%16 within
//    the MFMA's 128-k block, and 32-k scale block j = [32j, 32j+32) takes its E8M0 byte from
//    k-block lane j.  Mapping the MFMA's 128 k onto row k [128mi, 128mi + 128) in order
//    makes every scale block one MX group (4mi + j) of the row.
template <int MODE>
__device__ __forceinline__ int frag_k(int mi, int g, int p) {
  if (MODE == M_W8A16) {
    int c = mi >> 2, h = (mi >> 1) & 1, q = mi & 1;
    return 128 * c + 64 * h + 16 * g + 8 * q + p;
  } else if (MODE == M_W8A8) {
    int c = mi >> 1, h = mi & 1;
    return 128 * c + 64 * h + 16 * g + p;
  } else {
    return 128 * mi + 64 * (p >> 4) + 16 * g + (p & 15);
  }
}

struct LmArgs {
  const uint8_t* w;     // [M, KB] bytes
  const void* ws;       // per-row scales (fp16 or fp32) [M] or MX scales [M, K/32]
  const void* x;        // activations of this batch group, row stride ldx (or null)
  int xdt;              // dtype code of x (W8A16: fp16 only)
  const uint8_t* xq;    // pre-quantized e4m3 activations [Bg, K] (MX gemm forms) or null
  const uint8_t* xsq;   // pre-quantized E8M0 scales [Bg, K/32] or null
  const void* xall;     // W8A8: the whole activation tensor (amax is per-tensor)
  int64_t ldx;
  uint16_t* out;        // [Bg, ldo] (already offset to the group's first row)
  int64_t ldo;
  int32_t* acc;         // W8A8 optional [Bg, M]
  int M, K, Bg, Ball;
  int out_vec;          // 1 when 8-byte output stores are aligned
  float xs_val;         // W8A8 with pre-quantized activations: the per-tensor scale
  const float* xs_dev;  //   ... or, when not null, where to read it (device memory)
  int lds_x_bytes;      // LDS bytes of the staged activations (fragments + MX scales), 16-aligned
  int xr;               // LDS bytes per batch row of fragments (16 * odd)
  int xsr;              // MX: LDS dwords per batch row of activation scales (odd)
  int xs_off;           // MX: LDS byte offset of the activation scales
  int xvec;             // 1 when activation rows (x or xq) allow 16-byte loads
  // batch groups in one launch (XCD-grouped workgroups, see lmhead_lds_kernel), else 1;
  // group g's pointers are group 0's plus g times these strides; the last group's rows
  int ngrp;
  int64_t gs_x, gs_xq, gs_xsq, gs_out, gs_acc;
  int glast_Bg;
  int wide_cap;         // wide-batch kernel: tiles whose logits wait in LDS for the end
  // fused Gumbel-argmax epilogue (the sampling form only)
  const float* stemp;   // [Bg] temperatures or null (greedy)
  const void* sseeds;   // [Bg] int32 or int64 seeds
  int sseed64;
  unsigned long long* skeys;  // [Bg, waves of the launch] best key of each wave and row
};

// Per-lane state of the fused sampling epilogue: lane (g, j) sees batch row ct*16 + j of
// every column tile ct; its running best key over the rows it has scored, and that batch
// row's sampling parameters.
template <int NCT>
struct SmpLane {
  unsigned long long best[NCT];
  float T[NCT];
  uint32_t k0[NCT], k1[NCT];
  bool greedy[NCT];
};
template <int NCT>
__device__ __forceinline__ void smp_lane_init(const LmArgs& a, int lane, SmpLane<NCT>& sl) {
#pragma unroll
  for (int ct = 0; ct < NCT; ++ct) {
    const int b = min(ct * 16 + (lane & 15), a.Bg - 1);
    sl.best[ct] = 0ull;
    const float t = a.stemp ? a.stemp[b] : 0.f;
    sl.greedy[ct] = !a.stemp || t < 1e-5f;
    sl.T[ct] = t;
    uint64_t sd;
    if (a.sseed64) sd = ((const uint64_t*)a.sseeds)[b];
    else sd = (uint64_t)(int64_t)((const int32_t*)a.sseeds)[b];
    sl.k0[ct] = (uint32_t)sd;
    sl.k1[ct] = (uint32_t)(sd >> 32);
  }
}


// ---------------------------------------------------------------------------------------
// Prologue: stage the activations of this batch group into LDS in fragment order, one
// batch row after the other: fragment (mi, g) of row b lives at byte b*xr + (mi*4 + g)*FB, so
// consecutive MFMAs of a lane are a constant 4*FB apart.  xr/16 is odd, which puts the 16
// rows a ds_read_b128 serves in one pass on 16 different bank groups.
// MX scales: dword xs_off/4 + b*xsr + (mi/4)*4 + g holds byte (mi % 4) for fragment mi.
// Lanes of columns b >= Bg read row Bg-1 (their results are never stored), so no zero
// fragments are needed.
// A compile-time bool carried by value into a generic lambda (hoists a uniform branch out
// of an unrolled loop).
template <bool B_>
struct BoolTag {
  static constexpr bool value = B_;
};
template <int V_>
struct IntTag {
  static constexpr int value = V_;
};

template <int MODE, int DT>
__device__ __forceinline__ void stage_x_dt(const LmArgs& a, uint8_t* lds, uint32_t* lds_xs, float* lds_red) {
  typedef ModeTraits<MODE> T;
  const int tid = threadIdx.x, nth = blockDim.x;
  const int K = a.K, Bg = a.Bg;
  const int NMF = K / T::KPM;  // MFMAs per row
  const int nfrag = NMF * 4 * Bg;

  float xs_w8a8 = a.xs_val;
  // W8A8 with the whole activation in this group and at most 8 items per thread: one pass
  // (load, amax, scale, quantize from registers) instead of an amax pass and a quantize pass
  const bool w8a8_one = MODE == M_W8A8 && !a.xq && a.Ball == Bg && nfrag * (T::FB / 8) <= 8 * nth;
  if (MODE == M_W8A8 && !a.xq && !w8a8_one) {
    // per-tensor amax over the whole [Ball, K] activation (bit-exact max, order-free)
    float m = 0.f;
    if (a.xvec) {
      // 8 consecutive elements per step over the flattened [Ball, K/8] index space
      const int per_row = K >> 3, total = a.Ball * per_row;
#pragma unroll 4
      for (int c = tid; c < total; c += nth) {
        const int b = c / per_row, k8 = c - b * per_row;
        float v[8];
        load_run<DT, 8>(a.xall, (int64_t)b * a.ldx + 8 * k8, true, v);
#pragma unroll
        for (int e = 0; e < 8; ++e) m = fmaxf(m, fabsf(v[e]));
      }
    } else {
      for (int b = 0; b < a.Ball; ++b) {
#pragma unroll 8
        for (int k = tid; k < K; k += nth) m = fmaxf(m, fabsf(load_dt<DT>(a.xall, (int64_t)b * a.ldx + k)));
      }
    }
    for (int off = 32; off > 0; off >>= 1) m = fmaxf(m, __shfl_xor(m, off));
    if ((tid & 63) == 0) lds_red[tid >> 6] = m;
    __syncthreads();
    if (tid == 0) {
      float mm = 0.f;
      for (int i = 0; i < (nth >> 6); ++i) mm = fmaxf(mm, lds_red[i]);
      lds_red[16] = fmaxf(mm / 127.0f, 1e-12f);
    }
    __syncthreads();
    xs_w8a8 = lds_red[16];
  } else if (MODE == M_W8A8) {
    if (a.xs_dev) xs_w8a8 = *a.xs_dev;  // wave-uniform scalar read
    if (tid == 0) lds_red[16] = xs_w8a8;
  }
  const float xs_inv = 1.0f / xs_w8a8;  // W8A8: reciprocal for rint_div_i8 (IEEE division)

  if constexpr (T::MX) {
    const int G = K / 32;
    if (a.xq) {
      // pre-quantized bytes: one 32-element group (and its scale byte) per work item
      for (int f = tid; f < G * Bg; f += nth) {
        const int b = f % Bg, grp = f / Bg;
        const int mi = grp >> 2, j = grp & 3;
        const uint8_t* src = a.xq + (int64_t)b * K + 32 * grp;
        uint4 t0, t1;
        if (a.xvec) {
          t0 = ((const uint4*)src)[0];
          t1 = ((const uint4*)src)[1];
        } else {
          uint32_t v[8] = {0u, 0u, 0u, 0u, 0u, 0u, 0u, 0u};
#pragma unroll
          for (int e = 0; e < 32; ++e) v[e >> 2] |= (uint32_t)src[e] << (8 * (e & 3));
          t0 = make_uint4(v[0], v[1], v[2], v[3]);
          t1 = make_uint4(v[4], v[5], v[6], v[7]);
        }
        // the group's 32 bytes land in two 16-byte halves of the fragments of lanes
        // g = 2(j%2) and 2(j%2)+1 (j = group % 4), at byte 16*(j/2)
        uint8_t* d0 = lds + (size_t)b * a.xr + (size_t)(mi * 4 + 2 * (j & 1)) * T::FB + 16 * (j >> 1);
        *(uint4*)d0 = t0;
        *(uint4*)(d0 + T::FB) = t1;
        uint8_t* sdst = (uint8_t*)(lds_xs + (size_t)b * a.xsr + (mi >> 2) * 4 + j) + (mi & 3);
        *sdst = a.xsq[(int64_t)b * G + grp];
      }
    } else {
      // Quantize from the float activations: four lanes per group, 8 elements each (the
      // group's amax takes two lane exchanges), U items per thread and round with every
      // load of the round issued before the first encoding.  Lane quarter l of a group
      // writes bytes 8(l%2).. of half l/2 of the layout above.
      auto quantize = [&](auto vtag) {
        constexpr bool V = decltype(vtag)::value;
        constexpr int U = LM_XU;
        const int nit = 4 * G * Bg;  // a multiple of 4: a group's lanes share every trip
        for (int i0 = tid; i0 < nit; i0 += U * nth) {
          int f[U], l[U];
          bool ok[U];
          float xv[U][8];
#pragma unroll
          for (int u = 0; u < U; ++u) {
            const int it = i0 + u * nth;
            ok[u] = it < nit;  // the same for the 4 lanes of a group
            const int ic = ok[u] ? it : (it & 3);
            f[u] = ic >> 2;
            l[u] = ic & 3;
            const int b = f[u] % Bg, grp = f[u] / Bg;
            load_run<DT, 8>(a.x, (int64_t)b * a.ldx + 32 * grp + 8 * l[u], V, xv[u]);
          }
#pragma unroll
          for (int u = 0; u < U; ++u) {
            float amax = 0.f;
#pragma unroll
            for (int e = 0; e < 8; ++e) amax = fmaxf(amax, fabsf(xv[u][e]));
            amax = fmaxf(amax, __shfl_xor(amax, 1));
            amax = fmaxf(amax, __shfl_xor(amax, 2));
            const int kx = mx_exponent(amax, 448.0f);
            // x / 2^kx as x * 2^-kx: the same correctly rounded value (2^-kx is exact)
            const float isc = exp2i(-kx);
            float y[8];
#pragma unroll
            for (int e = 0; e < 8; ++e) y[e] = fminf(fmaxf(xv[u][e] * isc, -448.0f), 448.0f);
            const uint32_t v[2] = {e4m3x4_clamped(y[0], y[1], y[2], y[3]), e4m3x4_clamped(y[4], y[5], y[6], y[7])};
            if (!ok[u]) continue;
            const int b = f[u] % Bg, grp = f[u] / Bg;
            const int mi = grp >> 2, j = grp & 3;
            const int gl = 2 * (j & 1) + (l[u] >> 1), off = 16 * (j >> 1) + 8 * (l[u] & 1);
            *(uint2*)(lds + (size_t)b * a.xr + (size_t)(mi * 4 + gl) * T::FB + off) = make_uint2(v[0], v[1]);
            if (l[u] == 0) {
              uint8_t* sdst = (uint8_t*)(lds_xs + (size_t)b * a.xsr + (mi >> 2) * 4 + j) + (mi & 3);
              *sdst = (uint8_t)(kx + 127);
            }
          }
        }
      };
      if (a.xvec) quantize(BoolTag<true>{});
      else quantize(BoolTag<false>{});
    }
  } else if (MODE == M_W8A8 && w8a8_one) {
    auto one_pass = [&](auto vtag) {
      constexpr bool V = decltype(vtag)::value;
      constexpr int QU = 8, IPF = T::FB / 8;
      const int nit = nfrag * IPF;
      float xv[QU][8];
      int fb[QU], fgm[QU], sub[QU];
      bool ok[QU];
#pragma unroll
      for (int u = 0; u < QU; ++u) {
        const int it = tid + u * nth;
        ok[u] = it < nit;
        const int ic = ok[u] ? it : nit - 1;
        const int f = ic / IPF;
        sub[u] = ic - f * IPF;
        fb[u] = f % Bg;
        fgm[u] = f / Bg;
        const int g = fgm[u] & 3, mi = fgm[u] >> 2;
        load_run<DT, 8>(a.x, (int64_t)fb[u] * a.ldx + frag_k<MODE>(mi, g, 16 * (sub[u] >> 1)) + 8 * (sub[u] & 1),
                        V, xv[u]);
      }
      // the items cover the activation exactly once; idle slots repeat the last item,
      // which leaves a maximum unchanged
      float m = 0.f;
#pragma unroll
      for (int u = 0; u < QU; ++u)
#pragma unroll
        for (int e = 0; e < 8; ++e) m = fmaxf(m, fabsf(xv[u][e]));
      for (int off = 32; off > 0; off >>= 1) m = fmaxf(m, __shfl_xor(m, off));
      if ((tid & 63) == 0) lds_red[tid >> 6] = m;
      __syncthreads();
      if (tid == 0) {
        float mm = 0.f;
        for (int i = 0; i < (nth >> 6); ++i) mm = fmaxf(mm, lds_red[i]);
        lds_red[16] = fmaxf(mm / 127.0f, 1e-12f);
      }
      __syncthreads();
      const float xs = lds_red[16];
      const float xi = 1.0f / xs;
#pragma unroll
      for (int u = 0; u < QU; ++u) {
        uint32_t v[2] = {0u, 0u};
#pragma unroll
        for (int p = 0; p < 8; ++p) {
          float q = rint_div_i8(xv[u][p], xs, xi);
          q = fminf(fmaxf(q, -127.f), 127.f);
          v[p >> 2] |= (uint32_t)(uint8_t)(int8_t)(int)q << (8 * (p & 3));
        }
        if (ok[u]) *(uint2*)(lds + (size_t)fb[u] * a.xr + (size_t)fgm[u] * T::FB + 8 * sub[u]) = make_uint2(v[0], v[1]);
      }
    };
    if (a.xvec) one_pass(BoolTag<true>{});
    else one_pass(BoolTag<false>{});
  } else if (MODE != M_W8A16 && !a.xq) {
    // W8A8 (16-element fragments) or FP8 (32): quantize from the exact float, in items of 8
    // consecutive elements (a fragment's runs of 16 split in two), QU items per thread and
    // round with every load issued before the first conversion.
    auto quantize = [&](auto vtag) {
      constexpr bool V = decltype(vtag)::value;
      constexpr int QU = LM_XU, IPF = T::FB / 8;
      const int nit = nfrag * IPF;
      for (int i0 = tid; i0 < nit; i0 += QU * nth) {
        float xv[QU][8];
        int fb[QU], fgm[QU], sub[QU];
        bool ok[QU];
#pragma unroll
        for (int u = 0; u < QU; ++u) {
          const int it = i0 + u * nth;
          ok[u] = it < nit;
          const int ic = ok[u] ? it : nit - 1;
          const int f = ic / IPF;
          sub[u] = ic - f * IPF;
          fb[u] = f % Bg;
          fgm[u] = f / Bg;
          const int g = fgm[u] & 3, mi = fgm[u] >> 2;
          load_run<DT, 8>(a.x, (int64_t)fb[u] * a.ldx + frag_k<MODE>(mi, g, 16 * (sub[u] >> 1)) + 8 * (sub[u] & 1),
                          V, xv[u]);
        }
#pragma unroll
        for (int u = 0; u < QU; ++u) {
          uint32_t v[2] = {0u, 0u};
          if constexpr (MODE == M_W8A8) {
#pragma unroll
            for (int p = 0; p < 8; ++p) {
              float q = rint_div_i8(xv[u][p], xs_w8a8, xs_inv);
              q = fminf(fmaxf(q, -127.f), 127.f);
              v[p >> 2] |= (uint32_t)(uint8_t)(int8_t)(int)q << (8 * (p & 3));
            }
          } else {
            v[0] = e4m3x4_torch(xv[u][0], xv[u][1], xv[u][2], xv[u][3]);
            v[1] = e4m3x4_torch(xv[u][4], xv[u][5], xv[u][6], xv[u][7]);
          }
          if (ok[u]) *(uint2*)(lds + (size_t)fb[u] * a.xr + (size_t)fgm[u] * T::FB + 8 * sub[u]) = make_uint2(v[0], v[1]);
        }
      }
    };
    if (a.xvec) quantize(BoolTag<true>{});
    else quantize(BoolTag<false>{});
  } else {
    // W8A16 (fp16 copied as raw bits) or pre-quantized bytes: U fragments per thread per
    // round, every load of the round issued before the first store, so a round costs one
    // memory latency.
    constexpr int U = (MODE == M_FP8) ? 1 : 4;
    const bool vec = a.xvec != 0;
    for (int f0 = tid; f0 < nfrag; f0 += U * nth) {
      int fb[U], fgm[U];
      bool ok[U];
#pragma unroll
      for (int u = 0; u < U; ++u) {
        const int f = f0 + u * nth;
        ok[u] = f < nfrag;
        const int fc = ok[u] ? f : nfrag - 1;
        fb[u] = fc % Bg;
        fgm[u] = fc / Bg;
      }
      if constexpr (MODE == M_W8A16) {
        // fp16 fragments are 8 consecutive halves of the row: copied as raw bits
        uint4 raw[U];
#pragma unroll
        for (int u = 0; u < U; ++u) {
          const int g = fgm[u] & 3, mi = fgm[u] >> 2;
          const uint16_t* src = (const uint16_t*)a.x + (int64_t)fb[u] * a.ldx + frag_k<MODE>(mi, g, 0);
          if (vec) {
            raw[u] = *(const uint4*)src;
          } else {
            uint32_t v[4];
#pragma unroll
            for (int e = 0; e < 4; ++e) v[e] = (uint32_t)src[2 * e] | ((uint32_t)src[2 * e + 1] << 16);
            raw[u] = make_uint4(v[0], v[1], v[2], v[3]);
          }
        }
#pragma unroll
        for (int u = 0; u < U; ++u)
          if (ok[u]) *(uint4*)(lds + (size_t)fb[u] * a.xr + (size_t)fgm[u] * T::FB) = raw[u];
      } else {
        // pre-quantized bytes: element p of the fragment is row element frag_k(p), which
        // comes in runs of 16 consecutive bytes
        uint4 raw[U][T::FB / 16];
#pragma unroll
        for (int u = 0; u < U; ++u) {
          const int g = fgm[u] & 3, mi = fgm[u] >> 2;
#pragma unroll
          for (int r = 0; r < T::FB / 16; ++r) {
            const uint8_t* src = a.xq + (int64_t)fb[u] * K + frag_k<MODE>(mi, g, 16 * r);
            if (vec) {
              raw[u][r] = *(const uint4*)src;
            } else {
              uint32_t v[4] = {0u, 0u, 0u, 0u};
#pragma unroll
              for (int e = 0; e < 16; ++e) v[e >> 2] |= (uint32_t)src[e] << (8 * (e & 3));
              raw[u][r] = make_uint4(v[0], v[1], v[2], v[3]);
            }
          }
        }
#pragma unroll
        for (int u = 0; u < U; ++u) {
          if (!ok[u]) continue;
          uint8_t* dst = lds + (size_t)fb[u] * a.xr + (size_t)fgm[u] * T::FB;
#pragma unroll
          for (int r = 0; r < T::FB / 16; ++r) *(uint4*)(dst + 16 * r) = raw[u][r];
        }
      }
    }
  }
  __syncthreads();
}

// Activation prologue, dispatched on the activation dtype (pre-quantized input ignores it).
template <int MODE>
__device__ __forceinline__ void stage_x(const LmArgs& a, uint8_t* lds, uint32_t* lds_xs, float* lds_red) {
  if (MODE == M_W8A16 || a.xq || a.xdt == VQK_F16) stage_x_dt<MODE, VQK_F16>(a, lds, lds_xs, lds_red);
  else if (a.xdt == VQK_F32) stage_x_dt<MODE, VQK_F32>(a, lds, lds_xs, lds_red);
  else stage_x_dt<MODE, VQK_BF16>(a, lds, lds_xs, lds_red);
}

// ---------------------------------------------------------------------------------------
// One ring slot: the 32 weight bytes a lane owns in one 128-byte chunk of its row (plus the
// chunk's MX scale dwords).  FP8 modes keep them as one v8i so the MFMA A operand needs no
// register copy.
template <int MODE>
struct Slot {
  v4i lo, hi;
  uint32_t s0, s1;
};
template <>
struct Slot<M_FP8> {
  v8i w;
  uint32_t s0, s1;
};
template <>
struct Slot<M_MXFP8> {
  v8i w;
  uint32_t s0, s1;
};

// Loads lane k-block g's share of 128-byte chunk c of its row: two 16-byte pieces at
// [128c + 16g] and [128c + 64 + 16g], plus the chunk's MX scale dwords.  For the 8-bit
// operands the two pieces are the two halves the matrix core pairs with the activation
// halves (frag_k); for E2M1 each piece is one MFMA's A operand: 32 consecutive k of the row,
// i.e. one whole MX group (the fp4 A layout is 32 contiguous k per lane).
template <int MODE>
__device__ __forceinline__ void load_chunk(Slot<MODE>& s, const uint8_t* rowp, const uint32_t* srowp,
                                           int c, int g) {
  v4i lo = *(const v4i*)(rowp + 128 * c + 16 * g);
  v4i hi = *(const v4i*)(rowp + 128 * c + 64 + 16 * g);
  if constexpr (MODE == M_FP8 || MODE == M_MXFP8) {
    s.w = __builtin_shufflevector(lo, hi, 0, 1, 2, 3, 4, 5, 6, 7);
  } else {
    s.lo = lo;
    s.hi = hi;
  }
  if constexpr (MODE == M_MXFP8) {
    s.s0 = srowp[c];
  } else if constexpr (MODE == M_MXFP4) {
    s.s0 = srowp[2 * c];
    s.s1 = srowp[2 * c + 1];
  }
}

// int8 x4 (one dword) -> two packed fp16 pairs, exactly: (b ^ 0x80) | 0x6400 is the fp16
// value 1152 + b, so one packed subtraction of 1152 leaves b.
__device__ __forceinline__ void i8x4_to_h(uint32_t d, v2h& p0, v2h& p1) {
  uint32_t u = d ^ 0x80808080u;
  uint32_t a = __builtin_amdgcn_perm(0x64646464u, u, 0x04010400u);
  uint32_t b = __builtin_amdgcn_perm(0x64646464u, u, 0x04030402u);
  const v2h bias = {(_Float16)1152.0f, (_Float16)1152.0f};
  p0 = __builtin_bit_cast(v2h, a) - bias;
  p1 = __builtin_bit_cast(v2h, b) - bias;
}

template <int MODE>
struct AccT {
  typedef v4f type;
};
template <>
struct AccT<M_W8A8> {
  typedef v4i type;
};
template <int MODE, int NCT>
struct Acc {
  typename AccT<MODE>::type v[NCT];
  __device__ __forceinline__ void zero(int ct) { v[ct] = (typename AccT<MODE>::type)(0); }
};

// Per-lane activation pointers: xb[ct] = fragment (mi = 0, g) of column b = ct*16 + j
// (clamped to Bg-1), xsb[ct] = its MX scale dword for mi = 0.  Fragment mi is 4*FB*mi
// bytes further, its scale dword 4*(mi/4) dwords further.
template <int MODE, int NCT>
struct XPtr {
  const uint8_t* xb[NCT];
  const uint32_t* xsb[NCT];
};
template <int MODE, int NCT>
__device__ __forceinline__ XPtr<MODE, NCT> x_pointers(const LmArgs& a, const uint8_t* lds, const uint32_t* lds_xs,
                                                      int g, int j) {
  typedef ModeTraits<MODE> T;
  XPtr<MODE, NCT> p;
#pragma unroll
  for (int ct = 0; ct < NCT; ++ct) {
    const int b = (ct * 16 + j < a.Bg) ? ct * 16 + j : a.Bg - 1;
    p.xb[ct] = lds + b * a.xr + g * T::FB;
    p.xsb[ct] = lds_xs + b * a.xsr + g;
  }
  return p;
}

template <int MODE, int NCT>
__device__ __forceinline__ void compute_chunk(Acc<MODE, NCT>& acc, const Slot<MODE>& s, int c, int g,
                                              const XPtr<MODE, NCT>& xp) {
  typedef ModeTraits<MODE> T;
  constexpr int XS = 4 * T::FB;  // bytes between consecutive fragments of a lane
  if constexpr (MODE == M_W8A16) {
    uint32_t d[8] = {(uint32_t)s.lo.x, (uint32_t)s.lo.y, (uint32_t)s.lo.z, (uint32_t)s.lo.w,
                     (uint32_t)s.hi.x, (uint32_t)s.hi.y, (uint32_t)s.hi.z, (uint32_t)s.hi.w};
#pragma unroll
    for (int m = 0; m < 4; ++m) {  // m = 2h + q: dwords 2m, 2m+1
      v2h p0, p1, p2, p3;
      i8x4_to_h(d[2 * m], p0, p1);
      i8x4_to_h(d[2 * m + 1], p2, p3);
      v8h A = {p0.x, p0.y, p1.x, p1.y, p2.x, p2.y, p3.x, p3.y};
      const int mi = 4 * c + m;
#pragma unroll
      for (int ct = 0; ct < NCT; ++ct) {
        v8h Bv = *(const v8h*)(xp.xb[ct] + mi * XS);
        acc.v[ct] = __builtin_amdgcn_mfma_f32_16x16x32_f16(A, Bv, acc.v[ct], 0, 0, 0);
      }
    }
  } else if constexpr (MODE == M_W8A8) {
#pragma unroll
    for (int h = 0; h < 2; ++h) {
      v4i A = h ? s.hi : s.lo;
      const int mi = 2 * c + h;
#pragma unroll
      for (int ct = 0; ct < NCT; ++ct) {
        v4i Bv = *(const v4i*)(xp.xb[ct] + mi * XS);
        acc.v[ct] = __builtin_amdgcn_mfma_i32_16x16x64_i8(A, Bv, acc.v[ct], 0, 0, 0);
      }
    }
  } else if constexpr (MODE == M_FP8 || MODE == M_MXFP8) {
    const v8i A = s.w;
    const int mi = c;
    int sa = 127;
    if (MODE == M_MXFP8) sa = (int)(s.s0 >> (8 * g));
#pragma unroll
    for (int ct = 0; ct < NCT; ++ct) {
      const v4i* bp = (const v4i*)(xp.xb[ct] + mi * XS);
      v4i b0 = bp[0], b1 = bp[1];
      v8i Bv = __builtin_shufflevector(b0, b1, 0, 1, 2, 3, 4, 5, 6, 7);
      int sb = 127;
      if (MODE == M_MXFP8) sb = (int)(xp.xsb[ct][(mi >> 2) * 4] >> (8 * (mi & 3)));
      acc.v[ct] = __builtin_amdgcn_mfma_scale_f32_16x16x128_f8f6f4(A, Bv, acc.v[ct], 0, 0, 0, sa, 0, sb);
    }
  } else {  // MXFP4: two MFMAs per chunk, A = 32 E2M1 values (16 bytes) per lane
#pragma unroll
    for (int h = 0; h < 2; ++h) {
      v4i w = h ? s.hi : s.lo;
      // E2M1 operands occupy 4 VGPRs; the undefined upper half lets the backend pass
      // only those four to the MFMA.
      v8i A = __builtin_shufflevector(w, w, 0, 1, 2, 3, -1, -1, -1, -1);
      const int mi = 2 * c + h;
      int sa = (int)((h ? s.s1 : s.s0) >> (8 * g));
#pragma unroll
      for (int ct = 0; ct < NCT; ++ct) {
        const v4i* bp = (const v4i*)(xp.xb[ct] + mi * XS);
        v4i b0 = bp[0], b1 = bp[1];
        v8i Bv = __builtin_shufflevector(b0, b1, 0, 1, 2, 3, 4, 5, 6, 7);
        int sb = (int)(xp.xsb[ct][(mi >> 2) * 4] >> (8 * (mi & 3)));
        acc.v[ct] = __builtin_amdgcn_mfma_scale_f32_16x16x128_f8f6f4(A, Bv, acc.v[ct], 4, 0, 0, sa, 0, sb);
      }
    }
  }
}

// Epilogue of one 16-row tile: lane l holds D[4*(l/16) + e][l % 16], e = 0..3, i.e. rows
// m0 + 4*(l/16) + e of column b = ct*16 + (l % 16).
// Per-row dequantization scales of the 4 rows m0 + 4*(lane/16) + e a lane's accumulators
// hold (0 past M).  The loads are clamped to row M-1 rather than predicated, and the raw bits
// are kept apart from their conversion, so the loads can be issued a whole tile early.
template <int MODE>
__device__ __forceinline__ void row_scale_bits(const LmArgs& a, int m0, int lane, uint32_t (&raw)[4]) {
  const int mr = m0 + 4 * (lane >> 4);
#pragma unroll
  for (int e = 0; e < 4; ++e) {
    const int m = (mr + e < a.M) ? (mr + e) : (a.M - 1);
    if (MODE == M_W8A16 || MODE == M_FP8) raw[e] = ((const uint16_t*)a.ws)[m];
    else if (MODE == M_W8A8) raw[e] = ((const uint32_t*)a.ws)[m];
    else raw[e] = 0u;
  }
}
template <int MODE>
__device__ __forceinline__ void row_scales_from_bits(const LmArgs& a, int m0, int lane, const uint32_t (&raw)[4],
                                                     float (&sc)[4]) {
  const int mr = m0 + 4 * (lane >> 4);
#pragma unroll
  for (int e = 0; e < 4; ++e) {
    float v = 1.f;
    if (MODE == M_W8A16 || MODE == M_FP8) v = h2f((uint16_t)raw[e]);
    else if (MODE == M_W8A8) v = __uint_as_float(raw[e]);
    sc[e] = (mr + e < a.M) ? v : 0.f;
  }
}
template <int MODE>
__device__ __forceinline__ void row_scales(const LmArgs& a, int m0, int lane, float (&sc)[4]) {
  uint32_t raw[4];
  row_scale_bits<MODE>(a, m0, lane, raw);
  row_scales_from_bits<MODE>(a, m0, lane, raw, sc);
}

template <int MODE, int NCT>
__device__ __forceinline__ void epilogue(Acc<MODE, NCT>& acc, const LmArgs& a, int m0, int lane,
                                         float xs_w8a8, const float (&sc)[4], uint2 (&ov)[NCT],
                                         SmpLane<NCT>* sl = nullptr) {
  const int g = lane >> 4, j = lane & 15;
  const int mr = m0 + 4 * g;
#pragma unroll
  for (int ct = 0; ct < NCT; ++ct) {
    const int b = ct * 16 + j;
    if (b < a.Bg) {
      uint16_t o[4];
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        float r;
        if (MODE == M_W8A8) {
          r = ((float)acc.v[ct][e] * sc[e]) * xs_w8a8;
        } else if (MODE == M_W8A16 || MODE == M_FP8) {
          r = acc.v[ct][e] * sc[e];
        } else {
          r = acc.v[ct][e];
        }
        o[e] = f2h(r);
      }
      if (sl) {
        // Sampling epilogue: the score of each stored logit exactly as the stand-alone
        // sampler computes it from the fp16 logits converted to fp32 (y = fp32(fp16(r)),
        // then y / T + G(seed_b, m)), folded into the lane's running best key.
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          const int m = mr + e;
          if (m < a.M) {
            const float y = h2f(o[e]);
            float sy = y;
            if (!sl->greedy[ct]) {
              const float q = y / sl->T[ct];
              sy = q + gumbel_from_uniform(philox_uniform(philox_word0_vk((uint32_t)m, sl->k0[ct], sl->k1[ct])));
            }
            const unsigned long long k = make_key(sy, (uint32_t)m);
            sl->best[ct] = k > sl->best[ct] ? k : sl->best[ct];
          }
        }
      }
      ov[ct] = make_uint2((uint32_t)o[0] | ((uint32_t)o[1] << 16), (uint32_t)o[2] | ((uint32_t)o[3] << 16));
      if (MODE == M_W8A8) {
        if (a.acc) {
          int32_t* ap = a.acc + (int64_t)b * a.M + mr;
#pragma unroll
          for (int e = 0; e < 4; ++e)
            if (mr + e < a.M) ap[e] = acc.v[ct][e];
        }
      }
    }
    acc.zero(ct);
  }
}

// Store one tile's packed logits (lane (j, g): batch row ct*16 + j, rows mr..mr+3 of the
// tile at m0, mr = m0 + 4g), clipping the ragged last tile.
template <int NCT>
__device__ __forceinline__ void store_tile(const LmArgs& a, int m0, int lane, const uint2 (&ov)[NCT]) {
  const int g = lane >> 4, j = lane & 15;
  const int mr = m0 + 4 * g;
#pragma unroll
  for (int ct = 0; ct < NCT; ++ct) {
    const int b = ct * 16 + j;
    if (b >= a.Bg) continue;
    uint16_t* op = a.out + (int64_t)b * a.ldo + mr;
    if (mr + 3 < a.M && a.out_vec) {
      *(uint2*)op = ov[ct];
    } else {
      const uint32_t w[2] = {ov[ct].x, ov[ct].y};
#pragma unroll
      for (int e = 0; e < 4; ++e)
        if (mr + e < a.M) op[e] = (uint16_t)(w[e >> 1] >> (16 * (e & 1)));
    }
  }
}

template <int MODE, int NCT, int D>
__global__ void __launch_bounds__(512) __attribute__((amdgpu_waves_per_eu(4))) lmhead_kernel(LmArgs a) {
  typedef ModeTraits<MODE> T;
  extern __shared__ __attribute__((aligned(16))) uint8_t smem[];
  __shared__ float red[17];
  const int K = a.K;
  const int KB = (MODE == M_MXFP4) ? (K >> 1) : K;  // weight bytes per row
  uint8_t* lds = smem;
  uint32_t* lds_xs = (uint32_t*)(smem + a.xs_off);

  stage_x<MODE>(a, lds, lds_xs, red);
  const float xs_w8a8 = (MODE == M_W8A8) ? red[16] : 0.f;

  const int lane = threadIdx.x & 63;
  const int wave = threadIdx.x >> 6;
  const int nwaves = blockDim.x >> 6;
  const int r = lane & 15, g = lane >> 4;
  const XPtr<MODE, NCT> xp = x_pointers<MODE, NCT>(a, lds, lds_xs, g, r);
  const int ntiles = (a.M + 15) >> 4;
  const int wid = blockIdx.x * nwaves + wave;
  const int total = gridDim.x * nwaves;
  if (wid >= ntiles) return;
  const int my_tiles = (ntiles - 1 - wid) / total + 1;
  const int CPR = KB >> 7;  // 128-byte chunks per row; D divides CPR (host guarantees)
  const int nchunks = my_tiles * CPR;

  auto row_ptrs = [&](int tq, const uint8_t*& rp, const uint32_t*& sp) {
    int tile = wid + tq * total;
    int m = tile * 16 + r;
    m = (m < a.M) ? m : (a.M - 1);
    rp = a.w + (int64_t)m * KB;
    sp = T::MX ? (const uint32_t*)((const uint8_t*)a.ws + (int64_t)m * (K >> 5)) : nullptr;
  };

  Slot<MODE> ring[D];
  {
    const uint8_t* rp;
    const uint32_t* sp;
    row_ptrs(0, rp, sp);
#pragma unroll
    for (int d = 0; d < D; ++d) load_chunk<MODE>(ring[d], rp, sp, d, g);  // D <= CPR: all in tile 0
  }
  Acc<MODE, NCT> acc;
#pragma unroll
  for (int ct = 0; ct < NCT; ++ct) acc.zero(ct);

  for (int q0 = 0; q0 < nchunks; q0 += D) {
    const int tq = q0 / CPR;        // tile ordinal of this block of D chunks
    const int c0 = q0 - tq * CPR;   // first chunk index within the tile
    // the chunks loaded during this block are q0 + D .. q0 + 2D - 1 (same tile or next);
    // past the end of the wave's work the current chunks are re-read instead, so the loop
    // body has no branches and the loads stay unconditional (a few KB of extra reads)
    const int qn = q0 + D;
    const bool more = qn < nchunks;
    const int tqn = more ? qn / CPR : tq;
    const int cn0 = more ? qn - tqn * CPR : c0;
    const uint8_t* rpn;
    const uint32_t* spn;
    row_ptrs(tqn, rpn, spn);
#pragma unroll
    for (int d = 0; d < D; ++d) {
      compute_chunk<MODE, NCT>(acc, ring[d], c0 + d, g, xp);
      load_chunk<MODE>(ring[d], rpn, spn, cn0 + d, g);
      // keep each chunk's LDS reads next to its MFMAs: hoisting them across chunks only
      // raises register pressure (and occupancy is what hides the HBM latency here)
      __builtin_amdgcn_sched_barrier(0);
    }
    if (c0 + D == CPR) {
      float sc[4];
      row_scales<MODE>(a, (wid + tq * total) * 16, lane, sc);
      uint2 ov[NCT];
      epilogue<MODE, NCT>(acc, a, (wid + tq * total) * 16, lane, xs_w8a8, sc, ov);
      store_tile<NCT>(a, (wid + tq * total) * 16, lane, ov);
    }
  }
}

// ---------------------------------------------------------------------------------------
// LDS-staged variant (the default when K allows it).  Register loads in the MFMA layout touch
// 16 rows x 64 B per instruction; a plain stream of the weight measured ~6.0 TB/s that way,
// against ~6.6 TB/s for contiguous non-temporal loads.  So each wave streams its 16-row tile
// through LDS instead: a stage is 256 B of each of the 16 rows (4 KB), fetched with four
// global_load_lds_dwordx4 (instruction i: rows 4i..4i+3, 256 contiguous bytes each, 16 lanes
// per row, non-temporal) straight into the wave's LDS slot, and the MFMA operands are then
// read with ds_read_b128 in exactly the register layout load_chunk() produces.  Row r's byte c
// sits at slot + (r/4)*1024 + (r%4)*256 + ((c + 16r) & 255): the rotation by 16r makes the
// 16 rows of one ds_read_b128 hit distinct bank groups.  S slots per wave form the ring.
#define VQK_GPTR(p) ((const __attribute__((address_space(1))) void*)(p))
#define VQK_LPTR(p) ((__attribute__((address_space(3))) void*)(p))
constexpr int LDS_STAGE = 4096;
template <int N>
__device__ __forceinline__ void wait_vmcnt() {
  asm volatile("s_waitcnt vmcnt(%0)" ::"n"(N) : "memory");
}

// Row scales of a tile that lies inside M, through the scalar cache: one wave-uniform 32-byte
// (fp16 scales) or 64-byte (fp32) read per tile.  Scalar loads are counted by lgkmcnt, so the
// read neither waits for nor delays the weight stream's vmcnt accounting.  Needs a 4-byte
// aligned scale vector (host-checked).
template <int MODE>
__device__ __forceinline__ void tile_scales_smem(const LmArgs& a, int tile, uint32_t (&sdw)[16]) {
  typedef const __attribute__((address_space(4))) uint32_t* cp32;
  constexpr int ND = (MODE == M_W8A8) ? 16 : 8;
  const cp32 sp = (cp32)((uintptr_t)a.ws + (uintptr_t)tile * (4 * ND));
#pragma unroll
  for (int i = 0; i < ND; ++i) sdw[i] = sp[i];
}
// The 4 raw scales of rows 4g..4g+3 of the tile, out of its uniform dwords.  The dwords
// pass through readfirstlane so that the selects below stay register selects (a select
// between array elements would otherwise be folded into an indexed stack load).
__device__ __forceinline__ uint32_t pick4(uint32_t a0, uint32_t a1, uint32_t a2, uint32_t a3, int g) {
  const uint32_t x01 = (g & 1) ? a1 : a0;
  const uint32_t x23 = (g & 1) ? a3 : a2;
  return (g & 2) ? x23 : x01;
}
template <int MODE>
__device__ __forceinline__ void select_tile_scales(const uint32_t (&sdw)[16], int g, uint32_t (&raw)[4]) {
  constexpr int ND = (MODE == M_W8A8) ? 16 : 8;
  uint32_t d[16];
#pragma unroll
  for (int i = 0; i < ND; ++i) d[i] = __builtin_amdgcn_readfirstlane(sdw[i]);
  if constexpr (MODE == M_W8A8) {
#pragma unroll
    for (int e = 0; e < 4; ++e) raw[e] = pick4(d[e], d[4 + e], d[8 + e], d[12 + e], g);
  } else {
    const uint32_t lo = pick4(d[0], d[2], d[4], d[6], g);
    const uint32_t hi = pick4(d[1], d[3], d[5], d[7], g);
    raw[0] = lo & 0xFFFFu;
    raw[1] = lo >> 16;
    raw[2] = hi & 0xFFFFu;
    raw[3] = hi >> 16;
  }
}

// One stage of a wave: 256 weight bytes of each of its tile's 16 rows (4 KB, rows rotated as
// described above), then for MX modes the rows' E8M0 scales of those bytes (16 x 8 B for
// MXFP8, 16 x 16 B for MXFP4).  Weights and scales arrive by the same direct-to-LDS loads,
// so one vmcnt wait covers the whole stage.
template <int MODE>
struct StageGeom {
  static constexpr int SB = (MODE == M_MXFP8) ? 8 : (MODE == M_MXFP4) ? 16 : 0;  // scale bytes/row
  static constexpr int SLOT = LDS_STAGE + 16 * SB;
  static constexpr int NV = 4 + (SB ? 1 : 0);  // vector-memory instructions per stage
};

// Per-lane byte offsets, relative to the tile's first row, of the 4 weight pieces and of the
// scale piece this lane fetches for tile t (rows past M are clamped to M-1).
template <int MODE>
struct IssueOffsets {
  uint32_t w[4];
  uint32_t s;
};
template <int MODE>
__device__ __forceinline__ void issue_offsets(const LmArgs& a, int KB, int t, int lane, IssueOffsets<MODE>& o) {
  const int rr = lane >> 4, pp = 16 * (lane & 15);
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const int row = 4 * i + rr;
    const int m = min(16 * t + row, a.M - 1);
    o.w[i] = (uint32_t)((m - 16 * t) * KB + ((pp - 16 * row) & 255));
  }
  if constexpr (MODE == M_MXFP8) {  // lanes 0..31: row lane/2, dword lane%2 of its 8 bytes
    const int m = min(16 * t + ((lane >> 1) & 15), a.M - 1);
    o.s = (uint32_t)((m - 16 * t) * (a.K >> 5) + 4 * (lane & 1));
  } else if constexpr (MODE == M_MXFP4) {  // lanes 0..15: row lane, 16 bytes
    const int m = min(16 * t + (lane & 15), a.M - 1);
    o.s = (uint32_t)((m - 16 * t) * (a.K >> 5));
  } else {
    o.s = 0;
  }
}
template <int MODE>
__device__ __forceinline__ void issue_stage(const LmArgs& a, int KB, int t, int ks, uint8_t* slot, int lane,
                                            const IssueOffsets<MODE>& o) {
  typedef StageGeom<MODE> G;
  constexpr bool T8 = MODE == M_FP8 || MODE == M_MXFP8 || MODE == M_MXFP4;
  const uint8_t* tb = a.w + (int64_t)t * 16 * KB + 256 * ks;  // wave-uniform
  // One reader per weight line: non-temporal.  Several grouped readers (batch groups) of
  // the fp8/MX weights: the line stays cached for the others (measured: MXFP8 B=64
  // 237 -> 204 us; the int8 modes were slower with it, 211 -> 227 us for W8A16 B=32).
  if (T8 && a.ngrp >= 2) {
#pragma unroll
    for (int i = 0; i < 4; ++i)
      __builtin_amdgcn_global_load_lds(VQK_GPTR(tb + o.w[i]), VQK_LPTR(slot + 1024 * i), 16, 0, 0);
  } else {
#pragma unroll
    for (int i = 0; i < 4; ++i)
      __builtin_amdgcn_global_load_lds(VQK_GPTR(tb + o.w[i]), VQK_LPTR(slot + 1024 * i), 16, 0, LM_W_POLICY);
  }
  if constexpr (G::SB > 0) {
    const uint8_t* sb = (const uint8_t*)a.ws + (int64_t)t * 16 * (a.K >> 5) + G::SB * ks;
    if (MODE == M_MXFP8) {
      if (lane < 32)
        __builtin_amdgcn_global_load_lds(VQK_GPTR(sb + o.s), VQK_LPTR(slot + LDS_STAGE), 4, 0, LM_S_POLICY);
    } else {
      if (lane < 16)
        __builtin_amdgcn_global_load_lds(VQK_GPTR(sb + o.s), VQK_LPTR(slot + LDS_STAGE), 16, 0, LM_S_POLICY);
    }
  }
}

// Its LDS footprint allows one or two workgroups (one or two waves per SIMD) per CU, so
// the compiler may spend registers on keeping LDS reads in flight instead of aiming for an
// occupancy that cannot occur (without the hint the W8A16 loop waited on every fragment
// read once the held logits took their registers: 113 -> 131 us at batch 1).
template <int MODE, int NCT, int S, bool SMP = false>
__global__ void __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(1, 2))) lmhead_lds_kernel(LmArgs a0) {
  typedef ModeTraits<MODE> T;
  typedef StageGeom<MODE> G;
  extern __shared__ __attribute__((aligned(16))) uint8_t smem[];
  __shared__ float red[17];
  // G batch groups in one launch: the workgroups of run r of 8 consecutive workgroups
  // serve group r % G, so workgroups b, b + 8, ..., b + 8(G-1) (the same XCD under the
  // round-robin dispatch of workgroups to the 8 XCDs) stream the same weight tiles in
  // the same order for different batch rows, and all but the first reader of each line
  // find it in that XCD's L2 or in the last-level cache: the weight crosses HBM about
  // once instead of once per group.
  LmArgs a = a0;
  int bid = blockIdx.x, nwg = gridDim.x;
  if (a0.ngrp > 1) {
    const int G = a0.ngrp, run = bid >> 3;
    const int grp = run % G;
    bid = (run / G) * 8 + (bid & 7);
    nwg = gridDim.x / G;
    if (grp) {
      a.x = a0.x ? (const void*)((const char*)a0.x + grp * a0.gs_x) : nullptr;
      a.xq = a0.xq ? a0.xq + grp * a0.gs_xq : nullptr;
      a.xsq = a0.xsq ? a0.xsq + grp * a0.gs_xsq : nullptr;
      a.out = a0.out + grp * a0.gs_out;
      a.acc = a0.acc ? a0.acc + grp * a0.gs_acc : nullptr;
      if (grp == G - 1) a.Bg = a0.glast_Bg;
    }
  }
  const int K = a.K;
  const int KB = (MODE == M_MXFP4) ? (K >> 1) : K;
  uint8_t* lds = smem;
  uint32_t* lds_xs = (uint32_t*)(smem + a.xs_off);

  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);  // wave-uniform: scalar loop control
  const int r = lane & 15, g = lane >> 4;
  const int ntiles = (a.M + 15) >> 4;
  const int wid = bid * 4 + wave;
  const int total = nwg * 4;
  const bool live = wid < ntiles;
  const int my_tiles = live ? (ntiles - 1 - wid) / total + 1 : 0;
  const int SPT = KB >> 8;  // stages per tile (KB % 256 == 0, host guarantees)
  const int nst = my_tiles * SPT;
  uint8_t* ring = smem + a.lds_x_bytes + wave * (S * G::SLOT);

  // issue side: stage iq of the wave = (itile, iks)
  IssueOffsets<MODE> io;
  int itile = wid, iks = 0, iq = 0;
  issue_offsets<MODE>(a, KB, itile, lane, io);  // (idle waves, nst = 0, never use them)
  auto advance_issue = [&]() {
    ++iq;
    if (++iks == SPT) {
      iks = 0;
      itile += total;
      if (iq < nst) issue_offsets<MODE>(a, KB, itile, lane, io);
    }
  };
  auto fill_ring = [&]() {
#pragma unroll
    for (int s0 = 0; s0 < S; ++s0) {
      if (iq < nst) {
        issue_stage<MODE>(a, KB, itile, iks, ring + s0 * G::SLOT, lane, io);
        advance_issue();
      }
    }
  };

  stage_x<MODE>(a, lds, lds_xs, red);
  const float xs_w8a8 = (MODE == M_W8A8) ? red[16] : 0.f;

  if (!live) {
    if (SMP && (threadIdx.x & 63) < (unsigned)a.Bg) a.skeys[(int64_t)(threadIdx.x & 63) * total + wid] = 0ull;
    return;
  }
  const XPtr<MODE, NCT> xp = x_pointers<MODE, NCT>(a, lds, lds_xs, g, r);

  // lane (r, g) reads row r: its 4 pieces of a stage, rotated by 16r within the row's 256 B
  const uint32_t rbase = (uint32_t)((r >> 2) * 1024 + (r & 3) * 256);
  const uint8_t* wpc[4];
#pragma unroll
  for (int i = 0; i < 4; ++i) wpc[i] = ring + rbase + ((64 * i + 16 * g + 16 * r) & 255);
  const uint8_t* spc = ring + LDS_STAGE + G::SB * r;  // MX: row r's scale bytes of a stage

  fill_ring();

  Acc<MODE, NCT> acc;
#pragma unroll
  for (int ct = 0; ct < NCT; ++ct) acc.zero(ct);
  SmpLane<NCT> sl;
  if constexpr (SMP) smp_lane_init<NCT>(a, lane, sl);
  // From batch 2 up, the logits of up to HOLD tiles wait in registers and are stored
  // after the weight stream (measured: storing them tile by tile, in the same in-order
  // vector-memory queue as the weight stream, cost ~11 us at batch 16 and ~2 us at batch
  // 4; at batch 1 the per-tile stores are cheaper than the stores at the end, ~0.6 us).
  constexpr int HOLD = LM_HOLD_TILES;
  // With 32 batch columns a wave with more tiles flushes its HOLD held tiles at once
  // whenever the buffer is full (measured: FP8 / MXFP8 / W8A8 at batch 64, two paired
  // groups of 31 tiles per wave, 189-204 -> 179-192 us; MXFP4 there, and the 16-column
  // kernels at batch 4, were slower with the mid-stream flush compiled in).  Held tile k
  // (of nheld) is the wave's tile hfirst + k - (HOLD - nheld).
  constexpr bool MIDFLUSH = NCT == 2 && MODE != M_MXFP4;
  // smallest batch group that holds its logits (per-tile stores are cheaper below it;
  // medians at 248320 x 3072, held / per tile: MXFP4 B=2 62.0-62.5 / 61.2-61.3 us, B=3
  // 63.5-63.6 / 62.7-62.9, B=4 equal; MXFP8 B=2 114.7-115.0 / 114.2-114.3; FP8 and W8A8
  // B=4 114.8-117.5 / 116.3-118.8)
  constexpr int HOLD_MIN_B = (MODE == M_MXFP4) ? 4 : (MODE == M_MXFP8) ? 3 : 2;
  const bool hold = a.out_vec && a.Bg >= HOLD_MIN_B && (MIDFLUSH || my_tiles <= HOLD);
  uint2 ob[HOLD][NCT];
  int nheld = 0, hfirst = 0, wtile = 0;  // wave-uniform
  auto flush_held = [&]() {
#pragma unroll
    for (int k = 0; k < HOLD; ++k) {
      const int i = hfirst + k - (HOLD - nheld);
      if (k >= HOLD - nheld) store_tile<NCT>(a, (wid + i * total) * 16, lane, ob[k]);  // wave-uniform test
    }
    nheld = 0;
  };
  uint32_t sdw[16];  // the tile's row-scale dwords (wave-uniform), fetched at its first stage
  int ctile = wid, cks = 0;

  for (int q0 = 0; q0 < nst; q0 += S) {
#pragma unroll
    for (int s0 = 0; s0 < S; ++s0) {
      const int q = q0 + s0;
      if (q < nst) {
        // stage q has landed once at most the stages issued after it are outstanding
        if (iq == q + S) wait_vmcnt<(S - 1) * G::NV>();
        else wait_vmcnt<0>();
        const bool tile_full = ctile * 16 + 16 <= a.M;
        if (T::ROWSCALE && cks == 0 && tile_full) tile_scales_smem<MODE>(a, ctile, sdw);
        const int so = s0 * G::SLOT;
#pragma unroll
        for (int cc = 0; cc < 2; ++cc) {
          Slot<MODE> st;
          const v4i lo = *(const v4i*)(wpc[2 * cc] + so);
          const v4i hi = *(const v4i*)(wpc[2 * cc + 1] + so);
          if constexpr (MODE == M_FP8 || MODE == M_MXFP8) {
            st.w = __builtin_shufflevector(lo, hi, 0, 1, 2, 3, 4, 5, 6, 7);
          } else {
            st.lo = lo;
            st.hi = hi;
          }
          if constexpr (MODE == M_MXFP8) {
            st.s0 = *(const uint32_t*)(spc + so + 4 * cc);
          } else if constexpr (MODE == M_MXFP4) {
            typedef unsigned int v2u __attribute__((ext_vector_type(2)));
            const v2u t2 = *(const v2u*)(spc + so + 8 * cc);
            st.s0 = t2.x;
            st.s1 = t2.y;
          }
          compute_chunk<MODE, NCT>(acc, st, 2 * cks + cc, g, xp);
        }
        // Refill the slot before any epilogue work, so the stream keeps S stages in flight
        // while a tile's results are scaled, stored (and, in the sampling form, scored).
        // The slot's ds_reads have completed before the DMA may overwrite it.
        asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
        if (iq < nst) {
          issue_stage<MODE>(a, KB, itile, iks, ring + so, lane, io);
          advance_issue();
        }
        if (cks == SPT - 1) {
          float tsc[4];
          if (!T::ROWSCALE) {
            tsc[0] = tsc[1] = tsc[2] = tsc[3] = 1.f;
          } else if (tile_full) {
            uint32_t raw[4];
            select_tile_scales<MODE>(sdw, g, raw);
            row_scales_from_bits<MODE>(a, ctile * 16, lane, raw, tsc);
          } else {
            row_scales<MODE>(a, ctile * 16, lane, tsc);  // the ragged last tile
          }
          uint2 nv[NCT];
#pragma unroll
          for (int ct = 0; ct < NCT; ++ct) nv[ct] = make_uint2(0u, 0u);
          epilogue<MODE, NCT>(acc, a, ctile * 16, lane, xs_w8a8, tsc, nv, SMP ? &sl : nullptr);
          if (hold) {
            if (MIDFLUSH && nheld == HOLD) flush_held();
#pragma unroll
            for (int k = 0; k + 1 < HOLD; ++k)
#pragma unroll
              for (int ct = 0; ct < NCT; ++ct) ob[k][ct] = ob[k + 1][ct];
#pragma unroll
            for (int ct = 0; ct < NCT; ++ct) ob[HOLD - 1][ct] = nv[ct];
            if (nheld == 0) hfirst = wtile;
            ++nheld;
          } else {
            store_tile<NCT>(a, ctile * 16, lane, nv);
          }
          ++wtile;
        }
        if (++cks == SPT) {
          cks = 0;
          ctile += total;
        }
      }
    }
  }
  wait_vmcnt<0>();  // no DMA into LDS may still be in flight when the wave retires
  if (hold) flush_held();
  if constexpr (SMP) {
    // the wave's best key of each batch row: lanes j, j+16, j+32, j+48 hold row j's
#pragma unroll
    for (int ct = 0; ct < NCT; ++ct) {
      unsigned long long k = sl.best[ct];
#pragma unroll
      for (int off = 16; off <= 32; off <<= 1) {
        const unsigned long long o = __shfl_xor(k, off);
        k = o > k ? o : k;
      }
      const int b = ct * 16 + lane;
      if (lane < 16 && b < a.Bg) a.skeys[(int64_t)b * total + wid] = k;
    }
  }
}

// ---------------------------------------------------------------------------------------
// Wide-batch variant (33-64 batch rows in one pass over the weight).  With the activations
// of a 64-row batch in LDS there is no room for a weight ring (192 KB at K = 3072), and two
// 32-row groups stream every weight line through each CU twice while the activation
// fragments are re-read from LDS for every weight chunk (measured at FP8 batch 64: LDS
// traffic ~3x the weight bytes, 6-7x the bank conflicts of batch 1, MFMA busy 11%).
// Here the NW waves of a workgroup split K instead of rows: wave w owns bytes
// [w * SPW * 256, (w + 1) * SPW * 256) of every weight row and keeps the MFMA B fragments
// of its slice of all batch columns in VGPRs for the whole launch, so LDS holds only the
// weight ring (S stages per wave) and the accumulator hand-off.
// The waves form a pipeline over the workgroup's tiles: in step s wave w works on tile
// s - w, starting from the accumulators wave w - 1 left in LDS in step s - 1, and the last
// wave applies the epilogue.  Every tile's MFMA chain therefore runs over K in the same
// order as in lmhead_lds_kernel, so each batch row's logits are bit-identical to the same
// row computed in any other batch.  The weight stream runs ahead of the pipeline: every
// wave's ring is filled at the start, so the wave that starts computing NW - 1 steps late
// finds its stages landed.
template <int MODE>
struct FragT {
  typedef v8i type;  // 32-byte B fragments of the 16x16x128 f8f6f4 MFMA
};
template <>
struct FragT<M_W8A8> {
  typedef v4i type;
};
template <>
struct FragT<M_W8A16> {
  typedef v8h type;
};
template <int MODE, int NCT, int NMW>
struct XRegs {
  typename FragT<MODE>::type f[NCT][NMW];
  uint32_t sb[NCT][NMW];  // MX: the fragment's E8M0 byte in bits 0..7
};

// Copies this wave's fragments (MFMAs mi0 .. mi0 + NMW - 1 of every row) of the column tiles
// held by staged half h (batch rows 32h .. 32h + bh - 1) from the prologue's LDS layout into
// registers.  Columns past Bg repeat row Bg - 1, as in x_pointers().
template <int MODE, int NCT, int NMW>
__device__ __forceinline__ void load_xregs(XRegs<MODE, NCT, NMW>& xr, const LmArgs& a, const uint8_t* lds,
                                           const uint32_t* lxs, int h, int mi0, int g, int j) {
  typedef ModeTraits<MODE> T;
#pragma unroll
  for (int ct = 0; ct < NCT; ++ct) {
    if (ct / 2 != h) continue;
    const int b = min(ct * 16 + j, a.Bg - 1) - 32 * h;
    const uint8_t* xb = lds + b * a.xr + g * T::FB;
#pragma unroll
    for (int ml = 0; ml < NMW; ++ml) {
      const int mi = mi0 + ml;
      const v4i* p = (const v4i*)(xb + mi * 4 * T::FB);
      if constexpr (T::FB == 32) {
        const v4i b0 = p[0], b1 = p[1];
        xr.f[ct][ml] = __builtin_shufflevector(b0, b1, 0, 1, 2, 3, 4, 5, 6, 7);
      } else {
        xr.f[ct][ml] = __builtin_bit_cast(typename FragT<MODE>::type, p[0]);
      }
      if constexpr (T::MX) xr.sb[ct][ml] = lxs[b * a.xsr + (mi >> 2) * 4 + g] >> (8 * (mi & 3));
    }
  }
}

// Pre-quantized activations (a.xq, and a.xsq for MX): the wave's fragments straight from
// global memory into registers (row b's fragment (mi, g) is bytes frag_k(mi, g, 0..) of
// the row, in runs of 16; an MX fragment's scale is the E8M0 byte of group 4mi + g), every
// load issued before any is used, so the prologue costs one memory latency.
template <int MODE, int NCT, int NMW>
__device__ __forceinline__ void load_xregs_global(XRegs<MODE, NCT, NMW>& xr, const LmArgs& a, int mi0, int g, int j) {
  typedef ModeTraits<MODE> T;
  const int K = a.K;
  if constexpr (MODE == M_W8A16) {
    // fp16 activations as they are: fragment (mi, g) is the 8 elements from frag_k(mi, g, 0)
#pragma unroll
    for (int ct = 0; ct < NCT; ++ct) {
      const uint16_t* row = (const uint16_t*)a.x + (int64_t)min(ct * 16 + j, a.Bg - 1) * a.ldx;
#pragma unroll
      for (int ml = 0; ml < NMW; ++ml)
        xr.f[ct][ml] = __builtin_bit_cast(v8h, *(const v4i*)(row + frag_k<MODE>(mi0 + ml, g, 0)));
    }
    return;
  }
#pragma unroll
  for (int ct = 0; ct < NCT; ++ct) {
    const int b = min(ct * 16 + j, a.Bg - 1);
    const uint8_t* row = a.xq + (int64_t)b * K;
#pragma unroll
    for (int ml = 0; ml < NMW; ++ml) {
      const int mi = mi0 + ml;
      if constexpr (T::FB == 32) {
        const v4i b0 = *(const v4i*)(row + frag_k<MODE>(mi, g, 0));
        const v4i b1 = *(const v4i*)(row + frag_k<MODE>(mi, g, 16));
        xr.f[ct][ml] = __builtin_shufflevector(b0, b1, 0, 1, 2, 3, 4, 5, 6, 7);
      } else {
        xr.f[ct][ml] = __builtin_bit_cast(typename FragT<MODE>::type, *(const v4i*)(row + frag_k<MODE>(mi, g, 0)));
      }
      if constexpr (T::MX) xr.sb[ct][ml] = a.xsq[(int64_t)b * (K >> 5) + 4 * mi + g];
    }
  }
}

// compute_chunk() with the B fragments of the wave's local chunk cl taken from registers.
template <int MODE, int NCT, int NMW>
__device__ __forceinline__ void compute_chunk_reg(Acc<MODE, NCT>& acc, const Slot<MODE>& s, int cl, int g,
                                                  const XRegs<MODE, NCT, NMW>& xr) {
  if constexpr (MODE == M_W8A16) {
    uint32_t d[8] = {(uint32_t)s.lo.x, (uint32_t)s.lo.y, (uint32_t)s.lo.z, (uint32_t)s.lo.w,
                     (uint32_t)s.hi.x, (uint32_t)s.hi.y, (uint32_t)s.hi.z, (uint32_t)s.hi.w};
#pragma unroll
    for (int m = 0; m < 4; ++m) {
      v2h p0, p1, p2, p3;
      i8x4_to_h(d[2 * m], p0, p1);
      i8x4_to_h(d[2 * m + 1], p2, p3);
      v8h A = {p0.x, p0.y, p1.x, p1.y, p2.x, p2.y, p3.x, p3.y};
#pragma unroll
      for (int ct = 0; ct < NCT; ++ct)
        acc.v[ct] = __builtin_amdgcn_mfma_f32_16x16x32_f16(A, xr.f[ct][4 * cl + m], acc.v[ct], 0, 0, 0);
    }
  } else if constexpr (MODE == M_W8A8) {
#pragma unroll
    for (int h = 0; h < 2; ++h) {
      const v4i A = h ? s.hi : s.lo;
#pragma unroll
      for (int ct = 0; ct < NCT; ++ct)
        acc.v[ct] = __builtin_amdgcn_mfma_i32_16x16x64_i8(A, xr.f[ct][2 * cl + h], acc.v[ct], 0, 0, 0);
    }
  } else if constexpr (MODE == M_FP8 || MODE == M_MXFP8) {
    const int sa = (MODE == M_MXFP8) ? (int)(s.s0 >> (8 * g)) : 127;
#pragma unroll
    for (int ct = 0; ct < NCT; ++ct) {
      const int sb = (MODE == M_MXFP8) ? (int)xr.sb[ct][cl] : 127;
      acc.v[ct] = __builtin_amdgcn_mfma_scale_f32_16x16x128_f8f6f4(s.w, xr.f[ct][cl], acc.v[ct], 0, 0, 0, sa, 0, sb);
    }
  } else {  // MXFP4
#pragma unroll
    for (int h = 0; h < 2; ++h) {
      const v4i w = h ? s.hi : s.lo;
      const v8i A = __builtin_shufflevector(w, w, 0, 1, 2, 3, -1, -1, -1, -1);
      const int sa = (int)((h ? s.s1 : s.s0) >> (8 * g));
#pragma unroll
      for (int ct = 0; ct < NCT; ++ct)
        acc.v[ct] = __builtin_amdgcn_mfma_scale_f32_16x16x128_f8f6f4(A, xr.f[ct][2 * cl + h], acc.v[ct], 4, 0, 0,
                                                                     sa, 0, (int)xr.sb[ct][2 * cl + h]);
    }
  }
}

// How the K-split form deals its 16-row tiles to workgroups (µs per call at 248320 x 3072,
// contiguous ranges / groups of 4: FP8 B=64 135.4-135.6 / 134.5-135.3, MXFP8 B=64
// 138.4-138.5 / 136.9-137.0, W8A8 B=64 142.1-142.6 / 138.9-139.7, W8A16 B=32 within
// noise; MXFP4 B=32 72.9-73.0 / 75.3-76.2, and slower still with groups of 8, 16 or 32).
template <int MODE>
struct WideTileGroup {
  static constexpr int TG = (MODE == M_MXFP4) ? 0 : 4;
};

template <int MODE, int NCT, int NW, int SPW, int S>
__global__ void __launch_bounds__(64 * (NW + 1)) __attribute__((amdgpu_waves_per_eu(1, (NW + 4) / 4)))
lmhead_wide_kernel(LmArgs a) {
  typedef ModeTraits<MODE> T;
  typedef StageGeom<MODE> G;
  typedef typename AccT<MODE>::type AccV;
  constexpr int NMW = 2 * SPW * T::MPC;  // MFMAs per column tile of a wave's slice of a row
  extern __shared__ __attribute__((aligned(16))) uint8_t smem[];
  __shared__ float red[17];
  __shared__ int nreg_lds;
  // row stride of the writer's register tiles parked in the ring's LDS after the stream
  constexpr int HROW2 = LM_WIDE_HOLD_REGS * 32 + 16;
  static_assert(NCT * 16 * HROW2 <= NW * S * G::SLOT + 2 * NW * NCT * 64 * (int)sizeof(typename AccT<MODE>::type),
                "the parked tiles must fit the ring and hand-off space");
  const int K = a.K;
  const int KB = (MODE == M_MXFP4) ? (K >> 1) : K;
  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);  // NW = the writer
  const int r = lane & 15, g = lane >> 4;
  const int ntiles = (a.M + 15) >> 4;
  const int bid = blockIdx.x, nwg = gridDim.x;
  // Tiles go out in groups of TG consecutive tiles, group j to workgroup j mod nwg (TG = 0:
  // one contiguous range per workgroup), so the four tiles whose logits share a 128-byte
  // line of an output row are written from one CU; the tiles left after the last full round
  // go out one at a time (at most one more tile than another workgroup; >= 1 tile each: the
  // grid has at most ntiles workgroups).  Local tile i of a workgroup is global tile
  // gtile(i), increasing in i.
  constexpr int TG = WideTileGroup<MODE>::TG;
  const int full = TG ? ntiles / (TG * nwg) : 0;
  const int left = ntiles - TG * full * nwg;
  const int tpw = ntiles / nwg, trem = ntiles % nwg;
  const int my_tiles = TG ? TG * full + (bid < left ? (left - 1 - bid) / nwg + 1 : 0) : tpw + (bid < trem ? 1 : 0);
  const int t0 = bid * tpw + min(bid, trem);
  auto gtile = [&](int i) {
    if constexpr (TG == 0)
      return t0 + i;
    else
      return i < TG * full ? ((i / TG) * nwg + bid) * TG + (i % TG) : TG * full * nwg + bid + (i - TG * full) * nwg;
  };

  // Prologue: the activations in halves of up to 32 batch rows through the shared staging
  // code (which also quantizes them), each compute wave keeping its fragments in registers.
  XRegs<MODE, NCT, NMW> xr;
  float xs_w8a8 = 0.f;
  // (one pass per half, written out so the column tiles a pass fills are compile-time)
  auto stage_half = [&](auto htag) {
    constexpr int h = decltype(htag)::value;
    LmArgs ah = a;
    ah.Bg = min(32, a.Bg - 32 * h);
    if (h) {
      const int xes = (a.xdt == VQK_F32) ? 4 : 2;
      if (a.x) ah.x = (const void*)((const char*)a.x + (int64_t)32 * h * a.ldx * xes);
      if (a.xq) ah.xq = a.xq + (int64_t)32 * h * K;
      if (a.xsq) ah.xsq = a.xsq + (int64_t)32 * h * (K >> 5);
    }
    ah.xs_off = ah.Bg * a.xr;
    const uint32_t* lxs = (const uint32_t*)(smem + ah.xs_off);
    stage_x<MODE>(ah, smem, (uint32_t*)lxs, red);
    if (MODE == M_W8A8 && h == 0) xs_w8a8 = red[16];
    ah.Bg = a.Bg;  // load_xregs clamps against the whole group
    if (wave < NW) load_xregs<MODE, NCT, NMW>(xr, ah, smem, lxs, h, wave * NMW, g, r);
    __syncthreads();
  };
  // (pre-quantized activations in 16-byte aligned rows skip the staging, and so do W8A16's
  // fp16 activations, for which the host launches this form only with aligned rows)
  const bool direct = a.xq != nullptr && a.xvec && (!T::MX || a.xsq != nullptr);
  if constexpr (MODE == M_W8A16) {
    if (wave < NW) load_xregs_global<MODE, NCT, NMW>(xr, a, wave * NMW, g, r);
  } else if (direct) {
    if (MODE == M_W8A8) xs_w8a8 = a.xs_dev ? *a.xs_dev : a.xs_val;
    if (wave < NW) load_xregs_global<MODE, NCT, NMW>(xr, a, wave * NMW, g, r);
  } else {
    stage_half(IntTag<0>{});
    if constexpr (NCT > 2) stage_half(IntTag<1>{});
  }

  // LDS: the compute waves' rings, then the accumulator hand-off [2][NW][NCT][64 lanes]
  // (slot w of a step holds compute wave w's accumulators; slot NW - 1 the finished tile),
  // then the held logits [NCT * 16 batch rows][HROW bytes]: tile i's 16 rows at 32i.
  AccV* hand = (AccV*)(smem + NW * S * G::SLOT);
  uint8_t* hold = smem + NW * S * G::SLOT + 2 * NW * NCT * 64 * (int)sizeof(AccV);
  const int cap = a.wide_cap;
  const int hrow = cap * 32 + 16;  // +16: the 16 batch rows of one ds_write hit distinct banks
  const int nsteps = my_tiles + NW;
  if (wave == NW) {
    // The writer dequantizes each finished tile one step after the last compute wave
    // handed it over, and keeps its logits until the weight stream ends: the first cap
    // tiles in LDS, the next LM_WIDE_HOLD_REGS in its registers (each new tile shifts the
    // held ones down a slot), any further tile stored at once.  Logits written while the
    // weight streams cost ~20 % of the stream at batch 64, whatever their layout.
    uint32_t sdw[16];
    uint2 ob[LM_WIDE_HOLD_REGS][NCT];
    int nreg = 0;
    for (int s = 0; s < nsteps; ++s) {
      const int i = s - NW;
      if (i >= 0) {
        const int ctile = gtile(i);
        const bool tile_full = ctile * 16 + 16 <= a.M;
        if (T::ROWSCALE && tile_full) tile_scales_smem<MODE>(a, ctile, sdw);
        Acc<MODE, NCT> acc;
        const AccV* hp = hand + (((s - 1) & 1) * NW + NW - 1) * NCT * 64 + lane;
#pragma unroll
        for (int ct = 0; ct < NCT; ++ct) acc.v[ct] = hp[ct * 64];
        float tsc[4];
        if (!T::ROWSCALE) {
          tsc[0] = tsc[1] = tsc[2] = tsc[3] = 1.f;
        } else if (tile_full) {
          uint32_t raw[4];
          select_tile_scales<MODE>(sdw, g, raw);
          row_scales_from_bits<MODE>(a, ctile * 16, lane, raw, tsc);
        } else {
          row_scales<MODE>(a, ctile * 16, lane, tsc);
        }
        uint2 nv[NCT];
#pragma unroll
        for (int ct = 0; ct < NCT; ++ct) nv[ct] = make_uint2(0u, 0u);
        epilogue<MODE, NCT>(acc, a, ctile * 16, lane, xs_w8a8, tsc, nv, nullptr);
        if (i < cap) {
#pragma unroll
          for (int ct = 0; ct < NCT; ++ct) *(uint2*)(hold + (ct * 16 + r) * hrow + 32 * i + 8 * g) = nv[ct];
        } else if (nreg < LM_WIDE_HOLD_REGS) {
#pragma unroll
          for (int k = 0; k + 1 < LM_WIDE_HOLD_REGS; ++k)
#pragma unroll
            for (int ct = 0; ct < NCT; ++ct) ob[k][ct] = ob[k + 1][ct];
#pragma unroll
          for (int ct = 0; ct < NCT; ++ct) ob[LM_WIDE_HOLD_REGS - 1][ct] = nv[ct];
          ++nreg;
        } else {
          store_tile<NCT>(a, ctile * 16, lane, nv);
        }
      }
      asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory");
    }
    // the register-held tiles (slot k: tile cap + k - (LM_WIDE_HOLD_REGS - nreg)) go to the
    // ring's LDS once every compute wave is past its stream, in the held layout
    __syncthreads();
#pragma unroll
    for (int k = 0; k < LM_WIDE_HOLD_REGS; ++k) {
      const int i2 = k - (LM_WIDE_HOLD_REGS - nreg);
      if (i2 >= 0) {
#pragma unroll
        for (int ct = 0; ct < NCT; ++ct) *(uint2*)(smem + (ct * 16 + r) * HROW2 + 32 * i2 + 8 * g) = ob[k][ct];
      }
    }
    if (lane == 0) nreg_lds = nreg;
  } else {
  uint8_t* ring = smem + wave * (S * G::SLOT);
  IssueOffsets<MODE> io;
  const int nst = my_tiles * SPW;
  int ltile = 0, itile = gtile(0), iks = 0, iq = 0;
  issue_offsets<MODE>(a, KB, itile, lane, io);
  auto issue_next = [&](uint8_t* slot) {
    issue_stage<MODE>(a, KB, itile, wave * SPW + iks, slot, lane, io);
    ++iq;
    if (++iks == SPW) {
      iks = 0;
      itile = gtile(++ltile);
      if (iq < nst) issue_offsets<MODE>(a, KB, itile, lane, io);
    }
  };
#pragma unroll
  for (int s0 = 0; s0 < S; ++s0)
    if (iq < nst) issue_next(ring + s0 * G::SLOT);

  const uint32_t rbase = (uint32_t)((r >> 2) * 1024 + (r & 3) * 256);
  uint32_t wpo[4];
#pragma unroll
  for (int i = 0; i < 4; ++i) wpo[i] = rbase + ((64 * i + 16 * g + 16 * r) & 255);
  const uint32_t spo = LDS_STAGE + G::SB * r;

  int q = 0, slot = 0;
  for (int s = 0; s < nsteps; ++s) {
    const int i = s - wave;  // wave-uniform
    if (i >= 0 && i < my_tiles) {
      Acc<MODE, NCT> acc;
      if (wave == 0) {
#pragma unroll
        for (int ct = 0; ct < NCT; ++ct) acc.zero(ct);
      } else {
        const AccV* hp = hand + (((s - 1) & 1) * NW + wave - 1) * NCT * 64 + lane;
#pragma unroll
        for (int ct = 0; ct < NCT; ++ct) acc.v[ct] = hp[ct * 64];
      }
#pragma unroll
      for (int ks = 0; ks < SPW; ++ks) {
        if (iq == q + S) wait_vmcnt<(S - 1) * G::NV>();
        else wait_vmcnt<0>();
        const uint8_t* sp = ring + slot * G::SLOT;
#pragma unroll
        for (int cc = 0; cc < 2; ++cc) {
          Slot<MODE> st;
          const v4i lo = *(const v4i*)(sp + wpo[2 * cc]);
          const v4i hi = *(const v4i*)(sp + wpo[2 * cc + 1]);
          if constexpr (MODE == M_FP8 || MODE == M_MXFP8) {
            st.w = __builtin_shufflevector(lo, hi, 0, 1, 2, 3, 4, 5, 6, 7);
          } else {
            st.lo = lo;
            st.hi = hi;
          }
          if constexpr (MODE == M_MXFP8) {
            st.s0 = *(const uint32_t*)(sp + spo + 4 * cc);
          } else if constexpr (MODE == M_MXFP4) {
            typedef unsigned int v2u __attribute__((ext_vector_type(2)));
            const v2u t2 = *(const v2u*)(sp + spo + 8 * cc);
            st.s0 = t2.x;
            st.s1 = t2.y;
          }
          compute_chunk_reg<MODE, NCT, NMW>(acc, st, 2 * ks + cc, g, xr);
        }
        // the slot's ds_reads have completed before the DMA may overwrite it
        asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
        if (iq < nst) issue_next((uint8_t*)sp);
        ++q;
        if (++slot == S) slot = 0;
      }
      AccV* hp = hand + ((s & 1) * NW + wave) * NCT * 64 + lane;
#pragma unroll
      for (int ct = 0; ct < NCT; ++ct) hp[ct * 64] = acc.v[ct];
    }
    // hand-off written (lgkmcnt) before any wave reads it in the next step; the wave's
    // weight DMA stays in flight across the barrier
    asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory");
  }
  wait_vmcnt<0>();  // no DMA into LDS may still be in flight past this point
  __syncthreads();   // (the writer's first barrier after the stream)
  }
  // The weight stream is done: every wave stores the held logits, batch row by batch row,
  // in 16-byte pieces of consecutive rows (full 128-byte lines): first the cap tiles held
  // in LDS from the start, then the writer's register tiles parked in the ring's LDS.
  __syncthreads();
  const int nh = min(my_tiles, cap), n2 = nreg_lds;
  const bool vec16 = ((uintptr_t)a.out & 15) == 0 && (a.ldo & 7) == 0;
  auto flush = [&](const uint8_t* src, int rowb, int nt, int lfirst) {
    for (int u = threadIdx.x; u < a.Bg * 2 * nt; u += 64 * (NW + 1)) {
      const int b = u / (2 * nt), p = u - b * (2 * nt);
      const int r0 = gtile(lfirst + (p >> 1)) * 16 + 8 * (p & 1);
      const v4i v = *(const v4i*)(src + b * rowb + 16 * p);
      uint16_t* op = a.out + (int64_t)b * a.ldo + r0;
      if (vec16 && r0 + 8 <= a.M) {
        // non-temporal: the logits are not read back here, so they bypass the caches
        // (µs per call, cached / non-temporal: FP8 B=64 136.5-137.7 / 135.1-136.0, W8A8
        // B=64 142.3-143.3 / 140.3-141.3, W8A16 B=32 128.4-129.1 / 126.5-127.8, MXFP4 B=32
        // 73.8-74.1 / 72.8-73.8; MXFP8 B=64 138.1-138.4 / 138.9-139.8 keeps cached stores)
        if constexpr (MODE == M_MXFP8)
          *(v4i*)op = v;
        else
          __builtin_nontemporal_store(v, (v4i*)op);
      } else {
        const uint32_t w4[4] = {(uint32_t)v.x, (uint32_t)v.y, (uint32_t)v.z, (uint32_t)v.w};
#pragma unroll
        for (int e = 0; e < 8; ++e)
          if (r0 + e < a.M) op[e] = (uint16_t)(w4[e >> 1] >> (16 * (e & 1)));
      }
    }
  };
  flush(hold, hrow, nh, 0);
  if (n2 > 0) flush(smem, HROW2, n2, cap);
}

// The token of each batch row of a fused lm_head + sampling launch: one wave per row
// reduces the row's per-wave keys.
__global__ void __launch_bounds__(256) lmhead_sample_finish_kernel(const unsigned long long* skeys, int nslot,
                                                                   int B, int64_t* tokens) {
  const int row = blockIdx.x * 4 + (threadIdx.x >> 6), lane = threadIdx.x & 63;
  if (row >= B) return;
  unsigned long long k = 0ull;
  for (int i = lane; i < nslot; i += 64) {
    const unsigned long long o = skeys[(int64_t)row * nslot + i];
    k = o > k ? o : k;
  }
#pragma unroll
  for (int off = 32; off > 0; off >>= 1) {
    const unsigned long long o = __shfl_xor(k, off);
    k = o > k ? o : k;
  }
  if (lane == 0) tokens[row] = (int64_t)(~(uint32_t)(k & 0xFFFFFFFFull));
}

// ---------------------------------------------------------------------------------------
// Host side
// register-ring depth (chunks in flight per wave); 6 and 8 measured no faster than 4
static int pick_depth(int cpr) {
  if (cpr % 4 == 0) return 4;
  if (cpr % 2 == 0) return 2;
  return 1;
}

template <int MODE, int NCT>
static int launch_nct(const LmArgs& a, int depth, size_t lds_bytes, int grid, int threads,
                      hipStream_t st) {
  switch (depth) {
#define VQK_L(DD)                                                                                    \
  case DD:                                                                                           \
    hipLaunchKernelGGL((lmhead_kernel<MODE, NCT, DD>), dim3(grid), dim3(threads), lds_bytes, st, a); \
    break;
    VQK_L(1) VQK_L(2) VQK_L(4)
#undef VQK_L
    default:
      return VQK_EINVAL;
  }
  hipError_t e = hipGetLastError();
  return e == hipSuccess ? VQK_OK : (int)e;
}

template <int MODE, int NCT, bool SMP = false>
static int launch_lds(const LmArgs& a, int stages, size_t lds_bytes, int grid, hipStream_t st) {
  // gfx950 grants up to 160 KB of dynamic LDS per workgroup without an opt-in attribute;
  // rings of 6 and 8 stages measured no faster than 4
  if (stages == 4)
    hipLaunchKernelGGL((lmhead_lds_kernel<MODE, NCT, 4, SMP>), dim3(grid), dim3(256), lds_bytes, st, a);
  else if (stages == 3)
    hipLaunchKernelGGL((lmhead_lds_kernel<MODE, NCT, 3, SMP>), dim3(grid), dim3(256), lds_bytes, st, a);
  else
    hipLaunchKernelGGL((lmhead_lds_kernel<MODE, NCT, 2, SMP>), dim3(grid), dim3(256), lds_bytes, st, a);
  hipError_t e = hipGetLastError();
  return e == hipSuccess ? VQK_OK : (int)e;
}

// Wide-batch form: the K slice of a wave is SPW 256-byte stages of every weight row, and the
// waves of a workgroup cover the row (NW * SPW * 256 bytes).  Returns 0 when the row length
// has no such split.
// W8A16 keeps fp16 fragments (four per 128 weight bytes), so its K splits six ways (two
// waves per SIMD) and a launch covers at most 32 batch rows (2 column tiles: 128 VGPRs of
// fragments per wave).
template <int MODE>
struct WideShape {
  static constexpr int SPW = (MODE == M_MXFP4 || MODE == M_W8A16) ? 2 : 4;
  static constexpr int NW = (MODE == M_W8A16) ? 6 : 3;
  static constexpr int MAXB = (MODE == M_W8A16) ? 32 : 64;
  static constexpr int MINB = (MODE == M_W8A16) ? LM_WIDE_MIN_B_W8A16 : LM_WIDE_MIN_B;
  static constexpr int SPLIT_MIN_B = (MODE == M_W8A16 || MODE == M_MXFP4) ? MAXB + 1 : LM_WIDE_SPLIT_MIN_B;
  static bool fits(int KB) { return KB == NW * SPW * 256; }
};

template <int MODE, int NCT>
static int launch_wide(const LmArgs& a, size_t lds_bytes, int grid, hipStream_t st) {
  typedef WideShape<MODE> W;
  hipLaunchKernelGGL((lmhead_wide_kernel<MODE, NCT, W::NW, W::SPW, LM_WIDE_STAGES>), dim3(grid), dim3(64 * (W::NW + 1)),
                     lds_bytes, st, a);
  hipError_t e = hipGetLastError();
  return e == hipSuccess ? VQK_OK : (int)e;
}

// The fused sampling form's extra arguments.
struct SmpCall {
  const float* temp;
  const void* seeds;
  int seed64;
  int64_t* tokens;
  unsigned long long* skeys;
  int64_t slots_per_row;  // capacity of skeys per batch row
};
constexpr int64_t LM_SMP_SLOTS = 4096;  // per batch row: 4 waves x up to 1024 workgroups

// LDS layout of the staged activations (see stage_x_dt): fragment rows of xr bytes with
// xr/16 odd, then for MX modes scale rows of xsr dwords with xsr odd.
template <int MODE>
struct XLayout {
  int xr, xsr;
  static XLayout make(int64_t K) {
    typedef ModeTraits<MODE> T;
    XLayout l;
    const int NMF = (int)(K / T::KPM);
    l.xr = NMF * 4 * T::FB;
    if (((l.xr / 16) & 1) == 0) l.xr += 16;
    l.xsr = 0;
    if (T::MX) {
      l.xsr = ((NMF + 3) / 4) * 4;
      if ((l.xsr & 1) == 0) l.xsr += 1;
    }
    return l;
  }
  size_t per_row() const { return (size_t)xr + (size_t)xsr * 4; }
  size_t bytes(int Bg) const { return (((size_t)Bg * per_row()) + 15) & ~(size_t)15; }
};

template <int MODE>
static int lmhead_launch(const uint8_t* w, const void* ws, const void* x, int xdt, int64_t ldx,
                         const uint8_t* xq, const uint8_t* xsq, uint16_t* out, int64_t ldo,
                         int32_t* acc, int64_t M, int64_t K, int64_t B, hipStream_t st,
                         float xs_val = 0.f, const float* xs_dev = nullptr, const SmpCall* smp = nullptr) {
  typedef ModeTraits<MODE> T;
  typedef StageGeom<MODE> G;
  int rc = vqk_device_check();
  if (rc) return rc;
  if (!w || !ws || !out || (!x && !xq) || (xq && T::MX && !xsq)) return VQK_EINVAL;
  if (MODE == M_W8A16 && !x) return VQK_EINVAL;
  if (x && (xdt < VQK_F32 || xdt > VQK_BF16 || (MODE == M_W8A16 && xdt != VQK_F16))) return VQK_EINVAL;
  if (M < 1 || K < 1 || B < 0 || (x && ldx < K) || ldo < M) return VQK_EINVAL;
  if (B == 0) return VQK_OK;
  const int64_t kmult = (MODE == M_MXFP4) ? 256 : 128;
  // B is unbounded in practice (batch groups are launched in turn); the fused W8A8 prologue
  // indexes the whole [B, K/8] activation with 32-bit integers
  if (K % kmult != 0 || M > (int64_t)INT32_MAX - 16 || K > (1 << 20) || B > (1 << 24) ||
      B * (K / 8) > (int64_t)INT32_MAX)
    return VQK_EUNSUPPORTED;
  if (((uintptr_t)w & 15) != 0) return VQK_EUNSUPPORTED;

  const int KB = (int)((MODE == M_MXFP4) ? K / 2 : K);
  const int cpr = KB / 128;
  const int depth = pick_depth(cpr);
  const XLayout<MODE> xl = XLayout<MODE>::make(K);
  const size_t lds_cap = 150 * 1024;
  // The LDS-staged kernel needs whole 256-byte stages and 16-byte aligned scale rows; it
  // reserves 4 waves x 2 stages of ring next to the activations.
  const bool lds_path = KB % 256 == 0 && ((uintptr_t)ws & 15) == 0;
  const size_t ring2 = (size_t)4 * 2 * G::SLOT;
  // batch group size: up to 16*NCT rows, limited by LDS
  int gmax = (int)(((lds_path ? lds_cap - ring2 : lds_cap) - 64) / xl.per_row());
  if (gmax < 1) return VQK_EUNSUPPORTED;
  const int nct_max = (MODE == M_W8A16) ? 1 : 2;
  if (gmax > 16 * nct_max) gmax = 16 * nct_max;
  const int ngroups = (int)((B + gmax - 1) / gmax);
  const int gsize = (int)((B + ngroups - 1) / ngroups);  // balanced groups
  // the fused sampling form runs one batch group through the LDS kernel
  if (smp && (ngroups != 1 || !lds_path)) return VQK_EUNSUPPORTED;
  const int ncu = vqk_cu_count();
  const int threads = 512;

  int64_t adv = gsize;  // batch rows the iteration's launch covered
  for (int64_t b0 = 0; b0 < B; b0 += adv) {
    adv = gsize;
    const int Bg = (int)((B - b0) < gsize ? (B - b0) : gsize);
    LmArgs a;
    a.w = w;
    a.ws = ws;
    const int xes = (xdt == VQK_F32) ? 4 : 2;
    a.x = x ? (const void*)((const char*)x + b0 * ldx * xes) : nullptr;
    a.xdt = xdt;
    a.xq = xq ? xq + b0 * K : nullptr;
    a.xsq = xsq ? xsq + b0 * (K / 32) : nullptr;
    a.xall = x;
    a.ldx = ldx;
    a.out = out + b0 * ldo;
    a.ldo = ldo;
    a.acc = acc ? acc + b0 * M : nullptr;
    a.M = (int)M;
    a.K = (int)K;
    a.Bg = Bg;
    a.Ball = (int)B;
    a.out_vec = (((uintptr_t)out & 7) == 0 && (ldo & 3) == 0) ? 1 : 0;
    a.xs_val = xs_val;
    a.xs_dev = xs_dev;
    a.ngrp = 1;
    a.gs_x = a.gs_xq = a.gs_xsq = a.gs_out = a.gs_acc = 0;
    a.glast_Bg = Bg;
    a.stemp = smp ? smp->temp : nullptr;
    a.sseeds = smp ? smp->seeds : nullptr;
    a.sseed64 = smp ? smp->seed64 : 0;
    a.skeys = smp ? smp->skeys : nullptr;
    a.xr = xl.xr;
    if (xq) {
      a.xvec = ((uintptr_t)xq & 15) == 0 ? 1 : 0;  // rows are K bytes, K % 128 == 0
    } else {
      const int64_t es = (xdt == VQK_F32) ? 4 : 2;
      a.xvec = (((uintptr_t)x & 15) == 0 && (ldx * es) % 16 == 0) ? 1 : 0;
    }
    a.xsr = xl.xsr;
    a.xs_off = Bg * xl.xr;
    const size_t lds = xl.bytes(Bg);
    a.lds_x_bytes = (int)lds;
    const int ntiles = (int)((M + 15) / 16);
    {
      typedef WideShape<MODE> W;
      const int64_t left = B - b0;
      // W8A16 reads its fp16 activations straight into registers (aligned rows only).
      // Batches above MAXB rows run as balanced launches of at most MAXB, each streaming the
      // weight once (W8A16 and MXFP4 from MAXB + 1 rows, the 8-bit modes from 96).
      const bool xok = MODE != M_W8A16 || (xdt == VQK_F16 && a.xvec);
      const int64_t nwl = (left + W::MAXB - 1) / W::MAXB;
      const bool split_ok = left <= W::MAXB || left >= W::SPLIT_MIN_B;
      if (lds_path && !smp && xok && W::fits(KB) && left >= W::MINB && split_ok) {
        const int Bw = (int)((left + nwl - 1) / nwl);
        a.Bg = Bw;
        a.glast_Bg = Bw;
        // the kernel's column tiles (up to 16 rows on one tile: W8A16 from 9 rows, the other
        // modes from 13)
        const int nct_w = (Bw <= 16) ? 1 : (Bw <= 32 ? 2 : (Bw + 15) / 16);
        const size_t ring_w = (size_t)W::NW * LM_WIDE_STAGES * G::SLOT;
        const size_t hand_w = (size_t)2 * W::NW * nct_w * 64 * 16;
        const size_t pro_w = (MODE == M_W8A16) ? 0 : xl.bytes(Bw < 32 ? Bw : 32);
        const int grid_w = ntiles < ncu ? ntiles : ncu;
        // the most tiles a workgroup streams, and how many of them LDS can hold
        const int tmax = (ntiles + grid_w - 1) / grid_w;
        const size_t avail = (size_t)159 * 1024 - ring_w - hand_w;
        int cap = (int)((avail / ((size_t)nct_w * 16) - 16) / 32);
        if (cap > tmax) cap = tmax;
        a.wide_cap = cap;
        const size_t held_w = (size_t)nct_w * 16 * ((size_t)cap * 32 + 16);
        const size_t lds_w = (ring_w + hand_w + held_w > pro_w) ? ring_w + hand_w + held_w : pro_w;
        int rcw;
        if constexpr (W::MAXB <= 32)
          rcw = (nct_w == 1) ? launch_wide<MODE, 1>(a, lds_w, grid_w, st) : launch_wide<MODE, 2>(a, lds_w, grid_w, st);
        else
          rcw = (nct_w == 1)   ? launch_wide<MODE, 1>(a, lds_w, grid_w, st)
                : (nct_w <= 2)   ? launch_wide<MODE, 2>(a, lds_w, grid_w, st)
                : (nct_w == 3) ? launch_wide<MODE, 3>(a, lds_w, grid_w, st)
                               : launch_wide<MODE, 4>(a, lds_w, grid_w, st);
        if (rcw) return rcw;
        adv = Bw;
        continue;
      }
    }
    if (lds_path && lds + ring2 <= lds_cap) {
      // The deepest ring (4, 3 or 2 stages per wave) that fits next to the activations.
      // W8A16 prefers two workgroups per CU (two waves per SIMD) with a shallower ring when
      // both fit in the CU's 160 KB: its int8 -> fp16 conversion and four MFMAs per 128
      // bytes make one wave per SIMD issue-bound whenever the shader clock dips (measured
      // at batch 1 while the clock settles after a burst begins, 1.5-1.9 GHz: 135-158 us
      // with one workgroup per CU, 117-122 us with two); the other modes stream at the HBM
      // rate with one.
      auto fits = [&](int n, int per_cu) {
        return (size_t)per_cu * (lds + (size_t)4 * n * G::SLOT + 512) <= (per_cu == 1 ? lds_cap : 160 * 1024);
      };
      int per_cu_l = 1, stages = 0;
      // W8A16 at batch 1: four workgroups per CU on 2-stage rings where they fit (16 waves
      // hide the conversion and MFMA latency best while the shader clock settles: headline
      // window 118.9-119.6 vs 119.0-120.1 us, first 100 calls 117.2-117.4 vs 117.9-118.7,
      // steady state 112.5-112.8 vs 113.8-114.2 with two per CU; three per CU: 127)
      // FP8 and MXFP4 at 1-4 rows: two per CU (FP8 B=1 111.6-111.9 vs 113.1-114.5 us, MXFP4
      // B=4 63.2 vs 63.8-64.0; at 8 rows 0.5 us slower); MXFP8 keeps one (B=4 118.1-118.4 vs
      // 115.8-115.9), W8A8 measured the same either way.
      if (MODE == M_W8A16 && !smp && fits(2, 4)) stages = 2, per_cu_l = 4;
      if ((MODE == M_W8A16 || ((MODE == M_FP8 || MODE == M_MXFP4) && Bg <= 4)) && !smp)
        for (int n = 4; n >= 2 && !stages; --n)
          if (fits(n, 2)) stages = n, per_cu_l = 2;
      if (!stages) stages = fits(4, 1) ? 4 : fits(3, 1) ? 3 : 2;
      const size_t lds_l = lds + (size_t)4 * stages * G::SLOT;
      int grid_l = ncu * per_cu_l;
      const int max_grid_l = (ntiles + 3) / 4;
      if (grid_l > max_grid_l) grid_l = max_grid_l;
      if (Bg <= LM_BALANCE_MAX_B) {
        // as few waves as still give every wave the same (maximal) number of tiles, so
        // the stream keeps all of them busy to the end
        const int tpw = (ntiles + 4 * grid_l - 1) / (4 * grid_l);
        grid_l = ((ntiles + tpw - 1) / tpw + 3) / 4;
      }
      const int nct_l = (Bg + 15) / 16;
      int rcl;
      const int64_t left = (B - b0 + gsize - 1) / gsize;  // batch groups not yet launched
      const int G = (int)(left < LM_MAX_GROUPS ? left : LM_MAX_GROUPS);
      if (G >= 2 && !smp) {
        // G groups in one launch: 1/G of the CUs each, in XCD-aligned runs of 8
        // workgroups; every wave of the launch gets the same number of tiles (+-1)
        int gpg = (ncu / G) & ~7;
        const int maxg = (((ntiles + 3) / 4) + 7) & ~7;
        if (gpg > maxg) gpg = maxg;
        if (gpg >= 8) {
          const int xes2 = (xdt == VQK_F32) ? 4 : 2;
          a.ngrp = G;
          a.gs_x = (int64_t)gsize * ldx * xes2;
          a.gs_xq = (int64_t)gsize * K;
          a.gs_xsq = (int64_t)gsize * (K / 32);
          a.gs_out = (int64_t)gsize * ldo;
          a.gs_acc = (int64_t)gsize * M;
          a.glast_Bg = (int)(B - b0 - (int64_t)(G - 1) * gsize < gsize ? B - b0 - (int64_t)(G - 1) * gsize : gsize);
          const int nct_p = (gsize + 15) / 16;  // the larger groups' column tiles
          if constexpr (MODE == M_W8A16) {
            rcl = launch_lds<MODE, 1>(a, stages, lds_l, G * gpg, st);
          } else {
            rcl = (nct_p == 1) ? launch_lds<MODE, 1>(a, stages, lds_l, G * gpg, st)
                               : launch_lds<MODE, 2>(a, stages, lds_l, G * gpg, st);
          }
          if (rcl) return rcl;
          adv = (int64_t)G * gsize;
          continue;
        }
      }
      if (smp) {
        if (4 * (int64_t)grid_l > smp->slots_per_row) return VQK_EWORKSPACE;
        if constexpr (MODE == M_W8A16) {
          rcl = launch_lds<MODE, 1, true>(a, stages, lds_l, grid_l, st);
        } else {
          rcl = (nct_l == 1) ? launch_lds<MODE, 1, true>(a, stages, lds_l, grid_l, st)
                             : launch_lds<MODE, 2, true>(a, stages, lds_l, grid_l, st);
        }
        if (rcl) return rcl;
        hipLaunchKernelGGL(lmhead_sample_finish_kernel, dim3((unsigned)((Bg + 3) / 4)), dim3(256), 0, st,
                           smp->skeys, 4 * grid_l, Bg, smp->tokens);
        const hipError_t e = hipGetLastError();
        if (e != hipSuccess) return (int)e;
        continue;
      }
      if constexpr (MODE == M_W8A16) {
        rcl = launch_lds<MODE, 1>(a, stages, lds_l, grid_l, st);
      } else {
        rcl = (nct_l == 1) ? launch_lds<MODE, 1>(a, stages, lds_l, grid_l, st)
                           : launch_lds<MODE, 2>(a, stages, lds_l, grid_l, st);
      }
      if (rcl) return rcl;
      continue;
    }
    if (smp) return VQK_EUNSUPPORTED;  // the sampling form needs the LDS kernel
    int per_cu = (int)((150 * 1024) / (lds + 1024));
    if (per_cu > LM_RING_WG_PER_CU) per_cu = LM_RING_WG_PER_CU;
    if (per_cu < 1) per_cu = 1;
    int grid = ncu * per_cu;
    const int max_grid = (ntiles + (threads / 64) - 1) / (threads / 64);
    if (grid > max_grid) grid = max_grid;
    const int nct = (Bg + 15) / 16;
    int rc2;
    if constexpr (MODE == M_W8A16) {
      rc2 = launch_nct<MODE, 1>(a, depth, lds, grid, threads, st);
    } else {
      rc2 = (nct == 1) ? launch_nct<MODE, 1>(a, depth, lds, grid, threads, st)
                       : launch_nct<MODE, 2>(a, depth, lds, grid, threads, st);
    }
    if (rc2) return rc2;
  }
  return VQK_OK;
}

}  // namespace vqk

using namespace vqk;

extern "C" int vqk_lmhead_w8a16(const int8_t* w, const uint16_t* s_f16, const uint16_t* x_f16, int64_t ldx,
                                uint16_t* out_f16, int64_t ldo, int64_t M, int64_t K, int64_t B,
                                vqk_stream_t stream) {
  return lmhead_launch<M_W8A16>((const uint8_t*)w, s_f16, x_f16, VQK_F16, ldx, nullptr, nullptr, out_f16, ldo,
                                nullptr, M, K, B, (hipStream_t)stream);
}

extern "C" int vqk_lmhead_w8a8(const int8_t* w, const float* ws_f32, const void* x, int x_dtype, int64_t ldx,
                               uint16_t* out_f16, int64_t ldo, int32_t* acc_i32, int64_t M, int64_t K,
                               int64_t B, vqk_stream_t stream) {
  return lmhead_launch<M_W8A8>((const uint8_t*)w, ws_f32, x, x_dtype, ldx, nullptr, nullptr, out_f16, ldo,
                               acc_i32, M, K, B, (hipStream_t)stream);
}

extern "C" int vqk_lmhead_fp8(const uint8_t* w, const uint16_t* s_f16, const void* x, int x_dtype, int64_t ldx,
                              uint16_t* out_f16, int64_t ldo, int64_t M, int64_t K, int64_t B,
                              vqk_stream_t stream) {
  return lmhead_launch<M_FP8>(w, s_f16, x, x_dtype, ldx, nullptr, nullptr, out_f16, ldo, nullptr, M, K, B,
                              (hipStream_t)stream);
}

extern "C" int vqk_lmhead_mxfp8(const uint8_t* w, const uint8_t* ws, const void* x, int x_dtype, int64_t ldx,
                                uint16_t* out_f16, int64_t ldo, int64_t M, int64_t K, int64_t B,
                                vqk_stream_t stream) {
  return lmhead_launch<M_MXFP8>(w, ws, x, x_dtype, ldx, nullptr, nullptr, out_f16, ldo, nullptr, M, K, B,
                                (hipStream_t)stream);
}

extern "C" int vqk_lmhead_mxfp4(const uint8_t* w_packed, const uint8_t* ws, const void* x, int x_dtype,
                                int64_t ldx, uint16_t* out_f16, int64_t ldo, int64_t M, int64_t K, int64_t B,
                                vqk_stream_t stream) {
  return lmhead_launch<M_MXFP4>(w_packed, ws, x, x_dtype, ldx, nullptr, nullptr, out_f16, ldo, nullptr, M, K, B,
                                (hipStream_t)stream);
}

extern "C" int vqk_gemm_mxfp8(const uint8_t* w, const uint8_t* ws, const uint8_t* xq, const uint8_t* xs,
                              uint16_t* out_f16, int64_t ldo, int64_t M, int64_t K, int64_t B,
                              vqk_stream_t stream) {
  if (!xq || !xs) return VQK_EINVAL;
  return lmhead_launch<M_MXFP8>(w, ws, nullptr, VQK_F16, K, xq, xs, out_f16, ldo, nullptr, M, K, B,
                                (hipStream_t)stream);
}

extern "C" int vqk_gemm_mxfp4(const uint8_t* w_packed, const uint8_t* ws, const uint8_t* xq,
                              const uint8_t* xs, uint16_t* out_f16, int64_t ldo, int64_t M, int64_t K,
                              int64_t B, vqk_stream_t stream) {
  if (!xq || !xs) return VQK_EINVAL;
  return lmhead_launch<M_MXFP4>(w_packed, ws, nullptr, VQK_F16, K, xq, xs, out_f16, ldo, nullptr, M, K, B,
                                (hipStream_t)stream);
}

extern "C" int vqk_gemm_fp8(const uint8_t* w, const uint16_t* s_f16, const uint8_t* xq, uint16_t* out_f16,
                            int64_t ldo, int64_t M, int64_t K, int64_t B, vqk_stream_t stream) {
  if (!xq) return VQK_EINVAL;
  return lmhead_launch<M_FP8>(w, s_f16, nullptr, VQK_F16, K, xq, nullptr, out_f16, ldo, nullptr, M, K, B,
                              (hipStream_t)stream);
}

extern "C" int vqk_gemm_w8a8(const int8_t* w, const float* ws_f32, const int8_t* xq, float xs, uint16_t* out_f16,
                             int64_t ldo, int32_t* acc_i32, int64_t M, int64_t K, int64_t B, vqk_stream_t stream) {
  if (!xq) return VQK_EINVAL;
  return lmhead_launch<M_W8A8>((const uint8_t*)w, ws_f32, nullptr, VQK_F16, K, (const uint8_t*)xq, nullptr, out_f16,
                               ldo, acc_i32, M, K, B, (hipStream_t)stream, xs);
}

extern "C" int vqk_gemm_w8a8_devscale(const int8_t* w, const float* ws_f32, const int8_t* xq, const float* xs_dev,
                                      uint16_t* out_f16, int64_t ldo, int32_t* acc_i32, int64_t M, int64_t K,
                                      int64_t B, vqk_stream_t stream) {
  if (!xq || !xs_dev) return VQK_EINVAL;
  return lmhead_launch<M_W8A8>((const uint8_t*)w, ws_f32, nullptr, VQK_F16, K, (const uint8_t*)xq, nullptr, out_f16,
                               ldo, acc_i32, M, K, B, (hipStream_t)stream, 0.f, xs_dev);
}

extern "C" int64_t vqk_lmhead_sample_workspace_size(int64_t B) {
  return B < 0 ? 0 : B * LM_SMP_SLOTS * (int64_t)sizeof(unsigned long long);
}

extern "C" int vqk_lmhead_sample(int mode, const void* w, const void* ws, const void* x, int x_dtype, int64_t ldx,
                                 uint16_t* out_f16, int64_t ldo, int64_t M, int64_t K, int64_t B, const float* temp,
                                 const void* seeds, int seed_is_64bit, int64_t* tokens, void* workspace,
                                 int64_t ws_bytes, vqk_stream_t stream) {
  if (!x || !seeds || !tokens || !workspace) return VQK_EINVAL;
  if (B > 32 || M > (int64_t)UINT32_MAX / 2) return VQK_EUNSUPPORTED;
  if (ws_bytes < vqk_lmhead_sample_workspace_size(B)) return VQK_EWORKSPACE;
  if (((uintptr_t)workspace & 7) != 0) return VQK_EINVAL;
  SmpCall sc;
  sc.temp = temp;
  sc.seeds = seeds;
  sc.seed64 = seed_is_64bit ? 1 : 0;
  sc.tokens = tokens;
  sc.skeys = (unsigned long long*)workspace;
  sc.slots_per_row = LM_SMP_SLOTS;
  const hipStream_t st = (hipStream_t)stream;
  const uint8_t* wb = (const uint8_t*)w;
  switch (mode) {
    case VQK_MODE_W8A16:
      if (x_dtype != VQK_F16) return VQK_EINVAL;
      return lmhead_launch<M_W8A16>(wb, ws, x, VQK_F16, ldx, nullptr, nullptr, out_f16, ldo, nullptr, M, K, B, st,
                                    0.f, nullptr, &sc);
    case VQK_MODE_W8A8:
      return lmhead_launch<M_W8A8>(wb, ws, x, x_dtype, ldx, nullptr, nullptr, out_f16, ldo, nullptr, M, K, B, st,
                                   0.f, nullptr, &sc);
    case VQK_MODE_FP8:
      return lmhead_launch<M_FP8>(wb, ws, x, x_dtype, ldx, nullptr, nullptr, out_f16, ldo, nullptr, M, K, B, st,
                                  0.f, nullptr, &sc);
    case VQK_MODE_MXFP8:
      return lmhead_launch<M_MXFP8>(wb, ws, x, x_dtype, ldx, nullptr, nullptr, out_f16, ldo, nullptr, M, K, B, st,
                                    0.f, nullptr, &sc);
    case VQK_MODE_MXFP4:
      return lmhead_launch<M_MXFP4>(wb, ws, x, x_dtype, ldx, nullptr, nullptr, out_f16, ldo, nullptr, M, K, B, st,
                                    0.f, nullptr, &sc);
    default:
      return VQK_EINVAL;
  }
}
