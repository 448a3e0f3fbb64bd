/*
 * vqk.h - C ABI of the gfx950 (MI355X) kernels behind the vllm_quant_kernels plugin.
 *
 * The reference plugin (himikk/vllm-quant-kernels) has no native FFI: its hot path is
 * Python calling Triton kernels.  Each entry point below replaces one of those Triton
 * launches (or one torch op chain around them); the comment on each cites the
 * reference interface it stands in for.  A Python host binds these through ctypes
 * (vllm_quant_kernels/_lib.py).
 *
 * Conventions shared by every entry point:
 *   - All tensor pointers are DEVICE pointers.  fp16 / bf16 values are passed as their
 *     16-bit patterns (uint16_t); e4m3 (OCP float8_e4m3fn), packed E2M1 and E8M0 scales
 *     as uint8_t.  Matrices are row-major; ld* is the row stride in elements.
 *   - `stream` is a hipStream_t (NULL = the null stream).  Work is only enqueued; no
 *     entry point synchronises the stream.
 *   - Return value: VQK_OK (0) on success; a negative VQK_E* code when an argument is
 *     rejected before anything is launched; a positive hipError_t when the launch
 *     itself failed.
 *   - No entry point allocates device memory.  Stateless and reentrant, except
 *     vqk_gumbel_argmax, whose caller-provided workspace must not be shared by two
 *     launches that can run at the same time.
 */
#ifndef VQK_H
#define VQK_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

typedef struct ihipStream_t *vqk_stream_t;

enum {
  VQK_OK = 0,
  VQK_EINVAL = -1,       /* null pointer, negative size, bad enum value            */
  VQK_EUNSUPPORTED = -2, /* shape the kernels do not handle (see each function)    */
  VQK_ENODEVICE = -3,    /* no HIP device, or the device is not gfx950             */
  VQK_EWORKSPACE = -4    /* workspace too small                                    */
};

/* Element type codes for weight / activation inputs of the quantizers. */
enum { VQK_F32 = 0, VQK_F16 = 1, VQK_BF16 = 2 };

/* Library / device queries ---------------------------------------------------------- */

/* ABI version of this header (bumped on any signature change): 2. */
int vqk_abi_version(void);

/* Checks that the current HIP device is a gfx950 and records its CU count.
 * Returns VQK_OK or VQK_ENODEVICE.  Called implicitly by every launch. */
int vqk_device_check(void);

/* Human-readable text for a return code. */
const char *vqk_strerror(int code);

/* Weight quantizers (one-time, at the first _get_logits) ---------------------------- */

/* Per-row symmetric INT8: s[m] = max(amax_k |w[m,k]| / 127, 1e-12) (fp32);
 * q = clamp(round_half_even(w / s), -127, 127).
 * scale_out receives s as fp16 (scale_is_f32 = 0, the W8A16 layout) or fp32
 * (scale_is_f32 = 1, the W8A8 layout).
 * Replaces: QuantizedLogitsProcessor._init_int8_weights
 *           (src/vllm_quant_kernels/_quant.py:245-276) and _init_w8a8 (:278-302). */
int vqk_quant_rows_int8(const void *w, int w_dtype, int64_t M, int64_t K, int64_t ldw,
                        int8_t *q, void *scale_out, int scale_is_f32, vqk_stream_t stream);

/* Per-row FP8 e4m3: s[m] = max(amax/448, 1e-12); q = e4m3fn(clamp(w/s, -448, 448)) (RNE);
 * s stored as fp16.
 * Replaces: QuantizedLogitsProcessor._init_fp8 (src/vllm_quant_kernels/_quant.py:304-325). */
int vqk_quant_rows_fp8(const void *w, int w_dtype, int64_t M, int64_t K, int64_t ldw,
                       uint8_t *q, uint16_t *scale_f16, vqk_stream_t stream);

/* MXFP8: per 32-element group along K, k = clamp(ceil(log2(max(amax,1e-30)/448)), -127, 127),
 * scale byte k+127, q = e4m3fn(clamp(t / 2^k, -448, 448)).  K % 32 == 0.
 * q is [R,K] (row stride K), scales [R,K/32].
 * Replaces: _quantize_to_mxfp8 (src/vllm_quant_kernels/_quant.py:34-61). */
int vqk_quant_mxfp8(const void *t, int t_dtype, int64_t R, int64_t K, int64_t ldt,
                    uint8_t *q, uint8_t *scales, vqk_stream_t stream);

/* MXFP4: per 32-group, k = clamp(ceil(log2(max(amax,1e-30)/6)), -127, 127); y = t/2^k;
 * nibble = (y<0)<<3 | bucketize(min(|y|,6), [.25,.75,1.25,1.75,2.5,3.5,5]) (ties go to
 * the lower magnitude); byte j of a row = nib[2j] | nib[2j+1] << 4.  K % 32 == 0.
 * packed is [R,K/2], scales [R,K/32].
 * Replaces: _quantize_to_mxfp4 (src/vllm_quant_kernels/_quant.py:64-105). */
int vqk_quant_mxfp4(const void *t, int t_dtype, int64_t R, int64_t K, int64_t ldt,
                    uint8_t *packed, uint8_t *scales, vqk_stream_t stream);

/* Runtime activation quantizers (standalone forms; the lm_head entry points below fuse
 * the same arithmetic into their prologue) ------------------------------------------- */

/* Per-tensor INT8 over the whole [B,K] activation: xs = max(amax/127, 1e-12);
 * xq = clamp(round_half_even(x / xs), -127, 127).  xs is written to device memory.
 * Replaces: the torch chain in _w8a8_forward (src/vllm_quant_kernels/_quant.py:535-540),
 *           without its x_scale.item() host sync (:548). */
int vqk_act_quant_int8(const void *x, int x_dtype, int64_t ldx, int64_t B, int64_t K,
                       int8_t *xq, float *xs, vqk_stream_t stream);

/* Unscaled, unclamped cast to e4m3fn (RNE; |x| > 464 becomes NaN, as torch does).
 * Replaces: x.to(torch.float8_e4m3fn) in _fp8_forward (src/vllm_quant_kernels/_quant.py:413). */
int vqk_act_cast_e4m3(const void *x, int x_dtype, int64_t ldx, int64_t B, int64_t K,
                      uint8_t *xq, vqk_stream_t stream);

/* lm_head projections: out[b,m] (fp16, [B,M], row stride ldo) -------------------------
 * Shapes handled: K % 128 == 0 (K % 256 == 0 for MXFP4), M >= 1, 0 <= B <= 2^24 with
 * B * K / 8 < 2^31, row stride of every weight matrix = its logical width (contiguous
 * rows).  Batches larger than one launch's LDS budget are split in groups of up to 32
 * rows (W8A16: 16), launched up to four groups at a time; at K = 3072, 13-64 rows run as
 * one K-split launch (W8A16: 9-32 rows per launch, larger batches in balanced launches of
 * at most 32). */

/* W8A16: out = fp16( f32(s16[m]) * sum_k f32(w[m,k]) * f32(x[b,k]) ).
 * Replaces: int8_gmv (src/vllm_quant_kernels/_kernels.py:8-84) and int8_gemm (:148-250)
 *           as dispatched by _int8_forward (src/vllm_quant_kernels/_quant.py:560-643). */
int vqk_lmhead_w8a16(const int8_t *w, const uint16_t *s_f16, const uint16_t *x_f16,
                     int64_t ldx, uint16_t *out_f16, int64_t ldo, int64_t M, int64_t K,
                     int64_t B, vqk_stream_t stream);

/* The W8A8, FP8 and MX entry points read the activation x in its own dtype
 * (x_dtype = VQK_F16, VQK_BF16 or VQK_F32) and quantize it from its exact float32 value,
 * as the reference's x.float() / x.to(float8_e4m3fn) do.  W8A16 takes fp16 activations
 * (the reference converts them with x.to(torch.float16) before its kernel). */

/* W8A8: per-tensor INT8 activation quantization (as vqk_act_quant_int8) fused into the
 * prologue, acc = sum_k xq*wq in int32 (exact), out = fp16((f32(acc) * ws[m]) * xs).
 * acc_i32 (optional, [B,M] row stride M) receives the raw int32 accumulators.
 * Replaces: _w8a8_forward (src/vllm_quant_kernels/_quant.py:523-558) +
 *           int8_w8a8_gemm (src/vllm_quant_kernels/_kernels.py:369-479). */
int vqk_lmhead_w8a8(const int8_t *w, const float *ws_f32, const void *x, int x_dtype,
                    int64_t ldx, uint16_t *out_f16, int64_t ldo, int32_t *acc_i32,
                    int64_t M, int64_t K, int64_t B, vqk_stream_t stream);

/* FP8: e4m3 cast of x fused into the prologue; out = fp16(f32(s16[m]) * sum e4m3(w)*e4m3(x)).
 * Replaces: _fp8_forward (src/vllm_quant_kernels/_quant.py:399-430) +
 *           fp8_gemm (src/vllm_quant_kernels/_kernels.py:258-360). */
int vqk_lmhead_fp8(const uint8_t *w, const uint16_t *s_f16, const void *x, int x_dtype,
                   int64_t ldx, uint16_t *out_f16, int64_t ldo, int64_t M, int64_t K,
                   int64_t B, vqk_stream_t stream);

/* MXFP8: MXFP8 activation quantization fused into the prologue;
 * out = fp16( sum_g 2^(ws[m,g]-127) * 2^(xs[b,g]-127) * sum_{k in g} e4m3(w)*e4m3(x) ).
 * Replaces: _mxfp8_forward (src/vllm_quant_kernels/_quant.py:432-474) +
 *           mxfp8_gemm (src/vllm_quant_kernels/_kernels.py:491-634). */
int vqk_lmhead_mxfp8(const uint8_t *w, const uint8_t *ws, const void *x, int x_dtype,
                     int64_t ldx, uint16_t *out_f16, int64_t ldo, int64_t M, int64_t K,
                     int64_t B, vqk_stream_t stream);

/* MXFP4 (W4A8): E2M1 weights (two per byte, low nibble = even k), MXFP8 activations
 * quantized in the prologue; same output formula as MXFP8.
 * Replaces: _mxfp4_forward (src/vllm_quant_kernels/_quant.py:476-521) +
 *           mxfp4_gemm (src/vllm_quant_kernels/_kernels.py:649-804). */
int vqk_lmhead_mxfp4(const uint8_t *w_packed, const uint8_t *ws, const void *x,
                     int x_dtype, int64_t ldx, uint16_t *out_f16, int64_t ldo, int64_t M, int64_t K,
                     int64_t B, vqk_stream_t stream);

/* Pre-cast / pre-quantized activation forms, with the argument meaning of the reference's
 * factory-built kernels (activations already converted by the caller, [B,K] row stride K):
 *   vqk_gemm_fp8:  xq e4m3 (the reference casts on the host, _quant.py:413) -> fp8_gemm
 *                  (src/vllm_quant_kernels/_kernels.py:258-360, launched at _quant.py:419-425);
 *   vqk_gemm_w8a8: xq int8 + the per-tensor scale xs passed by value -> int8_w8a8_gemm
 *                  (src/vllm_quant_kernels/_kernels.py:369-479, launched at _quant.py:546-553). */
int vqk_gemm_fp8(const uint8_t *w, const uint16_t *s_f16, const uint8_t *xq, uint16_t *out_f16,
                 int64_t ldo, int64_t M, int64_t K, int64_t B, vqk_stream_t stream);
int vqk_gemm_w8a8(const int8_t *w, const float *ws_f32, const int8_t *xq, float xs,
                  uint16_t *out_f16, int64_t ldo, int32_t *acc_i32, int64_t M, int64_t K,
                  int64_t B, vqk_stream_t stream);
/* vqk_gemm_w8a8 with the per-tensor scale read from device memory (xs_dev: fp32 [1], as
 * vqk_act_quant_int8 writes it), so no host synchronisation separates the activation
 * quantization from the projection.  No counterpart in the reference, which passes
 * x_scale.item() by value (src/vllm_quant_kernels/_quant.py:548); the lm_head wrapper uses
 * it from batch 8 up, where quantizing the activations once per call beats doing it in
 * every workgroup's prologue. */
int vqk_gemm_w8a8_devscale(const int8_t *w, const float *ws_f32, const int8_t *xq,
                           const float *xs_dev, uint16_t *out_f16, int64_t ldo, int32_t *acc_i32,
                           int64_t M, int64_t K, int64_t B, vqk_stream_t stream);

/* Pre-quantized-activation forms of the two MX GEMMs: xq e4m3 [B,K] (row stride K) and
 * xs E8M0 [B,K/32] come from the caller, as the reference's factory-built kernels take them.
 * Replace: the kernels returned by _make_thor_mxfp8_gemm_kernel / _make_thor_mxfp4_gemm_kernel
 *          (src/vllm_quant_kernels/_kernels.py:491, :649), launched as in
 *          tests/test_mxfp4_kernel.py:28-54. */
int vqk_gemm_mxfp8(const uint8_t *w, const uint8_t *ws, const uint8_t *xq, const uint8_t *xs,
                   uint16_t *out_f16, int64_t ldo, int64_t M, int64_t K, int64_t B,
                   vqk_stream_t stream);
int vqk_gemm_mxfp4(const uint8_t *w_packed, const uint8_t *ws, const uint8_t *xq,
                   const uint8_t *xs, uint16_t *out_f16, int64_t ldo, int64_t M, int64_t K,
                   int64_t B, vqk_stream_t stream);

/* Fused Gumbel-argmax sampler ---------------------------------------------------------
 * For row b and vocab index v:  y = x                        if no temperature or T[b] < 1e-5
 *                               y = x / T[b] + G(seed_b, v)  otherwise,
 * G = -log(-log(max(u, 2^-126))), u = Philox4x32-10 word 0 of counter (v,0,0,0) and key
 * (seed lo32, seed hi32) mapped to [0,1) as Triton's uint_to_uniform_float does.
 * With topk_thr, y = -inf where x < thr[b] (raw logits).  out[b] = argmax_v y, smallest
 * index on ties.  Three launches on `stream` (candidates, survivors, finish); no host sync.
 *   logits   fp32 [B,V], row stride ld (elements), ld >= V.
 *   temp     fp32 [B] or NULL (NULL = plain argmax).
 *   seeds    int32 [B] (seed_is_64bit = 0; sign-extended to 64 bits) or int64 [B] (= 1).
 *   topk_thr fp32 [B] or NULL.
 *   out      int64 [B].
 *   workspace: >= vqk_gumbel_workspace_size(B, V) bytes of device memory, 8-byte aligned;
 *   no initialisation needed (every launch writes each value before reading it).
 * Replaces: fused_gumbel_sample + _gumbel_block_argmax_kernel
 *           (src/vllm_quant_kernels/_sampler_kernels.py:38-182). */
int64_t vqk_gumbel_workspace_size(int64_t B, int64_t V);
int vqk_gumbel_argmax(const float *logits, int64_t ld, int64_t B, int64_t V,
                      const float *temp, const void *seeds, int seed_is_64bit,
                      const float *topk_thr, int64_t *out, void *workspace,
                      int64_t ws_bytes, vqk_stream_t stream);

/* vqk_gumbel_argmax without a caller workspace, for callers that cannot allocate device
 * memory (code under HIP graph capture that may not hipMalloc, tight serving loops,
 * harnesses that forbid allocation).  It has no counterpart in the reference.  The
 * workspace is a static device array of vqk_gumbel_noalloc_max_bytes() = 1 MiB that the
 * library holds on each GPU it runs on until the process ends (at V = 248320, B <= 358
 * rows fit); larger calls return VQK_EWORKSPACE.  Calls that overlap on one GPU share the
 * array and race: issue them on one stream.  Same arguments and results as
 * vqk_gumbel_argmax minus the workspace; no allocation, no memset. */
int64_t vqk_gumbel_noalloc_max_bytes(void);
int vqk_gumbel_argmax_noalloc(const float *logits, int64_t ld, int64_t B, int64_t V,
                              const float *temp, const void *seeds, int seed_is_64bit,
                              const float *topk_thr, int64_t *out, vqk_stream_t stream);

/* Fused lm_head + Gumbel-argmax sampling (opt-in; one batch group: B <= 32 rows, and
 * B <= 16 for VQK_MODE_W8A16, else VQK_EUNSUPPORTED).
 * Runs the `mode` projection exactly as vqk_lmhead_<mode> does (same arguments: w, ws,
 * x, x_dtype, ldx, out_f16, ldo, M, K, B; for VQK_MODE_MXFP4, w is the packed [M,K/2] form
 * and K the logical K; W8A16 takes fp16 x only) and, in the same launch's epilogue,
 * scores every stored logit as vqk_gumbel_argmax does with the fp32 value of the fp16
 * logit: y = fp32(out[b,m]), greedy rows (temp NULL or T[b] < 1e-5) take y, the others
 * y / T[b] + G(seed_b, m).  A second, tiny launch reduces the per-wave best keys to
 * tokens[b] (int64 [B]).  The tokens equal those of vqk_lmhead_<mode> followed by
 * vqk_gumbel_argmax on the fp32-converted logits, bit for bit; the logits are still
 * written to out_f16.  No top-k (its threshold depends on the finished logits).
 *   workspace: >= vqk_lmhead_sample_workspace_size(B) bytes, 8-byte aligned, no
 *   initialisation needed.
 * Replaces: _quantized_forward (src/vllm_quant_kernels/_quant.py:382-397) followed by
 *           FusedSampler.sample's fast path (src/vllm_quant_kernels/_sampler.py:144-206);
 *           the reference runs them as separate launches with the logits in between. */
enum { VQK_MODE_W8A16 = 0, VQK_MODE_W8A8 = 1, VQK_MODE_FP8 = 2, VQK_MODE_MXFP8 = 3, VQK_MODE_MXFP4 = 4 };
int64_t vqk_lmhead_sample_workspace_size(int64_t B);
int vqk_lmhead_sample(int mode, const void *w, const void *ws, const void *x, int x_dtype,
                      int64_t ldx, uint16_t *out_f16, int64_t ldo, int64_t M, int64_t K, int64_t B,
                      const float *temp, const void *seeds, int seed_is_64bit, int64_t *tokens,
                      void *workspace, int64_t ws_bytes, vqk_stream_t stream);

/* Per-row top-k threshold on the device: thr[b] = the max(top_k[b], 1)-th largest raw
 * logit of row b (NaN ranked largest), or -inf for every row when max_b top_k[b] >= V
 * (the reference's "all rows disabled" case, where it passes no threshold; -inf masks
 * nothing).  Feeds vqk_gumbel_argmax's topk_thr with no host synchronisation.
 *   top_k    int32 [B] (top_k_is_64bit = 0) or int64 [B] (= 1), device memory.
 *   thr      fp32 [B].
 *   workspace: >= vqk_topk_threshold_workspace_size(B, V) bytes, 4-byte aligned, no
 *   initialisation needed.  Two launches.
 * Replaces: _compute_topk_threshold (src/vllm_quant_kernels/_sampler.py:62-93):
 *           top_k.max().item(), torch.topk and gather. */
int64_t vqk_topk_threshold_workspace_size(int64_t B, int64_t V);
int vqk_topk_threshold(const float *logits, int64_t ld, int64_t B, int64_t V, const void *top_k,
                       int top_k_is_64bit, float *thr, void *workspace, int64_t ws_bytes,
                       vqk_stream_t stream);

/* Debug form of the sampler arithmetic: writes y (the value the argmax is taken over,
 * -inf where masked) for every element to scores [B,V] (row stride V).  Same arguments
 * as vqk_gumbel_argmax minus the workspace.  Used by the parity tests to compare the
 * noise bit for bit; it has no counterpart in the reference. */
int vqk_gumbel_scores(const float *logits, int64_t ld, int64_t B, int64_t V,
                      const float *temp, const void *seeds, int seed_is_64bit,
                      const float *topk_thr, float *scores, vqk_stream_t stream);

/* Content hash of nbytes of device memory at p (16-byte aligned), for the identity of a
 * source weight in the on-disk quantized-lm_head cache: out[0], out[1] (device, zero
 * before the call) receive two 64-bit sums over the buffer's 16-byte chunks, each chunk
 * mixed with its index (splitmix64), so any changed byte or exchanged pair of chunks
 * changes both.  One launch; no counterpart in the reference, which re-quantizes on every
 * load instead of caching (src/vllm_quant_kernels/_quant.py:245-380). */
int vqk_hash128(const void *p, int64_t nbytes, uint64_t *out, vqk_stream_t stream);

/* Debug, no reference counterpart: over the float32 bit patterns [lo, hi) of magnitude
 * at most 448 (every pattern if full != 0), add to *count the number whose hardware e4m3
 * conversion differs from the library's encoder and lower *first to the smallest such
 * pattern.  *count and *first are device words the caller initialises (0 and 0xFFFFFFFF). */
int vqk_debug_e4m3_hw_check(uint32_t lo, uint32_t hi, int full, unsigned int *count, unsigned int *first,
                            vqk_stream_t stream);

#ifdef __cplusplus
}
#endif

#endif /* VQK_H */
