/*
 * hynomas_fp8.h -- C ABI of the MI355X (gfx950) FP8 quantized inference path.
 *
 * One shared library, libhynomas_fp8.so, built from the HIP sources in
 * hy-nomas_amd/csrc/.
 * Every pointer argument is a device pointer unless stated otherwise; sizes
 * and strides are in elements; `stream` is a hipStream_t (NULL = default
 * stream). Calls are asynchronous with respect to the host: they enqueue work
 * on `stream` and return. Each function returns HN_OK (0) or a negative HN_E*
 * code; hn_last_error() then describes the failure (thread-local). Argument
 * errors are detected on the host before anything is enqueued, so a failed
 * call has written nothing. A call with work to do on a device that is not a
 * gfx950 returns HN_E_DEVICE (the architecture check of the reference's
 * extension, cutlass_fp8.cu:21-34).
 *
 * Byte formats: bf16 is IEEE bfloat16; e4m3 is OCP FP8 E4M3 ("fn": no
 * infinities, 0x7F/0xFF NaN, max 448), the format of torch.float8_e4m3fn.
 *
 * Each entry point names the reference interface (upstream file:line) whose
 * work it performs; the Python mirror in hy-nomas_amd/ keeps those interfaces'
 * names, argument meaning and error behaviour on top of these calls.
 */
#ifndef HYNOMAS_FP8_H
#define HYNOMAS_FP8_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define HN_OK 0
#define HN_E_ARG (-1)     /* invalid shape, stride, alignment or mode */
#define HN_E_LAUNCH (-2)  /* the HIP runtime rejected a launch */
#define HN_E_DEVICE (-3)  /* no usable gfx950 device */

/* Scale rules for FP8 quantization (amax is the max |x| over the block):
 *   HN_SCALE_CLAMP:    s = max(amax, amax_floor) / 448
 *                      (cutlass_fp8.py:39, clamp_min(1e-4) / 448.0)
 *   HN_SCALE_ZERO_ONE: s = amax > 0 ? amax / 448 : 1
 *                      (int8_kv_cache.py:44,152 with 448 in place of 127)
 * Codes are e4m3_rne(x / s) with IEEE-754 binary32 division. */
#define HN_SCALE_CLAMP 0
#define HN_SCALE_ZERO_ONE 1

/* KV cache storage formats. */
#define HN_KV_FP8 0   /* e4m3 codes, s = amax>0 ? amax/448 : 1 */
#define HN_KV_INT8 1  /* int8 codes bit-exact with int8_kv_cache.py:22-58 */

/* GEMM epilogue activations. */
#define HN_ACT_NONE 0
#define HN_ACT_GELU_TANH 1  /* F.gelu(approximate="tanh"), nomas_compile_prepost.py:86 */

/* Message of the last failed call on this thread ("" if none). */
const char *hn_last_error(void);

/* ABI version of this library (bumped on any signature change). */
int hn_abi_version(void);

/* Per-row FP8 quantization of a bf16 matrix: one fp32 scale per row.
 * x: bf16 [rows, cols] with row stride `row_stride` (elements, >= cols, and
 *    the row start must be 16-byte aligned); q: e4m3 [rows, cols] contiguous;
 *    scale: fp32 [rows]. cols % 8 == 0, cols <= 16384.
 * Replaces the activation quantizer of the FP8 linear custom op,
 * hymm/models/vae/pixelumm_decoder/cutlass_fp8.py:35-41,49 (its recipe with
 * 1 x cols blocks: per-token activations, per-output-channel weights), whose
 * per-token form is the DeepGEMM call site fp8.py:19-21,30. */
int hn_quantize_rows_fp8(const void *x, int64_t rows, int64_t cols, int64_t row_stride,
                         int scale_mode, float amax_floor, void *q, float *scale,
                         void *stream);

/* LayerNorm (no affine, eps) + adaLN modulate + per-token FP8 quantization,
 * fused: o = bf16(bf16(bf16(LN(x)) * bf16(1 + scale_mod[b])) + shift[b]), then
 * the hn_quantize_rows_fp8 recipe (HN_SCALE_CLAMP, amax_floor) on o.
 * x: bf16 [rows, cols] contiguous; shift, scale_mod: bf16 [B, cols] with batch
 * stride mod_stride (elements), row r using batch r / rows_per_batch; q: e4m3
 * [rows, cols]; scale: fp32 [rows]. cols % 8 == 0, cols <= 8192.
 * Replaces the LayerNorm + _modulate in front of the block's FP8 linears,
 * nomas_compile_prepost.py:14-15,40-43 (QKV) and :81-84 (fc1), together with
 * the linear's activation quantizer (cutlass_fp8.py:35-41,49). */
int hn_ln_mod_quantize_fp8(const void *x, int64_t rows, int64_t cols, int64_t rows_per_batch,
                           const void *shift, const void *scale_mod, int64_t mod_stride, float eps,
                           float amax_floor, void *q, float *scale, void *stream);

/* 128x128 blockwise FP8 quantization, rows zero-padded to a multiple of 128.
 * x: bf16 [rows, cols] contiguous; q: e4m3 [rows, cols]; scale: fp32
 * [ceil(rows/128), cols/128]; cols % 128 == 0. Scale rule HN_SCALE_CLAMP with
 * floor 1e-4.
 * Replaces quantize_blockwise, cutlass_fp8.py:35-44. */
int hn_quantize_blockwise_fp8(const void *x, int64_t rows, int64_t cols, void *q,
                              float *scale, void *stream);

/* KV quantize-on-write of one tensor: values [B, L, H, D] (bf16, strides
 * xs[4]) are written into the cache q [B, cap, H, D] (strides qs[4], 1-byte
 * codes) and scale [B, cap, H, 1] (fp32, strides ss[3]) at token offset
 * `start`. One scale per (batch, token, head) row. D == 128, xs[3] == qs[3]
 * == 1. start + L > cap is refused (HN_E_ARG) before anything is written, as
 * the reference's capacity check does (int8_kv_cache.py:128-135).
 * status: NULL (the caller guarantees finite values) or a device int32. When
 * given, the values are validated on the device before the write, the
 * reference's validate-before-write (int8_kv_cache.py:140-141,176) without a
 * host synchronisation: *status is set to 0 if every value is finite, else to
 * 1, and then nothing (codes or scales) is written. The caller reads *status
 * after the stream reaches it.
 * Replaces _quantize_rows / quantize_kv_into, int8_kv_cache.py:22-58,125-158. */
int hn_kv_quantize(int fmt, const void *x, const int64_t *xs, int64_t B, int64_t L,
                   int64_t H, int64_t D, void *q, const int64_t *qs, float *scale,
                   const int64_t *ss, int64_t cap, int64_t start, int32_t *status,
                   void *stream);

/* K and V of one layer in a single launch (same shapes/strides for both,
 * capacity and status as in hn_kv_quantize; with a status, both K and V are
 * validated before either is written).
 * Replaces quantize_kv_pair_into, int8_kv_cache.py:161-179. */
int hn_kv_quantize_pair(int fmt, const void *k, const void *v, const int64_t *xs,
                        int64_t B, int64_t L, int64_t H, int64_t D, void *qk, void *qv,
                        const int64_t *qs, float *sk, float *sv, const int64_t *ss,
                        int64_t cap, int64_t start, int32_t *status, void *stream);

/* KV decode of the valid prefix: y[b,t,h,:] = bf16(decode(q[b,t,h,:]) * s[b,t,h]),
 * t < valid_len. q strides qs[4], scale strides ss[3], y bf16 strides ys[4];
 * D == 128 with unit innermost strides.
 * Replaces _dequantize_rows / dequantize_kv, int8_kv_cache.py:61-89,182-205. */
int hn_kv_dequantize(int fmt, const void *q, const int64_t *qs, const float *scale,
                     const int64_t *ss, int64_t B, int64_t valid_len, int64_t H, int64_t D,
                     void *y, const int64_t *ys, void *stream);

/* Row/column-scaled FP8 GEMM with fused epilogue:
 *   out[m, n] = act(acc[m, n] * sa[m] * sb[n] + bias[n]),  acc = sum_k a[m,k] b[n,k]
 * a: e4m3 [M, K] row-major; b: e4m3 [N, K] row-major (the nn.Linear weight
 * layout); sa: fp32 [M]; sb: fp32 [N]; bias: bf16 [N] or NULL; out: bf16
 * [M, N] with row stride ldc. fp32 accumulation. K % 128 == 0, N % 128 == 0,
 * a/b/out 16-byte aligned, ldc % 8 == 0, N <= ldc <= 2^22.
 * Replaces F.linear(x, linear_weight(m), b) of the DiT block
 * (nomas_compile_prepost.py:45-47,80-87 via int8_stored_bf16_linear.py:82-100)
 * for FP8 weights, and the DeepGEMM per-token GEMM of fp8.py:27-38.
 * Enqueues one kernel on `stream`, or two in order when the last row stripe
 * (M % 256 <= 64 rows, K >= 896) gets a launch of its own; nothing else. */
int hn_gemm_fp8_rowcol(const void *a, const void *b, const float *sa, const float *sb,
                       const void *bias, void *out, int64_t M, int64_t N, int64_t K,
                       int64_t ldc, int act, void *stream);

/* Blockwise-scaled FP8 GEMM, the `gemm(a, b, sa, sb)` contract of the
 * reference's native extension:
 *   out[m, n] = bf16( sum_kb sa[m/128, kb] * sb[n/128, kb] * sum_{k in kb} a[m,k] b[n,k] )
 * a: e4m3 [M, K]; b: e4m3 [N, K]; sa: fp32 [ceil(M/128), K/128]; sb: fp32
 * [N/128, K/128]; out: bf16 [M, N] contiguous. N % 128 == 0, K % 128 == 0.
 * Range: the accumulators are carried in units of the current K block's
 * factor f = sa * sb (rescaled by f_prev / f between blocks), so the result
 * stays finite while, within each 128 x 128 output block, no earlier factor
 * exceeds a later one by 2^99 or more (then |acc| < 24 K blocks x 2.6e7 x
 * 2^99 would stay below FLT_MAX; past it the rescale overflows to Inf). The
 * FP8Linear loader refuses weight scale rows spanning more than 2^60
 * (pixelumm_fp8.validate_serialized_tensors); activation scales from the
 * blockwise quantizer span more only for bf16 blocks 2^60 apart in magnitude.
 * When the last row stripe (M % 256 <= 64 rows) would add a round of tiles
 * and K >= 512, its rows are computed by a second kernel enqueued first on
 * the same stream, which adds each K block's product times its factor and
 * has no such range limit.
 * Replaces gemm / pixel_gemm, hymm/models/vae/pixelumm_decoder/csrc/cutlass_fp8.cu:20-57
 * and reactor/hy_nomas_fp8_sm100.cu:67-107. */
int hn_gemm_fp8_blockwise(const void *a, const void *b, const float *sa, const float *sb,
                          void *out, int64_t M, int64_t N, int64_t K, void *stream);

/* Attention of one chunk's queries over an FP8 KV cache, block-causal at chunk
 * granularity, optionally followed by an unquantized bf16 tail (the current
 * chunk's own K/V during denoising passes).
 *   q:     bf16 [B, Lq, H, D], strides qs[4] (qs[3] == 1), D == 128
 *   kc,vc: 1-byte codes [Bc, cap, H, D], strides cs[4] (cs[3] == 1)
 *   ks,vs: fp32 scales [Bc, cap, H, 1], strides ss[3]
 *          Bc == B, or one history slot read by every query batch (the
 *          read-only CFG broadcast of nomas_cpt.py:547-567): cs[0] == ss[0]
 *          == 0 (and cache_valid_stride == 0)
 *   cache_cap: tokens the cache holds; kv_len > cache_cap is refused
 *   kv_len: cached tokens attended, positions 0 .. kv_len-1
 *   cache_valid: NULL (every cached key valid) or bytes [Bc, >= kv_len]
 *          with batch stride cache_valid_stride; key t of batch b takes part
 *          iff cache_valid[b * stride + t] != 0 (the cache_mask history mask,
 *          nomas_cpt.py:536-546)
 *   kcur,vcur: bf16 [B, cur_len, H, D] (strides curs[4]) or NULL with cur_len 0;
 *          tail token j has position kv_len + j
 *   cur_valid: NULL or bytes [B, >= cur_len] (batch stride cur_valid_stride):
 *          validity of the tail keys (img ones | text_mask, nomas_cpt.py:488-504)
 *   q_pos0: position of query row 0; query i has position q_pos0 + i
 *   chunk_len: key at position p is visible to query at position r iff
 *          p / chunk_len <= r / chunk_len; chunk_len <= 0 makes every key visible
 *   softmax_scale: finite and > 0
 *   out:   bf16 [B, Lq, H, D], strides os[4]
 * O = softmax(Q K^T * softmax_scale) V over the visible valid keys, with K, V
 * the reference's dequantized values bf16(code * scale); query rows that see
 * no key are written as zeros (range_attention.py:212-239). The probabilities
 * multiply V as fp16 (relative rounding 2^-11) with fp32 accumulation.
 * Range: V (cached values bf16(code * scale) and the bf16 tail) is held as
 * fp16, converted toward zero, so a V value of magnitude above 65504 enters
 * the product as +-65504 (the reference attends the bf16 value); every other
 * bf16 V value is exact in fp16 down to 2^-24. A cached V exceeds 65504 only
 * when the written row held such a value (|bf16(code * s)| <= amax).
 * workspace: device scratch of at least hn_attn_fp8kv_workspace_size(...)
 *        bytes (16-byte aligned; NULL/0 when that size is 0). It holds per-split
 *        partial results when the key range is split across workgroups to fill
 *        the device (few queries, long cache); concurrent calls need separate
 *        workspaces.
 * Replaces the FP8/INT8-cache branch of causal_attention_with_cache_mp,
 * hymm/models/dit/nomas_cpt.py:529-531,614-625,771-829 (dequantize_kv, cat,
 * then Flex/FA3/SDPA), and flex_masked_attention, range_attention.py:212-239. */
int hn_attn_fp8kv(int fmt, const void *q, const int64_t *qs, int64_t B, int64_t Lq, int64_t H,
                  int64_t D, const void *kc, const void *vc, const int64_t *cs,
                  const float *ks, const float *vs, const int64_t *ss, int64_t cache_cap,
                  int64_t kv_len, const uint8_t *cache_valid, int64_t cache_valid_stride,
                  const void *kcur, const void *vcur, const int64_t *curs, int64_t cur_len,
                  const uint8_t *cur_valid, int64_t cur_valid_stride, int64_t q_pos0,
                  int64_t chunk_len, float softmax_scale, void *out, const int64_t *os,
                  void *workspace, int64_t workspace_bytes, void *stream);

/* Bytes of workspace hn_attn_fp8kv needs for these sizes on the current device
 * (0: none). Depends on the device's CU count. */
int64_t hn_attn_fp8kv_workspace_size(int64_t B, int64_t Lq, int64_t H, int64_t D,
                                     int64_t kv_len, int64_t cur_len);

/* hn_attn_fp8kv without the workspace arguments: a variant that allocates
 * nothing and takes no caller memory beyond its inputs and outputs. No
 * counterpart in the reference; it is for callers that cannot allocate device
 * memory (code under HIP graph capture, tight serving loops). The split-key
 * partials go to a scratch array the library holds on each device for the life
 * of the process, hn_attn_fp8kv_noalloc_scratch_bytes() bytes (40 MiB, above
 * the 34.1 MB that any call needs on 256 CUs); sizes whose
 * hn_attn_fp8kv_workspace_size() exceeds it are refused (HN_E_ARG). All
 * calls on one device share that array, so calls that overlap on one GPU (two
 * streams, or two threads) race. Arguments, results and errors are otherwise
 * those of hn_attn_fp8kv. */
int hn_attn_fp8kv_noalloc(int fmt, const void *q, const int64_t *qs, int64_t B, int64_t Lq,
                          int64_t H, int64_t D, const void *kc, const void *vc, const int64_t *cs,
                          const float *ks, const float *vs, const int64_t *ss, int64_t cache_cap,
                          int64_t kv_len, const uint8_t *cache_valid, int64_t cache_valid_stride,
                          const void *kcur, const void *vcur, const int64_t *curs, int64_t cur_len,
                          const uint8_t *cur_valid, int64_t cur_valid_stride, int64_t q_pos0,
                          int64_t chunk_len, float softmax_scale, void *out, const int64_t *os,
                          void *stream);

/* Bytes of the per-device scratch array of hn_attn_fp8kv_noalloc. */
int64_t hn_attn_fp8kv_noalloc_scratch_bytes(void);

/* Fused pre-attention tail of the DiT block's image stream, in place:
 *   q <- RoPE(RMSNorm_qw(q)),  k <- RoPE(RMSNorm_kw(k))
 * per (batch, token, head) row of D == 128, with the reference's op order and
 * bf16 rounding points: y = bf16(x * rsqrt(mean(x^2) + eps)); y = bf16(y * w);
 * out = bf16(y * cos + rotate_half(y) * sin), rotate_half(y0, y1) = (-y1, y0),
 * products and sums rounded separately in fp32.
 *   q, k, v: bf16 [B, L, H, D] sharing strides xs[4] (xs[3] == 1), e.g. views
 *            of one fused QKV projection output; q and k are overwritten
 *   q_weight, k_weight: bf16 [D]; cos, sin: fp32 [L, D] with row stride cs
 * When kc is non-NULL, the rotated k and v are also written into the KV cache
 * (kc, vc codes [B, cap, H, D] with strides qs[4]; ks, vs fp32 scales with
 * strides ss[3]) at token offset start, exactly as hn_kv_quantize_pair would
 * write them; start + L > cap is refused before anything is written. status
 * (only with a cache write): NULL, or a device int32 that validates the cache
 * write as in hn_kv_quantize: the rotated k and v are checked on the device
 * first (same arithmetic), and if any value is NaN/Inf *status becomes 1 and
 * the cache is not written (q and k are still rotated in place).
 * Replaces _rms_norm / _rotate_half and the q/k tail of pre_attention,
 * hymm/models/dit/modules/nomas_compile_prepost.py:18-27,49-54 (RMSNorm
 * norm_layers.py:49-63, RoPE posemb_layers.py:401-453), fused with the cache
 * write of quantize_kv_pair_into, int8_kv_cache.py:161-179. */
int hn_qk_norm_rope_kv(int fmt, void *q, void *k, const void *v, const int64_t *xs, int64_t B,
                       int64_t L, int64_t H, int64_t D, const void *q_weight,
                       const void *k_weight, const float *cos, const float *sin, int64_t cs,
                       float eps, void *kc, void *vc, const int64_t *qs, float *ks, float *vs,
                       const int64_t *ss, int64_t cap, int64_t start, int32_t *status,
                       void *stream);

/* Test support; it replaces no reference interface. Writes to out[i] the e4m3
 * byte that the quantizers' hardware conversion (v_cvt_pk_fp8_f32, round to
 * nearest even) gives for the fp32 value whose bit pattern is first + i, for
 * i in [0, n). n must be a multiple of 4 and first + n <= 2^32. Exists so
 * that tests can compare that conversion, over every input the quantizers can
 * produce (|x| <= 448.5), with the CPU oracle's encoder. */
int hn_e4m3_encode_range(uint32_t first, int64_t n, void *out, void *stream);

#ifdef __cplusplus
}
#endif

#endif /* HYNOMAS_FP8_H */
