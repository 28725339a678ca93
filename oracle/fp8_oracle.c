/*
 * CPU oracle for the FP8 quantized inference path -- TEST INFRASTRUCTURE ONLY.
 *
 * This file restates, in plain C, the reference's quantization recipes so the
 * HIP kernels can be checked bit-exactly. It is never linked into the product
 * library; only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg
 * load it (through oracle/oracle.py), and only as the checker.
 *
 * Build: oracle/Makefile -> oracle/liboracle.so (plain gcc, no fast-math, no
 * FMA contraction, so every float operation is one IEEE-754 binary32 op exactly
 * as ATen's CPU kernels perform it).
 *
 * Parity pins (tests/test_oracle.py):
 *   - e4m3 encode: exhaustive over all 2^16 bf16 bit patterns and a large
 *     random sample of fp32 patterns against torch's float8_e4m3fn cast,
 *     plus hand-derived known answers (448 -> 0x7E, 464 tie -> 0x7E,
 *     2^-10 tie -> 0x00, 1.5*2^-10 -> 0x01, >=480/NaN -> 0x7F|sign).
 *   - row / block / KV scale rules: closed-form known answers (power-of-two
 *     scales make x/s exact), invariants (|code| <= 0x7E, the amax element
 *     encodes to +-448), and the zero-row / clamp special cases.
 *   - INT8-compat: closed-form known answers including the fp32 "+0.5"
 *     rounding artefact of the reference recipe.
 */
#include <math.h>
#include <stdint.h>
#include <string.h>

/* ------------------------------------------------------------------------ */
/* OCP FP8 E4M3 ("fn" variant): 1 sign, 4 exponent bits (bias 7), 3 mantissa
 * bits, no infinities, S.1111.111 is NaN, largest finite 448 = 1.75 * 2^8,
 * subnormals m * 2^-9 for m in 1..7.
 *
 * Encoding is round-to-nearest-even on that grid, where the grid is extended by
 * one step past 448 (to 480, the bit pattern 0x7F). Anything that rounds to that
 * step, anything >= 480, and NaN/Inf all produce 0x7F | sign. This is the
 * behaviour of torch's Tensor.to(torch.float8_e4m3fn), which the reference's
 * recipes use (hymm/models/vae/pixelumm_decoder/cutlass_fp8.py:40). */
uint8_t hn_oracle_e4m3_encode(float f)
{
    uint32_t bits;
    memcpy(&bits, &f, sizeof bits);
    const uint8_t sign = (uint8_t)((bits >> 24) & 0x80u);
    const float a = fabsf(f);
    if (!(a < 480.0f))
        return sign | 0x7Fu;
    if (a < 0.015625f) { /* below 2^-6: subnormal grid, step 2^-9 */
        const float t = a * 512.0f;      /* exact: power-of-two scaling */
        const float r = nearbyintf(t);   /* RNE (default rounding mode) */
        return sign | (uint8_t)r;        /* r == 8 is 2^-6 == code 0x08 */
    }
    int e2;
    (void)frexpf(a, &e2);                /* a = m * 2^e2, m in [0.5, 1) */
    const int E = e2 - 1;                /* unbiased exponent, -6..8 */
    const float t = ldexpf(a, 3 - E);    /* exact, in [8, 16) */
    const int r = (int)nearbyintf(t);    /* 8..16; 16 carries into exponent */
    return sign | (uint8_t)(((E + 7) << 3) + (r - 8));
}

float hn_oracle_e4m3_decode(uint8_t c)
{
    const int e = (c >> 3) & 15, m = c & 7;
    const float s = (c & 0x80u) ? -1.0f : 1.0f;
    if (e == 15 && m == 7)
        return NAN;
    if (e == 0)
        return s * ldexpf((float)m, -9);
    return s * ldexpf(1.0f + (float)m / 8.0f, e - 7);
}

static inline float bf16_to_f32(uint16_t h)
{
    uint32_t u = (uint32_t)h << 16;
    float f;
    memcpy(&f, &u, sizeof f);
    return f;
}

void hn_oracle_e4m3_encode_f32(const float *x, int64_t n, uint8_t *q)
{
    for (int64_t i = 0; i < n; ++i)
        q[i] = hn_oracle_e4m3_encode(x[i]);
}

void hn_oracle_e4m3_decode_n(const uint8_t *q, int64_t n, float *y)
{
    for (int64_t i = 0; i < n; ++i)
        y[i] = hn_oracle_e4m3_decode(q[i]);
}

/* codes[i] against hn_oracle_e4m3_encode of the fp32 value whose bit pattern is
 * first + i, for i in [0, n): returns how many differ; *first_bad gets the
 * first differing index (-1 when none). Used to check a device conversion over
 * whole ranges of fp32 bit patterns. */
int64_t hn_oracle_e4m3_range_mismatches(uint32_t first, int64_t n, const uint8_t *codes,
                                        int64_t *first_bad)
{
    int64_t bad = 0;
    *first_bad = -1;
    for (int64_t i = 0; i < n; ++i) {
        const uint32_t b = first + (uint32_t)i;
        float f;
        memcpy(&f, &b, sizeof f);
        if (hn_oracle_e4m3_encode(f) != codes[i]) {
            if (bad == 0)
                *first_bad = i;
            ++bad;
        }
    }
    return bad;
}

/* ------------------------------------------------------------------------ */
/* Scale rules.
 *  mode 0 ("clamp"):  s = max(amax, floor) / 448
 *      cutlass_fp8.py:39  `amax(...).clamp_min(1e-4) / 448.0`  (floor = 1e-4f),
 *      used for linear activations (per token) and weights (per channel).
 *  mode 1 ("zero-one"): s = amax > 0 ? amax / 448 : 1
 *      int8_kv_cache.py:44,152 `where(peak > 0, peak / 127.0, 1.0)` with the
 *      e4m3 range 448 in place of 127; used for K/V rows.
 *  A NaN element makes the row / block amax NaN (torch's amax propagates it):
 *  in mode 0 the scale is then NaN (clamp_min keeps NaN) and every code of
 *  the row is a NaN code; in mode 1 the comparison is false and the scale is
 *  1. (The KV API rejects non-finite rows before they get here.) */
static inline float fp8_scale(float amax, int mode, float floor_)
{
    if (mode == 0)
        return (amax < floor_ ? floor_ : amax) / 448.0f;
    return amax > 0.0f ? amax / 448.0f : 1.0f;
}

/* Per-row FP8 quantization of a bf16 matrix [rows, cols] (row stride in
 * elements). One scale per row. This is the reference's blockwise recipe
 * (cutlass_fp8.py:35-41) with 1 x cols blocks instead of 128 x 128. */
void hn_oracle_quantize_rows_fp8(const uint16_t *x, int64_t rows, int64_t cols,
                                 int64_t row_stride, int mode, float floor_,
                                 uint8_t *q, float *scale)
{
    for (int64_t r = 0; r < rows; ++r) {
        const uint16_t *xr = x + r * row_stride;
        float amax = 0.0f;
        for (int64_t c = 0; c < cols; ++c) {
            const float v = fabsf(bf16_to_f32(xr[c]));
            amax = (v > amax || v != v) ? v : amax;   /* NaN propagates, as torch's amax */
        }
        const float s = fp8_scale(amax, mode, floor_);
        scale[r] = s;
        for (int64_t c = 0; c < cols; ++c)
            q[r * cols + c] = hn_oracle_e4m3_encode(bf16_to_f32(xr[c]) / s);
    }
}

/* 128 x 128 blockwise FP8 quantization, cutlass_fp8.py:35-41:
 * rows are zero-padded to a multiple of 128 (padding only lowers no amax),
 * scale[m/128, k/128] = max(amax_block, 1e-4) / 448, q = e4m3(x / scale).
 * cols must be a multiple of 128. */
void hn_oracle_quantize_blockwise_fp8(const uint16_t *x, int64_t rows, int64_t cols,
                                      uint8_t *q, float *scale)
{
    const int64_t mb = (rows + 127) / 128, kb = cols / 128;
    for (int64_t bi = 0; bi < mb; ++bi)
        for (int64_t bj = 0; bj < kb; ++bj) {
            float amax = 0.0f;
            for (int64_t r = bi * 128; r < rows && r < bi * 128 + 128; ++r)
                for (int64_t c = bj * 128; c < bj * 128 + 128; ++c) {
                    const float v = fabsf(bf16_to_f32(x[r * cols + c]));
                    amax = (v > amax || v != v) ? v : amax;   /* NaN propagates */
                }
            const float s = fp8_scale(amax, 0, 1e-4f);
            scale[bi * kb + bj] = s;
            for (int64_t r = bi * 128; r < rows && r < bi * 128 + 128; ++r)
                for (int64_t c = bj * 128; c < bj * 128 + 128; ++c)
                    q[r * cols + c] = hn_oracle_e4m3_encode(bf16_to_f32(x[r * cols + c]) / s);
        }
}

/* KV quantize-on-write, int8_kv_cache.py:125-158 restated for FP8:
 * values [B, L, H, D] (element strides xs[4]) are written into a cache
 * q [B, cap, H, D] (strides qs[4]) and scale [B, cap, H, 1] (strides ss[3]) at
 * token offset `start`. One scale per (batch, token, head) row of D.
 * fmt 0: FP8 e4m3, s = amax > 0 ? amax/448 : 1, q = e4m3(x / s)
 * fmt 1: INT8-compat, s = amax > 0 ? amax/127 : 1,
 *        q = clamp(x/s >= 0 ? floor(x/s + 0.5) : ceil(x/s - 0.5), -127, 127)
 *        with every operation in fp32 (int8_kv_cache.py:150-157). */
void hn_oracle_kv_quantize(const uint16_t *x, int64_t B, int64_t L, int64_t H, int64_t D,
                           const int64_t *xs, uint8_t *q, const int64_t *qs,
                           float *scale, const int64_t *ss, int64_t start, int fmt)
{
    for (int64_t b = 0; b < B; ++b)
        for (int64_t t = 0; t < L; ++t)
            for (int64_t h = 0; h < H; ++h) {
                const uint16_t *xr = x + b * xs[0] + t * xs[1] + h * xs[2];
                float amax = 0.0f;
                for (int64_t d = 0; d < D; ++d) {
                    const float v = fabsf(bf16_to_f32(xr[d * xs[3]]));
                    amax = v > amax ? v : amax;
                }
                float s;
                if (fmt == 0)
                    s = amax > 0.0f ? amax / 448.0f : 1.0f;
                else
                    s = amax > 0.0f ? amax / 127.0f : 1.0f;
                uint8_t *qr = q + b * qs[0] + (t + start) * qs[1] + h * qs[2];
                scale[b * ss[0] + (t + start) * ss[1] + h * ss[2]] = s;
                for (int64_t d = 0; d < D; ++d) {
                    const float v = bf16_to_f32(xr[d * xs[3]]) / s;
                    uint8_t code;
                    if (fmt == 0) {
                        code = hn_oracle_e4m3_encode(v);
                    } else {
                        float r = v >= 0.0f ? floorf(v + 0.5f) : ceilf(v - 0.5f);
                        r = r < -127.0f ? -127.0f : (r > 127.0f ? 127.0f : r);
                        code = (uint8_t)(int8_t)r;
                    }
                    qr[d * qs[3]] = code;
                }
            }
}

/* W8 weight quantization of the reference DiT linear (INT8-compat),
 * int8_stored_bf16_linear.py:46-61: per output channel and per 128-wide input
 * group, s = max > 0 ? max/127 : 1, q = clamp(floor(|x/s| + 0.5) * sign(x/s)).
 * w is fp32 [n, k]; q int8 [n, k]; scale fp32 [n, ceil(k/128)]. */
void hn_oracle_quantize_weight_int8(const float *w, int64_t n, int64_t k,
                                    int8_t *q, float *scale)
{
    const int64_t groups = (k + 127) / 128;
    for (int64_t r = 0; r < n; ++r)
        for (int64_t g = 0; g < groups; ++g) {
            float mx = 0.0f;
            for (int64_t c = g * 128; c < k && c < g * 128 + 128; ++c) {
                const float v = fabsf(w[r * k + c]);
                mx = v > mx ? v : mx;
            }
            const float s = mx > 0.0f ? mx / 127.0f : 1.0f;
            scale[r * groups + g] = s;
            for (int64_t c = g * 128; c < k && c < g * 128 + 128; ++c) {
                const float v = w[r * k + c] / s;
                const float sg = v > 0.0f ? 1.0f : (v < 0.0f ? -1.0f : 0.0f);
                float m = floorf(fabsf(v) + 0.5f) * sg;
                m = m < -127.0f ? -127.0f : (m > 127.0f ? 127.0f : m);
                q[r * k + c] = (int8_t)m;
            }
        }
}
