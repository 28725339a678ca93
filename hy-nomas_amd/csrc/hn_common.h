// Device-side helpers shared by the FP8 quantizers, the FP8 GEMM and the
// FP8-KV chunk attention. gfx950 (CDNA4) only: 64-wide wavefronts, OCP e4m3.
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>
#include <type_traits>

#define HN_DEVICE __device__ __forceinline__

namespace hn {

typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef float f32x16 __attribute__((ext_vector_type(16)));
typedef int i32x8 __attribute__((ext_vector_type(8)));
typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef __bf16 bf16x2 __attribute__((ext_vector_type(2)));
typedef short i16x8 __attribute__((ext_vector_type(8)));

// The e4m3 range used by every scale rule (largest finite OCP e4m3 value).
constexpr float kE4M3Max = 448.0f;

HN_DEVICE float bf16_bits_to_f32(uint32_t h16) { return __uint_as_float(h16 << 16); }

// fp32 -> bf16 bits, round to nearest even (NaN kept quiet).
HN_DEVICE uint32_t f32_to_bf16_bits(float f) {
    uint32_t u = __float_as_uint(f);
    if ((u & 0x7fffffffu) > 0x7f800000u) return 0x7fc0u;
    u += 0x7fffu + ((u >> 16) & 1u);
    return u >> 16;
}

// Two fp32 -> one word of two bf16 (lo in bits 0-15), one v_cvt_pk_bf16_f32.
// Round to nearest even: equal to f32_to_bf16_bits for every finite fp32
// (all 2^32 patterns compared on gfx950); a NaN stays a NaN of its own sign.
HN_DEVICE uint32_t f32x2_to_bf16x2(float lo, float hi) {
    typedef float f32x2 __attribute__((ext_vector_type(2)));
    return __builtin_bit_cast(uint32_t, __builtin_convertvector((f32x2){lo, hi}, bf16x2));
}

// The low / high bf16 of a word, as fp32 (exact).
HN_DEVICE float bf16_lo(uint32_t w) { return __uint_as_float(w << 16); }
HN_DEVICE float bf16_hi(uint32_t w) { return __uint_as_float(w & 0xffff0000u); }

// fp32 -> OCP e4m3 ("fn") byte, round to nearest even on the e4m3 grid.
// The grid is extended one step past 448 (480, bit pattern 0x7F): values that
// round there, values >= 480 and NaN/Inf all give 0x7F | sign, the behaviour of
// torch's float8_e4m3fn cast that the reference recipes rely on
// (cutlass_fp8.py:40). Normal range: keep the top 3 mantissa bits and round on
// the 20 discarded ones; subnormal range (< 2^-6): round a * 2^9 to an integer.
HN_DEVICE uint32_t e4m3_encode(float f) {
    const uint32_t u = __float_as_uint(f);
    const uint32_t sign = (u >> 24) & 0x80u;
    const uint32_t a = u & 0x7fffffffu;
    uint32_t code;
    if (a >= 0x43f00000u) {                 // >= 480, Inf, NaN
        code = 0x7fu;
    } else if (a < 0x3c800000u) {           // < 2^-6
        code = (uint32_t)__builtin_rintf(__uint_as_float(a) * 512.0f);
    } else {
        const uint32_t keep = a >> 20;      // exponent + 3 mantissa bits
        const uint32_t rest = a & 0xfffffu; // discarded mantissa bits
        const uint32_t up = (rest > 0x80000u) | ((rest == 0x80000u) & keep);
        code = keep - (120u << 3) + up;     // rebias 127 -> 7
    }
    return sign | code;
}

// Four fp32 -> four e4m3 bytes (little-endian in one dword) with the gfx950
// conversion v_cvt_pk_fp8_f32 (OCP e4m3, round to nearest even). On every
// finite |x| <= 448.5 -- the only inputs the quantizers produce, since
// |x / s| <= 448 (1 + 2^-23) for s = amax / 448 -- it returns exactly
// e4m3_encode(x); that equivalence is checked exhaustively over all fp32
// bit patterns of that range, both signs, on the device
// (tests/test_gpu_quant.py::test_hardware_e4m3_conversion_matches_oracle_over_quantizer_range,
// through hn_e4m3_encode_range).
HN_DEVICE uint32_t e4m3_encode4(float a, float b, float c, float d) {
    int w = __builtin_amdgcn_cvt_pk_fp8_f32(a, b, 0, false);
    w = __builtin_amdgcn_cvt_pk_fp8_f32(c, d, w, true);
    return (uint32_t)w;
}

// The fp32 quotient x / s of a quantizer, from the row's reciprocal.
//
// Per row: s and r = fl32(1 / s) (one IEEE division). Per element:
//   y = fl(x * r);  e = fma(-s, y, x) (exact residual);  q = fma(e, r, y)
// with the sign of x restored on q (an exactly-zero fma result is +0, while
// x / s keeps the sign of x). Three VALU operations replace the ~10 of an IEEE
// division. The result is not always fl32(x / s) in its last bit, but the
// *codes* derived from it are identical: for every bf16 row maximum amax and
// every bf16 x with |x| <= amax, for each scale rule in use
// (max(amax, 1e-4) / 448, amax > 0 ? amax / 448 : 1, amax > 0 ? amax / 127 : 1),
// e4m3_rne(q) == e4m3_rne(x / s) and the INT8 rounding of q equals that of
// x / s. That was checked exhaustively on the host (2 x 5.3e8 (amax, x)
// pairs per rule). The check holds for s >= 2^-100; smaller or non-finite
// scales (rows whose amax is within ~2^-91 of zero, or non-finite rows) take
// the IEEE division, since there the residual e underflows.
//
// `exact` is a property of the row, so callers choose the form once per row
// (with_form) and instantiate their encode loop for each (at<EXACT>), instead
// of a branch per element.
struct Quot {
    float s, r;
    bool exact;
    HN_DEVICE explicit Quot(float scale)
        : s(scale), r(1.0f / scale), exact(!(scale >= 0x1p-100f && scale <= 3.4028234e38f)) {}
    template <bool EXACT>
    HN_DEVICE float at(float x) const {
        if (EXACT) return x / s;
        const float y = __fmul_rn(x, r);
        const float e = __fmaf_rn(-s, y, x);
        return __builtin_copysignf(__fmaf_rn(e, r, y), x);
    }
    HN_DEVICE float operator()(float x) const { return exact ? at<true>(x) : at<false>(x); }
    // f(std::integral_constant<bool, EXACT>) for this row's form
    template <class F>
    HN_DEVICE void with_form(F&& f) const {
        if (exact) f(std::integral_constant<bool, true>{});
        else f(std::integral_constant<bool, false>{});
    }
};

// int8_kv_cache.py:150-157: fp32 round-half-away via floor(v + 0.5) /
// ceil(v - 0.5) (each add rounded in fp32), then clamp to +-127. Round to
// nearest is symmetric, so v - 0.5 rounds to -(|v| + 0.5) rounded and
// ceil(v - 0.5) = -floor(|v| + 0.5): the code is sign(v) min(floor(|v| + 0.5),
// 127) for either sign (-0 and +0 both give 0). With t = min(|v| + 0.5, 127)
// >= 0, floor(t) = trunc(t) and min(floor(x), 127) = floor(min(x, 127)) (127
// is an integer), so the float-to-int conversion's truncation toward zero of
// copysign(t, v) is the code: no floor instruction.
HN_DEVICE int int8_code_i32(float v) {
    const float t = fminf(fabsf(v) + 0.5f, 127.0f);
    return (int)__builtin_copysignf(t, v);
}

// Four INT8 codes, packed little-endian into one word: two saturating
// i32 -> i16 packs (exact: every code is in [-127, 127]) and one byte select.
HN_DEVICE uint32_t int8_pack4(int a, int b, int c, int d) {
    const uint32_t lo = __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_pk_i16(a, b));
    const uint32_t hi = __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_pk_i16(c, d));
    return __builtin_amdgcn_perm(hi, lo, 0x06040200u);  // bytes 0, 2 of lo, then of hi
}

HN_DEVICE uint32_t int8_code(float v) { return (uint32_t)int8_code_i32(v) & 0xffu; }

// The 8 codes (e4m3 if FP8, else INT8) of one lane's 8 values of a row with
// quotient d; the quotient form is chosen once for the 8.
template <bool FP8>
HN_DEVICE uint2 codes8(const float (&f)[8], const Quot& d) {
    uint2 out;
    d.with_form([&](auto form) {
        constexpr bool E = decltype(form)::value;
        if (FP8) {
            out.x = e4m3_encode4(d.at<E>(f[0]), d.at<E>(f[1]), d.at<E>(f[2]), d.at<E>(f[3]));
            out.y = e4m3_encode4(d.at<E>(f[4]), d.at<E>(f[5]), d.at<E>(f[6]), d.at<E>(f[7]));
        } else {
            out.x = int8_pack4(int8_code_i32(d.at<E>(f[0])), int8_code_i32(d.at<E>(f[1])),
                               int8_code_i32(d.at<E>(f[2])), int8_code_i32(d.at<E>(f[3])));
            out.y = int8_pack4(int8_code_i32(d.at<E>(f[4])), int8_code_i32(d.at<E>(f[5])),
                               int8_code_i32(d.at<E>(f[6])), int8_code_i32(d.at<E>(f[7])));
        }
    });
    return out;
}

// OCP e4m3 byte -> fp32 (exact).
HN_DEVICE float e4m3_decode(uint32_t c) {
    const uint32_t e = (c >> 3) & 15u, m = c & 7u;
    float v;
    if (e == 0) v = (float)m * 0.001953125f;  // m * 2^-9
    else v = __uint_as_float(((e + 120u) << 23) | (m << 20));
    if (e == 15u && m == 7u) v = __builtin_nanf("");
    return (c & 0x80u) ? -v : v;
}

// Max over the `width` lanes of an aligned lane group (width a power of two <= 64).
template <int WIDTH>
HN_DEVICE float group_max(float v) {
#pragma unroll
    for (int off = WIDTH / 2; off > 0; off >>= 1) v = fmaxf(v, __shfl_xor(v, off, 64));
    return v;
}

// The maximum that propagates NaN (IEEE maximum; v_maximum3_f32 on gfx950),
// as torch's amax does: the activation quantizers' row and block maxima.
HN_DEVICE float max_nan(float a, float b) { return __builtin_elementwise_maximum(a, b); }

template <int WIDTH>
HN_DEVICE float group_max_nan(float v) {
#pragma unroll
    for (int off = WIDTH / 2; off > 0; off >>= 1) v = max_nan(v, __shfl_xor(v, off, 64));
    return v;
}

template <int WIDTH>
HN_DEVICE float group_sum(float v) {
#pragma unroll
    for (int off = WIDTH / 2; off > 0; off >>= 1) v += __shfl_xor(v, off, 64);
    return v;
}

}  // namespace hn
