// Fused pre-attention tail of the DiT block (image stream), gfx950:
//
//   q, k <- RoPE(RMSNorm_w(q)), RoPE(RMSNorm_w(k))       in place, bf16
//   optionally: cache[start + t] <- quantize(k_rotated), quantize(v)
//
// One (batch, token, head) row of 128 dims per 16-lane group, 8 dims per lane.
// The arithmetic follows the reference's op sequence and rounding points
// (hymm/models/dit/modules/nomas_compile_prepost.py:18-27,49-54):
//   y  = bf16( x * rsqrt(mean(x^2) + eps) )          (fp32 math)
//   y  = bf16( y * w )                                (bf16 weight)
//   out = bf16( y * cos + rotate_half(y) * sin )      (fp32 math; rotate_half maps
//                                                      the pair (y0, y1) to (-y1, y0))
// with the products and the sum rounded separately (no fused multiply-add), as
// the element-wise tensor ops compute them. cos/sin are the fp32 tables with
// each frequency repeated for both members of a pair. The cache write is the
// per-row quantize-on-write of the KV cache (same scale rule and codes as
// hn_kv_quantize), applied to the rotated k and to v, so the separate
// reference passes (norm, rope, validate, quantize) become one read of q, k, v.
#include "hn_capi_internal.h"
#include "hn_common.h"

namespace hn {
namespace qkr {

struct Args {
    uint16_t* q;
    uint16_t* k;
    const uint16_t* v;
    int64_t xs0, xs1, xs2;       // strides of q, k and v (shared), elements
    const uint16_t* qw;
    const uint16_t* kw;
    const float* cos;
    const float* sin;
    int64_t cs;                  // row stride of cos / sin (elements)
    float eps;
    int64_t L, H, rows;          // rows = B * L * H
    // optional cache write
    uint8_t* ck;
    uint8_t* cv;
    float* sk;
    float* sv;
    int64_t qs0, qs1, qs2, ss0, ss1, ss2, start;
    // Device-side validation of the cache write (null: unchecked): set to 1 by
    // qk_check_kernel when a value to be written is NaN/Inf; the cache write
    // (not the in-place q/k update) is then skipped.
    int32_t* status;
};

HN_DEVICE void unpack8(const uint4& v, float (&f)[8]) {
    const uint32_t w[4] = {v.x, v.y, v.z, v.w};
#pragma unroll
    for (int j = 0; j < 4; ++j) {
        f[2 * j] = bf16_bits_to_f32(w[j] & 0xffffu);
        f[2 * j + 1] = bf16_bits_to_f32(w[j] >> 16);
    }
}

HN_DEVICE uint4 pack8(const float (&f)[8]) {
    uint32_t w[4];
#pragma unroll
    for (int j = 0; j < 4; ++j) w[j] = f32_to_bf16_bits(f[2 * j]) | (f32_to_bf16_bits(f[2 * j + 1]) << 16);
    return make_uint4(w[0], w[1], w[2], w[3]);
}

HN_DEVICE float bf16_round(float x) { return bf16_bits_to_f32(f32_to_bf16_bits(x)); }

// RMSNorm + RoPE of one row's 8 dims held by this lane (d0 = 8 * lane16).
// Every fp32 operation rounds on its own, as the reference's tensor ops do:
// contraction is off (the RoPE sum would otherwise fuse into an FMA) and the
// square root is the correctly rounded sqrtf (__fsqrt_rn is the native
// 1-ulp v_sqrt_f32).
HN_DEVICE void norm_rope(float (&x)[8], const float (&w)[8], const float (&c)[8], const float (&s)[8],
                         float eps) {
#pragma clang fp contract(off)
    float ss = 0.0f;
#pragma unroll
    for (int j = 0; j < 8; ++j) ss = ss + x[j] * x[j];
    ss = group_sum<16>(ss);
    const float r = 1.0f / sqrtf(ss * (1.0f / 128.0f) + eps);
    float y[8];
#pragma unroll
    for (int j = 0; j < 8; ++j) y[j] = bf16_round(bf16_round(x[j] * r) * w[j]);
#pragma unroll
    for (int j = 0; j < 8; j += 2) {
        x[j] = y[j] * c[j] + (-y[j + 1]) * s[j];
        x[j + 1] = y[j + 1] * c[j + 1] + y[j] * s[j + 1];
    }
}

// Per-row quantize-on-write of 8 values per lane (16 lanes = one row).
template <int FMT>
HN_DEVICE void quantize_row(const float (&f)[8], uint8_t* code_row, float* scale, int lane16) {
    float amax = 0.0f;
#pragma unroll
    for (int j = 0; j < 8; ++j) amax = fmaxf(amax, fabsf(f[j]));
    amax = group_max<16>(amax);
    const float qmax = FMT == HN_KV_FP8 ? kE4M3Max : 127.0f;
    const float s = amax > 0.0f ? amax / qmax : 1.0f;
    *reinterpret_cast<uint2*>(code_row + lane16 * 8) = codes8<FMT == HN_KV_FP8>(f, Quot(s));
    if (lane16 == 0) *scale = s;
}

// The values one row would write into the cache: the rotated k (bf16, as
// stored in place) and v, checked for NaN/Inf with the same arithmetic as
// qk_norm_rope_kernel, so the check tests exactly what would be written. Sets
// *a.status = 1 if any is not finite (the flag is cleared beforehand).
__global__ __launch_bounds__(256) void qk_check_kernel(Args a) {
    const int lane16 = threadIdx.x & 15;
    uint32_t bad = 0u;
    for (int64_t row = (int64_t)blockIdx.x * 16 + (threadIdx.x >> 4); row < a.rows;
         row += (int64_t)gridDim.x * 16) {  // grid-stride over whole 16-lane groups
        const int64_t h = row % a.H;
        const int64_t t = (row / a.H) % a.L;
        const int64_t b = row / (a.H * a.L);
        const int64_t off = b * a.xs0 + t * a.xs1 + h * a.xs2 + lane16 * 8;
        float kx[8], w[8], c[8], s[8];
        unpack8(*reinterpret_cast<const uint4*>(a.k + off), kx);
        const float4* cp = reinterpret_cast<const float4*>(a.cos + t * a.cs + lane16 * 8);
        const float4* sp = reinterpret_cast<const float4*>(a.sin + t * a.cs + lane16 * 8);
        const float4 c0 = cp[0], c1 = cp[1], s0 = sp[0], s1 = sp[1];
        c[0] = c0.x; c[1] = c0.y; c[2] = c0.z; c[3] = c0.w; c[4] = c1.x; c[5] = c1.y; c[6] = c1.z; c[7] = c1.w;
        s[0] = s0.x; s[1] = s0.y; s[2] = s0.z; s[3] = s0.w; s[4] = s1.x; s[5] = s1.y; s[6] = s1.z; s[7] = s1.w;
        unpack8(*reinterpret_cast<const uint4*>(a.kw + lane16 * 8), w);
        norm_rope(kx, w, c, s, a.eps);
        const uint4 ko = pack8(kx);
        const uint4 vo = *reinterpret_cast<const uint4*>(a.v + off);
        const uint32_t wd[8] = {ko.x, ko.y, ko.z, ko.w, vo.x, vo.y, vo.z, vo.w};
#pragma unroll
        for (int j = 0; j < 8; ++j)  // bf16 exponent all ones: Inf or NaN
            bad |= (uint32_t)((wd[j] & 0x7f80u) == 0x7f80u) | (uint32_t)(((wd[j] >> 16) & 0x7f80u) == 0x7f80u);
    }
    if (__any(bad != 0u) && (threadIdx.x & 63) == 0) *a.status = 1;
}

__global__ void qk_status_clear_kernel(int32_t* status) {
    if (threadIdx.x == 0) *status = 0;
}

template <int FMT, bool CACHE>
__global__ __launch_bounds__(256) void qk_norm_rope_kernel(Args a) {
    const int lane16 = threadIdx.x & 15;
    const int64_t row = (int64_t)blockIdx.x * 16 + (threadIdx.x >> 4);
    if (row >= a.rows) return;  // whole 16-lane groups exit; no barrier below
    const int64_t h = row % a.H;
    const int64_t t = (row / a.H) % a.L;
    const int64_t b = row / (a.H * a.L);
    const int64_t off = b * a.xs0 + t * a.xs1 + h * a.xs2 + lane16 * 8;
    float qx[8], kx[8], w[8], c[8], s[8];
    unpack8(*reinterpret_cast<const uint4*>(a.q + off), qx);
    unpack8(*reinterpret_cast<const uint4*>(a.k + off), kx);
    const float4* cp = reinterpret_cast<const float4*>(a.cos + t * a.cs + lane16 * 8);
    const float4* sp = reinterpret_cast<const float4*>(a.sin + t * a.cs + lane16 * 8);
    const float4 c0 = cp[0], c1 = cp[1], s0 = sp[0], s1 = sp[1];
    c[0] = c0.x; c[1] = c0.y; c[2] = c0.z; c[3] = c0.w; c[4] = c1.x; c[5] = c1.y; c[6] = c1.z; c[7] = c1.w;
    s[0] = s0.x; s[1] = s0.y; s[2] = s0.z; s[3] = s0.w; s[4] = s1.x; s[5] = s1.y; s[6] = s1.z; s[7] = s1.w;

    unpack8(*reinterpret_cast<const uint4*>(a.qw + lane16 * 8), w);
    norm_rope(qx, w, c, s, a.eps);
    unpack8(*reinterpret_cast<const uint4*>(a.kw + lane16 * 8), w);
    norm_rope(kx, w, c, s, a.eps);
    const uint4 qo = pack8(qx), ko = pack8(kx);
    *reinterpret_cast<uint4*>(a.q + off) = qo;
    *reinterpret_cast<uint4*>(a.k + off) = ko;

    if (CACHE && (a.status == nullptr || *a.status == 0)) {
        float kr[8], vx[8];
        unpack8(ko, kr);  // the rounded bf16 values that were stored
        unpack8(*reinterpret_cast<const uint4*>(a.v + off), vx);
        const int64_t tt = t + a.start;
        quantize_row<FMT>(kr, a.ck + b * a.qs0 + tt * a.qs1 + h * a.qs2,
                          a.sk + b * a.ss0 + tt * a.ss1 + h * a.ss2, lane16);
        quantize_row<FMT>(vx, a.cv + b * a.qs0 + tt * a.qs1 + h * a.qs2,
                          a.sv + b * a.ss0 + tt * a.ss1 + h * a.ss2, lane16);
    }
}

}  // namespace qkr
}  // namespace hn

using namespace hn;

extern "C" int hn_qk_norm_rope_kv(int fmt, void* q, void* k, const void* v, const int64_t* xs,
                                  int64_t B, int64_t L, int64_t H, int64_t D, const void* q_weight,
                                  const void* k_weight, const float* cos_t, const float* sin_t,
                                  int64_t cs, float eps, void* kc, void* vc, const int64_t* qs,
                                  float* ks, float* vs, const int64_t* ss, int64_t cap,
                                  int64_t start, int32_t* status, void* stream) {
    HN_REQUIRE(fmt == HN_KV_FP8 || fmt == HN_KV_INT8, HN_E_ARG, "hn_qk_norm_rope_kv: unknown KV format");
    HN_REQUIRE(D == 128, HN_E_ARG, "hn_qk_norm_rope_kv: head dim must be 128");
    HN_REQUIRE(B >= 0 && L >= 0 && H > 0 && start >= 0, HN_E_ARG, "hn_qk_norm_rope_kv: invalid shape");
    HN_REQUIRE(xs && xs[3] == 1 && xs[0] % 8 == 0 && xs[1] % 8 == 0 && xs[2] % 8 == 0, HN_E_ARG,
               "hn_qk_norm_rope_kv: q/k/v strides must be multiples of 8 with contiguous head dim");
    HN_REQUIRE(cs >= D && cs % 4 == 0, HN_E_ARG, "hn_qk_norm_rope_kv: cos/sin row stride");
    HN_REQUIRE(aligned(q, 16) && aligned(k, 16) && aligned(v, 16) && aligned(q_weight, 16) &&
                   aligned(k_weight, 16) && aligned(cos_t, 16) && aligned(sin_t, 16),
               HN_E_ARG, "hn_qk_norm_rope_kv: misaligned pointer");
    const bool cache = kc != nullptr;
    if (cache) {
        HN_REQUIRE(vc && ks && vs && qs && ss, HN_E_ARG, "hn_qk_norm_rope_kv: incomplete cache arguments");
        HN_REQUIRE(qs[3] == 1 && qs[0] % 8 == 0 && qs[1] % 8 == 0 && qs[2] % 8 == 0, HN_E_ARG,
                   "hn_qk_norm_rope_kv: cache strides must be multiples of 8 bytes");
        HN_REQUIRE(aligned(kc, 8) && aligned(vc, 8) && aligned(ks, 4) && aligned(vs, 4), HN_E_ARG,
                   "hn_qk_norm_rope_kv: misaligned cache pointer");
        HN_REQUIRE(cap >= 0 && start <= cap && L <= cap - start, HN_E_ARG,
                   "hn_qk_norm_rope_kv: KV write past the cache capacity (start + L > cap)");
        HN_REQUIRE(aligned(status, 4), HN_E_ARG, "hn_qk_norm_rope_kv: misaligned status pointer");
    } else {
        HN_REQUIRE(status == nullptr, HN_E_ARG, "hn_qk_norm_rope_kv: status without a cache write");
    }
    const int64_t rows = B * L * H;
    if (rows == 0) return HN_OK;
    HN_REQUIRE(q && k && v && q_weight && k_weight && cos_t && sin_t, HN_E_ARG,
               "hn_qk_norm_rope_kv: null pointer");
    if (const int rc = require_gfx950("hn_qk_norm_rope_kv"); rc != HN_OK) return rc;
    qkr::Args a;
    a.q = (uint16_t*)q; a.k = (uint16_t*)k; a.v = (const uint16_t*)v;
    a.xs0 = xs[0]; a.xs1 = xs[1]; a.xs2 = xs[2];
    a.qw = (const uint16_t*)q_weight; a.kw = (const uint16_t*)k_weight;
    a.cos = cos_t; a.sin = sin_t; a.cs = cs; a.eps = eps;
    a.L = L; a.H = H; a.rows = rows;
    a.ck = (uint8_t*)kc; a.cv = (uint8_t*)vc; a.sk = ks; a.sv = vs;
    a.qs0 = cache ? qs[0] : 0; a.qs1 = cache ? qs[1] : 0; a.qs2 = cache ? qs[2] : 0;
    a.ss0 = cache ? ss[0] : 0; a.ss1 = cache ? ss[1] : 0; a.ss2 = cache ? ss[2] : 0;
    a.start = start;
    a.status = status;
    const int64_t blocks = (rows + 15) / 16;
    HN_REQUIRE(blocks <= 0x7fffffffLL, HN_E_ARG, "hn_qk_norm_rope_kv: too many rows");
    hipStream_t st = (hipStream_t)stream;
    const dim3 grid((unsigned)blocks);
    if (status) {
        qkr::qk_status_clear_kernel<<<1, 64, 0, st>>>(status);
        qkr::qk_check_kernel<<<(unsigned)stream_grid(blocks, 8), 256, 0, st>>>(a);
    }
    if (!cache)
        qkr::qk_norm_rope_kernel<HN_KV_FP8, false><<<grid, 256, 0, st>>>(a);
    else if (fmt == HN_KV_FP8)
        qkr::qk_norm_rope_kernel<HN_KV_FP8, true><<<grid, 256, 0, st>>>(a);
    else
        qkr::qk_norm_rope_kernel<HN_KV_INT8, true><<<grid, 256, 0, st>>>(a);
    return check_launch("hn_qk_norm_rope_kv");
}
