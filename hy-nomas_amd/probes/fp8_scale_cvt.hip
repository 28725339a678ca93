// Device check of gfx950's scaled FP8 conversions: do
// v_cvt_scalef32_pk_{f32,bf16,f16}_fp8 multiply each e4m3 code by their fp32
// scale operand (code * s, rounded to nearest even), or by the power of two
// of that operand's exponent only (the E8M0 meaning of an MX block scale)?
// The answer decides whether the per-key scale of a KV cache row can be folded
// into the conversion that dequantizes it.
//
// Every one of the 256 codes is converted under 4096 scales (1, 0.5 and
// 2^u, u uniform in [-20, 4)); each result is compared with code * s and
// with code * 2^(e - 1), where s = m 2^e, m in [0.5, 1).
//
// Build: hy-nomas_amd/build.py (build_probes) -> hy-nomas_amd/probes/fp8_scale_cvt
// Run:   hy-nomas_amd/probes/fp8_scale_cvt   (one GPU, well under a second)
#include <hip/hip_runtime.h>

#include <cmath>
#include <cstdint>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <random>
#include <vector>

#define CHECK(x)                                                                       \
    do {                                                                               \
        hipError_t e_ = (x);                                                           \
        if (e_ != hipSuccess) {                                                        \
            fprintf(stderr, "%s: %s\n", #x, hipGetErrorString(e_));                    \
            exit(1);                                                                   \
        }                                                                              \
    } while (0)

typedef float f32x2 __attribute__((ext_vector_type(2)));
typedef __bf16 bf16x2 __attribute__((ext_vector_type(2)));
typedef _Float16 f16x2 __attribute__((ext_vector_type(2)));

// Codes 0 and 1 of word w[i] (bytes 0 and 1) under scale s[i].
__global__ void convert(const uint32_t* w, const float* s, f32x2* o32, bf16x2* obf, f16x2* of16, int n) {
    const int i = blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= n) return;
    o32[i] = __builtin_amdgcn_cvt_scalef32_pk_f32_fp8(w[i], s[i], false);
    obf[i] = __builtin_amdgcn_cvt_scalef32_pk_bf16_fp8(w[i], s[i], false);
    of16[i] = __builtin_amdgcn_cvt_scalef32_pk_f16_fp8(w[i], s[i], false);
}

// e4m3 (OCP, bias 7, no infinities, S.1111.111 = NaN) decoded from its bits.
static float e4m3_value(uint32_t c) {
    const int e = (c >> 3) & 15, m = c & 7;
    if (e == 15 && m == 7) return NAN;
    const float v = e == 0 ? ldexpf((float)m, -9) : ldexpf(8.0f + m, e - 10);
    return (c & 0x80) ? -v : v;
}

static uint16_t bf16_bits(float f) {  // round to nearest even
    uint32_t b;
    memcpy(&b, &f, 4);
    b += 0x7fffu + ((b >> 16) & 1u);
    return (uint16_t)(b >> 16);
}

static uint16_t f16_bits(float f) {
    const _Float16 h = (_Float16)f;
    uint16_t b;
    memcpy(&b, &h, 2);
    return b;
}

static bool same_or_zero(uint32_t a, uint32_t b, uint32_t sign_bit) {
    return a == b || ((a & ~sign_bit) == 0 && (b & ~sign_bit) == 0);
}

int main() {
    constexpr int NS = 4096, PAIRS = 128, n = NS * PAIRS;
    std::vector<uint32_t> w(n);
    std::vector<float> s(n);
    std::mt19937 gen(1);
    std::uniform_real_distribution<float> u(-20.0f, 4.0f);
    for (int j = 0; j < NS; ++j) {
        const float sc = j == 0 ? 1.0f : (j == 1 ? 0.5f : exp2f(u(gen)));
        for (int c = 0; c < PAIRS; ++c) {
            w[j * PAIRS + c] = (uint32_t)(2 * c) | ((uint32_t)(2 * c + 1) << 8);
            s[j * PAIRS + c] = sc;
        }
    }
    uint32_t* dw;
    float* ds;
    f32x2* d32;
    bf16x2* dbf;
    f16x2* d16;
    CHECK(hipMalloc(&dw, n * sizeof(uint32_t)));
    CHECK(hipMalloc(&ds, n * sizeof(float)));
    CHECK(hipMalloc(&d32, n * sizeof(f32x2)));
    CHECK(hipMalloc(&dbf, n * sizeof(bf16x2)));
    CHECK(hipMalloc(&d16, n * sizeof(f16x2)));
    CHECK(hipMemcpy(dw, w.data(), n * sizeof(uint32_t), hipMemcpyHostToDevice));
    CHECK(hipMemcpy(ds, s.data(), n * sizeof(float), hipMemcpyHostToDevice));
    convert<<<(n + 255) / 256, 256>>>(dw, ds, d32, dbf, d16, n);
    CHECK(hipGetLastError());
    CHECK(hipDeviceSynchronize());
    std::vector<float> r32(2 * n);
    std::vector<uint16_t> rbf(2 * n), r16(2 * n);
    CHECK(hipMemcpy(r32.data(), d32, n * sizeof(f32x2), hipMemcpyDeviceToHost));
    CHECK(hipMemcpy(rbf.data(), dbf, n * sizeof(bf16x2), hipMemcpyDeviceToHost));
    CHECK(hipMemcpy(r16.data(), d16, n * sizeof(f16x2), hipMemcpyDeviceToHost));

    long total = 0, f32_prod = 0, f32_exp = 0, bf_prod = 0, bf_exp = 0, h_prod = 0, h_exp = 0;
    for (int i = 0; i < n; ++i)
        for (int h = 0; h < 2; ++h) {
            const uint32_t c = (w[i] >> (8 * h)) & 0xffu;
            const float cv = e4m3_value(c);
            if (std::isnan(cv)) continue;
            ++total;
            int e;
            frexpf(s[i], &e);
            const float prod = cv * s[i], pexp = cv * ldexpf(1.0f, e - 1);
            uint32_t got, want_p, want_e;
            memcpy(&got, &r32[2 * i + h], 4);
            memcpy(&want_p, &prod, 4);
            memcpy(&want_e, &pexp, 4);
            f32_prod += same_or_zero(got, want_p, 0x80000000u);
            f32_exp += same_or_zero(got, want_e, 0x80000000u);
            bf_prod += same_or_zero(rbf[2 * i + h], bf16_bits(prod), 0x8000u);
            bf_exp += same_or_zero(rbf[2 * i + h], bf16_bits(pexp), 0x8000u);
            h_prod += same_or_zero(r16[2 * i + h], f16_bits(prod), 0x8000u);
            h_exp += same_or_zero(r16[2 * i + h], f16_bits(pexp), 0x8000u);
        }
    printf("%ld finite (code, scale) pairs; results equal to\n", total);
    printf("%-28s %14s %22s\n", "instruction", "code * s", "code * 2^(exp of s)");
    printf("%-28s %14ld %22ld\n", "v_cvt_scalef32_pk_f32_fp8", f32_prod, f32_exp);
    printf("%-28s %14ld %22ld\n", "v_cvt_scalef32_pk_bf16_fp8", bf_prod, bf_exp);
    printf("%-28s %14ld %22ld\n", "v_cvt_scalef32_pk_f16_fp8", h_prod, h_exp);
    CHECK(hipFree(dw));
    CHECK(hipFree(ds));
    CHECK(hipFree(d32));
    CHECK(hipFree(dbf));
    CHECK(hipFree(d16));
    return 0;
}
