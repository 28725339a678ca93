/*
 * Exhaustive host check of the quantizers' quotient (hy-nomas_amd/csrc/quant.hip,
 * struct Quot): for every bf16 row maximum amax > 0 and every bf16 x with
 * |x| <= amax, both signs, and each scale rule the kernels use,
 *
 *     y = fl(x * r), r = fl(1 / s);  e = fma(-s, y, x);  q = copysign(fma(e, r, y), x)
 *
 * gives the same code as the reference's fl32(x / s): the e4m3 RNE code
 * (oracle encoder) for the FP8 rules, and the fp32 round-half-away INT8 code
 * of int8_kv_cache.py:150-157 for the /127 rule. Rows with s < 2^-100 take the
 * IEEE division in the kernels and are skipped here.
 *
 * Build: gcc -O2 -fopenmp -ffp-contract=off fast_quotient_check.c ../oracle/fp8_oracle.c -lm
 * Prints one line per rule; exits non-zero on any mismatch.
 */
#include <math.h>
#include <stdint.h>
#include <stdio.h>
#include <string.h>

uint8_t hn_oracle_e4m3_encode(float f);

static float from_bits(uint32_t u) { float x; memcpy(&x, &u, 4); return x; }

static int int8_code(float v)
{
    float r = v >= 0.0f ? floorf(v + 0.5f) : ceilf(v - 0.5f);
    r = fminf(fmaxf(r, -127.0f), 127.0f);
    return (int)r;
}

static float scale_of(int rule, float amax)
{
    if (rule == 0) return fmaxf(amax, 1e-4f) / 448.0f;   /* linear activations / weights */
    if (rule == 1) return amax / 448.0f;                  /* FP8 KV (amax > 0 here) */
    return amax / 127.0f;                                 /* INT8-compatible KV */
}

int main(void)
{
    static const char *names[3] = {"max(amax,1e-4)/448", "amax/448", "amax/127"};
    int failed = 0;
    for (int rule = 0; rule < 3; ++rule) {
        unsigned long long pairs = 0, skipped = 0, bad = 0;
#pragma omp parallel for schedule(dynamic, 64) reduction(+ : pairs, skipped, bad)
        for (uint32_t ab = 1; ab < 0x7F80u; ++ab) {
            const float amax = from_bits(ab << 16);
            const float s = scale_of(rule, amax);
            if (!(s >= 0x1p-100f)) { skipped += 2ull * (ab + 1); continue; }
            const float r = 1.0f / s;
            for (uint32_t xs = 0; xs <= 2 * ab + 1; ++xs) {
                const float x = from_bits(((xs >> 1) << 16) | ((xs & 1u) << 31));
                const float exact = x / s;
                const float y = x * r;
                const float e = fmaf(-s, y, x);
                const float q = copysignf(fmaf(e, r, y), x);
                ++pairs;
                if (rule < 2) bad += hn_oracle_e4m3_encode(q) != hn_oracle_e4m3_encode(exact);
                else bad += int8_code(q) != int8_code(exact);
            }
        }
        printf("rule %s: %llu (amax, x) pairs checked, %llu on the exact path, %llu code mismatches\n",
               names[rule], pairs, skipped, bad);
        failed |= bad != 0;
    }
    return failed;
}
