// FP8 quantizers for the quantized inference path (gfx950):
//   * per-row (per-token activations / per-output-channel weights)
//   * 128x128 blockwise (the decoder GEMM's activation format)
//   * KV quantize-on-write into a token-major [B, cap, H, D] cache (FP8 and
//     the INT8-compatible recipe), and KV decode of a valid prefix.
// All are HBM-bound streaming kernels: 16-byte loads per lane, reductions in
// registers + cross-lane shuffles. Codes must be bit-identical to the
// reference's fp32 recipe e4m3_rne(fl32(x / s)) (or its INT8 rounding of
// fl32(x / s)); see Quot for how the quotient is formed.
#include "hn_capi_internal.h"
#include "hn_common.h"

namespace hn {

// Eight bf16 (one uint4) -> eight e4m3 codes of fl32(x / s), then RNE to
// e4m3, as two dwords.
template <bool EXACT>
HN_DEVICE uint2 encode8(const uint4& v, const Quot& d) {
    const uint32_t w[4] = {v.x, v.y, v.z, v.w};
    float f[8];
#pragma unroll
    for (int j = 0; j < 4; ++j) {
        f[2 * j] = d.at<EXACT>(bf16_lo(w[j]));
        f[2 * j + 1] = d.at<EXACT>(bf16_hi(w[j]));
    }
    return make_uint2(e4m3_encode4(f[0], f[1], f[2], f[3]), e4m3_encode4(f[4], f[5], f[6], f[7]));
}

// ---------------------------------------------------------------------------
// Per-row quantization. One wave per row, four rows per 256-thread block: the
// row max is a wave reduction (no block barrier), and each lane keeps its CPL
// chunks of 8 bf16 in registers between the max and the encode pass, so the
// row is read from HBM once with all of a lane's 16-byte loads in flight.
template <int CPL>
__global__ __launch_bounds__(256) void quantize_rows_kernel(
    const uint16_t* __restrict__ x, int64_t rows, int64_t cols, int64_t row_stride, int mode,
    float amax_floor, uint8_t* __restrict__ q, float* __restrict__ scale) {
    const int lane = threadIdx.x & 63;
    for (int64_t row = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6); row < rows;
         row += (int64_t)gridDim.x * 4) {  // grid-stride; whole waves, no barrier
    const uint16_t* xr = x + row * row_stride;
    const int nchunks = (int)(cols >> 3);
    uint4 v[CPL];
    float amax = 0.0f;
#pragma unroll
    for (int i = 0; i < CPL; ++i) {
        const int c = lane + i * 64;
        if (c < nchunks) v[i] = *reinterpret_cast<const uint4*>(xr + (int64_t)c * 8);
    }
#pragma unroll
    for (int i = 0; i < CPL; ++i) {
        const int c = lane + i * 64;
        if (c < nchunks) {
            const uint32_t w[4] = {v[i].x, v[i].y, v[i].z, v[i].w};
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                amax = max_nan(amax, fabsf(bf16_bits_to_f32(w[j] & 0xffffu)));
                amax = max_nan(amax, fabsf(bf16_bits_to_f32(w[j] >> 16)));
            }
        }
    }
    amax = group_max_nan<64>(amax);
    const float s = mode == HN_SCALE_CLAMP ? max_nan(amax, amax_floor) / kE4M3Max
                                           : (amax > 0.0f ? amax / kE4M3Max : 1.0f);
    if (lane == 0) scale[row] = s;
    const Quot d(s);
    uint8_t* qr = q + row * cols;
    d.with_form([&](auto form) {
#pragma unroll
        for (int i = 0; i < CPL; ++i) {
            const int c = lane + i * 64;
            if (c < nchunks) *reinterpret_cast<uint2*>(qr + (int64_t)c * 8) = encode8<decltype(form)::value>(v[i], d);
        }
    });
    }
}

// ---------------------------------------------------------------------------
// Per-row quantization of wide rows (more than 4096 columns): one 256-thread
// workgroup per row, thread t holding chunks t, t + 256, ... (CPT of 8 bf16).
// The row max is a wave reduction plus one exchange of the four wave maxima
// through LDS. Holding a 12288-column row in one wave took 24 chunks per lane
// and the register file limited the waves per SIMD: 3.9 TB/s.
template <int CPT>
__global__ __launch_bounds__(256) void quantize_rows_wide_kernel(
    const uint16_t* __restrict__ x, int64_t rows, int64_t cols, int64_t row_stride, int mode,
    float amax_floor, uint8_t* __restrict__ q, float* __restrict__ scale) {
    __shared__ float wave_max[4];
    const int t = threadIdx.x, lane = t & 63, wave = t >> 6;
    const int nchunks = (int)(cols >> 3);
    for (int64_t row = blockIdx.x; row < rows; row += gridDim.x) {  // grid-stride, uniform per block
        const uint16_t* xr = x + row * row_stride;
        uint4 v[CPT];
#pragma unroll
        for (int i = 0; i < CPT; ++i) {
            const int c = t + 256 * i;
            if (c < nchunks) v[i] = *reinterpret_cast<const uint4*>(xr + (int64_t)c * 8);
        }
        float amax = 0.0f;
#pragma unroll
        for (int i = 0; i < CPT; ++i) {
            const int c = t + 256 * i;
            if (c < nchunks) {
                const uint32_t w[4] = {v[i].x, v[i].y, v[i].z, v[i].w};
#pragma unroll
                for (int j = 0; j < 4; ++j)
                    amax = max_nan(amax, max_nan(fabsf(bf16_lo(w[j])), fabsf(bf16_hi(w[j]))));
            }
        }
        amax = group_max_nan<64>(amax);
        if (lane == 0) wave_max[wave] = amax;
        __syncthreads();
        amax = max_nan(max_nan(wave_max[0], wave_max[1]), max_nan(wave_max[2], wave_max[3]));
        __syncthreads();  // wave_max is rewritten for the next row
        const float s = mode == HN_SCALE_CLAMP ? max_nan(amax, amax_floor) / kE4M3Max
                                               : (amax > 0.0f ? amax / kE4M3Max : 1.0f);
        if (t == 0) scale[row] = s;
        const Quot d(s);
        uint8_t* qr = q + row * cols;
        d.with_form([&](auto form) {
#pragma unroll
            for (int i = 0; i < CPT; ++i) {
                const int c = t + 256 * i;
                if (c < nchunks)
                    *reinterpret_cast<uint2*>(qr + (int64_t)c * 8) = encode8<decltype(form)::value>(v[i], d);
            }
        });
    }
}

// ---------------------------------------------------------------------------
// LayerNorm (no affine) + adaLN modulate + per-token FP8 quantization, fused:
//   y = bf16((x - mean) * rsqrt(var + eps))            F.layer_norm on bf16
//   o = bf16(bf16(y * bf16(1 + scale[c])) + shift[c])  _modulate in bf16 ops
//   per-token e4m3 codes of o with the quantize_rows_kernel recipe.
// Each bf16 rounding is one of the reference's bf16 tensor ops
// (nomas_compile_prepost.py:14-15,40-43,81-84), so only the fp32 mean and
// variance differ from the unfused path (the order of their sums), which can
// move a LayerNorm output by one bf16 ulp at a rounding boundary. The sums have
// a fixed order and the kernel body turns FP contraction off (the compiler
// would otherwise fuse ss + d * d into one FMA; HIP's __fmul_rn / __fadd_rn
// are plain operators that keep the header's contraction setting, so the
// body uses operators under the pragma); lane l adds its values in storage
// order (chunks l, l + 64, ..., 8 values each),
// then the lanes combine by xor butterfly (every lane ends with the same sum,
// fp addition being commutative); mean = sum * (1 / cols), var = sum((x -
// mean)^2) * (1 / cols), rstd = 1 / sqrt(var + eps), all fp32 and correctly
// rounded (sqrtf, not __fsqrt_rn, which is the native 1-ulp v_sqrt_f32). One wave per row as in quantize_rows_kernel: the row is read once
// and kept in registers through the two reductions and the encode. Row r uses
// modulation vectors b = r / rows_per_batch (shift/scale [B, cols], batch
// stride mod_stride).
template <int CPL, bool FULL>
__global__ __launch_bounds__(256) void ln_mod_quantize_kernel(
    const uint16_t* __restrict__ x, int64_t rows, int64_t cols, int64_t rows_per_batch,
    const uint16_t* __restrict__ shift, const uint16_t* __restrict__ scl, int64_t mod_stride, float eps,
    float amax_floor, uint8_t* __restrict__ q, float* __restrict__ scale) {
#pragma clang fp contract(off)
    const int lane = threadIdx.x & 63;
    const float inv_cols = 1.0f / (float)cols;
    for (int64_t row = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6); row < rows;
         row += (int64_t)gridDim.x * 4) {  // grid-stride; whole waves, no barrier
        const uint16_t* xr = x + row * cols;
        const int nchunks = (int)(cols >> 3);
        const int64_t b = row / rows_per_batch;
        const uint16_t* sh = shift + b * mod_stride;
        const uint16_t* sc = scl + b * mod_stride;
        // every load of the row issued up front (x from HBM, the modulation
        // vectors from L2), so they are all in flight together
        uint4 v[CPL], s8[CPL], h8[CPL];
#pragma unroll
        for (int i = 0; i < CPL; ++i) {
            const int c = lane + i * 64;
            if (FULL || c < nchunks) v[i] = *reinterpret_cast<const uint4*>(xr + (int64_t)c * 8);
        }
#pragma unroll
        for (int i = 0; i < CPL; ++i) {
            const int c = lane + i * 64;
            if (FULL || c < nchunks) {
                s8[i] = *reinterpret_cast<const uint4*>(sc + (int64_t)c * 8);
                h8[i] = *reinterpret_cast<const uint4*>(sh + (int64_t)c * 8);
            }
        }
        float sum = 0.0f;
#pragma unroll
        for (int i = 0; i < CPL; ++i) {
            const int c = lane + i * 64;
            if (FULL || c < nchunks) {
                const uint32_t w[4] = {v[i].x, v[i].y, v[i].z, v[i].w};
#pragma unroll
                for (int j = 0; j < 4; ++j) {
                    sum = sum + bf16_bits_to_f32(w[j] & 0xffffu);
                    sum = sum + bf16_bits_to_f32(w[j] >> 16);
                }
            }
        }
        const float mean = group_sum<64>(sum) * inv_cols;
        float ss = 0.0f;
#pragma unroll
        for (int i = 0; i < CPL; ++i) {
            const int c = lane + i * 64;
            if (FULL || c < nchunks) {
                const uint32_t w[4] = {v[i].x, v[i].y, v[i].z, v[i].w};
#pragma unroll
                for (int j = 0; j < 4; ++j) {
                    const float d0 = bf16_bits_to_f32(w[j] & 0xffffu) - mean;
                    const float d1 = bf16_bits_to_f32(w[j] >> 16) - mean;
                    ss = ss + d0 * d0;
                    ss = ss + d1 * d1;
                }
            }
        }
        const float rstd = 1.0f / sqrtf(group_sum<64>(ss) * inv_cols + eps);
        float amax = 0.0f;
#pragma unroll
        for (int i = 0; i < CPL; ++i) {
            const int c = lane + i * 64;
            if (FULL || c < nchunks) {
                uint32_t w[4] = {v[i].x, v[i].y, v[i].z, v[i].w};
                const uint32_t ws[4] = {s8[i].x, s8[i].y, s8[i].z, s8[i].w};
                const uint32_t wh[4] = {h8[i].x, h8[i].y, h8[i].z, h8[i].w};
#pragma unroll
                for (int j = 0; j < 4; ++j) {
                    // each bf16 rounding is one v_cvt_pk_bf16_f32 for the pair
                    const uint32_t y = f32x2_to_bf16x2((bf16_lo(w[j]) - mean) * rstd,
                                                       (bf16_hi(w[j]) - mean) * rstd);
                    const uint32_t a = f32x2_to_bf16x2(1.0f + bf16_lo(ws[j]), 1.0f + bf16_hi(ws[j]));
                    const uint32_t m = f32x2_to_bf16x2(bf16_lo(y) * bf16_lo(a), bf16_hi(y) * bf16_hi(a));
                    w[j] = f32x2_to_bf16x2(bf16_lo(m) + bf16_lo(wh[j]), bf16_hi(m) + bf16_hi(wh[j]));
                    amax = max_nan(amax, max_nan(fabsf(bf16_lo(w[j])), fabsf(bf16_hi(w[j]))));
                }
                v[i] = make_uint4(w[0], w[1], w[2], w[3]);
            }
        }
        amax = group_max_nan<64>(amax);
        const float s = max_nan(amax, amax_floor) / kE4M3Max;
        if (lane == 0) scale[row] = s;
        const Quot d(s);
        uint8_t* qr = q + row * cols;
        d.with_form([&](auto form) {
#pragma unroll
            for (int i = 0; i < CPL; ++i) {
                const int c = lane + i * 64;
                if (FULL || c < nchunks) *reinterpret_cast<uint2*>(qr + (int64_t)c * 8) = encode8<decltype(form)::value>(v[i], d);
            }
        });
    }
}

// ---------------------------------------------------------------------------
// 128x128 blockwise quantization: one 256-thread block per (128-row, 128-col)
// tile; each thread holds 8 chunks of 8 bf16. Rows past `rows` are the zero
// padding of the reference recipe: they contribute nothing to amax and are
// not stored.
__global__ __launch_bounds__(256) void quantize_blockwise_kernel(
    const uint16_t* __restrict__ x, int64_t rows, int64_t cols, uint8_t* __restrict__ q,
    float* __restrict__ scale) {
    const int64_t r0 = (int64_t)blockIdx.x * 128, c0 = (int64_t)blockIdx.y * 128;
    uint4 v[8];
    float amax = 0.0f;
#pragma unroll
    for (int i = 0; i < 8; ++i) {
        const int id = threadIdx.x + i * 256;
        const int64_t r = r0 + (id >> 4);
        const int64_t c = c0 + (id & 15) * 8;
        if (r < rows) {
            v[i] = *reinterpret_cast<const uint4*>(x + r * cols + c);
            const uint32_t w[4] = {v[i].x, v[i].y, v[i].z, v[i].w};
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                amax = max_nan(amax, fabsf(bf16_bits_to_f32(w[j] & 0xffffu)));
                amax = max_nan(amax, fabsf(bf16_bits_to_f32(w[j] >> 16)));
            }
        }
    }
    amax = group_max_nan<64>(amax);
    __shared__ float red[4];
    if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = amax;
    __syncthreads();
    amax = max_nan(max_nan(red[0], red[1]), max_nan(red[2], red[3]));
    const float s = max_nan(amax, 1e-4f) / kE4M3Max;
    if (threadIdx.x == 0) scale[blockIdx.x * gridDim.y + blockIdx.y] = s;
    const Quot d(s);
    d.with_form([&](auto form) {
#pragma unroll
        for (int i = 0; i < 8; ++i) {
            const int id = threadIdx.x + i * 256;
            const int64_t r = r0 + (id >> 4);
            const int64_t c = c0 + (id & 15) * 8;
            if (r < rows) *reinterpret_cast<uint2*>(q + r * cols + c) = encode8<decltype(form)::value>(v[i], d);
        }
    });
}

// ---------------------------------------------------------------------------
// KV quantize-on-write. A row is one (batch, token, head) vector of D = 128
// values: 16 lanes x 8 values, so a wave covers 4 rows and a 256-thread block
// 16 rows. Rows are enumerated head-fastest, which makes consecutive rows
// consecutive 128-byte code lines of the token-major cache. blockIdx.y selects
// K (0) or V (1) for the paired launch.
struct KvArgs {
    const uint16_t* x[2];
    uint8_t* q[2];
    float* s[2];
    int64_t xs0, xs1, xs2;
    int64_t qs0, qs1, qs2;
    int64_t ss0, ss1, ss2;
    int64_t L, H, rows, start;
    // Work units of KV_UNIT = 64 rows. TOKEN_FAST: 8 tokens x 8 heads of one
    // batch (ttiles = ceil(L / 8) token tiles per head tile, htiles =
    // ceil(H / 8)); otherwise 64 consecutive (token, head) rows of one batch
    // (ttiles = ceil(L * H / 64) per batch, L * H < 2^31).
    int64_t ttiles, htiles, units;
    // Device-side validation (null: unchecked): set by kv_check_kernel when a
    // value is NaN/Inf; the write then stores nothing.
    const int32_t* status;
};

// Validate-before-write on the device (the reference's check,
// int8_kv_cache.py:140-141,176, without its host synchronisation):
// status_clear_kernel zeroes the flag, kv_check_kernel sets it to 1 when any
// value of the one or two sources (blockIdx.y) is NaN or Inf, and the write
// kernel that follows on the stream reads it and writes nothing when it is
// set. The flag is cleared by a kernel rather than a memset so that the
// sequence can be recorded in a graph.
__global__ void status_clear_kernel(int32_t* status) {
    if (threadIdx.x == 0) *status = 0;
}

struct KvCheckArgs {
    const uint16_t* x[2];
    int64_t xs0, xs1, xs2;
    int64_t L, H, rows;
    int32_t* status;
};

// One (batch, token, head) row of 128 bf16 per 16-lane group, 8 per lane, in
// a grid-stride loop; rows are walked token-fastest when the source's token
// stride is the smaller one, so that consecutive groups read adjacent rows.
template <bool TOKEN_FAST>
__global__ __launch_bounds__(256) void kv_check_kernel(KvCheckArgs a) {
    const uint16_t* x = a.x[blockIdx.y];
    const int lane16 = threadIdx.x & 15;
    uint32_t bad = 0u;
    for (int64_t row = (int64_t)blockIdx.x * 16 + (threadIdx.x >> 4); row < a.rows;
         row += (int64_t)gridDim.x * 16) {
        int64_t b, t, h;
        if (TOKEN_FAST) {
            t = row % a.L;
            h = (row / a.L) % a.H;
            b = row / (a.L * a.H);
        } else {
            h = row % a.H;
            t = (row / a.H) % a.L;
            b = row / (a.L * a.H);
        }
        const uint4 v = *reinterpret_cast<const uint4*>(x + b * a.xs0 + t * a.xs1 + h * a.xs2 + lane16 * 8);
        const uint32_t w[4] = {v.x, v.y, v.z, v.w};
#pragma unroll
        for (int j = 0; j < 4; ++j)  // bf16 exponent all ones: Inf or NaN
            bad |= (uint32_t)((w[j] & 0x7f80u) == 0x7f80u) | (uint32_t)(((w[j] >> 16) & 0x7f80u) == 0x7f80u);
    }
    if (__any(bad != 0u) && (threadIdx.x & 63) == 0) *a.status = 1;
}

constexpr int KV_ROWS_PER_GROUP = 4;  // rows each 16-lane group carries (loads issued together)
constexpr int KV_UNIT = 16 * KV_ROWS_PER_GROUP;

// TOKEN_FAST: rows are enumerated token-fastest within a (batch, head) instead
// of head-fastest, chosen when the values' token stride is the smaller one (a
// [B, H, L, D] source viewed as [B, L, H, D]): the loads of consecutive rows
// are then consecutive 256-byte rows of the source, and each 128-byte code row
// is still one whole cache line.
template <int FMT, bool TOKEN_FAST>
__global__ __launch_bounds__(256) void kv_quantize_kernel(KvArgs a) {
    const int sel = blockIdx.y;
    const int lane16 = threadIdx.x & 15;
    if (a.status != nullptr && *a.status != 0) return;  // rejected: write nothing
    for (int64_t unit = blockIdx.x; unit < a.units; unit += gridDim.x) {  // grid-stride
    // Group g (16 lanes) takes 4 rows, k = 0..3. TOKEN_FAST: token 8 tt + g % 8
    // of heads 8 ht + 4 (g / 8) + k -- for each k the loads are two runs of 8
    // consecutive tokens (2 KB each), and every token's 8 heads of codes
    // (1 KB) and scales (one 32-byte sector) are written by the unit.
    // Otherwise rows g + 16 k of the unit's 64 consecutive (token, head) rows.
    // Unit -> tiles is one wave-uniform division; per row there is no
    // division on the TOKEN_FAST path and one 32-bit division by H otherwise.
    const int g = threadIdx.x >> 4;
    uint4 v[KV_ROWS_PER_GROUP];
    int64_t rb[KV_ROWS_PER_GROUP], rt[KV_ROWS_PER_GROUP], rh[KV_ROWS_PER_GROUP];
#pragma unroll
    for (int k = 0; k < KV_ROWS_PER_GROUP; ++k) {
        // Rows past the end repeat the last token / head: they rewrite identical bytes.
        if (TOKEN_FAST) {
            const int64_t bh = unit / a.ttiles;          // b * htiles + ht
            const int64_t tt = unit - bh * a.ttiles;
            const int64_t b = bh / a.htiles;
            const int64_t t = tt * 8 + (g & 7);
            const int64_t h = (bh - b * a.htiles) * 8 + 4 * (g >> 3) + k;
            rb[k] = b;
            rt[k] = t < a.L ? t : a.L - 1;
            rh[k] = h < a.H ? h : a.H - 1;
        } else {
            const int64_t b = unit / a.ttiles;
            int64_t r = (unit - b * a.ttiles) * KV_UNIT + g + 16 * k;
            r = r < a.L * a.H ? r : a.L * a.H - 1;
            const uint32_t t = (uint32_t)r / (uint32_t)a.H;
            rb[k] = b;
            rt[k] = t;
            rh[k] = r - (int64_t)t * a.H;
        }
        v[k] = *reinterpret_cast<const uint4*>(a.x[sel] + rb[k] * a.xs0 + rt[k] * a.xs1 +
                                               rh[k] * a.xs2 + lane16 * 8);
    }
#pragma unroll
    for (int k = 0; k < KV_ROWS_PER_GROUP; ++k) {
        const uint32_t w[4] = {v[k].x, v[k].y, v[k].z, v[k].w};
        float f[8];
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            f[2 * j] = bf16_bits_to_f32(w[j] & 0xffffu);
            f[2 * j + 1] = bf16_bits_to_f32(w[j] >> 16);
        }
        float amax = 0.0f;
#pragma unroll
        for (int j = 0; j < 8; ++j) amax = fmaxf(amax, fabsf(f[j]));
        amax = group_max<16>(amax);
        const float qmax = FMT == HN_KV_FP8 ? kE4M3Max : 127.0f;
        const float s = amax > 0.0f ? amax / qmax : 1.0f;
        const int64_t tt = rt[k] + a.start;
        *reinterpret_cast<uint2*>(a.q[sel] + rb[k] * a.qs0 + tt * a.qs1 + rh[k] * a.qs2 + lane16 * 8) =
            codes8<FMT == HN_KV_FP8>(f, Quot(s));
        if (lane16 == 0) a.s[sel][rb[k] * a.ss0 + tt * a.ss1 + rh[k] * a.ss2] = s;
    }
    }
}

// KV decode of a valid prefix into bf16: y = bf16_rne(decode(q) * s).
struct KvDecArgs {
    const uint8_t* q;
    const float* s;
    uint16_t* y;
    int64_t qs0, qs1, qs2;
    int64_t ss0, ss1, ss2;
    int64_t ys0, ys1, ys2;
    int64_t L, H, rows;
};

template <int FMT>
__global__ __launch_bounds__(256) void kv_dequantize_kernel(KvDecArgs a) {
    const int64_t row = (int64_t)blockIdx.x * 16 + (threadIdx.x >> 4);
    if (row >= a.rows) return;
    const int lane16 = threadIdx.x & 15;
    const int64_t h = row % a.H;
    const int64_t t = (row / a.H) % a.L;
    const int64_t b = row / (a.H * a.L);
    const uint2 c = *reinterpret_cast<const uint2*>(a.q + b * a.qs0 + t * a.qs1 + h * a.qs2 +
                                                    lane16 * 8);
    const float s = a.s[b * a.ss0 + t * a.ss1 + h * a.ss2];
    const uint32_t cw[2] = {c.x, c.y};
    uint32_t out[4];
#pragma unroll
    for (int j = 0; j < 4; ++j) {
        const uint32_t word = cw[j >> 1];
        const uint32_t b0 = (word >> (16 * (j & 1))) & 0xffu;
        const uint32_t b1 = (word >> (16 * (j & 1) + 8)) & 0xffu;
        float v0, v1;
        if (FMT == HN_KV_FP8) {
            v0 = e4m3_decode(b0);
            v1 = e4m3_decode(b1);
        } else {
            v0 = (float)(int8_t)b0;
            v1 = (float)(int8_t)b1;
        }
        out[j] = f32_to_bf16_bits(v0 * s) | (f32_to_bf16_bits(v1 * s) << 16);
    }
    *reinterpret_cast<uint4*>(a.y + b * a.ys0 + t * a.ys1 + h * a.ys2 + lane16 * 8) =
        make_uint4(out[0], out[1], out[2], out[3]);
}

}  // namespace hn

using namespace hn;

// ---------------------------------------------------------------------------
// C ABI

extern "C" int hn_quantize_rows_fp8(const void* x, int64_t rows, int64_t cols,
                                    int64_t row_stride, int scale_mode, float amax_floor,
                                    void* q, float* scale, void* stream) {
    HN_REQUIRE(rows >= 0 && cols > 0 && cols % 8 == 0 && cols <= 16384, HN_E_ARG,
               "hn_quantize_rows_fp8: cols must be a positive multiple of 8 and <= 16384");
    HN_REQUIRE(row_stride >= cols && row_stride % 8 == 0, HN_E_ARG,
               "hn_quantize_rows_fp8: row_stride must be >= cols and a multiple of 8");
    HN_REQUIRE(scale_mode == HN_SCALE_CLAMP || scale_mode == HN_SCALE_ZERO_ONE, HN_E_ARG,
               "hn_quantize_rows_fp8: unknown scale mode");
    HN_REQUIRE(aligned(x, 16) && aligned(q, 8) && aligned(scale, 4), HN_E_ARG,
               "hn_quantize_rows_fp8: x must be 16-byte and q 8-byte aligned");
    if (rows == 0) return HN_OK;
    HN_REQUIRE(x && q && scale, HN_E_ARG, "hn_quantize_rows_fp8: null pointer");
    if (const int rc = require_gfx950("hn_quantize_rows_fp8"); rc != HN_OK) return rc;
    HN_REQUIRE(rows <= 0x7fffffffLL, HN_E_ARG, "hn_quantize_rows_fp8: too many rows");
    const int per_lane = (int)((cols / 8 + 63) / 64);  // 16-byte chunks per lane, <= 32
    const dim3 grid((unsigned)stream_grid((rows + 3) / 4, 8));
    hipStream_t st = (hipStream_t)stream;
    const uint16_t* xp = (const uint16_t*)x;
    uint8_t* qp = (uint8_t*)q;
    if (per_lane > 8) {  // > 4096 columns: one workgroup per row
        const int per_thread = (int)((cols / 8 + 255) / 256);  // <= 8
        const dim3 wgrid((unsigned)stream_grid(rows, 8));
#define HN_WIDE_CASE(N)                                                                              \
        if (per_thread <= N) {                                                                       \
            quantize_rows_wide_kernel<N><<<wgrid, 256, 0, st>>>(xp, rows, cols, row_stride, scale_mode, \
                                                                amax_floor, qp, scale);              \
            return check_launch("hn_quantize_rows_fp8");                                             \
        }
        HN_WIDE_CASE(4)
        HN_WIDE_CASE(6)
        HN_WIDE_CASE(8)
#undef HN_WIDE_CASE
    }
#define HN_ROWS_CASE(N)                                                                       \
    if (per_lane <= N) {                                                                      \
        quantize_rows_kernel<N><<<grid, 256, 0, st>>>(xp, rows, cols, row_stride, scale_mode, \
                                                      amax_floor, qp, scale);                 \
        return check_launch("hn_quantize_rows_fp8");                                          \
    }
    HN_ROWS_CASE(1)
    HN_ROWS_CASE(2)
    HN_ROWS_CASE(4)
    HN_ROWS_CASE(6)
    HN_ROWS_CASE(8)
#undef HN_ROWS_CASE
    return fail(HN_E_ARG, "hn_quantize_rows_fp8: unsupported width");
}

extern "C" int hn_ln_mod_quantize_fp8(const void* x, int64_t rows, int64_t cols, int64_t rows_per_batch,
                                      const void* shift, const void* scale_mod, int64_t mod_stride, float eps,
                                      float amax_floor, void* q, float* scale, void* stream) {
    HN_REQUIRE(rows >= 0 && cols > 0 && cols % 8 == 0 && cols <= 8192, HN_E_ARG,
               "hn_ln_mod_quantize_fp8: cols must be a positive multiple of 8 and <= 8192");
    HN_REQUIRE(rows_per_batch > 0 && mod_stride >= cols && mod_stride % 8 == 0, HN_E_ARG,
               "hn_ln_mod_quantize_fp8: invalid rows_per_batch or modulation stride");
    HN_REQUIRE(eps >= 0.0f && amax_floor >= 0.0f, HN_E_ARG, "hn_ln_mod_quantize_fp8: negative eps or floor");
    HN_REQUIRE(aligned(x, 16) && aligned(shift, 16) && aligned(scale_mod, 16) && aligned(q, 8) &&
                   aligned(scale, 4),
               HN_E_ARG, "hn_ln_mod_quantize_fp8: x, shift, scale_mod must be 16-byte and q 8-byte aligned");
    if (rows == 0) return HN_OK;
    HN_REQUIRE(x && shift && scale_mod && q && scale, HN_E_ARG, "hn_ln_mod_quantize_fp8: null pointer");
    if (const int rc = require_gfx950("hn_ln_mod_quantize_fp8"); rc != HN_OK) return rc;
    HN_REQUIRE(rows <= 0x7fffffffLL, HN_E_ARG, "hn_ln_mod_quantize_fp8: too many rows");
    const int per_lane = (int)((cols / 8 + 63) / 64);  // 16-byte chunks per lane, <= 16
    const dim3 grid((unsigned)stream_grid((rows + 3) / 4, 8));
    hipStream_t st = (hipStream_t)stream;
#define HN_LNQ_CASE(N)                                                                                  \
    if (per_lane <= N) {                                                                                \
        if (cols == N * 512)                                                                            \
            ln_mod_quantize_kernel<N, true><<<grid, 256, 0, st>>>(                                      \
                (const uint16_t*)x, rows, cols, rows_per_batch, (const uint16_t*)shift,                 \
                (const uint16_t*)scale_mod, mod_stride, eps, amax_floor, (uint8_t*)q, scale);           \
        else                                                                                            \
            ln_mod_quantize_kernel<N, false><<<grid, 256, 0, st>>>(                                     \
                (const uint16_t*)x, rows, cols, rows_per_batch, (const uint16_t*)shift,                 \
                (const uint16_t*)scale_mod, mod_stride, eps, amax_floor, (uint8_t*)q, scale);           \
        return check_launch("hn_ln_mod_quantize_fp8");                                                  \
    }
    HN_LNQ_CASE(1)
    HN_LNQ_CASE(2)
    HN_LNQ_CASE(4)
    HN_LNQ_CASE(6)
    HN_LNQ_CASE(8)
    HN_LNQ_CASE(16)
#undef HN_LNQ_CASE
    return fail(HN_E_ARG, "hn_ln_mod_quantize_fp8: unsupported width");
}

extern "C" int hn_quantize_blockwise_fp8(const void* x, int64_t rows, int64_t cols, void* q,
                                         float* scale, void* stream) {
    HN_REQUIRE(rows >= 0 && cols > 0 && cols % 128 == 0, HN_E_ARG,
               "hn_quantize_blockwise_fp8: cols must be a positive multiple of 128");
    HN_REQUIRE(aligned(x, 16) && aligned(q, 8) && aligned(scale, 4), HN_E_ARG,
               "hn_quantize_blockwise_fp8: misaligned pointer");
    if (rows == 0) return HN_OK;
    HN_REQUIRE(x && q && scale, HN_E_ARG, "hn_quantize_blockwise_fp8: null pointer");
    if (const int rc = require_gfx950("hn_quantize_blockwise_fp8"); rc != HN_OK) return rc;
    const dim3 grid((unsigned)((rows + 127) / 128), (unsigned)(cols / 128));
    quantize_blockwise_kernel<<<grid, 256, 0, (hipStream_t)stream>>>(
        (const uint16_t*)x, rows, cols, (uint8_t*)q, scale);
    return check_launch("hn_quantize_blockwise_fp8");
}

static int kv_quantize_impl(int fmt, const void* const x[2], int n, const int64_t* xs,
                            int64_t B, int64_t L, int64_t H, int64_t D, void* const q[2],
                            const int64_t* qs, float* const s[2], const int64_t* ss,
                            int64_t cap, int64_t start, int32_t* status, void* stream,
                            const char* who) {
    if (fmt != HN_KV_FP8 && fmt != HN_KV_INT8) return fail(HN_E_ARG, "unknown KV format");
    HN_REQUIRE(D == 128, HN_E_ARG, "KV quantization requires head dim 128");
    HN_REQUIRE(B >= 0 && L >= 0 && H > 0 && start >= 0, HN_E_ARG, "invalid KV shape");
    HN_REQUIRE(cap >= 0 && start <= cap && L <= cap - start, HN_E_ARG,
               "KV write past the cache capacity (start + L > cap)");
    HN_REQUIRE(xs && qs && ss, HN_E_ARG, "null stride array");
    HN_REQUIRE(xs[3] == 1 && qs[3] == 1, HN_E_ARG, "KV head dim must be contiguous");
    HN_REQUIRE(xs[0] % 8 == 0 && xs[1] % 8 == 0 && xs[2] % 8 == 0, HN_E_ARG,
               "KV value strides must be multiples of 8 elements");
    HN_REQUIRE(qs[0] % 8 == 0 && qs[1] % 8 == 0 && qs[2] % 8 == 0, HN_E_ARG,
               "KV cache strides must be multiples of 8 bytes");
    for (int i = 0; i < n; ++i)
        HN_REQUIRE(aligned(x[i], 16) && aligned(q[i], 8) && aligned(s[i], 4), HN_E_ARG,
                   "misaligned KV pointer");
    HN_REQUIRE(aligned(status, 4), HN_E_ARG, "misaligned KV status pointer");
    const int64_t rows = B * L * H;
    if (rows == 0) return HN_OK;
    for (int i = 0; i < n; ++i) HN_REQUIRE(x[i] && q[i] && s[i], HN_E_ARG, "null KV pointer");
    if (const int rc = require_gfx950(who); rc != HN_OK) return rc;
    KvArgs a;
    for (int i = 0; i < 2; ++i) {
        a.x[i] = (const uint16_t*)x[i < n ? i : 0];
        a.q[i] = (uint8_t*)q[i < n ? i : 0];
        a.s[i] = s[i < n ? i : 0];
    }
    a.xs0 = xs[0]; a.xs1 = xs[1]; a.xs2 = xs[2];
    a.qs0 = qs[0]; a.qs1 = qs[1]; a.qs2 = qs[2];
    a.ss0 = ss[0]; a.ss1 = ss[1]; a.ss2 = ss[2];
    a.L = L; a.H = H; a.rows = rows; a.start = start;
    const bool token_fast = xs[1] < xs[2];
    HN_REQUIRE(token_fast || L * H < 0x7fffffffLL, HN_E_ARG, "KV write: too many rows per batch");
    static_assert(KV_UNIT == 64, "token-fast units are 8 tokens x 8 heads");
    a.htiles = token_fast ? (H + 7) / 8 : 1;
    a.ttiles = token_fast ? (L + 7) / 8 : (L * H + KV_UNIT - 1) / KV_UNIT;
    a.units = B * a.htiles * a.ttiles;
    const dim3 grid((unsigned)stream_grid(a.units, 16 / n), (unsigned)n);
    a.status = status;
    if (status) {
        const hipStream_t st = (hipStream_t)stream;
        status_clear_kernel<<<1, 64, 0, st>>>(status);
        KvCheckArgs c;
        for (int i = 0; i < 2; ++i) c.x[i] = a.x[i];
        c.xs0 = xs[0]; c.xs1 = xs[1]; c.xs2 = xs[2];
        c.L = L; c.H = H; c.rows = rows; c.status = status;
        const dim3 cgrid((unsigned)stream_grid((rows + 15) / 16, 8 / n), (unsigned)n);
        if (token_fast) kv_check_kernel<true><<<cgrid, 256, 0, st>>>(c);
        else kv_check_kernel<false><<<cgrid, 256, 0, st>>>(c);
    }
    if (fmt == HN_KV_FP8) {
        if (token_fast) kv_quantize_kernel<HN_KV_FP8, true><<<grid, 256, 0, (hipStream_t)stream>>>(a);
        else kv_quantize_kernel<HN_KV_FP8, false><<<grid, 256, 0, (hipStream_t)stream>>>(a);
    } else {
        if (token_fast) kv_quantize_kernel<HN_KV_INT8, true><<<grid, 256, 0, (hipStream_t)stream>>>(a);
        else kv_quantize_kernel<HN_KV_INT8, false><<<grid, 256, 0, (hipStream_t)stream>>>(a);
    }
    return check_launch(who);
}

extern "C" int hn_kv_quantize(int fmt, const void* x, const int64_t* xs, int64_t B, int64_t L,
                              int64_t H, int64_t D, void* q, const int64_t* qs, float* scale,
                              const int64_t* ss, int64_t cap, int64_t start, int32_t* status,
                              void* stream) {
    const void* xx[2] = {x, x};
    void* qq[2] = {q, q};
    float* sss[2] = {scale, scale};
    return kv_quantize_impl(fmt, xx, 1, xs, B, L, H, D, qq, qs, sss, ss, cap, start, status, stream,
                            "hn_kv_quantize");
}

extern "C" int hn_kv_quantize_pair(int fmt, const void* k, const void* v, const int64_t* xs,
                                   int64_t B, int64_t L, int64_t H, int64_t D, void* qk,
                                   void* qv, const int64_t* qs, float* sk, float* sv,
                                   const int64_t* ss, int64_t cap, int64_t start, int32_t* status,
                                   void* stream) {
    const void* xx[2] = {k, v};
    void* qq[2] = {qk, qv};
    float* sss[2] = {sk, sv};
    return kv_quantize_impl(fmt, xx, 2, xs, B, L, H, D, qq, qs, sss, ss, cap, start, status, stream,
                            "hn_kv_quantize_pair");
}

extern "C" int hn_kv_dequantize(int fmt, const void* q, const int64_t* qs, const float* scale,
                                const int64_t* ss, int64_t B, int64_t valid_len, int64_t H,
                                int64_t D, void* y, const int64_t* ys, void* stream) {
    if (fmt != HN_KV_FP8 && fmt != HN_KV_INT8) return fail(HN_E_ARG, "unknown KV format");
    HN_REQUIRE(D == 128, HN_E_ARG, "KV decode requires head dim 128");
    HN_REQUIRE(B >= 0 && valid_len >= 0 && H > 0, HN_E_ARG, "invalid KV decode shape");
    HN_REQUIRE(qs && ss && ys, HN_E_ARG, "null stride array");
    HN_REQUIRE(qs[3] == 1 && ys[3] == 1, HN_E_ARG, "KV head dim must be contiguous");
    HN_REQUIRE(qs[0] % 8 == 0 && qs[1] % 8 == 0 && qs[2] % 8 == 0 && ys[0] % 8 == 0 &&
                   ys[1] % 8 == 0 && ys[2] % 8 == 0,
               HN_E_ARG, "KV decode strides must be multiples of 8");
    HN_REQUIRE(aligned(q, 8) && aligned(y, 16) && aligned(scale, 4), HN_E_ARG,
               "misaligned KV decode pointer");
    const int64_t rows = B * valid_len * H;
    if (rows == 0) return HN_OK;
    HN_REQUIRE(q && scale && y, HN_E_ARG, "null KV decode pointer");
    if (const int rc = require_gfx950("hn_kv_dequantize"); rc != HN_OK) return rc;
    KvDecArgs a;
    a.q = (const uint8_t*)q; a.s = scale; a.y = (uint16_t*)y;
    a.qs0 = qs[0]; a.qs1 = qs[1]; a.qs2 = qs[2];
    a.ss0 = ss[0]; a.ss1 = ss[1]; a.ss2 = ss[2];
    a.ys0 = ys[0]; a.ys1 = ys[1]; a.ys2 = ys[2];
    a.L = valid_len; a.H = H; a.rows = rows;
    const int64_t blocks = (rows + 15) / 16;
    if (fmt == HN_KV_FP8)
        kv_dequantize_kernel<HN_KV_FP8><<<(unsigned)blocks, 256, 0, (hipStream_t)stream>>>(a);
    else
        kv_dequantize_kernel<HN_KV_INT8><<<(unsigned)blocks, 256, 0, (hipStream_t)stream>>>(a);
    return check_launch("hn_kv_dequantize");
}

// Encodes the fp32 values with bit patterns first, first + 1, ... with the
// quantizers' own conversion (e4m3_encode4), four per thread in one word.
__global__ __launch_bounds__(256) void e4m3_encode_range_kernel(uint32_t first, int64_t words,
                                                                uint32_t* out) {
    const int64_t stride = (int64_t)gridDim.x * blockDim.x;
    for (int64_t w = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; w < words; w += stride) {
        const uint32_t b = first + (uint32_t)(w * 4);
        out[w] = e4m3_encode4(__uint_as_float(b), __uint_as_float(b + 1u), __uint_as_float(b + 2u),
                              __uint_as_float(b + 3u));
    }
}

extern "C" int hn_e4m3_encode_range(uint32_t first, int64_t n, void* out, void* stream) {
    HN_REQUIRE(n >= 0 && n % 4 == 0, HN_E_ARG, "hn_e4m3_encode_range: n must be a multiple of 4");
    HN_REQUIRE((uint64_t)first + (uint64_t)n <= (1ull << 32), HN_E_ARG,
               "hn_e4m3_encode_range: the range passes the last fp32 bit pattern");
    HN_REQUIRE(aligned(out, 4), HN_E_ARG, "hn_e4m3_encode_range: out must be 4-byte aligned");
    if (n == 0) return HN_OK;
    HN_REQUIRE(out, HN_E_ARG, "hn_e4m3_encode_range: null output");
    if (const int rc = require_gfx950("hn_e4m3_encode_range"); rc != HN_OK) return rc;
    const int64_t words = n / 4;
    const int64_t grid = stream_grid((words + 255) / 256, 8);
    e4m3_encode_range_kernel<<<(unsigned)grid, 256, 0, (hipStream_t)stream>>>(first, words,
                                                                              (uint32_t*)out);
    return check_launch("hn_e4m3_encode_range");
}
