// Block-causal chunk attention over an FP8 (or INT8-compat) KV cache, gfx950.
//
//   O = softmax(Q K^T * scale) V,   K, V = code * per-(token, head) scale
//
// Work decomposition: one workgroup = 4 waves = 128 queries of one (batch,
// head); each wave owns 32 queries (one 32-column MFMA block), and two
// workgroups share a CU (2 waves per SIMD), so one wave's softmax VALU work
// overlaps the other's MFMAs. Keys stream
// through LDS in tiles of 64. K codes are widened to bf16 once per workgroup
// as they are written to LDS (exact: every e4m3 and int8 code is a bf16
// value) and the per-token K scale (times softmax_scale * log2 e) multiplies
// the fp32 logits, so K enters as code * scale in fp32. V codes are widened to
// fp16 (also exact) and the per-token V scale multiplies the fp32 probability
// before it is packed to fp16 for the PV MFMA: P' = fp16(p * s_v), so the PV
// product carries fp16's 2^-11 relative rounding instead of bf16's 2^-8. The
// optional unquantized tail (the current chunk's bf16 K/V) is copied into the
// same LDS formats with unit scales, so one compute path serves both segments.
//
// Per tile the wave computes S^T = K Q^T with v_mfma_f32_32x32x16_bf16: the
// MFMA output puts one query per lane column, so the online-softmax max/sum
// are lane-local plus one exchange with lane ^ 32. P^T is packed to fp16 in
// registers and reused as the B operand of O^T += V^T P^T on
// v_mfma_f32_32x32x16_f16. V is stored in LDS in its natural [key][dim] order
// and the V^T operand is fetched with gfx950's transposing LDS read
// (ds_read_b64_tr_b16), in the key order of the S^T registers. Two LDS
// stages: the next tile's global loads are in flight in registers while the
// MFMAs consume the current one.
//
// Mask: key position p is visible to query position r iff p / chunk <= r / chunk
// (chunk <= 0: all visible). Tiles wholly beyond the last query's chunk are
// never visited; tiles wholly visible to every query of the workgroup skip
// the per-element test.
#include "hn_capi_internal.h"
#include "hn_common.h"

namespace hn {
namespace attn {

constexpr int D = 128;
constexpr int BKV = 64;            // keys per tile
constexpr int NW = 4;              // waves per workgroup
constexpr int NT = 64 * NW;
constexpr int QW = 32;             // queries per wave
constexpr int BQ = QW * NW;        // queries per workgroup
constexpr int KROW = D * 2 + 16;   // K tile row: 128 bf16 + 16 B pad (bank spread)
// V tile: [key][dim] fp16 rows of 256 B, padded to 320 B (80 dwords: row k
// starts 16 banks after row k - 1); 16-byte chunk c of key row k is stored at
// position vchunk(k, c) (see below).
constexpr int VROW = D * 2 + 64;
constexpr int K_BYTES = BKV * KROW;
constexpr int V_BYTES = BKV * VROW;
constexpr int S_BYTES = 2 * BKV * 4;  // per-key K and V scales (fp32)
constexpr int STAGE = K_BYTES + V_BYTES + S_BYTES;

struct Params {
    const uint16_t* q;
    const uint8_t* kc;
    const uint8_t* vc;
    const float* ks;
    const float* vs;
    const uint16_t* kcur;
    const uint16_t* vcur;
    uint16_t* out;
    int64_t qs0, qs1, qs2;
    int64_t cs0, cs1, cs2;
    int64_t ss0, ss1, ss2;
    int64_t us0, us1, us2;
    int64_t os0, os1, os2;
    int64_t Lq, H, kv_len, cur_len, q_pos0, chunk;
    float scale_log2;  // softmax_scale * log2(e)
    int fmt;
    int q_tiles;       // ceil(Lq / BQ)
    int splits;        // key-range splits per (batch, head, query tile)
    int work;          // B * H * q_tiles * splits
    int per_xcd;       // ceil(work / 8)
    float* ws_o;       // splits > 1: unnormalized O, [split][B][H][Lq][D] fp32
    float* ws_ml;      // splits > 1: running max and sum, [split][B][H][Lq][2]
};

typedef _Float16 f16x2 __attribute__((ext_vector_type(2)));
typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));
typedef float f32x2 __attribute__((ext_vector_type(2)));

// Position of the 16-byte chunk c (8 dims) of key row k in the V tile: the two
// low bits of c are XORed with bits 2-3 of k. With the 16-bank row shift this
// makes both access patterns conflict-free over the 64 LDS banks: the row
// writes (16 lanes = keys 16 i .. 16 i + 15 at one chunk index: bank groups
// 16 (k % 4) + 4 ((c % 4) ^ (k / 4 % 4)) all differ) and the transposing reads
// (keys 4 i .. 4 i + 3 x chunks 4 b .. 4 b + 3). Chunk groups 4 b .. 4 b + 3
// stay in place, so a dim block is a constant offset.
HN_DEVICE int vchunk(int k, int c) { return (c & ~3) | ((c & 3) ^ ((k >> 2) & 3)); }

typedef _Float16 f16x4 __attribute__((ext_vector_type(4)));
typedef short i16x4 __attribute__((ext_vector_type(4)));

// V^T fragment of the PV MFMA for dim block db and 16-key slice `slice`:
// lane l needs dim 32 db + l % 32 and keys 16 slice + 4 (l / 32) + {0..3} and
// + 8 + {0..3} (the order of the P^T registers, see compute loop). The
// transposing read gives lane i of each 16-lane group element i % 4 of the
// 8-byte rows addressed by lanes i / 4 + 4 e, e = 0..3; so lane j of group g
// addresses key (base + j / 4) at dims 32 db + 16 (g % 2) + 4 (j % 4), and
// every lane receives four consecutive keys of its own dim.
HN_DEVICE f16x8 read_vt(const uint8_t* vl, int db, int slice, int lane) {
    const int g = lane >> 4, j = lane & 15;
    const int c = 4 * db + 2 * (g & 1) + ((j & 3) >> 1);
    const int byte = 8 * (j & 1);
    f16x4 r[2];
#pragma unroll
    for (int h2 = 0; h2 < 2; ++h2) {
        const int k = 16 * slice + 8 * h2 + 4 * (g >> 1) + (j >> 2);
        const uint8_t* a = vl + k * VROW + vchunk(k, c) * 16 + byte;
        r[h2] = __builtin_bit_cast(f16x4, __builtin_amdgcn_ds_read_tr16_b64_v4i16(
            (__attribute__((address_space(3))) i16x4*)(__attribute__((address_space(3))) void*)a));
    }
    f16x8 v;
    v[0] = r[0][0]; v[1] = r[0][1]; v[2] = r[0][2]; v[3] = r[0][3];
    v[4] = r[1][0]; v[5] = r[1][1]; v[6] = r[1][2]; v[7] = r[1][3];
    return v;
}

// Two codes (bytes 2 hi, 2 hi + 1 of w) -> their two exact bf16 values. The
// gfx950 conversion is used with a unit scale only: its scale operand applies
// just the exponent of the fp32 value, so per-token scales are applied in fp32
// by the caller instead.
template <int FMT>
HN_DEVICE uint32_t cvt2(uint32_t w, bool hi) {
    if (FMT == HN_KV_FP8) {
        bf16x2 r = hi ? __builtin_amdgcn_cvt_scalef32_pk_bf16_fp8(w, 1.0f, true)
                      : __builtin_amdgcn_cvt_scalef32_pk_bf16_fp8(w, 1.0f, false);
        return __builtin_bit_cast(uint32_t, r);
    }
    const uint32_t sh = hi ? 16 : 0;
    const float a = (float)(int8_t)((w >> sh) & 0xffu);
    const float b = (float)(int8_t)((w >> (sh + 8)) & 0xffu);
    return f32_to_bf16_bits(a) | (f32_to_bf16_bits(b) << 16);
}

// 16 codes (one uint4) -> 16 bf16 as 8 dwords.
template <int FMT>
HN_DEVICE void cvt16(const uint4& c, uint32_t (&o)[8]) {
    const uint32_t w[4] = {c.x, c.y, c.z, c.w};
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        o[2 * i] = cvt2<FMT>(w[i], false);
        o[2 * i + 1] = cvt2<FMT>(w[i], true);
    }
}


HN_DEVICE uint32_t pack_f16(float a, float b) {
    const f32x2 f = {a, b};
    return __builtin_bit_cast(uint32_t, __builtin_convertvector(f, f16x2));
}

// 16 codes (one uint4) -> their 16 exact fp16 values, as 8 dwords.
template <int FMT>
HN_DEVICE void codes16_f16(const uint4& c, uint32_t (&o)[8]) {
    const uint32_t w[4] = {c.x, c.y, c.z, c.w};
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        if (FMT == HN_KV_FP8) {
            o[2 * i] = __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_scalef32_pk_f16_fp8(w[i], 1.0f, false));
            o[2 * i + 1] = __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_scalef32_pk_f16_fp8(w[i], 1.0f, true));
        } else {
            o[2 * i] = pack_f16((float)(int8_t)(w[i] & 0xffu), (float)(int8_t)((w[i] >> 8) & 0xffu));
            o[2 * i + 1] = pack_f16((float)(int8_t)((w[i] >> 16) & 0xffu), (float)(int8_t)(w[i] >> 24));
        }
    }
}

// Two bf16 (one dword) -> two fp16.
HN_DEVICE uint32_t bf16x2_to_f16x2(uint32_t w) {
    return pack_f16(bf16_bits_to_f32(w & 0xffffu), bf16_bits_to_f32(w >> 16));
}

// Registers holding one cache tile between its global load and its LDS
// write (the load is issued before the tile in LDS is consumed).
// K: thread t owns units u = t + 256 i (i < 2): key u / 8, 16 dims at 16 (u % 8).
// V: lane l of wave w owns key l, dims 32 w .. 32 w + 31.
struct CacheRegs {
    uint4 k[2];
    uint4 v[2];
    float sk[2], sv;
};

HN_DEVICE void load_cache_tile(const Params& p, CacheRegs& r, int64_t b, int64_t h,
                               int64_t first, int64_t count) {
    const int t = threadIdx.x;
#pragma unroll
    for (int i = 0; i < 2; ++i) {
        const int u = t + NT * i;
        int64_t j = u >> 3;
        j = j < count ? j : count - 1;  // clamp inside the segment; masked later
        const int64_t tok = first + j;
        r.k[i] = *reinterpret_cast<const uint4*>(p.kc + b * p.cs0 + tok * p.cs1 + h * p.cs2 + (u & 7) * 16);
        r.sk[i] = p.ks[b * p.ss0 + tok * p.ss1 + h * p.ss2];
    }
    int64_t j = t & 63;
    j = j < count ? j : count - 1;
    const int64_t tok = first + j;
    const uint8_t* src = p.vc + b * p.cs0 + tok * p.cs1 + h * p.cs2 + (t >> 6) * 32;
    r.v[0] = *reinterpret_cast<const uint4*>(src);
    r.v[1] = *reinterpret_cast<const uint4*>(src + 16);
    r.sv = p.vs[b * p.ss0 + tok * p.ss1 + h * p.ss2];
}

// V row write: key t % 64, chunks 4 (t / 64) .. +3 (32 dims), from 16 dwords of fp16 pairs.
HN_DEVICE void store_v_row(uint8_t* vl, const uint32_t (&cv)[16]) {
    const int t = threadIdx.x;
    const int k = t & 63, c0 = 4 * (t >> 6);
#pragma unroll
    for (int c = 0; c < 4; ++c)
        *reinterpret_cast<uint4*>(vl + k * VROW + vchunk(k, c0 + c) * 16) =
            make_uint4(cv[4 * c], cv[4 * c + 1], cv[4 * c + 2], cv[4 * c + 3]);
}

// Per-key scales in LDS: [0, 64) K scale * softmax_scale * log2 e, [64, 128) V scale.
HN_DEVICE float* stage_scales(uint8_t* st) { return reinterpret_cast<float*>(st + K_BYTES + V_BYTES); }

template <int FMT>
HN_DEVICE void store_cache_tile(const Params& p, const CacheRegs& r, uint8_t* st) {
    const int t = threadIdx.x;
    float* sc = stage_scales(st);
#pragma unroll
    for (int i = 0; i < 2; ++i) {
        const int u = t + NT * i;
        uint32_t o[8];
        cvt16<FMT>(r.k[i], o);
        uint4* dst = reinterpret_cast<uint4*>(st + (u >> 3) * KROW + (u & 7) * 32);
        dst[0] = make_uint4(o[0], o[1], o[2], o[3]);
        dst[1] = make_uint4(o[4], o[5], o[6], o[7]);
        if ((u & 7) == 0) sc[u >> 3] = r.sk[i] * p.scale_log2;
    }
    uint32_t cv[16];
    codes16_f16<FMT>(r.v[0], *reinterpret_cast<uint32_t(*)[8]>(&cv[0]));
    codes16_f16<FMT>(r.v[1], *reinterpret_cast<uint32_t(*)[8]>(&cv[8]));
    store_v_row(st + K_BYTES, cv);
    if (t < BKV) sc[BKV + t] = r.sv;  // wave 0: lane t holds key t
}

// Unquantized tail tile (bf16 K/V of the current chunk): load and write to LDS
// in one go (not prefetched: it is at most one chunk of the keys).
HN_DEVICE void copy_tail_tile(const Params& p, int64_t b, int64_t h, int64_t first,
                              int64_t count, uint8_t* st) {
    const int t = threadIdx.x;
#pragma unroll
    for (int i = 0; i < 2; ++i) {
        const int u = t + NT * i;
        int64_t j = u >> 3;
        j = j < count ? j : count - 1;
        const uint16_t* src = p.kcur + b * p.us0 + (first + j) * p.us1 + h * p.us2 + (u & 7) * 16;
        const uint4 lo = *reinterpret_cast<const uint4*>(src);
        const uint4 hi = *reinterpret_cast<const uint4*>(src + 8);
        uint4* dst = reinterpret_cast<uint4*>(st + (u >> 3) * KROW + (u & 7) * 32);
        dst[0] = lo;
        dst[1] = hi;
    }
    {
        int64_t j = t & 63;
        j = j < count ? j : count - 1;
        const uint16_t* src = p.vcur + b * p.us0 + (first + j) * p.us1 + h * p.us2 + (t >> 6) * 32;
        uint32_t cv[16];
#pragma unroll
        for (int c = 0; c < 4; ++c) {
            const uint4 w = *reinterpret_cast<const uint4*>(src + 8 * c);
            cv[4 * c] = bf16x2_to_f16x2(w.x);
            cv[4 * c + 1] = bf16x2_to_f16x2(w.y);
            cv[4 * c + 2] = bf16x2_to_f16x2(w.z);
            cv[4 * c + 3] = bf16x2_to_f16x2(w.w);
        }
        store_v_row(st + K_BYTES, cv);
    }
    float* sc = stage_scales(st);
    if (t < BKV) sc[t] = p.scale_log2;
    else if (t < 2 * BKV) sc[t] = 1.0f;
}

HN_DEVICE f32x16 mfma_bf16(const bf16x8& a, const bf16x8& b, const f32x16& c) {
    return __builtin_amdgcn_mfma_f32_32x32x16_bf16(a, b, c, 0, 0, 0);
}

HN_DEVICE bf16x8 ld_bf16x8(const uint8_t* p) {
    return __builtin_bit_cast(bf16x8, *reinterpret_cast<const uint4*>(p));
}

template <int FMT>
__global__ __launch_bounds__(NT, 2) void attn_fp8kv_kernel(Params p) {
    __shared__ __attribute__((aligned(16))) uint8_t smem[2 * STAGE];

    // XCD-aware work order: workgroup ids are dealt round-robin to the 8 XCDs,
    // so id % 8 picks a contiguous range of work items -- the query tiles of
    // the same few heads share that XCD's L2 while they stream its K/V.
    const int id = blockIdx.x;
    const int w = (id & 7) * p.per_xcd + (id >> 3);
    if (w >= p.work) return;
    const int split = w % p.splits;
    const int wq = w / p.splits;
    const int qt = wq % p.q_tiles;
    const int64_t h = (wq / p.q_tiles) % p.H;
    const int64_t b = wq / (p.q_tiles * (int)p.H);

    const int lane = threadIdx.x & 63;
    const int wave = threadIdx.x >> 6;
    const int col = lane & 31, half = lane >> 5;
    const int64_t row = (int64_t)qt * BQ + wave * QW + col;  // this lane's query row
    const bool qvalid = row < p.Lq;
    const int64_t qrow = qvalid ? row : p.Lq - 1;
    const int64_t qpos = p.q_pos0 + qrow;

    // Q^T fragments (B operand): query column `col`, dims 16 s + 8 half .. +8
    // for K slice s (the K fragments use the same dim mapping).
    bf16x8 qf[8];
    {
        const uint16_t* src = p.q + b * p.qs0 + qrow * p.qs1 + h * p.qs2 + half * 8;
#pragma unroll
        for (int sl = 0; sl < 8; ++sl)
            qf[sl] = __builtin_bit_cast(bf16x8, *reinterpret_cast<const uint4*>(src + 16 * sl));
    }

    // Visible key range for this workgroup (positions): up to the end of the
    // last query's chunk.
    const int64_t wg_first_q = (int64_t)qt * BQ;
    int64_t wg_last_q = wg_first_q + BQ - 1;
    wg_last_q = wg_last_q < p.Lq - 1 ? wg_last_q : p.Lq - 1;
    const int64_t r_first = p.q_pos0 + wg_first_q, r_last = p.q_pos0 + wg_last_q;
    int64_t pos_end = p.kv_len + p.cur_len;
    if (p.chunk > 0) {
        const int64_t lim = (r_last / p.chunk + 1) * p.chunk;
        pos_end = pos_end < lim ? pos_end : lim;
    }
    const int64_t cache_end = p.kv_len < pos_end ? p.kv_len : pos_end;
    const int64_t tail_end = pos_end - p.kv_len;  // tail keys visited (may be <= 0)
    const int n_cache = (int)((cache_end + BKV - 1) / BKV);
    const int n_tail = tail_end > 0 ? (int)((tail_end + BKV - 1) / BKV) : 0;
    const int n_all = n_cache + n_tail;
    // This split's share of the tile list [t_begin, t_end).
    const int t_begin = (int)((int64_t)n_all * split / p.splits);
    const int t_end = (int)((int64_t)n_all * (split + 1) / p.splits);
    // Visibility limits (exclusive key positions): this lane's query, and the
    // workgroup's first query (every key below it is visible to all lanes).
    const int64_t no_limit = p.kv_len + p.cur_len;
    const int64_t key_limit = p.chunk > 0 ? (qpos / p.chunk + 1) * p.chunk : no_limit;
    const int64_t wg_key_limit = p.chunk > 0 ? (r_first / p.chunk + 1) * p.chunk : no_limit;

    f32x16 o[4];  // O^T: [dim block], column = this lane's query
#pragma unroll
    for (int i = 0; i < 4; ++i)
#pragma unroll
        for (int v = 0; v < 16; ++v) o[i][v] = 0.0f;
    float mrow = -INFINITY;
    float lsum = 0.0f;

    CacheRegs regs;
    auto tile_geom = [&](int t, bool& cache_seg, int64_t& first, int64_t& count, int64_t& pos0) {
        if (t < n_cache) {
            cache_seg = true;
            first = (int64_t)t * BKV;
            count = cache_end - first;
            pos0 = first;
        } else {
            cache_seg = false;
            first = (int64_t)(t - n_cache) * BKV;
            count = tail_end - first;
            pos0 = p.kv_len + first;
        }
        count = count < BKV ? count : BKV;
    };

    if (t_end > t_begin) {
        bool cs;
        int64_t first, count, pos0;
        tile_geom(t_begin, cs, first, count, pos0);
        if (cs) {
            load_cache_tile(p, regs, b, h, first, count);
            store_cache_tile<FMT>(p, regs, smem);
        } else {
            copy_tail_tile(p, b, h, first, count, smem);
        }
    }
    __syncthreads();

    for (int t = t_begin; t < t_end; ++t) {
        const uint8_t* st = smem + ((t - t_begin) & 1) * STAGE;
        bool cs;
        int64_t first, count, pos0;
        tile_geom(t, cs, first, count, pos0);
        bool ncs = false;
        int64_t nf = 0, nc = 0, np = 0;
        if (t + 1 < t_end) {
            tile_geom(t + 1, ncs, nf, nc, np);
            if (ncs) load_cache_tile(p, regs, b, h, nf, nc);
        }

        // ---- S^T = K Q^T: two 32-key blocks x this wave's 32 queries
        f32x16 sacc[2];
#pragma unroll
        for (int kb = 0; kb < 2; ++kb)
#pragma unroll
            for (int v = 0; v < 16; ++v) sacc[kb][v] = 0.0f;
#pragma unroll
        for (int sl = 0; sl < 8; ++sl)
#pragma unroll
            for (int kb = 0; kb < 2; ++kb) {
                const bf16x8 kf = ld_bf16x8(st + (kb * 32 + col) * KROW + (16 * sl + 8 * half) * 2);
                sacc[kb] = mfma_bf16(kf, qf[sl], sacc[kb]);
            }

        // ---- mask: keys past the segment end, and the chunk-causal rule.
        // Positions increase with the key index, so the keys this lane's query
        // sees in the tile are exactly j < lim (lane-local, 32-bit compare).
        // Register v of block kb holds key 32 kb + 8 (v/4) + 4 half + v%4.
        const bool full = count == BKV && pos0 + BKV <= wg_key_limit;
        if (!full) {
            int64_t lim64 = key_limit - pos0;
            lim64 = lim64 < count ? lim64 : count;
            const int lim = lim64 < 0 ? 0 : (int)lim64;
#pragma unroll
            for (int kb = 0; kb < 2; ++kb)
#pragma unroll
                for (int v = 0; v < 16; ++v) {
                    const int j = kb * 32 + 8 * (v >> 2) + 4 * half + (v & 3);
                    if (j >= lim) sacc[kb][v] = -INFINITY;
                }
        }

        // ---- logits in log2 units: t = s * (k_scale * softmax_scale * log2 e).
        // Register v of block kb holds key 32 kb + 8 (v/4) + 4 half + v%4, so
        // each group of 4 registers takes 4 consecutive scales (one 16-byte read).
        const float* sc = reinterpret_cast<const float*>(st + K_BYTES + V_BYTES);
#pragma unroll
        for (int kb = 0; kb < 2; ++kb)
#pragma unroll
            for (int g4 = 0; g4 < 4; ++g4) {
                const float4 ks4 = *reinterpret_cast<const float4*>(sc + kb * 32 + 8 * g4 + 4 * half);
                sacc[kb][4 * g4 + 0] *= ks4.x;
                sacc[kb][4 * g4 + 1] *= ks4.y;
                sacc[kb][4 * g4 + 2] *= ks4.z;
                sacc[kb][4 * g4 + 3] *= ks4.w;
            }

        // ---- online softmax for this lane's query (keys split over lane ^ 32)
        float mx = -INFINITY;
#pragma unroll
        for (int kb = 0; kb < 2; ++kb)
#pragma unroll
            for (int v = 0; v < 16; ++v) mx = fmaxf(mx, sacc[kb][v]);
        mx = fmaxf(mx, __shfl_xor(mx, 32, 64));
        const float mnew = fmaxf(mrow, mx);
        const float muse = mnew == -INFINITY ? 0.0f : mnew;
        const float alpha = __builtin_amdgcn_exp2f(mrow - muse);
        mrow = mnew;
        float rs = 0.0f;
        f16x8 pf[2][2];  // [kb][t]: P^T registers 8t .. 8t+7 of block kb, times the V scale
#pragma unroll
        for (int kb = 0; kb < 2; ++kb)
#pragma unroll
            for (int tt = 0; tt < 2; ++tt) {
                // registers 8t .. 8t+3 hold keys 32 kb + 16 t + 4 half + 0..3,
                // registers 8t+4 .. 8t+7 keys 32 kb + 16 t + 8 + 4 half + 0..3
                const float4 va = *reinterpret_cast<const float4*>(sc + BKV + kb * 32 + 16 * tt + 4 * half);
                const float4 vb = *reinterpret_cast<const float4*>(sc + BKV + kb * 32 + 16 * tt + 8 + 4 * half);
                const float vsc[8] = {va.x, va.y, va.z, va.w, vb.x, vb.y, vb.z, vb.w};
                float pv[8];
#pragma unroll
                for (int e2 = 0; e2 < 8; ++e2) {
                    pv[e2] = __builtin_amdgcn_exp2f(sacc[kb][8 * tt + e2] - muse);
                    rs += pv[e2];
                }
                f16x8 x;
#pragma unroll
                for (int e2 = 0; e2 < 8; ++e2) x[e2] = (_Float16)(pv[e2] * vsc[e2]);
                pf[kb][tt] = x;
            }
        rs += __shfl_xor(rs, 32, 64);
        lsum = lsum * alpha + rs;
        // Rescale O only when some lane's running max moved (wave-uniform test).
        if (__any(alpha != 1.0f)) {
#pragma unroll
            for (int db = 0; db < 4; ++db)
#pragma unroll
                for (int v = 0; v < 16; ++v) o[db][v] *= alpha;
        }

        // ---- O^T += V^T P^T over the four 16-key slices of the tile
        const uint8_t* vl = st + K_BYTES;
#pragma unroll
        for (int kb = 0; kb < 2; ++kb)
#pragma unroll
            for (int tt = 0; tt < 2; ++tt) {
                const int slice = kb * 2 + tt;
#pragma unroll
                for (int db = 0; db < 4; ++db) {
                    const f16x8 vf = read_vt(vl, db, slice, lane);
                    o[db] = __builtin_amdgcn_mfma_f32_32x32x16_f16(vf, pf[kb][tt], o[db], 0, 0, 0);
                }
            }

        if (t + 1 < t_end) {
            uint8_t* nst = smem + ((t + 1 - t_begin) & 1) * STAGE;
            if (ncs) store_cache_tile<FMT>(p, regs, nst);
            else copy_tail_tile(p, b, h, nf, nc, nst);
        }
        __syncthreads();
    }

    // ---- epilogue: O = O^T / l; the lane holds dims 32 db + 8 (v/4) + 4 half + v%4
    if (p.splits > 1) {
        // Unnormalized partial result of this key range, merged by attn_combine_kernel.
        if (qvalid) {
            const int64_t qi = ((((int64_t)split * (p.work / p.splits / p.q_tiles / p.H)) + b) * p.H + h) * p.Lq + row;
            float* dst = p.ws_o + qi * D;
#pragma unroll
            for (int db = 0; db < 4; ++db)
#pragma unroll
                for (int vq = 0; vq < 4; ++vq) {
                    const int d = db * 32 + vq * 8 + half * 4;
                    *reinterpret_cast<float4*>(dst + d) =
                        make_float4(o[db][vq * 4], o[db][vq * 4 + 1], o[db][vq * 4 + 2], o[db][vq * 4 + 3]);
                }
            if (half == 0) *reinterpret_cast<float2*>(p.ws_ml + qi * 2) = make_float2(mrow, lsum);
        }
        return;
    }
    if (qvalid) {
        const float inv = lsum > 0.0f ? 1.0f / lsum : 0.0f;
        uint16_t* dst = p.out + b * p.os0 + row * p.os1 + h * p.os2;
#pragma unroll
        for (int db = 0; db < 4; ++db)
#pragma unroll
            for (int vq = 0; vq < 4; ++vq) {
                const int d = db * 32 + vq * 8 + half * 4;
                const uint32_t w0 = f32_to_bf16_bits(o[db][vq * 4] * inv) |
                                    (f32_to_bf16_bits(o[db][vq * 4 + 1] * inv) << 16);
                const uint32_t w1 = f32_to_bf16_bits(o[db][vq * 4 + 2] * inv) |
                                    (f32_to_bf16_bits(o[db][vq * 4 + 3] * inv) << 16);
                *reinterpret_cast<uint2*>(dst + d) = make_uint2(w0, w1);
            }
    }
}

// Merge of the per-split partial results: with M = max_s m_s,
// O = sum_s 2^(m_s - M) O_s / sum_s 2^(m_s - M) l_s (0 when no key was visible).
// One 128-thread block per (batch, head, query); thread d owns one dimension.
__global__ __launch_bounds__(128) void attn_combine_kernel(const float* __restrict__ ws_o,
                                                           const float* __restrict__ ws_ml,
                                                           int splits, int64_t rows_per_split,
                                                           int64_t Lq, int64_t H, uint16_t* out,
                                                           int64_t os0, int64_t os1, int64_t os2) {
    const int64_t r = blockIdx.x;  // (b * H + h) * Lq + q
    const int d = threadIdx.x;
    float M = -INFINITY;
    for (int sp = 0; sp < splits; ++sp) M = fmaxf(M, ws_ml[(sp * rows_per_split + r) * 2]);
    const float Muse = M == -INFINITY ? 0.0f : M;
    float num = 0.0f, den = 0.0f;
    for (int sp = 0; sp < splits; ++sp) {
        const int64_t idx = sp * rows_per_split + r;
        const float wgt = __builtin_amdgcn_exp2f(ws_ml[idx * 2] - Muse);
        den = fmaf(wgt, ws_ml[idx * 2 + 1], den);
        num = fmaf(wgt, ws_o[idx * D + d], num);
    }
    const int64_t q = r % Lq, h = (r / Lq) % H, b = r / (Lq * H);
    out[b * os0 + q * os1 + h * os2 + d] = (uint16_t)f32_to_bf16_bits(den > 0.0f ? num / den : 0.0f);
}

}  // namespace attn
}  // namespace hn

using namespace hn;

// Split selection: a launch wants at least two workgroups per CU (two fit per
// CU by LDS and registers). When (batch x heads x query tiles) falls short, the
// key range of each query tile is split so that the grid fills the device
// (the decode-style case: a few hundred queries over a long cache); each split
// keeps at least 16 key tiles.
static int attn_splits(int64_t B, int64_t Lq, int64_t H, int64_t kv_len, int64_t cur_len) {
    int dev = 0, cus = 256;
    if (hipGetDevice(&dev) == hipSuccess) {
        int v = 0;
        if (hipDeviceGetAttribute(&v, hipDeviceAttributeMultiprocessorCount, dev) == hipSuccess && v > 0) cus = v;
    }
    const int64_t work = B * H * ((Lq + attn::BQ - 1) / attn::BQ);
    const int64_t target = 2LL * cus;
    if (work <= 0 || work >= target) return 1;
    const int64_t tiles = (kv_len + cur_len + attn::BKV - 1) / attn::BKV;
    // Round down: the kernel holds two workgroups per CU, so work * sp <= target
    // keeps the whole launch in one round (one more workgroup would need a second).
    int64_t sp = target / work;
    const int64_t cap = tiles / 16;
    if (sp > cap) sp = cap;
    return sp > 1 ? (int)sp : 1;
}

extern "C" int64_t hn_attn_fp8kv_workspace_size(int64_t B, int64_t Lq, int64_t H, int64_t D,
                                                int64_t kv_len, int64_t cur_len) {
    if (B <= 0 || Lq <= 0 || H <= 0 || D != attn::D || kv_len < 0 || cur_len < 0) return 0;
    const int sp = attn_splits(B, Lq, H, kv_len, cur_len);
    if (sp <= 1) return 0;
    return (int64_t)sp * B * H * Lq * (D + 2) * (int64_t)sizeof(float);
}

extern "C" int hn_attn_fp8kv(int fmt, const void* q, const int64_t* qs, int64_t B, int64_t Lq,
                             int64_t H, int64_t D, const void* kc, const void* vc,
                             const int64_t* cs, const float* ks, const float* vs,
                             const int64_t* ss, int64_t kv_len, const void* kcur,
                             const void* vcur, const int64_t* curs, int64_t cur_len,
                             int64_t q_pos0, int64_t chunk_len, float softmax_scale, void* out,
                             const int64_t* os, void* workspace, int64_t workspace_bytes,
                             void* stream) {
    HN_REQUIRE(fmt == HN_KV_FP8 || fmt == HN_KV_INT8, HN_E_ARG, "hn_attn_fp8kv: unknown KV format");
    HN_REQUIRE(D == attn::D, HN_E_ARG, "hn_attn_fp8kv: head dim must be 128");
    HN_REQUIRE(B >= 0 && Lq >= 0 && H > 0 && kv_len >= 0 && cur_len >= 0 && q_pos0 >= 0, HN_E_ARG,
               "hn_attn_fp8kv: invalid shape");
    HN_REQUIRE(qs && os && (kv_len == 0 || (cs && ss)) && (cur_len == 0 || curs), HN_E_ARG,
               "hn_attn_fp8kv: null stride array");
    HN_REQUIRE(qs[3] == 1 && os[3] == 1, HN_E_ARG, "hn_attn_fp8kv: head dim must be contiguous");
    HN_REQUIRE(qs[0] % 8 == 0 && qs[1] % 8 == 0 && qs[2] % 8 == 0 && os[0] % 4 == 0 &&
                   os[1] % 4 == 0 && os[2] % 4 == 0,
               HN_E_ARG, "hn_attn_fp8kv: q/out strides misaligned");
    HN_REQUIRE(aligned(q, 16) && aligned(out, 8), HN_E_ARG, "hn_attn_fp8kv: q/out misaligned");
    if (kv_len > 0) {
        HN_REQUIRE(kc && vc && ks && vs, HN_E_ARG, "hn_attn_fp8kv: null cache pointer");
        HN_REQUIRE(cs[3] == 1 && cs[0] % 16 == 0 && cs[1] % 16 == 0 && cs[2] % 16 == 0, HN_E_ARG,
                   "hn_attn_fp8kv: cache strides must be multiples of 16 bytes");
        HN_REQUIRE(aligned(kc, 16) && aligned(vc, 16), HN_E_ARG, "hn_attn_fp8kv: cache misaligned");
    }
    if (cur_len > 0) {
        HN_REQUIRE(kcur && vcur, HN_E_ARG, "hn_attn_fp8kv: null tail pointer");
        HN_REQUIRE(curs[3] == 1 && curs[0] % 8 == 0 && curs[1] % 8 == 0 && curs[2] % 8 == 0,
                   HN_E_ARG, "hn_attn_fp8kv: tail strides must be multiples of 8");
        HN_REQUIRE(aligned(kcur, 16) && aligned(vcur, 16), HN_E_ARG, "hn_attn_fp8kv: tail misaligned");
    }
    if (B == 0 || Lq == 0) return HN_OK;
    HN_REQUIRE(out && q, HN_E_ARG, "hn_attn_fp8kv: null q/out");
    attn::Params p;
    p.q = (const uint16_t*)q;
    p.kc = (const uint8_t*)kc; p.vc = (const uint8_t*)vc;
    p.ks = ks; p.vs = vs;
    p.kcur = (const uint16_t*)kcur; p.vcur = (const uint16_t*)vcur;
    p.out = (uint16_t*)out;
    p.qs0 = qs[0]; p.qs1 = qs[1]; p.qs2 = qs[2];
    if (kv_len > 0) {
        p.cs0 = cs[0]; p.cs1 = cs[1]; p.cs2 = cs[2];
        p.ss0 = ss[0]; p.ss1 = ss[1]; p.ss2 = ss[2];
    } else {
        p.cs0 = p.cs1 = p.cs2 = p.ss0 = p.ss1 = p.ss2 = 0;
    }
    if (cur_len > 0) {
        p.us0 = curs[0]; p.us1 = curs[1]; p.us2 = curs[2];
    } else {
        p.us0 = p.us1 = p.us2 = 0;
    }
    p.os0 = os[0]; p.os1 = os[1]; p.os2 = os[2];
    p.Lq = Lq; p.H = H; p.kv_len = kv_len; p.cur_len = cur_len;
    p.q_pos0 = q_pos0; p.chunk = chunk_len;
    p.scale_log2 = softmax_scale * 1.4426950408889634f;
    p.fmt = fmt;
    const int64_t qt = (Lq + attn::BQ - 1) / attn::BQ;
    const int sp = attn_splits(B, Lq, H, kv_len, cur_len);
    const int64_t need = sp > 1 ? (int64_t)sp * B * H * Lq * (D + 2) * (int64_t)sizeof(float) : 0;
    HN_REQUIRE(workspace_bytes >= need && (need == 0 || (workspace && aligned(workspace, 16))), HN_E_ARG,
               "hn_attn_fp8kv: workspace smaller than hn_attn_fp8kv_workspace_size() or misaligned");
    const int64_t work = B * H * qt * sp;
    HN_REQUIRE(work <= 0x3fffffffLL, HN_E_ARG, "hn_attn_fp8kv: too much work for one launch");
    p.q_tiles = (int)qt;
    p.splits = sp;
    p.work = (int)work;
    p.per_xcd = (int)((work + 7) / 8);
    p.ws_o = sp > 1 ? (float*)workspace : nullptr;
    p.ws_ml = sp > 1 ? (float*)workspace + (int64_t)sp * B * H * Lq * D : nullptr;
    const dim3 grid((unsigned)(8 * (int64_t)p.per_xcd));
    if (fmt == HN_KV_FP8)
        attn::attn_fp8kv_kernel<HN_KV_FP8><<<grid, attn::NT, 0, (hipStream_t)stream>>>(p);
    else
        attn::attn_fp8kv_kernel<HN_KV_INT8><<<grid, attn::NT, 0, (hipStream_t)stream>>>(p);
    int rc = check_launch("hn_attn_fp8kv");
    if (rc != HN_OK || sp <= 1) return rc;
    const int64_t rows = B * H * Lq;
    HN_REQUIRE(rows <= 0x7fffffffLL, HN_E_ARG, "hn_attn_fp8kv: too many rows to combine");
    attn::attn_combine_kernel<<<(unsigned)rows, attn::D, 0, (hipStream_t)stream>>>(
        p.ws_o, p.ws_ml, sp, rows, Lq, H, (uint16_t*)out, os[0], os[1], os[2]);
    return check_launch("hn_attn_fp8kv (combine)");
}
