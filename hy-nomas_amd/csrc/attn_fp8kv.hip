// Block-causal chunk attention over an FP8 (or INT8-compat) KV cache, gfx950.
//
//   O = softmax(Q K^T * scale) V,   K, V = code * per-(token, head) scale
//
// Work decomposition: one workgroup = NW waves = 32 NW queries of one (batch,
// head); each wave owns 32 queries (one 32-column MFMA block). Two shapes:
// 4 waves (128 queries, two workgroups per CU) and 8 waves (256 queries, one
// per CU); both put 2 waves on each SIMD, and the 8-wave shape dequantizes
// each K/V tile once for twice the queries. Keys stream through LDS in tiles
// of 64. Each tile is dequantized once per workgroup as it is written to LDS,
// to the reference's own dequantized values: K = bf16(code * k_scale) and
// V = bf16(code * v_scale) (fp32 product, rounded to nearest even), so the
// MFMAs consume exactly the K/V the reference attends over, and no per-key
// scale is needed in the compute loop. The optional unquantized tail (the
// current chunk's bf16 K/V) is copied into the same LDS formats.
//
// Per 32-key block the wave computes S^T = K Q^T with
// v_mfma_f32_32x32x16_bf16: the MFMA output puts one query per lane column,
// so a block's max is lane-local. The running max m moves only when a block's
// logits pass m + 8 (one exchange with lane ^ 32 then makes it the pair's
// exact max): probabilities stay <= 2^8, and the common path has no
// cross-lane step. The row sum (of the fp16 probabilities, v_dot2) stays
// lane-local until the end. P^T is packed to fp16 in
// registers and is the B operand of O^T += V^T P^T (v_mfma_f32_32x32x16_f16).
// fp16 probabilities round at 2^-11 relative instead of bf16's 2^-8; V^T is
// held as the fp16 form of its bf16 value, which is the same number (a bf16
// value in fp16's normal range is exactly representable; fp16 subnormals
// round below 2^-24 and magnitudes past 65504 saturate). V is kept
// transposed in LDS ([dim][key], keys of each 16-key slice in the order of
// the P^T registers), so each V^T operand is one 16-byte LDS read.
//
// The loop is software-pipelined over half tiles (32-key blocks) so that each
// wave's MFMAs run beside independent VALU work of its own (see step_a /
// step_b).
//
// Mask: key position p is visible to query position r iff p / chunk <= r / chunk
// (chunk <= 0: all visible), and, in the MASK instantiation, iff the key's
// validity byte is non-zero (padded text keys, holes in the cached history:
// the kv_mask of nomas_cpt.py:611-685). Tiles wholly beyond the last query's
// chunk are never visited; tiles wholly visible to every query of the
// workgroup skip the per-element test.
#include <mutex>

#include "hn_capi_internal.h"
#include "hn_common.h"

namespace hn {
namespace attn {

constexpr int D = 128;
constexpr int BKV = 64;            // keys per tile
constexpr int QW = 32;             // queries per wave
constexpr int KROW = D * 2 + 16;   // K tile row: 128 bf16 + 16 B pad (bank spread)
// V^T tile: 128 dim rows of 64 fp16 keys (128 B) padded to 144 B = 9 16-byte
// units, so 16 consecutive rows at one column fall in 16 different bank
// groups (9 is odd). Column unit c of a row holds the 8 keys 16 (c / 2) +
// 4 (c % 2) + {0..3} and + 8 + {0..3}: the keys lane half c % 2 feeds to the
// PV MFMA for 16-key slice c / 2.
constexpr int VTROW = 144;
constexpr int K_BYTES = BKV * KROW;
constexpr int VT_BYTES = D * VTROW;
// After K and V^T, each stage holds the tile's 64-bit key-validity word (bit
// j: key j of the tile exists and is valid), written only by the MASK
// instantiation.
constexpr int MASK_OFF = K_BYTES + VT_BYTES;
constexpr int STAGE = K_BYTES + VT_BYTES + 16;
constexpr uint64_t ALL_KEYS = ~0ull;
// Per-key scales of a tile in flight ([0, 64) K, [64, 128) V), two buffers.
constexpr int SB_FLOATS = 2 * BKV;
// K/V stages in LDS: three for the 8-wave shape (one workgroup per CU), so
// that a tile is written two tiles ahead of its use and one barrier per tile
// suffices; two for the 4-wave shape, whose two workgroups per CU could not
// hold three each.
template <int NW>
constexpr int stages() { return NW == 8 ? 3 : 2; }
template <int NW>
constexpr int smem_bytes() { return stages<NW>() * STAGE + 2 * SB_FLOATS * 4; }

// Workgroup shape for NW (4 or 8) waves.
template <int NW>
struct Shape {
    static_assert(NW == 4 || NW == 8, "4 or 8 waves");
    static constexpr int NT = 64 * NW;   // threads
    static constexpr int BQ = QW * NW;   // queries
    static constexpr int KU = 512 / NT;  // 16-code K units per thread (64 keys x 8 units)
    static constexpr int VD = 2048 / NT; // V dims per thread (64 keys x 128 dims, 4-key quads)
};

struct Params {
    const uint16_t* q;
    const uint8_t* kc;
    const uint8_t* vc;
    const float* ks;
    const float* vs;
    const uint16_t* kcur;
    const uint16_t* vcur;
    uint16_t* out;
    // Key-validity bytes (MASK instantiation; null = every key valid): cache
    // keys kvalid[b * kvs + t], tail keys uvalid[b * uvs + j].
    const uint8_t* kvalid;
    const uint8_t* uvalid;
    int64_t kvs, uvs;
    int64_t qs0, qs1, qs2;
    int64_t cs0, cs1, cs2;   // cs0 == 0 (and ss0 == 0): one cache slot read by every batch
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

typedef float f32x2 __attribute__((ext_vector_type(2)));
typedef _Float16 f16x2 __attribute__((ext_vector_type(2)));
typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));

// ---------------------------------------------------------------------------
// Dequantization to the reference's bf16 values.

// Two codes (bytes 2 hi, 2 hi + 1 of w) -> their exact fp32 values. The gfx950
// conversion is used with a unit scale only: its scale operand applies just
// the exponent of the fp32 value.
template <int FMT>
HN_DEVICE f32x2 codes2_f32(uint32_t w, bool hi) {
    if (FMT == HN_KV_FP8)
        return hi ? __builtin_amdgcn_cvt_scalef32_pk_f32_fp8(w, 1.0f, true)
                  : __builtin_amdgcn_cvt_scalef32_pk_f32_fp8(w, 1.0f, false);
    const uint32_t sh = hi ? 16 : 0;
    f32x2 r;
    r[0] = (float)(int8_t)((w >> sh) & 0xffu);
    r[1] = (float)(int8_t)((w >> (sh + 8)) & 0xffu);
    return r;
}

// bf16 bits of fp32 a and b, packed (a low), round to nearest even.
HN_DEVICE uint32_t pack_bf16(float a, float b) {
    const f32x2 f = {a, b};
    return __builtin_bit_cast(uint32_t, __builtin_convertvector(f, bf16x2));
}

// fp16 bits of fp32 a and b, packed (a low), round to nearest even.
HN_DEVICE uint32_t pack_f16(float a, float b) {
    const f32x2 f = {a, b};
    return __builtin_bit_cast(uint32_t, __builtin_convertvector(f, f16x2));
}

// fp16 bits of the two bf16 values of word w (lo, hi), packed (lo low). Exact
// for bf16 values in fp16's range; round toward zero, so magnitudes past
// 65504 saturate instead of overflowing.
HN_DEVICE uint32_t bf16x2_to_f16x2(uint32_t w) {
    return __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_pkrtz(bf16_lo(w), bf16_hi(w)));
}

// fp16 bits of bf16(a), bf16(b): the reference's bf16 dequantized values held
// as fp16 operands of the PV MFMA.
HN_DEVICE uint32_t pack_f16_of_bf16(float a, float b) { return bf16x2_to_f16x2(pack_bf16(a, b)); }

// ---------------------------------------------------------------------------
// Tile loads and LDS writes.
//
// K: thread t owns units i < KU: key k_key(t) + NT / 8 i, 16 dims at 16 k_unit(t).
// In each wave, lane bits 0-1 give the unit's low bits, bit 2 the key's low
// bit, bit 3 the unit's high bit and bits 4-5 the key's high bits: 16 lanes
// cover two whole key rows (256 contiguous bytes of the cache), and the
// 16-byte LDS writes of any 8 consecutive lanes (two keys, rows 272 B apart)
// fall in 8 different 16-byte bank groups -- a 16-byte LDS write is served 8
// lanes at a time over 128 bytes of banks, so one key's 8 units 32 B apart
// would pair up.
// V^T: thread t (wave w, lane λ) owns key quad qd = λ % 16 (keys quad_key(qd, j),
// j < 4: the 8-byte half qd % 2 of column unit qd / 2) and the VD dims VD dg ..
// VD dg + VD - 1 (v_group). Per 8-byte LDS write a 32-lane group covers 2 dim
// groups 8 rows apart x 16 quads, whose bank pairs (18 row + qd) mod 32 are all
// distinct (row pitch 144 B, 18 x 8 = 16 mod 32); per global load each wave
// reads 16 keys x 4 VD contiguous bytes.
// Scales: threads 0-63 load the K scale of key t, threads 64-127 the V scale
// of key t - 64, into the tile's scale buffer.
// Validity (MASK): threads 128-191 (wave 2) load the validity byte of key
// t - 128; the wave's ballot is the tile's validity word.

// Key (within the tile, for i = 0) and unit (16-code run of the key) of
// thread t's K unit.
HN_DEVICE uint32_t k_key(uint32_t t) { return 8u * (t >> 6) + 2u * ((t >> 4) & 3u) + ((t >> 2) & 1u); }
HN_DEVICE uint32_t k_unit(uint32_t t) { return (t & 3u) + 4u * ((t >> 3) & 1u); }

// Key (0..63) of entry j (0..3) of quad qd.
HN_DEVICE int quad_key(int qd, int j) {
    return 16 * (qd >> 2) + 4 * ((qd >> 1) & 1) + 8 * (qd & 1) + j;
}

// Dim group of this thread's V^T quad: lanes 0-31 and 32-63 of a wave take
// groups whose first rows are 8 apart.
template <int NW>
HN_DEVICE int v_group_of(int tid) {
    const int w = tid >> 6, hh = (tid & 63) >> 4;
    if constexpr (NW == 4) return 4 * w + hh;                       // 8 dims per group
    else return 4 * w + 2 * (hh & 1) + (hh >> 1);                   // 4 dims per group
}
template <int NW>
HN_DEVICE int v_group() { return v_group_of<NW>(threadIdx.x); }

// Registers holding one cache tile between its global load and its LDS
// write (issued about one tile ahead).
template <int NW>
struct CacheRegs {
    uint4 k[Shape<NW>::KU];
    uint32_t v[4][Shape<NW>::VD / 4];  // VD codes (dims VD dg ..) of quad key j
    float s;                           // one per-key scale (threads < 128)
    uint32_t mk;                       // MASK: validity of key t - 128 (wave 2)
};

// A cache tile's loads are buffer loads: per tile one scalar descriptor per
// array (base = the tile's first key; size = the tile's bytes, so rows past
// the tile's key count read as zeros -- they are masked out of the softmax --
// with no per-lane clamp), and per lane a fixed 32-bit offset inside the
// tile, computed once (LaneOffs).
constexpr int BUF_FLAGS = 0x00020000;  // raw (stride 0) buffer, 32-bit dwords

struct TileBase {
    __amdgpu_buffer_rsrc_t k, v, ks, vs;
    const uint8_t* mk;  // validity bytes of the tile's keys, or null (all valid)
};

HN_DEVICE __amdgpu_buffer_rsrc_t tile_rsrc(const void* base, int64_t bytes) {
    return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(base), (short)0, (int)bytes, BUF_FLAGS);
}

// count = 0 gives empty descriptors: every load through them reads zeros and
// touches no memory (the loop issues its prefetch loads unconditionally, so
// that their order, and with it every wait on them, is the same on all paths).
HN_DEVICE TileBase tile_base(const Params& p, int64_t b, int64_t h, int64_t first, int count) {
    TileBase tb;
    const int64_t c = b * p.cs0 + first * p.cs1 + h * p.cs2;
    const int64_t s = b * p.ss0 + first * p.ss1 + h * p.ss2;
    const int64_t cb = count > 0 ? (int64_t)(count - 1) * p.cs1 + D : 0;  // codes of keys 0 .. count - 1
    const int64_t sb = count > 0 ? ((int64_t)(count - 1) * p.ss1 + 1) * 4 : 0;
    tb.k = tile_rsrc(p.kc + c, cb);
    tb.v = tile_rsrc(p.vc + c, cb);
    tb.ks = tile_rsrc(p.ks + s, sb);
    tb.vs = tile_rsrc(p.vs + s, sb);
    tb.mk = p.kvalid ? p.kvalid + b * p.kvs + first : nullptr;
    return tb;
}

// This thread's byte offsets inside a tile: K units (key u / 8, 16 codes at
// 16 (u % 8)), the VD codes of its V^T quad keys, and its per-key scale
// (threads < 128: K scales for threads 0-63, V for 64-127).
template <int NW>
struct LaneOffs {
    uint32_t k[Shape<NW>::KU];
    uint32_t v[4];
    uint32_t s;
};

template <int NW>
HN_DEVICE LaneOffs<NW> lane_offsets(const Params& p) {
    LaneOffs<NW> o;
    const uint32_t t = threadIdx.x;
#pragma unroll
    for (int i = 0; i < Shape<NW>::KU; ++i)
        o.k[i] = (k_key(t) + (uint32_t)(Shape<NW>::NT / 8) * i) * (uint32_t)p.cs1 + k_unit(t) * 16u;
    const int qd = t & 15, dg = v_group<NW>();
#pragma unroll
    for (int j = 0; j < 4; ++j) o.v[j] = (uint32_t)quad_key(qd, j) * (uint32_t)p.cs1 + (uint32_t)(Shape<NW>::VD * dg);
    o.s = (t & 63u) * (uint32_t)p.ss1 * 4u;
    return o;
}

// `co` / `so`: a tile's byte offset inside descriptors that start before it
// (the steady loop's span descriptors), added to every lane's code / scale
// offset; `mk0` the tile's first key in the span's validity bytes; 0 with
// per-tile descriptors.
template <int NW, bool MASK>
HN_DEVICE void load_k(const LaneOffs<NW>& lo, CacheRegs<NW>& r, const TileBase& tb, int count, uint32_t co = 0,
                      uint32_t so = 0, int64_t mk0 = 0) {
    const uint32_t t = threadIdx.x;
    // Wave 0 reads the K scales, wave 1 the V scales. The wave index goes
    // through readfirstlane so that the descriptor choice is a scalar one (a
    // per-lane choice of descriptor would be a loop over its distinct values).
    // The scale load is issued before the codes: its consumer (the scale
    // buffer write) then waits for it alone.
    const uint32_t wv = __builtin_amdgcn_readfirstlane(t >> 6);
    if (wv < 2u) {
        const __amdgpu_buffer_rsrc_t sr = wv == 0u ? tb.ks : tb.vs;
        r.s = __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(sr, lo.s + so, 0, 0));
    }
#pragma unroll
    for (int i = 0; i < Shape<NW>::KU; ++i)
        r.k[i] = __builtin_bit_cast(uint4, __builtin_amdgcn_raw_buffer_load_b128(tb.k, lo.k[i] + co, 0, 0));
    if constexpr (MASK) {
        if ((t >> 6) == 2u) {
            const uint32_t j = t & 63u;
            r.mk = (int)j < count ? (tb.mk ? (uint32_t)tb.mk[mk0 + j] : 1u) : 0u;
        }
    }
}

// The validity word of a cache tile, from the bytes wave 2 loaded with its
// codes, into the stage (MASK only). Called with the tile's K write.
template <int NW, bool MASK>
HN_DEVICE void store_mask(const CacheRegs<NW>& r, uint8_t* st) {
    if constexpr (MASK) {
        if ((threadIdx.x >> 6) == 2) {
            const uint64_t bits = __ballot(r.mk != 0u);
            if ((threadIdx.x & 63) == 0) *reinterpret_cast<uint64_t*>(st + MASK_OFF) = bits;
        }
    }
}

// The validity word of the tile in stage st (ALL_KEYS without MASK). Every
// lane reads the same 8 bytes; the word is made wave-uniform.
template <bool MASK>
HN_DEVICE uint64_t tile_mask(const uint8_t* st) {
    if constexpr (!MASK) return ALL_KEYS;
    const uint64_t w = *reinterpret_cast<const uint64_t*>(st + MASK_OFF);
    const uint32_t lo = __builtin_amdgcn_readfirstlane((uint32_t)w);
    const uint32_t hi = __builtin_amdgcn_readfirstlane((uint32_t)(w >> 32));
    return ((uint64_t)hi << 32) | lo;
}

template <int NW>
HN_DEVICE void load_v(const LaneOffs<NW>& lo, CacheRegs<NW>& r, const TileBase& tb, uint32_t co = 0) {
    constexpr int VD = Shape<NW>::VD;
#pragma unroll
    for (int j = 0; j < 4; ++j) {
        if constexpr (VD == 8) {
            const uint2 x = __builtin_bit_cast(uint2, __builtin_amdgcn_raw_buffer_load_b64(tb.v, lo.v[j] + co, 0, 0));
            r.v[j][0] = x.x;
            r.v[j][1] = x.y;
        } else {
            r.v[j][0] = __builtin_amdgcn_raw_buffer_load_b32(tb.v, lo.v[j] + co, 0, 0);
        }
    }
}

HN_DEVICE uint32_t word(const uint4& c, int q) { return q == 0 ? c.x : q == 1 ? c.y : q == 2 ? c.z : c.w; }

// Dequantized K write, part i (0..7): the thread's codes 2 KU i .. +2 KU - 1
// (unit code / 16) into bf16 dwords of kd; each completed run of 8 codes is
// one 16-byte write (every second part with 2 units, every fourth with 1).
template <int FMT, int NW>
HN_DEVICE void store_k_part(const CacheRegs<NW>& r, uint8_t* st, int i, const float (&ks)[Shape<NW>::KU],
                            uint32_t (&kd)[4]) {
    constexpr int CP = 2 * Shape<NW>::KU;  // codes per part
    const int code0 = CP * i, un = code0 >> 4, c = code0 & 15;
#pragma unroll
    for (int c2 = 0; c2 < CP / 2; ++c2) {
        const int cc = c + 2 * c2;
        const f32x2 a = codes2_f32<FMT>(word(r.k[un], cc >> 2), (cc & 2) != 0);
        kd[(cc >> 1) & 3] = pack_bf16(a[0] * ks[un], a[1] * ks[un]);
    }
    if (((c + CP) & 7) == 0) {
        const uint32_t key = k_key(threadIdx.x) + (Shape<NW>::NT / 8) * un;
        *reinterpret_cast<uint4*>(st + key * KROW + k_unit(threadIdx.x) * 32 + ((c + CP - 8) >> 3) * 16) =
            make_uint4(kd[0], kd[1], kd[2], kd[3]);
    }
}

// The K scales of the thread's units, from the tile's scale buffer.
template <int NW>
HN_DEVICE void k_scales(const float* sb, float (&ks)[Shape<NW>::KU]) {
#pragma unroll
    for (int i = 0; i < Shape<NW>::KU; ++i) ks[i] = sb[k_key(threadIdx.x) + (Shape<NW>::NT / 8) * i];
}

// Dequantized V^T write, part i (0..7): quad key j = i / 2, dims VD/2 (i % 2)
// .. + VD/2 - 1 of the thread's VD; keys (0, 1) and (2, 3) pair into dwords
// of fp16-held bf16 values (vd[2 d + pair], dim d), and parts 6 and 7 write
// the two halves of the dims (8 bytes = 4 keys each).
// `vc` holds the thread's codes (as CacheRegs::v), `vt` is the V^T tile.
template <int FMT, int NW>
HN_DEVICE void store_v_part(const uint32_t (&vc)[4][Shape<NW>::VD / 4], uint8_t* vt, int i, const float4& vs,
                            float (&vp)[Shape<NW>::VD], uint32_t (&vd)[2 * Shape<NW>::VD]) {
    constexpr int VD = Shape<NW>::VD, DP = VD / 2;
    const int j = i >> 1, hf = i & 1;
    const float s = j == 0 ? vs.x : j == 1 ? vs.y : j == 2 ? vs.z : vs.w;
    float x[DP];
#pragma unroll
    for (int c2 = 0; c2 < DP / 2; ++c2) {
        const int code = DP * hf + 2 * c2;
        const f32x2 a = codes2_f32<FMT>(vc[j][code >> 2], (code & 2) != 0);
        x[2 * c2] = a[0] * s;
        x[2 * c2 + 1] = a[1] * s;
    }
#pragma unroll
    for (int dd = 0; dd < DP; ++dd) {
        const int d = DP * hf + dd;
        if (j & 1) vd[2 * d + (j >> 1)] = pack_f16_of_bf16(vp[d], x[dd]);
        else vp[d] = x[dd];
    }
    if (j == 3) {
        const int qd = threadIdx.x & 15, dg = v_group<NW>();
#pragma unroll
        for (int dd = 0; dd < DP; ++dd) {
            const int d = DP * hf + dd;
            *reinterpret_cast<uint2*>(vt + (VD * dg + d) * VTROW + 8 * qd) = make_uint2(vd[2 * d], vd[2 * d + 1]);
        }
    }
}

// The V scales of the thread's quad (4 consecutive keys), from the scale buffer.
HN_DEVICE float4 v_scales(const float* sb) {
    const int qd = threadIdx.x & 15;
    return *reinterpret_cast<const float4*>(sb + BKV + quad_key(qd, 0));
}

// Whole-tile write (prologue), scales from the tile's scale buffer.
template <int FMT, int NW, bool MASK>
HN_DEVICE void store_tile(const CacheRegs<NW>& r, uint8_t* st, const float* sb) {
    store_mask<NW, MASK>(r, st);
    float ks[Shape<NW>::KU];
    k_scales<NW>(sb, ks);
    const float4 vs = v_scales(sb);
    uint32_t kd[4];
    float vp[Shape<NW>::VD];
    uint32_t vd[2 * Shape<NW>::VD];
#pragma unroll
    for (int i = 0; i < 8; ++i) {
        store_k_part<FMT, NW>(r, st, i, ks, kd);
        store_v_part<FMT, NW>(r.v, st + K_BYTES, i, vs, vp, vd);
    }
}

// Unquantized tail tile (bf16 K/V of the current chunk), written with the
// same thread-to-location mapping as the cache writes (so it cleanly
// replaces what those wrote to the same stage). The loads and the LDS writes
// are separate steps: the 8-wave loop issues a tail tile's loads one tile
// ahead, as it does a cache tile's, into TailRegs; the 4-wave loop (two
// stages, registers already near the limit) loads and writes in one go.
template <int NW>
struct TailRegs {
    uint4 k[2 * Shape<NW>::KU];        // unit i: dims 16 u .. + 7 in k[2 i], + 8 .. + 15 in k[2 i + 1]
    uint32_t v[4][Shape<NW>::VD / 2];  // dims VD dg .. + VD - 1 of quad key j (bf16 pairs)
    uint32_t mk;                       // MASK: validity of key t - 128 (wave 2)
};

template <int NW, bool MASK>
HN_DEVICE void load_tail_k(const Params& p, int64_t b, int64_t h, int64_t first, int count, TailRegs<NW>& r) {
    const int t = threadIdx.x;
    if constexpr (MASK) {
        if ((t >> 6) == 2) {
            const int j = t & 63;
            r.mk = j < count ? (p.uvalid ? (uint32_t)p.uvalid[b * p.uvs + first + j] : 1u) : 0u;
        }
    }
#pragma unroll
    for (int i = 0; i < Shape<NW>::KU; ++i) {
        const int key = (int)k_key(t) + (Shape<NW>::NT / 8) * i, unit = (int)k_unit(t);
        const int j = min(key, count - 1);
        const uint16_t* src = p.kcur + b * p.us0 + (first + j) * p.us1 + h * p.us2 + unit * 16;
        r.k[2 * i] = *reinterpret_cast<const uint4*>(src);
        r.k[2 * i + 1] = *reinterpret_cast<const uint4*>(src + 8);
    }
}

template <int NW, bool MASK>
HN_DEVICE void store_tail_k(const TailRegs<NW>& r, uint8_t* st) {
    const int t = threadIdx.x;
    if constexpr (MASK) {
        if ((t >> 6) == 2) {
            const uint64_t bits = __ballot(r.mk != 0u);
            if ((t & 63) == 0) *reinterpret_cast<uint64_t*>(st + MASK_OFF) = bits;
        }
    }
#pragma unroll
    for (int i = 0; i < Shape<NW>::KU; ++i) {
        const int key = (int)k_key(t) + (Shape<NW>::NT / 8) * i, unit = (int)k_unit(t);
        uint4* dst = reinterpret_cast<uint4*>(st + key * KROW + unit * 32);
        dst[0] = r.k[2 * i];
        dst[1] = r.k[2 * i + 1];
    }
}

template <int NW>
HN_DEVICE void load_tail_v(const Params& p, int64_t b, int64_t h, int64_t first, int count, TailRegs<NW>& r) {
    constexpr int VD = Shape<NW>::VD;
    const int qd = threadIdx.x & 15, dg = v_group<NW>();
#pragma unroll
    for (int j = 0; j < 4; ++j) {
        const int key = min(quad_key(qd, j), count - 1);
        const uint16_t* src = p.vcur + b * p.us0 + (first + key) * p.us1 + h * p.us2 + VD * dg;
        if constexpr (VD == 8) {
            const uint4 x = *reinterpret_cast<const uint4*>(src);
            r.v[j][0] = x.x; r.v[j][1] = x.y; r.v[j][2] = x.z; r.v[j][3] = x.w;
        } else {
            const uint2 x = *reinterpret_cast<const uint2*>(src);
            r.v[j][0] = x.x; r.v[j][1] = x.y;
        }
    }
}

// V^T holds fp16: the bf16 values converted (exactly, in fp16's range).
template <int NW>
HN_DEVICE void store_tail_v(const TailRegs<NW>& r, uint8_t* st) {
    constexpr int VD = Shape<NW>::VD;
    const int qd = threadIdx.x & 15, dg = v_group<NW>();
#pragma unroll
    for (int d = 0; d < VD; ++d) {
        uint32_t o[2];
        const uint32_t sh = (d & 1) * 16;
#pragma unroll
        for (int pr = 0; pr < 2; ++pr)
            o[pr] = bf16x2_to_f16x2(((r.v[2 * pr][d >> 1] >> sh) & 0xffffu) |
                                    (((r.v[2 * pr + 1][d >> 1] >> sh) & 0xffffu) << 16));
        *reinterpret_cast<uint2*>(st + K_BYTES + (VD * dg + d) * VTROW + 8 * qd) = make_uint2(o[0], o[1]);
    }
}

template <int NW, bool MASK>
HN_DEVICE void copy_tail_k(const Params& p, int64_t b, int64_t h, int64_t first, int count, uint8_t* st) {
    TailRegs<NW> r;
    load_tail_k<NW, MASK>(p, b, h, first, count, r);
    store_tail_k<NW, MASK>(r, st);
}

template <int NW>
HN_DEVICE void copy_tail_v(const Params& p, int64_t b, int64_t h, int64_t first, int count, uint8_t* st) {
    TailRegs<NW> r;
    load_tail_v<NW>(p, b, h, first, count, r);
    store_tail_v<NW>(r, st);
}

HN_DEVICE f32x16 mfma_bf16(const bf16x8& a, const bf16x8& b, const f32x16& c) {
    return __builtin_amdgcn_mfma_f32_32x32x16_bf16(a, b, c, 0, 0, 0);
}

HN_DEVICE f32x16 mfma_f16(const f16x8& a, const f16x8& b, const f32x16& c) {
    return __builtin_amdgcn_mfma_f32_32x32x16_f16(a, b, c, 0, 0, 0);
}

HN_DEVICE bf16x8 ld_bf16x8(const uint8_t* p) {
    return __builtin_bit_cast(bf16x8, *reinterpret_cast<const uint4*>(p));
}

HN_DEVICE f16x8 ld_f16x8(const uint8_t* p) {
    return __builtin_bit_cast(f16x8, *reinterpret_cast<const uint4*>(p));
}

// Max of v over the lane pair (l, l ^ 32), through the LDS crossbar
// (ds_bpermute). gfx950's v_permlane32_swap is not used: in this kernel's
// instruction stream the compiler issues it two wait states after the VALU
// write of its operand, and the swapped values were then stale (the running
// max came out lane-local, which fp16 probabilities turn into overflow).
HN_DEVICE float pair_max(float v) { return fmaxf(v, __shfl_xor(v, 32, 64)); }

// ---------------------------------------------------------------------------
// Half-tile steps. A "half" is one 32-key block kb of a 64-key tile; for it
// the wave holds S^T as one f32x16 (register v: key 32 kb + 8 (v/4) + 4 half
// + v%4, query = this lane's column).

// S^T block kb of the tile in stage st: 8 MFMAs over the 128 dims (prologue).
HN_DEVICE f32x16 s_block(const uint8_t* ka, const bf16x8 (&qf)[8]) {
    f32x16 acc;
#pragma unroll
    for (int v = 0; v < 16; ++v) acc[v] = 0.0f;
#pragma unroll
    for (int sl = 0; sl < 8; ++sl) acc = mfma_bf16(ld_bf16x8(ka + 32 * sl), qf[sl], acc);
    return acc;
}

// Running state of this lane's query: m, the reference point of the
// probabilities in log2 units (-inf before any visible key); nm = -m (0 while
// m = -inf); l, this lane's share of the softmax denominator.
struct Run {
    float m, nm, l;
};

// m may lag the true running max by up to REBASE_SLACK: the probabilities
// 2^(s c - m) then stay <= 2^REBASE_SLACK, far inside fp16's range, and O, l
// and m stay consistent (both are relative to m), so the softmax is the same
// for any such m.
constexpr float REBASE_SLACK = 8.0f;

// Max of a raw S^T block over this lane's 16 keys of the query (the pair
// lane holds the other 16; rebase exchanges the two only when it acts).
HN_DEVICE float raw_max(const f32x16& s) {
    float mx = s[0];
#pragma unroll
    for (int v = 1; v < 16; ++v) mx = fmaxf(mx, s[v]);
    return mx;
}

// Partial tiles: keys j >= lim of the tile, and keys whose bit of the tile's
// validity word mw is clear, are masked to -inf; returns the new max.
HN_DEVICE float mask_raw(f32x16& u, int kb, int half, int lim, uint64_t mw) {
    const uint32_t bits = (uint32_t)(mw >> (kb * 32 + 4 * half));
    float mx = -INFINITY;
#pragma unroll
    for (int v = 0; v < 16; ++v) {
        const int j = kb * 32 + 8 * (v >> 2) + 4 * half + (v & 3);
        if (j >= lim || !((bits >> (8 * (v >> 2) + (v & 3))) & 1u)) u[v] = -INFINITY;
        mx = fmaxf(mx, u[v]);
    }
    return mx;
}

// Before a block's probabilities, with the lane's raw block max mx (its
// logit max in log2 units is mx * c, c = softmax_scale * log2 e > 0): taken,
// wave-uniformly, only when some lane's logit max passes m + REBASE_SLACK
// (always when a lane sees its first visible key, m = -inf). Then m moves to
// the pair's exact max (an LDS-crossbar exchange with lane ^ 32), and O and l
// are rescaled by 2^(m_old - m_new).
HN_DEVICE void rebase(float mx, float c, Run& run, f32x16 (&o)[4]) {
    if (!__any(mx * c > run.m + REBASE_SLACK)) return;
    const float mnew = fmaxf(run.m, pair_max(mx) * c);
    const float alpha = run.m == -INFINITY ? 1.0f : __builtin_amdgcn_exp2f(run.m - mnew);
    run.m = mnew;
    run.nm = mnew == -INFINITY ? 0.0f : -mnew;  // m = -inf: every s is -inf (masked)
    run.l *= alpha;
    if (__any(alpha != 1.0f)) {
#pragma unroll
        for (int db = 0; db < 4; ++db)
#pragma unroll
            for (int v = 0; v < 16; ++v) o[db][v] *= alpha;
    }
}

// Ties values to this point of the instruction stream: the empty asm is
// ordered with the sched_barrier that ends a slot, so the arithmetic feeding
// it cannot drift into later slots (pure operations are otherwise placed
// freely before the machine scheduler sees the barrier).
template <typename A, typename B, typename C>
HN_DEVICE void pin(A& a, B& b, C& c) {
    asm volatile("" : "+v"(a), "+v"(b), "+v"(c));
}
template <typename A, typename B>
HN_DEVICE void pin(A& a, B& b) {
    asm volatile("" : "+v"(a), "+v"(b));
}
template <typename A>
HN_DEVICE void pin(A& a) {
    asm volatile("" : "+v"(a));
}

// ---------------------------------------------------------------------------
// The two software-pipelined steps of a half tile. Each pairs one 8-MFMA chain
// with the independent VALU work of the other chain, spread over 8 slots (one
// MFMA + about 8 VALU instructions, ~32 cycles each) that sched_barrier keeps
// in place: a wave's VALU instructions execute while its own MFMAs occupy the
// matrix core, so the overlap is built into each wave's instruction stream
// rather than left to the other wave on the SIMD. Operand reads from LDS are
// issued two slots ahead.

// Step A: S^T of the next block from the K rows at ka (this lane's row in the
// stage) beside the probabilities of the current block (raw S^T in s):
// p = 2^(s c - m), l += fp16(p), P^T = fp16(p) for the two 16-key slices
// (registers 8t .. 8t+7 hold keys 16 t + 4 half + {0..3} and + 8 + {0..3} of
// the block).
HN_DEVICE f32x16 step_a(const f32x16& s, float c, float nm, float& l, f16x8 (&pf)[2], const uint8_t* ka,
                        const bf16x8 (&qf)[8]) {
    bf16x8 kf[8];
    kf[0] = ld_bf16x8(ka);
    kf[1] = ld_bf16x8(ka + 32);
    f32x16 acc;
#pragma unroll
    for (int v = 0; v < 16; ++v) acc[v] = 0.0f;
    float ls = 0.0f;
    const f16x2 ones = {(_Float16)1.0f, (_Float16)1.0f};
    uint32_t x[8];
#pragma unroll
    for (int i = 0; i < 8; ++i) {
        if (i + 2 < 8) kf[i + 2] = ld_bf16x8(ka + 32 * (i + 2));
        acc = mfma_bf16(kf[i], qf[i], acc);
        const float p0 = __builtin_amdgcn_exp2f(__builtin_fmaf(s[2 * i], c, nm));
        const float p1 = __builtin_amdgcn_exp2f(__builtin_fmaf(s[2 * i + 1], c, nm));
        x[i] = pack_f16(p0, p1);
        // l sums the fp16 probabilities the PV MFMA multiplies (v_dot2_f32_f16)
        ls = __builtin_amdgcn_fdot2(__builtin_bit_cast(f16x2, x[i]), ones, ls, false);
        pin(x[i], ls);
        __builtin_amdgcn_sched_barrier(0);
    }
    l += ls;
    pf[0] = __builtin_bit_cast(f16x8, make_uint4(x[0], x[1], x[2], x[3]));
    pf[1] = __builtin_bit_cast(f16x8, make_uint4(x[4], x[5], x[6], x[7]));
    return acc;
}

// Step B: O^T += V^T P^T of block kb (V^T operand reads at va: this lane's
// row and column in the stage) beside the raw max of the next block (s) and,
// per STORE (1: K, 2: V^T), half of the write of the prefetched tile to stage
// nst with the scales of buffer sb. Returns the next block's raw max over this
// lane's keys.
template <int FMT, int NW, int STORE>
HN_DEVICE float step_b(const f16x8 (&pf)[2], const uint8_t* va, int kb, f32x16 (&o)[4], const f32x16& s,
                       const CacheRegs<NW>& r, uint8_t* nst, const float* sb) {
    // operand i (= 4 tt + db): dim block db, 16-key slice 2 kb + tt
    f16x8 vf[8];
    vf[0] = ld_f16x8(va + 64 * kb);
    vf[1] = ld_f16x8(va + 64 * kb + 32 * VTROW);
    float ks[Shape<NW>::KU] = {};
    float4 vs = make_float4(0.0f, 0.0f, 0.0f, 0.0f);
    if (STORE == 1) k_scales<NW>(sb, ks);
    if (STORE == 2) vs = v_scales(sb);
    float mx = -INFINITY;
    uint32_t kd[4];
    float vp[Shape<NW>::VD];
    uint32_t vd[2 * Shape<NW>::VD];
#pragma unroll
    for (int i = 0; i < 8; ++i) {
        const int tt = i >> 2, db = i & 3;
        if (i + 2 < 8) {
            const int i2 = i + 2;
            vf[i2] = ld_f16x8(va + 64 * kb + 32 * (i2 >> 2) + (i2 & 3) * 32 * VTROW);
        }
        o[db] = mfma_f16(vf[i], pf[tt], o[db]);
        mx = fmaxf(mx, fmaxf(s[2 * i], s[2 * i + 1]));
        pin(mx);
        if (STORE == 1) store_k_part<FMT, NW>(r, nst, i, ks, kd);
        if (STORE == 2) store_v_part<FMT, NW>(r.v, nst + K_BYTES, i, vs, vp, vd);
        __builtin_amdgcn_sched_barrier(0);
    }
    return mx;
}

template <int FMT, int NW, bool MASK>
__global__ __launch_bounds__(64 * NW, 8 / NW) void attn_fp8kv_kernel(Params p) {
    constexpr int BQ = Shape<NW>::BQ;
    constexpr int NS = stages<NW>();
    __shared__ __attribute__((aligned(16))) uint8_t smem[smem_bytes<NW>()];
    float* const sbuf = reinterpret_cast<float*>(smem + NS * STAGE);  // [2][128]

    // XCD-aware work order: workgroup ids are dealt round-robin to the 8 XCDs,
    // so id % 8 picks a contiguous range of work items.
    //  * No key split: items run (b, h, query tile) with the tile fastest, so
    //    the query tiles of the same few heads share an XCD's L2 while they
    //    stream those heads' K/V.
    //  * Key splits: items run (b, query tile, split, h) with the head
    //    fastest, so an XCD holds whole key ranges of every head. A token's
    //    per-head scales are adjacent ([B, cap, H, 1]): the heads of one key
    //    range then share each scale sector in one L2, where a head-major
    //    order had every XCD fetch every sector for its few heads.
    const int id = blockIdx.x;
    const int w = (id & 7) * p.per_xcd + (id >> 3);
    if (w >= p.work) return;
    int split, qt;
    int64_t h, b;
    if (p.splits > 1) {
        h = w % p.H;
        const int ws = w / (int)p.H;
        split = ws % p.splits;
        const int wt = ws / p.splits;
        qt = wt % p.q_tiles;
        b = wt / p.q_tiles;
    } else {
        split = 0;
        qt = w % p.q_tiles;
        h = (w / p.q_tiles) % p.H;
        b = w / (p.q_tiles * (int)p.H);
    }

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
    Run run{-INFINITY, 0.0f, 0.0f};  // shared by the lane pair (but l)
    const float c = p.scale_log2;

    // Tile t: segment, first key index within it, key count;
    // `full`: every key exists and is visible to every query of the workgroup;
    // `lim`: keys j < lim of the tile are visible to this lane's query.
    struct Geom {
        bool cache;
        int64_t first;
        int count;
        bool full;
        int64_t pos0;  // position of the tile's key 0
    };
    auto geom = [&](int t) {
        Geom g;
        int64_t count, pos0;
        if (t < n_cache) {
            g.cache = true;
            g.first = (int64_t)t * BKV;
            count = cache_end - g.first;
            pos0 = g.first;
        } else {
            g.cache = false;
            g.first = (int64_t)(t - n_cache) * BKV;
            count = tail_end - g.first;
            pos0 = p.kv_len + g.first;
        }
        g.count = (int)(count < BKV ? count : BKV);
        g.full = g.count == BKV && pos0 + BKV <= wg_key_limit;
        g.pos0 = pos0;
        return g;
    };
    // Keys j < lim_of(g) of tile g are visible to this lane's query (taken only
    // on the masked path).
    auto lim_of = [&](const Geom& g) {
        int64_t lim64 = key_limit - g.pos0;
        lim64 = lim64 < g.count ? lim64 : g.count;
        return lim64 < 0 ? 0 : (int)lim64;
    };
    // This lane's K row (block 0) at dims 8 half .., and its V^T row (dim
    // block 0) at column unit `half` (slice 0).
    const uint32_t ka_off = col * KROW + 16 * half;
    const uint32_t va_off = K_BYTES + col * VTROW + 16 * half;
    CacheRegs<NW> regs;
    regs.s = 0.0f;
    const LaneOffs<NW> lo = lane_offsets<NW>(p);

    // Steady tiles: the prefix [t_begin, t_fast) of the range in which the
    // current and the next tile are full cache tiles (every key exists and is
    // visible to every query: nothing to mask) and the tiles written and
    // fetched are cache tiles -- the bulk of any long range. They run a loop
    // with no per-tile geometry, tail or mask branches, loading through
    // descriptors that span the (b, h) cache rows [0, cache_end) at the
    // tile's byte offset (so the span must fit 31 bits). Kernels with
    // validity masks take the general loop throughout.
    const int64_t full_end = cache_end < wg_key_limit ? cache_end : wg_key_limit;
    const int n_full = full_end > 0 ? (int)(full_end / BKV) : 0;
    const bool span_ok = cache_end > 0 && p.cs1 > 0 && p.ss1 > 0 &&
                         (cache_end - 1) * p.cs1 + D < ((int64_t)1 << 31) &&
                         ((cache_end - 1) * p.ss1 + 1) * 4 < ((int64_t)1 << 31);
    int t_fast = t_begin;
    if (span_ok) {
        int tf = n_full - 1;
        tf = tf < t_end - NS ? tf : t_end - NS;
        tf = tf < n_cache - NS ? tf : n_cache - NS;
        t_fast = tf > t_begin ? tf : t_begin;
    }
    const TileBase span = tile_base(p, b, h, 0, span_ok ? (int)cache_end : 0);
    const uint32_t tile_co = (uint32_t)(BKV * p.cs1), tile_so = (uint32_t)(BKV * p.ss1 * 4);

    // Software pipeline over half tiles. Tile t (u = t - t_begin) is in
    // stage u % NS; during it the wave writes tile t + NS - 1 (dequantized from
    // the prefetch registers, scales from buffer (u + NS - 1) % 2) to stage
    // (u + NS - 1) % NS and fetches the codes and scales of tile t + NS:
    //   half 0: rebase; S(t, kb 1) || probs(kb 0)
    //           PV(t, kb 0) || max(kb 1), K of t + NS - 1 written; K codes +
    //           scales of t + NS fetched
    //   half 1: rebase; S(t + 1, kb 0) || probs(kb 1)
    //           PV(t, kb 1) || max(t + 1, kb 0), V^T of t + NS - 1 written;
    //           scales of t + NS to buffer (u + NS) % 2, V codes fetched
    // NS = 2 (the loop below, written for it): K of t + 1 is written in half
    // 0 and read by S(t + 1) in half 1, so a barrier ends half 0 as well as
    // the tile. NS = 3 (the generic loop after it): every tile a half
    // reads was written before the barrier that ended an earlier tile, and
    // the stage written during tile t (that of t - 1) was last read in half 1
    // of t - 1, before the barrier ending it; one barrier per tile.
    // Scale buffer (u + NS) % 2 last served the write of tile t + NS - 2,
    // during tile t - 2 (NS = 3) or t - 1 (NS = 2), before a barrier.
    if constexpr (NS == 2) {
        if (t_end > t_begin) {
            f32x16 sa, sb;
            float mxa, mxb;
            uint64_t mw;  // validity word of tile t
            Geom g = geom(t_begin);
            {
                if (g.cache) {
                    const TileBase tb = tile_base(p, b, h, g.first, g.count);
                    load_k<NW, MASK>(lo, regs, tb, g.count);
                    load_v<NW>(lo, regs, tb);
                    __builtin_amdgcn_s_waitcnt(0);
                    if (threadIdx.x < 2 * BKV) sbuf[threadIdx.x] = regs.s;
                    __syncthreads();
                    store_tile<FMT, NW, MASK>(regs, smem, sbuf);
                } else {
                    copy_tail_k<NW, MASK>(p, b, h, g.first, g.count, smem);
                    copy_tail_v<NW>(p, b, h, g.first, g.count, smem);
                }
                if (t_begin + 1 < t_end) {
                    const Geom g1 = geom(t_begin + 1);
                    if (g1.cache) {
                        const TileBase tb = tile_base(p, b, h, g1.first, g1.count);
                        load_k<NW, MASK>(lo, regs, tb, g1.count);
                        load_v<NW>(lo, regs, tb);
                    }
                }
                // Everything issued so far (the Q fragments included) has landed;
                // inside the loop the only loads in flight are the prefetch.
                __builtin_amdgcn_s_waitcnt(0);
                if (threadIdx.x < 2 * BKV) sbuf[SB_FLOATS + threadIdx.x] = regs.s;
                __syncthreads();
                mw = tile_mask<MASK>(smem);
                sa = s_block(smem + ka_off, qf);
                mxa = raw_max(sa);
                if (!g.full || mw != ALL_KEYS) mxa = mask_raw(sa, 0, half, lim_of(g), mw);
            }
            int t = t_begin;
            {
                // steady tiles (see t_fast): fetch tile t + 2 at offsets fco / fso.
                // With validity masks (MASK) each tile's word travels with its
                // K write; a tile whose word is not all ones masks its blocks.
                uint32_t fco = (uint32_t)((int64_t)(t + 2) * BKV * p.cs1);
                uint32_t fso = (uint32_t)((int64_t)(t + 2) * BKV * p.ss1 * 4);
                for (; t < t_fast; ++t) {
                    const int u = t - t_begin;
                    const uint8_t* st = smem + (u & 1) * STAGE;
                    uint8_t* nst = smem + ((u & 1) ^ 1) * STAGE;
                    const float* nsb = sbuf + ((u & 1) ^ 1) * SB_FLOATS;
                    f16x8 pf[2];
                    rebase(mxa, c, run, o);
                    sb = step_a(sa, c, run.nm, run.l, pf, st + ka_off + 32 * KROW, qf);
                    mxb = step_b<FMT, NW, 1>(pf, st + va_off, 0, o, sb, regs, nst, nsb);
                    if constexpr (MASK) {
                        store_mask<NW, MASK>(regs, nst);
                        if (mw != ALL_KEYS) mxb = mask_raw(sb, 1, half, BKV, mw);
                    }
                    load_k<NW, MASK>(lo, regs, span, BKV, fco, fso, (int64_t)(t + 2) * BKV);
                    __syncthreads();
                    rebase(mxb, c, run, o);
                    sa = step_a(sb, c, run.nm, run.l, pf, nst + ka_off, qf);
                    mxa = step_b<FMT, NW, 2>(pf, st + va_off, 1, o, sa, regs, nst, nsb);
                    if constexpr (MASK) {
                        mw = tile_mask<MASK>(nst);  // tile t + 1
                        if (mw != ALL_KEYS) mxa = mask_raw(sa, 0, half, BKV, mw);
                    }
                    if (threadIdx.x < 2 * BKV) sbuf[(u & 1) * SB_FLOATS + threadIdx.x] = regs.s;
                    load_v<NW>(lo, regs, span, fco);
                    __syncthreads();
                    fco += tile_co;
                    fso += tile_so;
                }
                if (t > t_begin) g = geom(t);
            }
            for (; t < t_end; ++t) {
                const int u = t - t_begin;
                const uint8_t* st = smem + (u & 1) * STAGE;
                uint8_t* nst = smem + ((u & 1) ^ 1) * STAGE;
                const float* nsb = sbuf + ((u & 1) ^ 1) * SB_FLOATS;  // scales of tile t + 1
                const bool has_next = t + 1 < t_end;
                const Geom gn = geom(has_next ? t + 1 : t);
                const bool fetch2 = t + 2 < t_end;
                const Geom g2 = geom(fetch2 ? t + 2 : t);
                f16x8 pf[2];

                // ---- half 0
                rebase(mxa, c, run, o);
                sb = step_a(sa, c, run.nm, run.l, pf, st + ka_off + 32 * KROW, qf);
                // K (and validity word) of tile t + 1 from the prefetch registers
                // (a tail tile or the end of the range is handled right after:
                // the stage is not read before the barrier).
                mxb = step_b<FMT, NW, 1>(pf, st + va_off, 0, o, sb, regs, nst, nsb);
                store_mask<NW, MASK>(regs, nst);
                if (!g.full || mw != ALL_KEYS) mxb = mask_raw(sb, 1, half, lim_of(g), mw);
                if (has_next && !gn.cache) copy_tail_k<NW, MASK>(p, b, h, gn.first, gn.count, nst);
                const int n2 = fetch2 && g2.cache ? g2.count : 0;  // 0: no fetch (zeros)
                load_k<NW, MASK>(lo, regs, tile_base(p, b, h, g2.first, n2), n2);
                __syncthreads();

                // ---- half 1 (on the last tile the S block of "tile t + 1" reads
                // stale LDS; its result is never used)
                const uint64_t mwn = tile_mask<MASK>(nst);
                rebase(mxb, c, run, o);
                sa = step_a(sb, c, run.nm, run.l, pf, nst + ka_off, qf);
                mxa = step_b<FMT, NW, 2>(pf, st + va_off, 1, o, sa, regs, nst, nsb);
                if (!gn.full || mwn != ALL_KEYS) mxa = mask_raw(sa, 0, half, lim_of(gn), mwn);
                if (has_next && !gn.cache) copy_tail_v<NW>(p, b, h, gn.first, gn.count, nst);
                // (without a fetch: zeros into a scale buffer no write reads)
                if (threadIdx.x < 2 * BKV) sbuf[(u & 1) * SB_FLOATS + threadIdx.x] = regs.s;
                load_v<NW>(lo, regs, tile_base(p, b, h, g2.first, n2));
                __syncthreads();
                g = gn;
                mw = mwn;
            }
        }
    } else {
        if (t_end > t_begin) {
            f32x16 sa, sb;
            float mxa, mxb;
            // Prologue: tiles t_begin .. t_begin + NS - 2 written, the codes of
            // t_begin + NS - 1 in the prefetch registers with their scales in
            // buffer (NS - 1) % 2. Tiles k < NS - 1: load, scales to buffer k % 2,
            // barrier, dequantizing write to stage k (buffer k % 2 is rewritten
            // only after the next barrier, which follows this write).
#pragma unroll
            for (int k = 0; k < NS - 1; ++k) {
                const int t = t_begin + k;
                if (t >= t_end) break;
                const Geom gk = geom(t);
                if (gk.cache) {
                    const TileBase tb = tile_base(p, b, h, gk.first, gk.count);
                    load_k<NW, MASK>(lo, regs, tb, gk.count);
                    load_v<NW>(lo, regs, tb);
                    __builtin_amdgcn_s_waitcnt(0);
                    if (threadIdx.x < 2 * BKV) sbuf[(k & 1) * SB_FLOATS + threadIdx.x] = regs.s;
                    __syncthreads();
                    store_tile<FMT, NW, MASK>(regs, smem + k * STAGE, sbuf + (k & 1) * SB_FLOATS);
                } else {
                    copy_tail_k<NW, MASK>(p, b, h, gk.first, gk.count, smem + k * STAGE);
                    copy_tail_v<NW>(p, b, h, gk.first, gk.count, smem + k * STAGE);
                }
            }
            TailRegs<NW> tregs;  // a tail tile's bf16 K/V, loaded one tile ahead of its write
            if (t_begin + NS - 1 < t_end) {
                const Geom gk = geom(t_begin + NS - 1);
                if (gk.cache) {
                    const TileBase tb = tile_base(p, b, h, gk.first, gk.count);
                    load_k<NW, MASK>(lo, regs, tb, gk.count);
                    load_v<NW>(lo, regs, tb);
                } else {
                    load_tail_k<NW, MASK>(p, b, h, gk.first, gk.count, tregs);
                    load_tail_v<NW>(p, b, h, gk.first, gk.count, tregs);
                }
            }
            // Everything issued so far (the Q fragments included) has landed;
            // inside the loop the only loads in flight are the prefetch.
            __builtin_amdgcn_s_waitcnt(0);
            if (threadIdx.x < 2 * BKV) sbuf[((NS - 1) & 1) * SB_FLOATS + threadIdx.x] = regs.s;
            __syncthreads();
            Geom g = geom(t_begin);
            uint64_t mw = tile_mask<MASK>(smem);  // validity word of tile t
            sa = s_block(smem + ka_off, qf);
            mxa = raw_max(sa);
                if (!g.full || mw != ALL_KEYS) mxa = mask_raw(sa, 0, half, lim_of(g), mw);
            int t = t_begin;
            {
                // steady tiles (see t_fast): fetch tile t + NS at offsets fco / fso
                // (validity words as in the two-stage loop above)
                uint32_t fco = (uint32_t)((int64_t)(t + NS) * BKV * p.cs1);
                uint32_t fso = (uint32_t)((int64_t)(t + NS) * BKV * p.ss1 * 4);
                int s0 = 0;  // stage of tile t, (t - t_begin) % NS
                for (; t < t_fast; ++t) {
                    const int u = t - t_begin;
                    const int s1 = s0 == NS - 1 ? 0 : s0 + 1;  // tile t + 1
                    const int sw = s0 == 0 ? NS - 1 : s0 - 1;  // tile t + NS - 1
                    const uint8_t* st = smem + s0 * STAGE;
                    const uint8_t* st1 = smem + s1 * STAGE;
                    uint8_t* wst = smem + sw * STAGE;
                    const float* wsb = sbuf + ((u + NS - 1) & 1) * SB_FLOATS;
                    f16x8 pf[2];
                    const uint64_t mwn = tile_mask<MASK>(st1);  // tile t + 1
                    rebase(mxa, c, run, o);
                    sb = step_a(sa, c, run.nm, run.l, pf, st + ka_off + 32 * KROW, qf);
                    mxb = step_b<FMT, NW, 1>(pf, st + va_off, 0, o, sb, regs, wst, wsb);
                    if constexpr (MASK) {
                        store_mask<NW, MASK>(regs, wst);
                        if (mw != ALL_KEYS) mxb = mask_raw(sb, 1, half, BKV, mw);
                    }
                    load_k<NW, MASK>(lo, regs, span, BKV, fco, fso, (int64_t)(t + NS) * BKV);
                    rebase(mxb, c, run, o);
                    sa = step_a(sb, c, run.nm, run.l, pf, st1 + ka_off, qf);
                    mxa = step_b<FMT, NW, 2>(pf, st + va_off, 1, o, sa, regs, wst, wsb);
                    if constexpr (MASK) {
                        if (mwn != ALL_KEYS) mxa = mask_raw(sa, 0, half, BKV, mwn);
                        mw = mwn;
                    }
                    if (threadIdx.x < 2 * BKV) sbuf[((u + NS) & 1) * SB_FLOATS + threadIdx.x] = regs.s;
                    load_v<NW>(lo, regs, span, fco);
                    __syncthreads();
                    fco += tile_co;
                    fso += tile_so;
                    s0 = s1;
                }
                if (t > t_begin) g = geom(t);
            }
            for (; t < t_end; ++t) {
                const int u = t - t_begin;
                const uint8_t* st = smem + (u % NS) * STAGE;              // tile t
                const uint8_t* st1 = smem + ((u + 1) % NS) * STAGE;       // tile t + 1
                uint8_t* wst = smem + ((u + NS - 1) % NS) * STAGE;        // tile t + NS - 1
                const float* wsb = sbuf + ((u + NS - 1) & 1) * SB_FLOATS; // its scales
                const bool has_next = t + 1 < t_end;
                const Geom gn = geom(has_next ? t + 1 : t);
                const bool write = t + NS - 1 < t_end;
                const Geom gw = geom(write ? t + NS - 1 : t);
                const bool fetch = t + NS < t_end;
                const Geom gf = geom(fetch ? t + NS : t);
                f16x8 pf[2];
                const uint64_t mwn = tile_mask<MASK>(st1);  // tile t + 1 (stale on the last tile)

                // ---- half 0
                rebase(mxa, c, run, o);
                sb = step_a(sa, c, run.nm, run.l, pf, st + ka_off + 32 * KROW, qf);
                // K (and validity word) of tile t + NS - 1 from the prefetch
                // registers (a tail tile or the end of the range is handled
                // right after: the stage is not read before the barrier).
                mxb = step_b<FMT, NW, 1>(pf, st + va_off, 0, o, sb, regs, wst, wsb);
                store_mask<NW, MASK>(regs, wst);
                if (!g.full || mw != ALL_KEYS) mxb = mask_raw(sb, 1, half, lim_of(g), mw);
                if (write && !gw.cache) store_tail_k<NW, MASK>(tregs, wst);
                const int nf = fetch && gf.cache ? gf.count : 0;  // 0: no fetch (zeros)
                load_k<NW, MASK>(lo, regs, tile_base(p, b, h, gf.first, nf), nf);
                if (fetch && !gf.cache) load_tail_k<NW, MASK>(p, b, h, gf.first, gf.count, tregs);

                // ---- half 1 (on the last tile the S block of "tile t + 1" reads
                // stale LDS; its result is never used)
                rebase(mxb, c, run, o);
                sa = step_a(sb, c, run.nm, run.l, pf, st1 + ka_off, qf);
                mxa = step_b<FMT, NW, 2>(pf, st + va_off, 1, o, sa, regs, wst, wsb);
                if (!gn.full || mwn != ALL_KEYS) mxa = mask_raw(sa, 0, half, lim_of(gn), mwn);
                if (write && !gw.cache) store_tail_v<NW>(tregs, wst);
                // (without a fetch: zeros into a scale buffer no write reads)
                if (threadIdx.x < 2 * BKV) sbuf[((u + NS) & 1) * SB_FLOATS + threadIdx.x] = regs.s;
                load_v<NW>(lo, regs, tile_base(p, b, h, gf.first, nf));
                if (fetch && !gf.cache) load_tail_v<NW>(p, b, h, gf.first, gf.count, tregs);
                __syncthreads();
                g = gn;
                mw = mwn;
            }
        }
    }
    const float l = run.l + __shfl_xor(run.l, 32, 64);
    const float m = run.m;

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
            if (half == 0) *reinterpret_cast<float2*>(p.ws_ml + qi * 2) = make_float2(m, l);
        }
        return;
    }
    if (qvalid) {
        const float inv = l > 0.0f ? 1.0f / l : 0.0f;
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
// 8 (batch, head, query) rows per 256-thread block, 32 threads per row, each
// owning 4 consecutive dimensions: 16-byte loads of the partials and one
// 8-byte store. Every element is the same chain of operations in split order
// as with one thread per dimension, so the result does not depend on the
// block shape.
constexpr int COMBINE_ROWS = 8;
__global__ __launch_bounds__(256) void attn_combine_kernel(const float* __restrict__ ws_o,
                                                           const float* __restrict__ ws_ml,
                                                           int splits, int64_t rows_per_split,
                                                           int64_t Lq, int64_t H, uint16_t* out,
                                                           int64_t os0, int64_t os1, int64_t os2) {
    const int64_t r = (int64_t)blockIdx.x * COMBINE_ROWS + (threadIdx.x >> 5);  // (b * H + h) * Lq + q
    if (r >= rows_per_split) return;
    const int d = (threadIdx.x & 31) * 4;
    float M = -INFINITY;
    for (int sp = 0; sp < splits; ++sp) M = fmaxf(M, ws_ml[(sp * rows_per_split + r) * 2]);
    const float Muse = M == -INFINITY ? 0.0f : M;
    float den = 0.0f;
    float num[4] = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll 4
    for (int sp = 0; sp < splits; ++sp) {
        const int64_t idx = sp * rows_per_split + r;
        const float2 ml = *reinterpret_cast<const float2*>(ws_ml + idx * 2);
        const float4 ov = *reinterpret_cast<const float4*>(ws_o + idx * D + d);
        const float wgt = __builtin_amdgcn_exp2f(ml.x - Muse);
        den = fmaf(wgt, ml.y, den);
        num[0] = fmaf(wgt, ov.x, num[0]);
        num[1] = fmaf(wgt, ov.y, num[1]);
        num[2] = fmaf(wgt, ov.z, num[2]);
        num[3] = fmaf(wgt, ov.w, num[3]);
    }
    const int64_t q = r % Lq, h = (r / Lq) % H, b = r / (Lq * H);
    uint32_t o[4];
#pragma unroll
    for (int e = 0; e < 4; ++e) o[e] = f32_to_bf16_bits(den > 0.0f ? num[e] / den : 0.0f);
    *reinterpret_cast<uint2*>(out + b * os0 + q * os1 + h * os2 + d) =
        make_uint2(o[0] | (o[1] << 16), o[2] | (o[3] << 16));
}

}  // namespace attn
}  // namespace hn

using namespace hn;

// Split selection for the 4-wave kernel: a launch wants at least two
// workgroups per CU (two fit per CU by LDS and registers). When (batch x heads
// x query tiles) falls short, the key range of each query tile is split so
// that the grid fills the device (the decode-style case: a few hundred
// queries over a long cache); each split keeps at least 16 key tiles.
static int attn_splits(int64_t B, int64_t Lq, int64_t H, int64_t kv_len, int64_t cur_len, int cus) {
    const int64_t work = B * H * ((Lq + attn::Shape<4>::BQ - 1) / attn::Shape<4>::BQ);
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

// Launch plan: query rows [0, rows8) go to the 8-wave kernel (whole 256-query
// tiles, no key split), rows [rows8, Lq) to the 4-wave kernel with `splits`
// key-range splits.
//
// Model, in units of one full round of 4-wave workgroups (2 per CU, 128
// queries each, which takes as long per key tile as one round of 8-wave
// workgroups, 1 per CU, 256 queries each -- the 8-wave round measures 0.92 of
// it at 86400 keys, so K8_ROUND = 0.92):
//   4-wave only: ceil(n4 / 2C) rounds, n4 = B H ceil(Lq / 128);
//   8-wave over k tiles of 256 rows per (batch, head): ceil(B H k / C)
//                K8_ROUND rounds, plus the other Lq - 256 k rows on the
//                4-wave kernel, split sp ways: ceil(nr sp / 2C) / sp rounds.
// Every k from floor(Lq / 256) down is tried, so that a few rows past a
// whole number of 8-wave rounds (a chunk's text tokens beside its 10 800
// image tokens: 43 tiles x 24 heads = 4.03 rounds, i.e. 5) go to the split
// 4-wave launch instead of a nearly empty extra round. The 8-wave kernel is
// used only when it fills every CU at least once (B H k >= C) and the model
// says it is faster: a partial last round of 1-per-CU workgroups idles half
// the SIMD slots a 4-wave round would keep busy.
struct AttnPlan {
    int64_t rows8;
    int splits;
};

static AttnPlan attn_plan(int64_t B, int64_t Lq, int64_t H, int64_t kv_len, int64_t cur_len) {
    constexpr double K8_ROUND = 0.92;
    const int cus = device_cus();
    AttnPlan plan{0, 1};
    const int64_t bh = B * H;
    const int64_t n4 = bh * ((Lq + attn::Shape<4>::BQ - 1) / attn::Shape<4>::BQ);
    double best = (double)((n4 + 2 * cus - 1) / (2 * cus));
    for (int64_t k = Lq / attn::Shape<8>::BQ; k > 0 && bh * k >= cus; --k) {
        const int64_t n8 = bh * k;
        double r8 = K8_ROUND * (double)((n8 + cus - 1) / cus);
        const int64_t rows8 = k * attn::Shape<8>::BQ;
        const int64_t rest = Lq - rows8;
        if (rest > 0) {
            const int sp = attn_splits(B, rest, H, kv_len, cur_len, cus);
            const int64_t nr = bh * ((rest + attn::Shape<4>::BQ - 1) / attn::Shape<4>::BQ) * sp;
            r8 += (double)((nr + 2 * cus - 1) / (2 * cus)) / sp;
        }
        if (r8 < best) {
            best = r8;
            plan.rows8 = rows8;
        }
        if (r8 > best + 1.0) break;  // fewer tiles only add 4-wave rounds from here
    }
    plan.splits = attn_splits(B, Lq - plan.rows8, H, kv_len, cur_len, cus);
    return plan;
}

static int64_t plan_workspace(const AttnPlan& plan, int64_t B, int64_t Lq, int64_t H) {
    if (plan.splits <= 1) return 0;
    return (int64_t)plan.splits * B * H * (Lq - plan.rows8) * (attn::D + 2) * (int64_t)sizeof(float);
}

extern "C" int64_t hn_attn_fp8kv_workspace_size(int64_t B, int64_t Lq, int64_t H, int64_t D,
                                                int64_t kv_len, int64_t cur_len) {
    if (B <= 0 || Lq <= 0 || H <= 0 || D != attn::D || kv_len < 0 || cur_len < 0) return 0;
    return plan_workspace(attn_plan(B, Lq, H, kv_len, cur_len), B, Lq, H);
}

// The kernel instantiation for the format, with or without key-validity masks.
template <int NW, bool MASK>
static void launch_kernel(const attn::Params& p, dim3 grid, hipStream_t stream) {
    if (p.fmt == HN_KV_FP8)
        attn::attn_fp8kv_kernel<HN_KV_FP8, NW, MASK><<<grid, attn::Shape<NW>::NT, 0, stream>>>(p);
    else
        attn::attn_fp8kv_kernel<HN_KV_INT8, NW, MASK><<<grid, attn::Shape<NW>::NT, 0, stream>>>(p);
}


// One launch of the NW-wave kernel over query rows [row0, row0 + rows) of p's
// problem (p.Lq = all rows), with `sp` key-range splits merged through the
// workspace by attn_combine_kernel.
template <int NW>
static int launch_rows(attn::Params p, int64_t B, int64_t row0, int64_t rows, int sp, void* workspace,
                       hipStream_t stream) {
    constexpr int BQ = attn::Shape<NW>::BQ;
    p.q += row0 * p.qs1;
    p.out += row0 * p.os1;
    p.q_pos0 += row0;
    p.Lq = rows;
    const int64_t qt = (rows + BQ - 1) / BQ;
    const int64_t work = B * p.H * qt * sp;
    HN_REQUIRE(work <= 0x3fffffffLL, HN_E_ARG, "hn_attn_fp8kv: too much work for one launch");
    p.q_tiles = (int)qt;
    p.splits = sp;
    p.work = (int)work;
    p.per_xcd = (int)((work + 7) / 8);
    p.ws_o = sp > 1 ? (float*)workspace : nullptr;
    p.ws_ml = sp > 1 ? (float*)workspace + (int64_t)sp * B * p.H * rows * attn::D : nullptr;
    const dim3 grid((unsigned)(8 * (int64_t)p.per_xcd));
    if (p.kvalid || p.uvalid) launch_kernel<NW, true>(p, grid, stream);
    else launch_kernel<NW, false>(p, grid, stream);
    int rc = check_launch("hn_attn_fp8kv");
    if (rc != HN_OK || sp <= 1) return rc;
    const int64_t nrows = B * p.H * rows;
    HN_REQUIRE(nrows <= 0x7fffffffLL, HN_E_ARG, "hn_attn_fp8kv: too many rows to combine");
    attn::attn_combine_kernel<<<(unsigned)((nrows + attn::COMBINE_ROWS - 1) / attn::COMBINE_ROWS), 256, 0, stream>>>(
        p.ws_o, p.ws_ml, sp, nrows, rows, p.H, p.out, p.os0, p.os1, p.os2);
    return check_launch("hn_attn_fp8kv (combine)");
}

// Argument checks and parameter block shared by the attention entry points.
// Returns HN_OK with *pp and *plan filled, or an error code (nothing enqueued).
static int attn_setup(int fmt, const void* q, const int64_t* qs, int64_t B, int64_t Lq, int64_t H,
                      int64_t D, const void* kc, const void* vc, const int64_t* cs, const float* ks,
                      const float* vs, const int64_t* ss, int64_t cache_cap, int64_t kv_len,
                      const uint8_t* cache_valid, int64_t cvs, const void* kcur, const void* vcur,
                      const int64_t* curs, int64_t cur_len, const uint8_t* cur_valid, int64_t uvs,
                      int64_t q_pos0, int64_t chunk_len, float softmax_scale, void* out,
                      const int64_t* os, attn::Params* pp, AttnPlan* plan, bool* empty) {
    HN_REQUIRE(fmt == HN_KV_FP8 || fmt == HN_KV_INT8, HN_E_ARG, "hn_attn_fp8kv: unknown KV format");
    HN_REQUIRE(D == attn::D, HN_E_ARG, "hn_attn_fp8kv: head dim must be 128");
    HN_REQUIRE(B >= 0 && Lq >= 0 && H > 0 && kv_len >= 0 && cur_len >= 0 && q_pos0 >= 0, HN_E_ARG,
               "hn_attn_fp8kv: invalid shape");
    HN_REQUIRE(kv_len <= cache_cap, HN_E_ARG, "hn_attn_fp8kv: kv_len exceeds the cache capacity");
    HN_REQUIRE(softmax_scale > 0.0f && softmax_scale <= 3.4028234e38f, HN_E_ARG,
               "hn_attn_fp8kv: softmax_scale must be finite and positive");
    HN_REQUIRE(cvs >= 0 && uvs >= 0, HN_E_ARG, "hn_attn_fp8kv: negative validity stride");
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
        HN_REQUIRE(cs[0] >= 0 && cs[1] > 0 && cs[2] >= 0 && ss[0] >= 0 && ss[1] > 0 && ss[2] >= 0,
                   HN_E_ARG, "hn_attn_fp8kv: invalid cache strides");
        HN_REQUIRE(aligned(kc, 16) && aligned(vc, 16), HN_E_ARG, "hn_attn_fp8kv: cache misaligned");
    }
    if (cur_len > 0) {
        HN_REQUIRE(kcur && vcur, HN_E_ARG, "hn_attn_fp8kv: null tail pointer");
        HN_REQUIRE(curs[3] == 1 && curs[0] % 8 == 0 && curs[1] % 8 == 0 && curs[2] % 8 == 0,
                   HN_E_ARG, "hn_attn_fp8kv: tail strides must be multiples of 8");
        HN_REQUIRE(aligned(kcur, 16) && aligned(vcur, 16), HN_E_ARG, "hn_attn_fp8kv: tail misaligned");
    }
    *empty = B == 0 || Lq == 0;
    if (*empty) return HN_OK;
    HN_REQUIRE(out && q, HN_E_ARG, "hn_attn_fp8kv: null q/out");
    const int rc = require_gfx950("hn_attn_fp8kv");
    if (rc != HN_OK) return rc;
    attn::Params& p = *pp;
    p.q = (const uint16_t*)q;
    p.kc = (const uint8_t*)kc; p.vc = (const uint8_t*)vc;
    p.ks = ks; p.vs = vs;
    p.kcur = (const uint16_t*)kcur; p.vcur = (const uint16_t*)vcur;
    p.out = (uint16_t*)out;
    p.kvalid = kv_len > 0 ? cache_valid : nullptr;
    p.uvalid = cur_len > 0 ? cur_valid : nullptr;
    p.kvs = cvs; p.uvs = uvs;
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
    *plan = attn_plan(B, Lq, H, kv_len, cur_len);
    return HN_OK;
}

static int attn_run(const attn::Params& p, const AttnPlan& plan, int64_t B, int64_t Lq, void* workspace,
                    hipStream_t st) {
    if (plan.rows8 > 0) {
        const int rc = launch_rows<8>(p, B, 0, plan.rows8, 1, nullptr, st);
        if (rc != HN_OK || plan.rows8 == Lq) return rc;
    }
    return launch_rows<4>(p, B, plan.rows8, Lq - plan.rows8, plan.splits, workspace, st);
}

extern "C" int hn_attn_fp8kv(int fmt, const void* q, const int64_t* qs, int64_t B, int64_t Lq,
                             int64_t H, int64_t D, const void* kc, const void* vc,
                             const int64_t* cs, const float* ks, const float* vs,
                             const int64_t* ss, int64_t cache_cap, int64_t kv_len,
                             const uint8_t* cache_valid, int64_t cache_valid_stride,
                             const void* kcur, const void* vcur, const int64_t* curs,
                             int64_t cur_len, const uint8_t* cur_valid, int64_t cur_valid_stride,
                             int64_t q_pos0, int64_t chunk_len, float softmax_scale, void* out,
                             const int64_t* os, void* workspace, int64_t workspace_bytes,
                             void* stream) {
    attn::Params p;
    AttnPlan plan;
    bool empty = false;
    int rc = attn_setup(fmt, q, qs, B, Lq, H, D, kc, vc, cs, ks, vs, ss, cache_cap, kv_len, cache_valid,
                        cache_valid_stride, kcur, vcur, curs, cur_len, cur_valid, cur_valid_stride, q_pos0,
                        chunk_len, softmax_scale, out, os, &p, &plan, &empty);
    if (rc != HN_OK || empty) return rc;
    const int64_t need = plan_workspace(plan, B, Lq, H);
    HN_REQUIRE(workspace_bytes >= need && (need == 0 || (workspace && aligned(workspace, 16))), HN_E_ARG,
               "hn_attn_fp8kv: workspace smaller than hn_attn_fp8kv_workspace_size() or misaligned");
    return attn_run(p, plan, B, Lq, workspace, (hipStream_t)stream);
}

// ---------------------------------------------------------------------------
// hn_attn_fp8kv_noalloc: hn_attn_fp8kv with the split-key workspace in a
// file-scope device array, for callers that cannot allocate. Each GPU holds
// its own copy of `scratch` until the process ends. Host code never passes the
// array's name (a host-side stand-in) to a kernel: the device address comes
// from hipGetSymbolAddress, looked up once per device with that device current.
// Every call on a device shares its scratch, so calls that overlap on one GPU
// race; the kernels write every partial they read, so nothing needs clearing.
// Size: a split launch keeps at most 2 workgroups per CU in one round, each
// with 128 query rows of (128 + 2) fp32 partials, so a call needs at most
// 2 * CUs * 128 * 130 * 4 bytes: 34.1 MB on MI355X's 256 CUs.
constexpr int64_t NOALLOC_SCRATCH_BYTES = 40ll << 20;
static __device__ __align__(256) uint8_t scratch[NOALLOC_SCRATCH_BYTES];

static std::mutex g_scratch_mu;
static void* g_scratch_ptr[64] = {};

static int scratch_for_current_device(void** out) {
    int dev = -1;
    if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) {
        (void)hipGetLastError();
        return fail(HN_E_DEVICE, "hn_attn_fp8kv_noalloc: no usable current device");
    }
    std::lock_guard<std::mutex> lock(g_scratch_mu);
    if (g_scratch_ptr[dev] == nullptr) {
        void* ptr = nullptr;
        const hipError_t e = hipGetSymbolAddress(&ptr, HIP_SYMBOL(scratch));
        if (e != hipSuccess || ptr == nullptr) {
            (void)hipGetLastError();
            set_error("hn_attn_fp8kv_noalloc: hipGetSymbolAddress of the scratch array failed on device %d: %s",
                      dev, hipGetErrorString(e));
            return HN_E_DEVICE;
        }
        g_scratch_ptr[dev] = ptr;
    }
    *out = g_scratch_ptr[dev];
    return HN_OK;
}

extern "C" int64_t hn_attn_fp8kv_noalloc_scratch_bytes(void) { return NOALLOC_SCRATCH_BYTES; }

extern "C" int hn_attn_fp8kv_noalloc(int fmt, const void* q, const int64_t* qs, int64_t B, int64_t Lq,
                                     int64_t H, int64_t D, const void* kc, const void* vc,
                                     const int64_t* cs, const float* ks, const float* vs,
                                     const int64_t* ss, int64_t cache_cap, int64_t kv_len,
                                     const uint8_t* cache_valid, int64_t cache_valid_stride,
                                     const void* kcur, const void* vcur, const int64_t* curs,
                                     int64_t cur_len, const uint8_t* cur_valid,
                                     int64_t cur_valid_stride, int64_t q_pos0, int64_t chunk_len,
                                     float softmax_scale, void* out, const int64_t* os,
                                     void* stream) {
    attn::Params p;
    AttnPlan plan;
    bool empty = false;
    int rc = attn_setup(fmt, q, qs, B, Lq, H, D, kc, vc, cs, ks, vs, ss, cache_cap, kv_len, cache_valid,
                        cache_valid_stride, kcur, vcur, curs, cur_len, cur_valid, cur_valid_stride, q_pos0,
                        chunk_len, softmax_scale, out, os, &p, &plan, &empty);
    if (rc != HN_OK || empty) return rc;
    const int64_t need = plan_workspace(plan, B, Lq, H);
    if (need > NOALLOC_SCRATCH_BYTES) {
        set_error("hn_attn_fp8kv_noalloc: these sizes need %lld bytes of split-key scratch, more than the "
                  "%lld the library holds per device; call hn_attn_fp8kv with a workspace",
                  (long long)need, (long long)NOALLOC_SCRATCH_BYTES);
        return HN_E_ARG;
    }
    void* ws = nullptr;
    if (need > 0) {
        rc = scratch_for_current_device(&ws);
        if (rc != HN_OK) return rc;
    }
    return attn_run(p, plan, B, Lq, ws, (hipStream_t)stream);
}
