// FP8 (OCP e4m3) GEMM for gfx950 with fp32 accumulation on the CDNA4
// f8f6f4 matrix cores (v_mfma_f32_32x32x64_f8f6f4).
//
//   out[m, n] = epilogue( sum_k a[m, k] * b[n, k] )
//
// a: activations [M, K] and b: weights [N, K], both K-contiguous e4m3 (the
// nn.Linear weight layout). Two scale modes:
//   ROWCOL    per-token x per-output-channel scales, bias and optional
//             GELU-tanh fused in the epilogue (gemm_rowcol_oe_kernel, a
//             persistent 4-wave kernel; gemm_rowcol_kernel for short K);
//   BLOCKWISE 128x128 block scales on both operands (the decoder contract):
//             each 128-wide K step is promoted with its own sa * sb factor
//             (gemm_bw8_kernel, 8 waves).
//
// Tiling: a workgroup owns a 256 x 256 output tile; with 4 waves (2 x 2) each
// wave owns 128 x 128 = 4 x 4 MFMA blocks of 32 x 32 (256 fp32 accumulators
// per lane), with 8 waves (2 x 4) 128 x 64. K advances 128 bytes per step
// through LDS buffers filled by direct global -> LDS loads. Rows are 128
// bytes in LDS with their eight 16-byte chunks XOR-swizzled (swz_pos), so the
// 16-byte fragment reads of consecutive rows hit distinct bank groups.
//
// The MFMA's first operand is the weight tile and its second the activation
// tile, i.e. the wave computes out^T: each lane then holds four consecutive
// output columns n..n+3 of one row m and stores them as one 8-byte write.
#include <cstdlib>
#include <type_traits>

#include "hn_capi_internal.h"
#include "hn_common.h"
#include "gemm_dma.h"

namespace hn {
namespace gemm {

constexpr int BM = 256, BN = 256, BK = 128;
constexpr int NT = 256;
constexpr int TILE_BYTES = BM * BK;         // one operand tile, 32 KB
constexpr int STAGE_BYTES = 2 * TILE_BYTES;  // A + B

enum Mode { ROWCOL = 0, BLOCKWISE = 1 };
// Epilogue staging: each wave's 128 x 128 bf16 result, rows padded to 272 B so
// the 16-byte row reads of the store pass are conflict-free.
constexpr int OUT_ROW = 128 * 2 + 16;
constexpr int OUT_WAVE_BYTES = 128 * OUT_ROW;
constexpr int SMEM_BYTES = (4 * OUT_WAVE_BYTES > 2 * STAGE_BYTES) ? 4 * OUT_WAVE_BYTES : 2 * STAGE_BYTES;
constexpr int kMaxKT = 256;  // K <= 32768

struct Params {
    const uint8_t* a;
    const uint8_t* b;
    const float* sa;
    const float* sb;
    const uint16_t* bias;
    uint16_t* out;
    int64_t M, N, K, ldc;
    int act;
    int tiles_m, tiles_n;
    int per_xcd;  // work items per XCD (grid = 8 * per_xcd)
    // Row/column kernel order: the tiles_full = tm_full * tn_full tiles that
    // lie wholly inside M x N come first, then the tiles_part edge tiles
    // (the last row stripe if M % 256 != 0, then the last column stripe if
    // N % 256 != 0); each class is split evenly over the 8 XCDs.
    int tm_full, tn_full, tiles_full, tiles_part, m_tail;
    // Tile width in columns: 256, except in the persistent row/column kernel,
    // which takes 192 when a launch has fewer 256-wide tiles than CUs and
    // more, still at most one per CU, at 192 (its WC template argument).
    int bn;
    // Persistent kernel: rows [M, tail_M) (tail_M > M only when the tail
    // stripe rides on the light workgroups, tail_wide) in items of tail_cols
    // columns, item i for light workgroup i.
    int64_t tail_M;
    int tail_cols;
};

// 16-byte chunk c of LDS row r lives at chunk position c ^ ((r >> 1) & 7).
// gfx950 serves a 16-byte LDS read 16 lanes at a time across 64 banks
// (256 bytes): the 16 lanes of a fragment read hit 16 consecutive rows at one
// logical chunk, and with 128-byte rows the bank group of (r, c) is
// 8 (r & 1) + position, so the swizzle must spread rows of equal parity --
// hence (r >> 1), not r.
HN_DEVICE int swz(int row, int chunk) { return row * BK + (swz_pos(row, chunk) << 4); }

// Direct global -> LDS loads of one operand tile (global_load_lds_dwordx4:
// 16 bytes per lane, written at M0 + 16 * lane). Each wave fills 8 regions of
// 1 KB = 8 rows; a lane's bytes land at row lane / 8, physical chunk lane % 8,
// so the lane fetches the logical chunk the swizzle puts there. Rows past the operand's end are clamped to its last row: the
// loads stay in bounds and the rows they fill are never stored.
//
// The load is issued from inline asm so the compiler does not track its LDS
// write: it would otherwise wait for every DMA in flight before any LDS read,
// serialising the prefetch of stage s^1 behind the MFMAs on stage s. The
// kernel instead waits explicitly (vmcnt(0) + barrier) at the end of each K
// step, and its K loop issues no other vector-memory loads.
HN_DEVICE void dma_16B(const uint8_t* gsrc, uint32_t lds_addr) {
    asm volatile(
        "s_mov_b32 m0, %1\n\t"
        "global_load_lds_dwordx4 %0, off"
        :
        : "v"(gsrc), "s"(lds_addr)
        : "memory", "m0");
}

HN_DEVICE uint32_t lds_addr(const void* p) {
    return (uint32_t)(uintptr_t)(const __attribute__((address_space(3))) void*)p;
}

// One 32 x 64 fragment: lane l reads row (l % 32) of the block and the 32
// bytes [32 (l / 32), +32) of the 64-byte K slice `kh`. A and B use the same
// lane -> K mapping, so any order of K inside a slice gives the same sum.
HN_DEVICE i32x8 read_frag(const uint8_t* lds, int row, int kh, int lane) {
    const int c0 = kh * 4 + (lane >> 5) * 2;
    const uint4 lo = *reinterpret_cast<const uint4*>(lds + swz(row, c0));
    const uint4 hi = *reinterpret_cast<const uint4*>(lds + swz(row, c0 + 1));
    i32x8 f;
    f[0] = lo.x; f[1] = lo.y; f[2] = lo.z; f[3] = lo.w;
    f[4] = hi.x; f[5] = hi.y; f[6] = hi.z; f[7] = hi.w;
    return f;
}

HN_DEVICE f32x16 mfma(const i32x8& a, const i32x8& b, const f32x16& c) {
    return __builtin_amdgcn_mfma_scale_f32_32x32x64_f8f6f4(a, b, c, 0, 0, 0, 0, 0, 0);
}

// The eight fragments (4 weight blocks, 4 activation blocks) of one 64-byte
// K slice of a stage, for the wave's 128 x 128 sub-tile.
struct Frags {
    i32x8 b[4];
    i32x8 a[4];
};

HN_DEVICE void mfma_slice(f32x16 (&acc)[4][4], const Frags& f) {
#pragma unroll
    for (int i = 0; i < 4; ++i)
#pragma unroll
        for (int j = 0; j < 4; ++j) acc[i][j] = mfma(f.b[i], f.a[j], acc[i][j]);
}

// Interleave the 16 LDS reads of the next slice with this slice's 16 MFMAs.
HN_DEVICE void interleave_reads_with_mfma() {
#pragma unroll
    for (int i = 0; i < 16; ++i) {
        __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);  // one DS read
        __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);  // one MFMA
    }
}

HN_DEVICE float gelu_tanh(float x) {
    // 0.5 x (1 + tanh(u)) with u = sqrt(2/pi) (x + 0.044715 x^3), written as
    // x * sigmoid(2u) = x / (1 + 2^t), t = -2 u log2(e) = x (c0 + c1 x^2), on
    // v_exp_f32 / v_rcp_f32 (about 1 ulp each: far below the bf16 output's
    // rounding). Saturates correctly: x -> -inf gives 2^t = inf and -0;
    // x -> +inf gives 2^t = 0 and x.
    constexpr float c0 = -2.0f * 0.7978845608028654f * 1.4426950408889634f;
    constexpr float c1 = c0 * 0.044715f;
    const float t = x * fmaf(c1, x * x, c0);
    return x * __builtin_amdgcn_rcpf(1.0f + __builtin_amdgcn_exp2f(t));
}

typedef float f32x2_t __attribute__((ext_vector_type(2)));
HN_DEVICE uint32_t pack_bf16(float a, float b) {
    const f32x2_t f = {a, b};
    return __builtin_bit_cast(uint32_t, __builtin_convertvector(f, bf16x2));
}

// Epilogue shared by the kernels. acc[i][j][v] holds out^T for n = wn*128 +
// 32 i + 8 (v/4) + 4 (lane/32) + v%4 and m = wm*128 + 32 j + lane%32
// (tile-local). Each wave scales its 128 x 128 sub-tile, packs it to bf16 and
// parks it in its own LDS slice; then it writes the slice out as 256-byte row
// segments (16 lanes x 16 bytes per row, 4 rows per store).
//
// The per-row / per-column scales and the bias the lane needs (4 + 16 x 4 +
// 16 x 4 values) are loaded in one batch up front: with one wave per SIMD
// nothing else hides a load's latency, so loading them group by group would
// expose it sixteen times.
template <int MODE, int ACT>
HN_DEVICE void epilogue_act(f32x16 (&acc)[4][4], const Params& p, int64_t m0, int64_t n0, uint8_t* smem,
                            int wave, int wm, int wn, int lane, int imax, int jmax) {
    float sam[4];
#pragma unroll
    for (int j = 0; j < 4; ++j) {
        int64_t m = m0 + wm * 128 + j * 32 + (lane & 31);
        m = m < p.M ? m : p.M - 1;
        sam[j] = MODE == ROWCOL ? p.sa[m] : 1.0f;
    }
    float4 sbn[4][4];
    uint2 bias[4][4];
#pragma unroll
    for (int i = 0; i < 4; ++i)
#pragma unroll
        for (int vq = 0; vq < 4; ++vq) {
            int64_t n = n0 + wn * 128 + i * 32 + vq * 8 + (lane >> 5) * 4;
            n = n < p.N ? n : p.N - 4;  // stays in bounds; columns past N are not stored
            sbn[i][vq] = make_float4(1.0f, 1.0f, 1.0f, 1.0f);
            bias[i][vq] = make_uint2(0u, 0u);
            if (MODE == ROWCOL) {
                sbn[i][vq] = *reinterpret_cast<const float4*>(p.sb + n);
                if (p.bias) bias[i][vq] = *reinterpret_cast<const uint2*>(p.bias + n);
            }
        }
    __syncthreads();  // the last K step's LDS reads are done (all waves)
    uint8_t* ow = smem + wave * OUT_WAVE_BYTES;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        if (i >= imax) continue;  // weight block wholly past N (wave-uniform)
#pragma unroll
        for (int vq = 0; vq < 4; ++vq) {
            const float sb4[4] = {sbn[i][vq].x, sbn[i][vq].y, sbn[i][vq].z, sbn[i][vq].w};
            const uint2 bb = bias[i][vq];
            const float bn[4] = {bf16_bits_to_f32(bb.x & 0xffffu), bf16_bits_to_f32(bb.x >> 16),
                                 bf16_bits_to_f32(bb.y & 0xffffu), bf16_bits_to_f32(bb.y >> 16)};
            const int nl = i * 32 + vq * 8 + (lane >> 5) * 4;
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                if (j >= jmax) continue;  // activation block wholly past M (wave-uniform)
                float y[4];
#pragma unroll
                for (int e = 0; e < 4; ++e) {
                    y[e] = fmaf(acc[i][j][vq * 4 + e], sam[j] * sb4[e], bn[e]);
                    if (ACT == HN_ACT_GELU_TANH) y[e] = gelu_tanh(y[e]);
                }
                const int ml = j * 32 + (lane & 31);
                *reinterpret_cast<uint2*>(ow + ml * OUT_ROW + nl * 2) =
                    make_uint2(pack_bf16(y[0], y[1]), pack_bf16(y[2], y[3]));
            }
        }
    }
    // Each wave reads back only its own slice: no barrier needed beyond the
    // wave's own LDS ordering.
    __builtin_amdgcn_s_waitcnt(0);
    const int64_t nbase = n0 + wn * 128 + (lane & 15) * 8;
#pragma unroll 4
    for (int r = 0; r < 32; ++r) {
        const int ml = r * 4 + (lane >> 4);
        const int64_t m = m0 + wm * 128 + ml;
        const uint4 v = *reinterpret_cast<const uint4*>(ow + ml * OUT_ROW + (lane & 15) * 16);
        if (m < p.M && nbase < p.N) *reinterpret_cast<uint4*>(p.out + m * p.ldc + nbase) = v;
    }
}

template <int MODE>
HN_DEVICE void epilogue(f32x16 (&acc)[4][4], const Params& p, int64_t m0, int64_t n0, uint8_t* smem,
                        int wave, int wm, int wn, int lane, int imax = 4, int jmax = 4) {
    if (MODE == ROWCOL && p.act == HN_ACT_GELU_TANH)
        epilogue_act<MODE, HN_ACT_GELU_TANH>(acc, p, m0, n0, smem, wave, wm, wn, lane, imax, jmax);
    else
        epilogue_act<MODE, HN_ACT_NONE>(acc, p, m0, n0, smem, wave, wm, wn, lane, imax, jmax);
}

// ---------------------------------------------------------------------------
// Row/column-scaled kernel: 128-byte K steps through five single-operand LDS
// buffers.
//
// The stage DMA costs per cache line touched: one CU moves a 32 KB stage of
// 128-byte row segments in about 810 cycles, but one of 64-byte segments (half
// lines) in about 1360 -- more than the 1024 MFMA cycles a 64-byte K step of a
// 256 x 256 tile takes. So every LDS buffer holds whole lines: one operand's
// 256 rows x 128 bytes (32 KB, 16-byte chunks swizzled as swz()). Five buffers
// fill the 160 KB of LDS; load L(i) -- A of K step i / 2 for even i, B for odd
// i -- goes to buffer i % 5.
//
// K step k (128 bytes) runs as two halves of 16 MFMAs, one per 64-byte K slice,
// each interleaved with the 16 LDS reads of the next slice's fragments:
//   half 0: MFMAs on slice (k, 0); reads of slice (k, 1)
//   mid:    wait for step k + 1's buffers and barrier; step k's buffers are
//           then free (their last reads completed before the barrier)
//   half 1: MFMAs on slice (k, 1); reads of slice (k + 1, 0); the loads
//           L(2k + 5) = B(k + 2) and L(2k + 6) = A(k + 3) into step k's
//           buffers, one 1 KB DMA per MFMA
// B of a step is requested about one step (32 MFMAs) before its wait, A two
// steps; with that lead the waits measure ~0 cycles per tile.
constexpr int R_BUFS = 5;
constexpr int R_BUF = BM * BK;            // one operand of one K step, 32 KB
constexpr int R_SMEM = R_BUFS * R_BUF;    // 160 KB
static_assert(R_SMEM >= 4 * OUT_WAVE_BYTES, "epilogue staging must fit in the stage buffers");

// Stage loads use global_load_lds with a scalar base: the address is
// sbase (SGPR pair: operand + tile row0 * K + k0) + voff (per-lane 32-bit
// offset of the lane's row and chunk inside the tile, fixed for the tile), and
// the LDS destination M0 is scalar too. Issuing a 1 KB load is then one s_mov
// and the load -- no per-load vector address arithmetic or readfirstlane.
HN_DEVICE void dma_16B_sbase(const uint8_t* sbase, uint32_t voff, uint32_t lds) {
    asm volatile(
        "s_mov_b32 m0, %2\n\t"
        "global_load_lds_dwordx4 %0, %1"
        :
        : "v"(voff), "s"(sbase), "s"(lds)
        : "memory", "m0");
}

// Per-lane offsets of a wave's eight 1 KB regions (8 rows of 128 bytes) of one
// 256 x 128 buffer. Lane l lands at row l / 8, physical chunk l % 8 of region
// wave * 8 + q and fetches the logical chunk that position holds (the swizzle
// is an involution). Rows past the operand's end are clamped to its last row:
// in bounds, never stored.
HN_DEVICE void buffer_offsets(uint32_t (&off)[8], int64_t row0, int64_t rows, int64_t K, int wave, int lane) {
#pragma unroll
    for (int q = 0; q < 8; ++q) {
        const int r = (wave * 8 + q) * 8 + (lane >> 3);
        const int c = swz_pos(r, lane & 7);
        const int64_t row = row0 + r < rows ? row0 + r : rows - 1;
        off[q] = (uint32_t)((row - row0) * K + (c << 4));
    }
}

// The fragments of K slice kh of step buffers (a_buf, b_buf).
HN_DEVICE void read_slice(Frags& f, const uint8_t* a_buf, const uint8_t* b_buf, int kh, int wm, int wn,
                          int lane) {
#pragma unroll
    for (int i = 0; i < 4; ++i) f.b[i] = read_frag(b_buf, wn * 128 + i * 32 + (lane & 31), kh, lane);
#pragma unroll
    for (int j = 0; j < 4; ++j) f.a[j] = read_frag(a_buf, wm * 128 + j * 32 + (lane & 31), kh, lane);
}

// mfma_slice for an edge tile: only blocks inside the matrix (wave-uniform tests).
HN_DEVICE void mfma_slice_partial(f32x16 (&acc)[4][4], const Frags& f, int imax, int jmax) {
#pragma unroll
    for (int i = 0; i < 4; ++i)
#pragma unroll
        for (int j = 0; j < 4; ++j)
            if (i < imax && j < jmax) acc[i][j] = mfma(f.b[i], f.a[j], acc[i][j]);
}

// One workgroup per queue entry (id = x + 8 i).
HN_DEVICE bool tile_of(const Params& p, int id, int& tm, int& tn) { return tile_at(p, id & 7, id >> 3, tm, tn); }

// ---------------------------------------------------------------------------
// Blockwise-scaled kernel, 8 waves: a 512-thread workgroup owns a 256 x 256
// output tile; wave w owns rows 128 (w % 2) .. + 127 and columns 64 (w / 2)
// .. + 63, i.e. 4 x 2 MFMA blocks of 32 x 32 (128 fp32 accumulators per
// lane, held in VGPRs), two waves per SIMD. The K pipeline is the row/column
// kernel's: five single-operand 32 KB buffers, L(2 s) = A(s) and L(2 s + 1)
// = B(s) in buffer L % 5; step k's half 0 runs the MFMAs of K slice (k, 0)
// beside the reads of slice (k, 1); a mid-step wait and barrier make step
// k + 1's buffers complete and free step k's; half 1 runs slice (k, 1)
// beside the reads of slice (k + 1, 0) and the DMAs of B(k + 2) and
// A(k + 3) into step k's buffers, one 1 KB DMA per MFMA (each wave fills 4
// of a buffer's 32 regions).
//
// Scale promotion without a second accumulator set: the wave's sub-tile lies
// inside one 128 x 128 scale block of each operand, so K block k has one
// factor f_k = sa[mb][k] * sb[nb][k] for the whole sub-tile. The accumulators
// are kept in units of the current block's factor:
//     acc_k = acc_(k-1) * (f_(k-1) / f_k) + A_k B_k^T,  out = acc * f_last,
// which is sum_k f_k A_k B_k^T up to fp32 rounding of the rescale (one
// multiply per accumulator per K block, ~2^-24 relative each). A block with
// f_k = 0 contributes nothing: its MFMAs are skipped (the wave still takes
// part in every read, DMA and barrier), so f is never divided by 0. The
// rescale of an MFMA block is issued right before that block's first MFMA of
// the step, beside the previous block's MFMA.
constexpr int NT8 = 512;

// Per-lane offsets of a wave's four 1 KB regions of one 256 x 128 buffer
// (region q: 8 rows of 128 bytes; lane l lands at row 32 w + 8 q + l / 8,
// physical chunk l % 8, and fetches the logical chunk the swizzle puts
// there). Rows past the operand's end are clamped to its last row: in
// bounds, never stored.
HN_DEVICE void buffer_offsets8(uint32_t (&off)[4], int64_t row0, int64_t rows, int64_t K, int wave, int lane) {
#pragma unroll
    for (int q = 0; q < 4; ++q) {
        const int r = (wave * 4 + q) * 8 + (lane >> 3);
        const int c = swz_pos(r, lane & 7);
        const int64_t row = row0 + r < rows ? row0 + r : rows - 1;
        off[q] = (uint32_t)((row - row0) * K + (c << 4));
    }
}

// The fragments of one 64-byte K slice for the wave's 128 x 64 sub-tile.
struct Frags8 {
    i32x8 b[2];
    i32x8 a[4];
};

// Fragment t (0..5) of a slice: weight blocks b[0], b[1], then activation
// blocks a[0..3].
HN_DEVICE void read_frag8(Frags8& f, int t, const uint8_t* a_buf, const uint8_t* b_buf, int kh, int wm, int wn,
                          int lane) {
    if (t < 2) f.b[t] = read_frag(b_buf, wn * 64 + t * 32 + (lane & 31), kh, lane);
    else f.a[t - 2] = read_frag(a_buf, wm * 128 + (t - 2) * 32 + (lane & 31), kh, lane);
}

__global__ __launch_bounds__(NT8, 1) void gemm_bw8_kernel(Params p) {
    __shared__ __attribute__((aligned(16))) uint8_t smem[R_SMEM];

    // Tile order. Workgroup ids are dealt round-robin to the 8 XCDs, each with
    // its own L2, so id % 8 selects a contiguous range of work items for that
    // XCD. Work items are laid out in groups of GROUP_M tile rows, walking N
    // inside a group: the tiles an XCD runs at once then share their A and B
    // panels in that L2.
    const int w = (blockIdx.x & 7) * p.per_xcd + (blockIdx.x >> 3);
    if (w >= p.tiles_m * p.tiles_n) return;
    const int per_group = GROUP_M * p.tiles_n;
    const int first_m = (w / per_group) * GROUP_M;
    const int gm = min(GROUP_M, p.tiles_m - first_m);
    const int tm = first_m + (w % per_group) % gm;
    const int tn = (w % per_group) / gm;
    const int64_t m0 = (int64_t)tm * BM, n0 = (int64_t)tn * BN;

    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int wm = wave & 1, wn = wave >> 1;  // rows 128 wm .., columns 64 wn ..
    const int KT = (int)(p.K / BK);
    const uint8_t* const a_tile = p.a + m0 * p.K;
    const uint8_t* const b_tile = p.b + n0 * p.K;
    uint32_t off_a[4], off_b[4];
    buffer_offsets8(off_a, m0, p.M, p.K, wave, lane);
    buffer_offsets8(off_b, n0, p.N, p.K, wave, lane);
    const uint32_t lds_base = lds_addr(smem) + wave * 4 * 1024;

    // Block factors of this wave's sub-tile (0 for a sub-tile past M or N:
    // its MFMAs are skipped and it is never stored).
    // The scale rows are read through the constant address space: wave-uniform
    // loads of memory the kernel never writes become scalar loads, outside
    // the vector-memory counter that the DMA waits count.
    typedef const __attribute__((address_space(4))) float cfloat;
    const int64_t mb = (m0 >> 7) + wm, nb = (n0 >> 7) + (wn >> 1);
    const bool live = mb * 128 < p.M && nb * 128 < p.N;
    cfloat* const sa_row = (cfloat*)p.sa + (live ? mb : 0) * KT;
    cfloat* const sb_row = (cfloat*)p.sb + (live ? nb : 0) * KT;
    auto factor = [&](int k) { return live ? sa_row[k] * sb_row[k] : 0.0f; };

    f32x16 acc[2][4];  // [n block][m block]
#pragma unroll
    for (int i = 0; i < 2; ++i)
#pragma unroll
        for (int j = 0; j < 4; ++j)
#pragma unroll
            for (int v = 0; v < 16; ++v) acc[i][j][v] = 0.0f;

    auto a_buf = [&](int s) { return smem + ((2 * s) % R_BUFS) * R_BUF; };
    auto b_buf = [&](int s) { return smem + ((2 * s + 1) % R_BUFS) * R_BUF; };
    auto issue_a = [&](int s) {
        const uint32_t dst = lds_base + ((2 * s) % R_BUFS) * R_BUF;
#pragma unroll
        for (int q = 0; q < 4; ++q) dma_16B_sbase(a_tile + (int64_t)s * BK, off_a[q], dst + q * 1024);
    };
    auto issue_b = [&](int s) {
        const uint32_t dst = lds_base + ((2 * s + 1) % R_BUFS) * R_BUF;
#pragma unroll
        for (int q = 0; q < 4; ++q) dma_16B_sbase(b_tile + (int64_t)s * BK, off_b[q], dst + q * 1024);
    };
    // Prologue: L(0) .. L(4), then wait for step 0 (L(0), L(1)).
    issue_a(0);
    issue_b(0);
    if (KT > 1) {
        issue_a(1);
        issue_b(1);
        if (KT > 2) {
            issue_a(2);
            asm volatile("s_waitcnt vmcnt(12)" ::: "memory");
        } else {
            asm volatile("s_waitcnt vmcnt(8)" ::: "memory");
        }
    } else {
        asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
    }
    __syncthreads();

    Frags8 cur, nxt;
#pragma unroll
    for (int t = 0; t < 6; ++t) read_frag8(cur, t, a_buf(0), b_buf(0), 0, wm, wn, lane);
    float f_prev = 0.0f;

    // A block whose factor is 0 contributes nothing: its fragments are zeroed
    // (so its MFMAs add 0) and the rescale is 1 (the rare wave-uniform branch
    // keeps one copy of the step's code).
    auto zero = [&](Frags8& f) {
#pragma unroll
        for (int t = 0; t < 2; ++t) f.b[t] = i32x8{};
#pragma unroll
        for (int t = 0; t < 4; ++t) f.a[t] = i32x8{};
    };
    // half 0 of step k: slot s = 4 i + j rescales block (i, j) by r and
    // issues its MFMA on slice (k, 0); slots 0..5 also read fragment s of
    // slice (k, 1).
    auto half0 = [&](int k, float r) {
#pragma unroll
        for (int s8 = 0; s8 < 8; ++s8) {
            const int i = s8 >> 2, j = s8 & 3;
            if (s8 < 6) read_frag8(nxt, s8, a_buf(k), b_buf(k), 1, wm, wn, lane);
#pragma unroll
            for (int v = 0; v < 16; ++v) acc[i][j][v] *= r;
            acc[i][j] = mfma(cur.b[i], cur.a[j], acc[i][j]);
            __builtin_amdgcn_sched_barrier(0);
        }
    };
    // half 1 of step k: MFMAs on slice (k, 1); with NEXT, slots 0..5 read
    // fragment s of slice (k + 1, 0); with DB, slots 0..3 issue B(k + 2)'s
    // regions and, with DA, slots 4..7 A(k + 3)'s.
    auto half1 = [&](int k, auto next_tag, auto db_tag, auto da_tag) {
        constexpr bool NEXT = decltype(next_tag)::value;
        constexpr bool DB = decltype(db_tag)::value, DA = decltype(da_tag)::value;
        const uint32_t db = lds_base + ((2 * (k + 2) + 1) % R_BUFS) * R_BUF;
        const uint32_t da = lds_base + ((2 * (k + 3)) % R_BUFS) * R_BUF;
        const uint8_t* bsrc = b_tile + (int64_t)(k + 2) * BK;
        const uint8_t* asrc = a_tile + (int64_t)(k + 3) * BK;
#pragma unroll
        for (int s8 = 0; s8 < 8; ++s8) {
            const int i = s8 >> 2, j = s8 & 3;
            if (NEXT && s8 < 6) read_frag8(cur, s8, a_buf(k + 1), b_buf(k + 1), 0, wm, wn, lane);
            acc[i][j] = mfma(nxt.b[i], nxt.a[j], acc[i][j]);
            if (DB && s8 < 4) dma_16B_sbase(bsrc, off_b[s8], db + s8 * 1024);
            if (DA && s8 >= 4) dma_16B_sbase(asrc, off_a[s8 - 4], da + (s8 - 4) * 1024);
            __builtin_amdgcn_sched_barrier(0);
        }
    };
    using T = std::true_type;
    using F = std::false_type;
    // One step k before the last: half 0, the mid-step wait (step k + 1's
    // buffers landed in this wave: in flight after them at most A(k + 2),
    // issued in half 1 of step k - 1 or the prologue) and barrier (every
    // wave; step k's buffers free), half 1 with the DMAs DB / DA.
    float f = factor(0);
    auto step = [&](int k, auto next_tag, auto db_tag, auto da_tag) {
        const float f_next = decltype(next_tag)::value ? factor(k + 1) : 0.0f;  // scalar loads, issued early
        if (f == 0.0f) zero(cur);
        half0(k, f != 0.0f ? f_prev / f : 1.0f);
        if (f == 0.0f) zero(nxt);
        if (decltype(next_tag)::value) {
            if (decltype(db_tag)::value) asm volatile("s_waitcnt vmcnt(4)" ::: "memory");
            else asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
            __syncthreads();
        }
        half1(k, next_tag, db_tag, da_tag);
        if (f != 0.0f) f_prev = f;
        f = f_next;
    };
    int k = 0;
    for (; k + 3 < KT; ++k) step(k, T{}, T{}, T{});
    if (k + 2 < KT) step(k++, T{}, T{}, F{});
    if (k + 1 < KT) step(k++, T{}, F{}, F{});
    step(k, F{}, F{}, F{});  // k = KT - 1: nothing further to read or issue

    // Epilogue: out = acc * f_last in bf16. A lane holds 4 consecutive
    // columns of one row per (block, register quad): one 8-byte store each;
    // the 8 stores of a block write whole 64-byte row segments, which the L2
    // merges.
#pragma unroll
    for (int i = 0; i < 2; ++i)
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            const int64_t m = m0 + wm * 128 + j * 32 + (lane & 31);
#pragma unroll
            for (int vq = 0; vq < 4; ++vq) {
                const int64_t n = n0 + wn * 64 + i * 32 + vq * 8 + (lane >> 5) * 4;
                const f32x16& a = acc[i][j];
                const uint2 o = make_uint2(pack_bf16(a[4 * vq] * f_prev, a[4 * vq + 1] * f_prev),
                                           pack_bf16(a[4 * vq + 2] * f_prev, a[4 * vq + 3] * f_prev));
                if (m < p.M && n < p.N) *reinterpret_cast<uint2*>(p.out + m * p.ldc + n) = o;
            }
        }
}

__global__ __launch_bounds__(NT, 1) void gemm_rowcol_kernel(Params p) {
    __shared__ __attribute__((aligned(16))) uint8_t smem[R_SMEM];
    int tm, tn;
    if (!tile_of(p, blockIdx.x, tm, tn)) return;
    const int64_t m0 = (int64_t)tm * BM, n0 = (int64_t)tn * BN;

    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int wm = wave & 1, wn = wave >> 1;
    const int KT = (int)(p.K / BK);
    const uint8_t* const a_tile = p.a + m0 * p.K;
    const uint8_t* const b_tile = p.b + n0 * p.K;
    uint32_t off_a[8], off_b[8];
    buffer_offsets(off_a, m0, p.M, p.K, wave, lane);
    buffer_offsets(off_b, n0, p.N, p.K, wave, lane);
    const uint32_t lds_base = lds_addr(smem) + wave * 8 * 1024;
    // Blocks of this wave inside the matrix: imax weight blocks (N % 128 == 0,
    // so 0 or 4), jmax activation blocks of 32 rows. Wave-uniform.
    const int64_t rows_w = p.M - (m0 + wm * 128), cols_w = p.N - (n0 + wn * 128);
    const int jmax = rows_w >= 128 ? 4 : (rows_w <= 0 ? 0 : (int)((rows_w + 31) >> 5));
    const int imax = cols_w >= 128 ? 4 : (cols_w <= 0 ? 0 : (int)(cols_w >> 5));
    const bool whole = imax == 4 && jmax == 4;

    f32x16 acc[4][4];
#pragma unroll
    for (int i = 0; i < 4; ++i)
#pragma unroll
        for (int j = 0; j < 4; ++j)
#pragma unroll
            for (int v = 0; v < 16; ++v) acc[i][j][v] = 0.0f;

    // Buffers of step s: A in (2 s) % 5, B in (2 s + 1) % 5.
    auto a_buf = [&](int s) { return smem + ((2 * s) % R_BUFS) * R_BUF; };
    auto b_buf = [&](int s) { return smem + ((2 * s + 1) % R_BUFS) * R_BUF; };
    auto issue_a = [&](int s) {
        const uint32_t dst = lds_base + ((2 * s) % R_BUFS) * R_BUF;
#pragma unroll
        for (int q = 0; q < 8; ++q) dma_16B_sbase(a_tile + (int64_t)s * BK, off_a[q], dst + q * 1024);
    };
    auto issue_b = [&](int s) {
        const uint32_t dst = lds_base + ((2 * s + 1) % R_BUFS) * R_BUF;
#pragma unroll
        for (int q = 0; q < 8; ++q) dma_16B_sbase(b_tile + (int64_t)s * BK, off_b[q], dst + q * 1024);
    };
    // Prologue: L(0) .. L(4), then wait for step 0 (L(0), L(1)).
    issue_a(0);
    issue_b(0);
    if (KT > 1) {
        issue_a(1);
        issue_b(1);
        if (KT > 2) {
            issue_a(2);
            asm volatile("s_waitcnt vmcnt(24)" ::: "memory");
        } else {
            asm volatile("s_waitcnt vmcnt(16)" ::: "memory");
        }
    } else {
        asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
    }
    __syncthreads();

    // The K loop, instantiated for whole tiles and for edge tiles (blocks
    // outside the matrix skipped); the choice is made once per tile.
    auto kloop = [&](auto edge_tag) {
        constexpr bool EDGE = decltype(edge_tag)::value;
        Frags cur, nxt;
        auto mfmas = [&](const Frags& f) {
            if (EDGE) {
                mfma_slice_partial(acc, f, imax, jmax);
            } else {
                mfma_slice(acc, f);
                interleave_reads_with_mfma();
            }
        };
        // half 0 of step k: MFMAs on slice (k, 0), reads of slice (k, 1)
        auto half0 = [&](int k) {
            read_slice(nxt, a_buf(k), b_buf(k), 1, wm, wn, lane);
            mfmas(cur);
        };
        // half 1 of step k: MFMAs on slice (k, 1), reads of slice (k + 1, 0)
        auto half1 = [&](int k) {
            read_slice(cur, a_buf(k + 1), b_buf(k + 1), 0, wm, wn, lane);
            mfmas(nxt);
        };
        read_slice(cur, a_buf(0), b_buf(0), 0, wm, wn, lane);
        int k = 0;
        // Steady state: at the mid-step wait, A(k + 2) is still in flight.
        // Half 1 of a steady-state step with the step's 16 DMA issues spread
        // one per MFMA: a DMA issue stalls the wave while the address unit
        // takes its 1 KB, and back to back after the barrier the 16 of them
        // kept the matrix core idle for about 1000 cycles per step. Slot s
        // holds one fragment read of slice (k + 1, 0) (s < 8), MFMA s on slice
        // (k, 1) and DMA s (B(k + 2) regions, then A(k + 3) regions); the
        // sched_barrier keeps each slot's instructions together.
        auto half1_dma = [&](int k, auto with_a_tag) {
            constexpr bool WITH_A = decltype(with_a_tag)::value;
            const uint8_t* an = a_buf(k + 1);
            const uint8_t* bn = b_buf(k + 1);
            const uint32_t db = lds_base + ((2 * (k + 2) + 1) % R_BUFS) * R_BUF;
            const uint32_t da = lds_base + ((2 * (k + 3)) % R_BUFS) * R_BUF;
            const uint8_t* bsrc = b_tile + (int64_t)(k + 2) * BK;
            const uint8_t* asrc = a_tile + (int64_t)(k + 3) * BK;
#pragma unroll
            for (int s = 0; s < 16; ++s) {
                if (s < 4) cur.b[s] = read_frag(bn, wn * 128 + s * 32 + (lane & 31), 0, lane);
                else if (s < 8) cur.a[s - 4] = read_frag(an, wm * 128 + (s - 4) * 32 + (lane & 31), 0, lane);
                acc[s >> 2][s & 3] = mfma(nxt.b[s >> 2], nxt.a[s & 3], acc[s >> 2][s & 3]);
                if (s < 8) dma_16B_sbase(bsrc, off_b[s], db + s * 1024);
                else if (WITH_A) dma_16B_sbase(asrc, off_a[s - 8], da + (s - 8) * 1024);
                __builtin_amdgcn_sched_barrier(0);
            }
        };
        if constexpr (!EDGE) {
            for (; k + 3 < KT; ++k) {
                half0(k);
                asm volatile("s_waitcnt vmcnt(8)" ::: "memory");  // step k + 1 landed (this wave)
                __syncthreads();                                  // ... every wave; step k's buffers free
                half1_dma(k, std::true_type{});
            }
            if (k + 2 < KT) {
                half0(k);
                asm volatile("s_waitcnt vmcnt(8)" ::: "memory");
                __syncthreads();
                half1_dma(k, std::false_type{});
                ++k;
            }
        } else {
            for (; k + 2 < KT; ++k) {
                half0(k);
                asm volatile("s_waitcnt vmcnt(8)" ::: "memory");  // step k + 1 landed (this wave)
                __syncthreads();                                  // ... every wave; step k's buffers free
                issue_b(k + 2);
                if (k + 3 < KT) issue_a(k + 3);
                half1(k);
            }
        }
        if (k + 1 < KT) {  // k = KT - 2: nothing left to issue
            half0(k);
            asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
            __syncthreads();
            half1(k);
            ++k;
        }
        // k = KT - 1: the last slice's MFMAs read nothing further.
        read_slice(nxt, a_buf(k), b_buf(k), 1, wm, wn, lane);
        mfmas(cur);
        if (EDGE) mfma_slice_partial(acc, nxt, imax, jmax);
        else mfma_slice(acc, nxt);
    };
    if (whole) kloop(std::false_type{});
    else kloop(std::true_type{});
    epilogue<ROWCOL>(acc, p, m0, n0, smem, wave, wm, wn, lane, imax, jmax);
}

// ===========================================================================
// Overlapped-epilogue row/column kernel (K >= O_MIN_KT x 128): persistent,
// one workgroup per CU walking its XCD's tile queue (tile_of order).
//
// With one wave per SIMD holding a 128 x 128 accumulator, an epilogue's VALU
// work cannot overlap another wave's MFMAs -- only the same wave's. So the
// wave carries half of each finished tile's output into the next tile's K loop:
//   * after a tile's K loop it converts row blocks 0 .. O_JO - 1 of its
//     accumulator to y = bf16(acc * sa * sb + bias) (64 VGPRs of packed
//     pairs; the reference's linear output, rounded to bf16 before the
//     activation as in the reference) and writes row blocks O_JO .. 3
//     straight to memory (direct_passes);
//   * during the next tile's first O_PASSES K steps it applies the activation
//     to y and writes it out through a 4 KB LDS staging area -- O_PASSES
//     passes of 32 rows x 64 columns, one per step, one element per MFMA
//     slot -- with the 128-byte row read-back and the stores of pass p in
//     step p + 1.
// Fragments are read "rolling" into the registers their last MFMA of the
// slice has just read (slot s = 4 i + j runs MFMA (i, j); B block i is
// replaced after slot 4 i + 3, A block j after slot 12 + j). LDS: four 32 KB
// stage buffers (two K steps: step s in pair (s + par) & 1), the staging
// areas and the epilogue parameters (DMA'd in step 0).
//
// Step k: half 0 -- MFMAs of slice (k, 0), reads of slice (k, 1); wait for
// step k + 1 (vmcnt(0)) and barrier; half 1 -- MFMAs of slice (k, 1), reads of
// slice (k + 1, 0), and the 16 DMAs of step k + 2 into step k's pair (one per
// slot). Step KT - 2 loads the next tile's step 0 instead, and after the last
// step the next tile's step 1 goes into the last pair: the next tile's first
// wait finds its data landed. Stores issued in a half 1 are drained by the
// following mid-step wait; every load wait is either vmcnt(0) or a count that
// a pending wanted load cannot satisfy (loads complete in order among
// themselves).
constexpr int O_BUFS = 4;
constexpr int O_STAGE = 32 * 128;                   // per wave: 32 rows x 64 bf16
constexpr int O_PARAMS = 1792;                      // per wave: 128 + 128 floats, 128 bf16, 128 floats
constexpr int O_BIAS_F32 = 1280;                    // the bias as fp32 (bias_to_f32), in the param area
constexpr int O_STAGE_BASE = O_BUFS * R_BUF;
constexpr int O_PARAM_BASE = O_STAGE_BASE + 4 * O_STAGE;
constexpr int O_SMEM = O_PARAM_BASE + 4 * O_PARAMS;
constexpr int O_JO = 2;                             // row blocks carried into the next tile
constexpr int O_PASSES = 2 * O_JO;                  // overlapped passes (steps 0 .. O_PASSES - 1)
constexpr int O_MIN_KT = O_PASSES + 3;              // + the tail step + the last two steps
static_assert(O_SMEM <= 160 * 1024, "LDS");

// Output window of one wave's 128 x wc sub-tile (first row m0w, first column
// n0w): a raw buffer whose range check drops the stores to rows past M (the
// store geometry and the window's size are gemm_dma.h's, shared with the CPU
// checker), so the stores carry no per-lane test and no 64-bit address
// arithmetic. The launcher bounds ldc (<= 2^22) so that 128 rows of pitch fit
// the 32-bit offsets.
constexpr int OUT_RSRC_FLAGS = 0x00020000;  // raw (stride 0) buffer, 32-bit dwords
typedef uint32_t u32x4_t __attribute__((ext_vector_type(4)));
typedef uint32_t u32x2_t __attribute__((ext_vector_type(2)));

HN_DEVICE __amdgpu_buffer_rsrc_t out_window(const Params& p, int64_t m0w, int64_t n0w, int imax) {
    const int64_t bytes = out_window_bytes(p.M, p.ldc, m0w, imax);
    uint16_t* const base = bytes > 0 ? p.out + m0w * p.ldc + n0w : p.out;
    return __builtin_amdgcn_make_buffer_rsrc(base, (short)0, (int)bytes, OUT_RSRC_FLAGS);
}

// The lane id, regenerated in place (v_mbcnt) by a volatile asm: values
// derived from it are recomputed where used rather than hoisted and held live
// across the tile loop.
HN_DEVICE int fresh_lane() {
    int l;
    asm volatile("v_mbcnt_lo_u32_b32 %0, -1, 0\n\tv_mbcnt_hi_u32_b32 %0, -1, %0" : "=v"(l));
    return l;
}

HN_DEVICE void dma_4B_sbase(const void* sbase, uint32_t voff, uint32_t lds) {
    asm volatile(
        "s_mov_b32 m0, %2\n\t"
        "global_load_lds_dword %0, %1"
        :
        : "v"(voff), "s"(sbase), "s"(lds)
        : "memory", "m0");
}

// Parameter DMA q (0..4) of a wave's sub-tile, 256 bytes each: row scales at
// [0, 512), column scales at [512, 1024), bias pairs at [1024, 1280). Indices
// are clamped to the operand's end (in bounds; never used). bias_to_f32 then
// widens the bias to fp32 at [1280, 1792), so the epilogue reads 4 biases as
// one 16-byte load with no per-value conversion.
template <int WC>
HN_DEVICE void param_dma(const Params& p, int64_t m0, int64_t n0, int wm, int wn, int lane, uint32_t lds, int q) {
    if (q < 2) {
        int64_t m = m0 + wm * 128 + 64 * q + lane;
        m = m < p.M ? m : p.M - 1;
        dma_4B_sbase(p.sa, (uint32_t)(m * 4), lds + 256 * q);
    } else if (q < 4) {
        int64_t n = n0 + wn * WC + 64 * (q - 2) + lane;
        n = n < p.N ? n : p.N - 1;
        dma_4B_sbase(p.sb, (uint32_t)(n * 4), lds + 512 + 256 * (q - 2));
    } else if (p.bias) {
        int64_t n = n0 + wn * WC + 2 * lane;
        n = n < p.N ? n : p.N - 2;
        dma_4B_sbase(p.bias, (uint32_t)(n * 2), lds + 1024);
    } else {
        // No bias: zeros, so the conversion reads the area unconditionally.
        __attribute__((address_space(3))) uint32_t* z =
            (__attribute__((address_space(3))) uint32_t*)(uintptr_t)(lds + 1024);
        z[lane] = 0u;
    }
}


// The wave's 128 bf16 biases (2 per lane) widened to fp32 in its param area,
// from the wave's own LDS (the param DMA has landed: every step after step 0
// waits for its loads).
HN_DEVICE void bias_to_f32(uint8_t* prm, int lane) {
    const uint32_t w = *reinterpret_cast<const uint32_t*>(prm + 1024 + 4 * lane);
    *reinterpret_cast<float2*>(prm + O_BIAS_F32 + 8 * lane) =
        make_float2(__uint_as_float(w << 16), __uint_as_float(w & 0xffff0000u));
}

// y[i][j][w] (j < O_JO) = bf16 pair (2 w, 2 w + 1) of block (i, j): columns
// 32 i + 16 (w / 4) + 8 (lane / 32) + 2 (w % 4) + {0, 1}, row 32 j +
// oe_row(lane % 32) of the sub-tile (the fragment reads' row order, in
// gemm_dma.h, puts 8 consecutive columns in each 4 words). Value group vq (4 values) covers columns
// 32 i + oe_cols(vq, h) + {0..3}.
// Column groups outer, row blocks inner: one group's scales and bias live at a
// time. The bias area holds zeros when the layer has no bias.
HN_DEVICE int oe_cols(int vq, int h) { return 16 * (vq >> 1) + 8 * h + 4 * (vq & 1); }

HN_DEVICE void convert_tile(const f32x16 (&acc)[4][4], uint32_t (&y)[4][4][8], const uint8_t* prm, int lane) {
    const float* const psa = reinterpret_cast<const float*>(prm);
    const float* const psb = reinterpret_cast<const float*>(prm + 512);
    const float* const pbias = reinterpret_cast<const float*>(prm + O_BIAS_F32);
    const int h = lane >> 5, r = oe_row(lane & 31);
    float sam[O_JO];
#pragma unroll
    for (int j = 0; j < O_JO; ++j) sam[j] = psa[32 * j + r];
#pragma unroll
    for (int i = 0; i < 4; ++i)
#pragma unroll
        for (int vq = 0; vq < 4; ++vq) {
            const int nl = 32 * i + oe_cols(vq, h);
            const float4 sb4 = *reinterpret_cast<const float4*>(psb + nl);
            const float4 bn = *reinterpret_cast<const float4*>(pbias + nl);
#pragma unroll
            for (int j = 0; j < O_JO; ++j) {
                const float y0 = fmaf(acc[i][j][4 * vq + 0], sam[j] * sb4.x, bn.x);
                const float y1 = fmaf(acc[i][j][4 * vq + 1], sam[j] * sb4.y, bn.y);
                const float y2 = fmaf(acc[i][j][4 * vq + 2], sam[j] * sb4.z, bn.z);
                const float y3 = fmaf(acc[i][j][4 * vq + 3], sam[j] * sb4.w, bn.w);
                y[i][j][2 * vq] = pack_bf16(y0, y1);
                y[i][j][2 * vq + 1] = pack_bf16(y2, y3);
            }
        }
}

// Pass P (block row j = P / 2, weight blocks 2 (P % 2) + {0, 1}) covers the
// 32 carried values x = 16 ii + 8 hv + 4 (vq % 2) + e of a lane; each 8 of
// them (ii, hv) are 8 consecutive columns, one 16-byte staging write
// (128-byte staging rows with 16-byte chunk c at position c ^ ((r >> 1) & 7)).
//
// oe_act: the activation of value x in place (bf16 in, bf16 out; the even
// value of a pair is held in glo until the odd one repacks the word).
template <int ACT>
HN_DEVICE void oe_act(uint32_t (&y)[4][4][8], float& glo, int P, int x) {
    if (ACT != HN_ACT_GELU_TANH) return;
    const int j = P >> 1, i = 2 * (P & 1) + (x >> 4), vq = (x >> 2) & 3, e = x & 3;
    uint32_t& w = y[i][j][2 * vq + (e >> 1)];
    if ((e & 1) == 0) glo = gelu_tanh(__uint_as_float(w << 16));
    else w = pack_bf16(glo, gelu_tanh(__uint_as_float(w & 0xffff0000u)));
}

// Staging write of half hv (0, 1) of weight block ii of pass P: 16 bytes,
// columns 32 ii + 16 hv + 8 (lane / 32) + {0..7} of the pass (16-byte chunk
// c = 4 ii + 2 hv + lane / 32) in staging row oe_row(lane % 32), from the
// pair words 4 hv .. 4 hv + 3 of block (2 (P % 2) + ii, P / 2).
HN_DEVICE void oe_stage16(uint8_t* stg, int ii, int hv, int lane, uint4 v) {
    const int r = oe_row(lane & 31), c = 4 * ii + 2 * hv + (lane >> 5);
    *reinterpret_cast<uint4*>(stg + r * 128 + ((c ^ ((r >> 1) & 7)) << 4)) = v;
}

HN_DEVICE void oe_write(const uint32_t (&y)[4][4][8], uint8_t* stg, int P, int ii, int hv, int lane) {
    const int j = P >> 1, i = 2 * (P & 1) + ii;
    oe_stage16(stg, ii, hv, lane, make_uint4(y[i][j][4 * hv], y[i][j][4 * hv + 1], y[i][j][4 * hv + 2], y[i][j][4 * hv + 3]));
}

// Staging read-back q (0..3) of a pass: rows 8 q + lane / 8, 16-byte chunk lane % 8.
HN_DEVICE uint4 oe_readback(const uint8_t* stg, int q, int lane) {
    const int rr = 8 * q + (lane >> 3), c = lane & 7;
    return *reinterpret_cast<const uint4*>(stg + rr * 128 + ((c ^ ((rr >> 1) & 7)) << 4));
}

// Store q of pass P of the pending sub-tile (gemm_dma.h: oe_store_off), through
// its output window (pimax: its column blocks inside the matrix).
template <int WC>
HN_DEVICE void oe_store(__amdgpu_buffer_rsrc_t win, int pimax, uint32_t pitch, int P, int q, const uint4& v,
                        int lane) {
    if (oe_store_on(WC, pimax, P, lane))
        __builtin_amdgcn_raw_buffer_store_b128(__builtin_bit_cast(u32x4_t, v), win,
                                               (int)oe_store_off(pitch, lane, P, q), 0, 0);
}

// All eight passes of a pending tile without overlap (before an edge tile and
// after a workgroup's last tile).
template <int ACT, int WC>
HN_DEVICE void oe_flush(const Params& p, uint32_t (&y)[4][4][8], uint8_t* stg, __amdgpu_buffer_rsrc_t win,
                        int pimax, int lane) {
    const uint32_t pitch = (uint32_t)p.ldc * 2;
#pragma unroll
    for (int P = 0; P < O_PASSES; ++P) {
        float glo = 0.0f;
#pragma unroll
        for (int x = 0; x < 32; ++x) oe_act<ACT>(y, glo, P, x);
#pragma unroll
        for (int g = 0; g < 4; ++g) oe_write(y, stg, P, g >> 1, g & 1, lane);
#pragma unroll
        for (int q = 0; q < 4; ++q) oe_store<WC>(win, pimax, pitch, P, q, oe_readback(stg, q, lane), lane);
    }
}

// Passes 2 j, 2 j + 1 for the row blocks j >= O_JO straight from the
// accumulator (not carried): scale, bias, activation and stores. With the
// fragment reads' row order each 8 values of a lane are 8 consecutive columns
// of one row, stored as 16 bytes (gemm_dma.h: direct_store_off) without the
// LDS staging of the carried passes: a store writes 32 bytes of each of 32
// rows (the two half waves side by side), and the 4 stores of a pass fill its
// rows' 128-byte lines, which the L2 merges.
template <int ACT, int WC>
HN_DEVICE void direct_passes(const Params& p, const f32x16 (&acc)[4][4], const uint8_t* prm,
                             __amdgpu_buffer_rsrc_t win, int imax, int lane) {
    const int h = lane >> 5, r = oe_row(lane & 31);
    const uint32_t pitch = (uint32_t)p.ldc * 2;
#pragma unroll
    for (int P = O_PASSES; P < 8; ++P) {
        // Parameters re-read per pass (opaque offset): common loads kept
        // across the passes would hold 32 column-scale vectors live.
        int z = 0;
        asm volatile("" : "+s"(z));
        const float* const psa = reinterpret_cast<const float*>(prm + z);
        const float* const psb = reinterpret_cast<const float*>(prm + z + 512);
        const float* const pbias = reinterpret_cast<const float*>(prm + z + O_BIAS_F32);
        const int j = P >> 1, ih = P & 1;
        const float sam = psa[32 * j + r];
#pragma unroll
        for (int ii = 0; ii < 2; ++ii) {
            const int i = 2 * ih + ii;
            if (32 * i >= WC) continue;  // block past a 96-column wave
            uint32_t w[8];
#pragma unroll
            for (int vq = 0; vq < 4; ++vq) {
                const int nl = 32 * i + oe_cols(vq, h);
                const float4 sb4 = *reinterpret_cast<const float4*>(psb + nl);
                const float4 bn = *reinterpret_cast<const float4*>(pbias + nl);
                float v[4] = {fmaf(acc[i][j][4 * vq + 0], sam * sb4.x, bn.x),
                              fmaf(acc[i][j][4 * vq + 1], sam * sb4.y, bn.y),
                              fmaf(acc[i][j][4 * vq + 2], sam * sb4.z, bn.z),
                              fmaf(acc[i][j][4 * vq + 3], sam * sb4.w, bn.w)};
                // The activation sees the bf16-rounded linear output, as when carried.
                uint2 o = make_uint2(pack_bf16(v[0], v[1]), pack_bf16(v[2], v[3]));
                if (ACT == HN_ACT_GELU_TANH) {
                    v[0] = gelu_tanh(__uint_as_float(o.x << 16));
                    v[1] = gelu_tanh(__uint_as_float(o.x & 0xffff0000u));
                    v[2] = gelu_tanh(__uint_as_float(o.y << 16));
                    v[3] = gelu_tanh(__uint_as_float(o.y & 0xffff0000u));
                    o = make_uint2(pack_bf16(v[0], v[1]), pack_bf16(v[2], v[3]));
                }
                w[2 * vq] = o.x;
                w[2 * vq + 1] = o.y;
            }
            if (direct_store_on(WC, imax, i)) {
                __builtin_amdgcn_raw_buffer_store_b128(u32x4_t{w[0], w[1], w[2], w[3]}, win,
                                                       (int)direct_store_off(pitch, lane, P, ii, 0), 0, 0);
                __builtin_amdgcn_raw_buffer_store_b128(u32x4_t{w[4], w[5], w[6], w[7]}, win,
                                                       (int)direct_store_off(pitch, lane, P, ii, 1), 0, 0);
            }
        }
    }
}

#ifdef HN_GEMM_PHASE_STAMPS
// Measurement build only (libhynomas_fp8_stamps.so, read by bench.py --only
// gemm_phases): thread 0 of workgroups 0-15 records the shader clock
// (s_memtime) at each phase boundary of its first 12 tiles.
constexpr int STAMP_WGS = 16, STAMP_TILES = 12, STAMP_PHASES = 8;
__device__ unsigned long long g_stamps[STAMP_WGS][STAMP_TILES][STAMP_PHASES];
#endif

// The tail stripe's columns [n0, n0 + ncols) (ncols <= TAIL_WIDE_COLS, a
// multiple of 32) over the whole K, by one 4-wave workgroup of the persistent
// kernel after its last tile: the "light" workgroups (one full tile fewer than
// the rest, see light_index) run one such item each in the launch's last tile
// round, where they would otherwise sit idle, instead of a launch of its own
// for the stripe. Wave w owns columns 96 w .. 96 w + 95 (three 32-column
// blocks) of the JB row blocks. Each K step's stage -- the stripe's A rows,
// then the item's B rows -- is filled by the four waves' whole-line direct
// loads (8 rows per 1 KB load, load q by wave q % 4; tail_wide_src) and
// shared; two stages, with one barrier after a step's loads land and one after
// every wave has read its fragments, before that stage is refilled. The
// epilogue is the persistent kernel's, 8 bytes (4 columns) per store.
constexpr int TAIL_WIDE_COLS = 384;
// Where the fused stripe gains (same-box A/B against the separate launch, two
// runs): the north star (32 light workgroups, K 3072) 0.978x and 0.981x, QKV
// (24, N 9216) 0.989x and 0.986x. Where it does not: past K 4096 an item
// outlasts the light workgroups' idle round (fc2, K 12 288: 1.013x), and with
// 8 light workgroups (out-projection, N 3072) it measured 0.991x and 1.017x.
constexpr int64_t TAIL_WIDE_MAX_K = 4096;
constexpr int TAIL_WIDE_MIN_LIGHT = 16;

template <int JB>
constexpr int tail_wide_stage_bytes() { return (32 * JB + TAIL_WIDE_COLS) * BK; }

template <int ACT, int JB>
HN_DEVICE void tail_wide(const Params& p, int64_t m0, int64_t M, int64_t n0, int ncols, uint8_t* smem) {
    constexpr int AR = 32 * JB, NQ = (AR + TAIL_WIDE_COLS) / 8, QW = NQ / 4, STG = tail_wide_stage_bytes<JB>();
    static_assert(NQ % 4 == 0, "the stage's loads split evenly over the four waves");
    const int lane = threadIdx.x & 63;
    const int w = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int64_t K = p.K;
    const uint32_t s_lds = lds_addr(smem);
    const uint8_t* src[QW];
#pragma unroll
    for (int k = 0; k < QW; ++k) {
        const TailSrc ts = tail_wide_src(w + 4 * k, lane, AR, m0, M, n0, n0 + ncols - 1, K);
        src[k] = (ts.a ? p.a : p.b) + ts.off;
    }
    const int KT = (int)(K / BK);  // >= O_MIN_KT >= 2
    auto issue = [&](int st, int t) {
        const int64_t off = (int64_t)t * BK;
        const uint32_t base = s_lds + st * STG;
#pragma unroll
        for (int k = 0; k < QW; ++k) dma_16B(src[k] + off, base + (w + 4 * k) * 1024);
    };
    int nb = (ncols - 96 * w) / 32;  // the wave's column blocks inside the item (wave-uniform)
    nb = nb < 0 ? 0 : (nb > 3 ? 3 : nb);
    f32x16 acc[3][JB];
#pragma unroll
    for (int i = 0; i < 3; ++i)
#pragma unroll
        for (int j = 0; j < JB; ++j)
#pragma unroll
            for (int v = 0; v < 16; ++v) acc[i][j][v] = 0.0f;
    issue(0, 0);
    issue(1, 1);
    for (int t = 0; t < KT; ++t) {
        const int st = t & 1;
        // Step t's loads are the older of at most two steps in flight.
        if (t + 1 < KT) asm volatile("s_waitcnt vmcnt(%0)" ::"n"(QW) : "memory");
        else asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
        __syncthreads();  // every wave's loads of step t have landed
        const uint8_t* const sb = smem + st * STG;
        i32x8 fa[2][JB], fb[2][3];
#pragma unroll
        for (int kh = 0; kh < 2; ++kh) {
#pragma unroll
            for (int j = 0; j < JB; ++j) fa[kh][j] = read_frag(sb, 32 * j + (lane & 31), kh, lane);
#pragma unroll
            for (int i = 0; i < 3; ++i)
                if (i < nb) fb[kh][i] = read_frag(sb, AR + 96 * w + 32 * i + (lane & 31), kh, lane);
        }
        asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
        __syncthreads();  // every wave has read stage st
        if (t + 2 < KT) issue(st, t + 2);
#pragma unroll
        for (int kh = 0; kh < 2; ++kh)
#pragma unroll
            for (int i = 0; i < 3; ++i)
                if (i < nb)
#pragma unroll
                    for (int j = 0; j < JB; ++j) acc[i][j] = mfma(fb[kh][i], fa[kh][j], acc[i][j]);
    }
    // acc[i][j][v] of lane l is out^T for column 96 w + 32 i + 8 (v / 4) + 4 (l / 32) + v % 4
    // and row 32 j + l % 32 of the item.
#pragma unroll
    for (int j = 0; j < JB; ++j) {
        const int64_t m = m0 + 32 * j + (lane & 31);
        if (m >= M) continue;
        const float sam = p.sa[m];
#pragma unroll
        for (int i = 0; i < 3; ++i) {
            if (i >= nb) continue;
#pragma unroll
            for (int vq = 0; vq < 4; ++vq) {
                const int64_t n = n0 + 96 * w + 32 * i + 8 * vq + 4 * (lane >> 5);
                const float4 sb4 = *reinterpret_cast<const float4*>(p.sb + n);
                float bn[4] = {0.0f, 0.0f, 0.0f, 0.0f};
                if (p.bias) {
                    const uint2 bb = *reinterpret_cast<const uint2*>(p.bias + n);
                    bn[0] = bf16_bits_to_f32(bb.x & 0xffffu);
                    bn[1] = bf16_bits_to_f32(bb.x >> 16);
                    bn[2] = bf16_bits_to_f32(bb.y & 0xffffu);
                    bn[3] = bf16_bits_to_f32(bb.y >> 16);
                }
                const float v0 = fmaf(acc[i][j][4 * vq + 0], sam * sb4.x, bn[0]);
                const float v1 = fmaf(acc[i][j][4 * vq + 1], sam * sb4.y, bn[1]);
                const float v2 = fmaf(acc[i][j][4 * vq + 2], sam * sb4.z, bn[2]);
                const float v3 = fmaf(acc[i][j][4 * vq + 3], sam * sb4.w, bn[3]);
                uint2 o = make_uint2(pack_bf16(v0, v1), pack_bf16(v2, v3));
                if (ACT == HN_ACT_GELU_TANH)
                    o = make_uint2(pack_bf16(gelu_tanh(__uint_as_float(o.x << 16)),
                                             gelu_tanh(__uint_as_float(o.x & 0xffff0000u))),
                                   pack_bf16(gelu_tanh(__uint_as_float(o.y << 16)),
                                             gelu_tanh(__uint_as_float(o.y & 0xffff0000u))));
                *reinterpret_cast<uint2*>(p.out + m * p.ldc + n) = o;
            }
        }
    }
}

// WC: columns per wave, 128 (256 x 256 tiles) or 96 (256 x 192 tiles, which
// take the edge-tile path: no carried epilogue).
template <int ACT, int WC>
__global__ __launch_bounds__(NT, 1) void gemm_rowcol_oe_kernel(Params p) {
    constexpr int TBN = 2 * WC;  // tile columns
    __shared__ __attribute__((aligned(16))) uint8_t smem[O_SMEM];
    const int xcd = blockIdx.x & 7;
    const int stride = (int)(gridDim.x >> 3);  // workgroups per XCD
    int slot = (int)(blockIdx.x >> 3);
    int tm, tn;
    if (!tile_of_slot(p, xcd, slot, stride, tm, tn)) return;

    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int wm = wave & 1, wn = wave >> 1;
    const int KT = (int)(p.K / BK);
    const uint32_t lds_base = lds_addr(smem) + wave * 8 * 1024;
    uint8_t* const stg = smem + O_STAGE_BASE + wave * O_STAGE;
    uint8_t* const prm = smem + O_PARAM_BASE + wave * O_PARAMS;
    const uint32_t prm_lds = lds_addr(prm);

    // DMA source: the tile whose stages are being loaded. A 1 KB load q of
    // a buffer fills rows 8 (8 wave + q) .. + 7 (lane / 8 each) with the
    // swizzled logical chunk of physical chunk lane % 8; its per-lane offset
    // is computed at issue from the lane's row (lrow + 8 q, clamped to the
    // operand's last row: in bounds, never stored) and chunk offset, which
    // depends only on q % 2 (chunk[q & 1]).
    const uint8_t* a_src = nullptr;
    const uint8_t* b_src = nullptr;
    // Largest offset a load may take from its K step's source address
    // (src + 128 step): the last 16-byte chunk of the step's 128-byte window
    // of the source tile's last row inside the operand, last K + 112.
    uint32_t a_lim = 0, b_lim = 0;
    auto set_src = [&](int tm_, int tn_) {
        const int64_t m0_ = (int64_t)tm_ * BM, n0_ = (int64_t)tn_ * TBN;
        a_src = p.a + m0_ * p.K;
        b_src = p.b + n0_ * p.K;
        const int64_t a_rows = p.M - m0_ < BM ? p.M - m0_ : BM;
        // A 192-wide tile still fills all 256 stage rows; rows past its width
        // are clamped like rows past N (never read by an MFMA).
        const int64_t b_rows = p.N - n0_ < TBN ? p.N - n0_ : TBN;
        a_lim = dma_limit(a_rows, p.K);
        b_lim = dma_limit(b_rows, p.K);
    };
    // Per-lane DMA geometry from a regenerated lane id l (gemm_dma.h: the
    // lane's row in load 0, its chunk offsets for even and odd loads, row K),
    // and the offset of load q capped at the source tile's limit, so every
    // load of every wave stays inside the operand, whichever rows the wave
    // itself multiplies.
    auto dma_lane = [&](int l) { return dma_lane_of(wave, l, p.K); };
    auto dma_off = [&](const DmaLane& d, int q, uint32_t lim) { return dma_offset(d, q, p.K, lim); };
    // Current tile: origin and blocks inside the matrix (imax weight blocks of
    // the wave's wc columns, 4 or 3 in the interior; jmax activation blocks of
    // 32 rows). Wave-uniform. Tiles with every block inside the matrix take
    // the carried path.
    int64_t cm0 = 0, cn0 = 0;
    int cimax = 0, cjmax = 0;
    auto set_cur = [&](int tm_, int tn_) {
        cm0 = (int64_t)tm_ * BM;
        cn0 = (int64_t)tn_ * TBN;
        const WaveExtent e = wave_extent(p.M, p.N, cm0 + wm * 128, cn0 + wn * WC, WC);
        cimax = e.imax;
        cjmax = e.jmax;
    };
    int par = 0;  // step s of the current tile uses buffer pair (s + par) & 1
    auto pair_of = [&](int s) { return (s + par) & 1; };
    auto dma_a = [&](const DmaLane& d, int src_step, int pr, int q) {
        dma_16B_sbase(a_src + (int64_t)src_step * BK, dma_off(d, q, a_lim), lds_base + (2 * pr) * R_BUF + q * 1024);
    };
    auto dma_b = [&](const DmaLane& d, int src_step, int pr, int q) {
        dma_16B_sbase(b_src + (int64_t)src_step * BK, dma_off(d, q, b_lim),
                      lds_base + (2 * pr + 1) * R_BUF + q * 1024);
    };

    f32x16 acc[4][4];
    i32x8 fa[4], fb[4];
    uint32_t y[4][4][8];         // carried rows (j < O_JO) of the pending tile
    // Pending tile: its output window and column blocks inside (none yet: an
    // empty window, every store dropped).
    __amdgpu_buffer_rsrc_t pwin = out_window(p, p.M, 0, 0);
    int pimax = 0;
    bool pending = false;

    // Fragment reads. A fragment of block row base + 32 q is 16-byte chunks
    // c0 = 4 kh + 2 (lane / 32) and c0 + 1 of row base + 32 q + oe_row(lane % 32); the
    // swizzle depends only on the lane (32 q and base are multiples of 16), so
    // a lane needs four offsets (kh x chunk), computed per step from a
    // regenerated lane id (hoisted, they would be held live and spilled).
    struct RdLane {
        uint32_t off[2][2];
    };
    auto rd_lane = [&](int l) {
        RdLane d;
        const int r = oe_row(l & 31), c0 = (l >> 5) * 2;
#pragma unroll
        for (int kh = 0; kh < 2; ++kh)
#pragma unroll
            for (int hi = 0; hi < 2; ++hi)
                d.off[kh][hi] = (uint32_t)(r * BK + (swz_pos(r, 4 * kh + c0 + hi) << 4));
        return d;
    };
    auto frag_at = [&](const uint8_t* buf, int row0, int kh, const RdLane& d) {
        const uint4 lo = *reinterpret_cast<const uint4*>(buf + row0 * BK + d.off[kh][0]);
        const uint4 hi = *reinterpret_cast<const uint4*>(buf + row0 * BK + d.off[kh][1]);
        i32x8 f;
        f[0] = lo.x; f[1] = lo.y; f[2] = lo.z; f[3] = lo.w;
        f[4] = hi.x; f[5] = hi.y; f[6] = hi.z; f[7] = hi.w;
        return f;
    };
    auto read_a = [&](const uint8_t* buf, int j, int kh, const RdLane& d) {
        fa[j] = frag_at(buf, wm * 128 + j * 32, kh, d);
    };
    auto read_b = [&](const uint8_t* buf, int i, int kh, const RdLane& d) {
        fb[i] = frag_at(buf, wn * WC + i * 32, kh, d);
    };
    // Rolling reads of the next slice after slot s's MFMA.
    auto roll = [&](int s, const uint8_t* abuf, const uint8_t* bbuf, int kh, const RdLane& d) {
        if (s == 3 || s == 7 || s == 11) read_b(bbuf, s >> 2, kh, d);
        if (s >= 12) read_a(abuf, s - 12, kh, d);
        if (s == 15 && WC == 128) read_b(bbuf, 3, kh, d);  // no fourth block at 96 columns
    };

    // One K step. EDGE: edge tile (blocks outside the matrix skipped). PASS:
    // -1 none, 0 .. O_PASSES - 1 epilogue pass of the pending tile (plus the
    // read-back and stores of pass PASS - 1), O_PASSES only the read-back and
    // stores of the last pass.
    // DMA: 0 none, 1 this tile's step k + 2, 2 the next tile's step 0, 3 as 1
    // plus this tile's epilogue parameters. NEXT: reads of slice (k + 1, 0)
    // and the mid-step wait (false on the last step). FIRST: the accumulator
    // starts at zero (step 0).
    auto step = [&](int k, auto edge_t, auto pass_t, auto dma_t, auto next_t, auto first_t) {
        constexpr bool EDGE = decltype(edge_t)::value;
        constexpr int PASS = decltype(pass_t)::value;
        constexpr int DMA = decltype(dma_t)::value;
        constexpr bool NEXT = decltype(next_t)::value;
        constexpr bool FIRST = decltype(first_t)::value;
        const uint8_t* const ab = smem + (2 * pair_of(k)) * R_BUF;
        const uint8_t* const bb = ab + R_BUF;
        const uint8_t* const an = smem + (2 * pair_of(k + 1)) * R_BUF;
        const uint8_t* const bnx = an + R_BUF;
        const int dst = pair_of(k);
        float glo = 0.0f;
        uint4 rb[4];
        const int el = fresh_lane();
        const DmaLane dl = dma_lane(el);
        const RdLane rl = rd_lane(el);
        const uint32_t pitch = (uint32_t)p.ldc * 2;
#pragma unroll
        for (int s = 0; s < 16; ++s) {
            const int i = s >> 2, j = s & 3;
            if (i < WC / 32 && (!EDGE || (i < cimax && j < cjmax))) {
                if (FIRST) acc[i][j] = mfma(fb[i], fa[j], f32x16{});
                else acc[i][j] = mfma(fb[i], fa[j], acc[i][j]);
            } else if (FIRST) {
                acc[i][j] = f32x16{};
            }
            roll(s, ab, bb, 1, rl);
            if (PASS >= 0 && PASS < O_PASSES) oe_act<ACT>(y, glo, PASS, s);
            __builtin_amdgcn_sched_barrier(0);
        }
        if (NEXT) {
            asm volatile("s_waitcnt vmcnt(0)" ::: "memory");  // step k + 1 landed (this wave)
            __syncthreads();                                  // ... every wave; step k's pair free
        }
#pragma unroll
        for (int s = 0; s < 16; ++s) {
            // Read-back of the previous pass (slots 0-3) before this pass's
            // staging writes (slots 3-15), stores two slots after each read.
            if (PASS >= 1 && s < 4) rb[s] = oe_readback(stg, s, el);
            if (PASS >= 1 && s >= 2 && s < 6)
                oe_store<WC>(pwin, pimax, pitch, PASS - 1, s - 2, rb[s - 2], el);
            const int i = s >> 2, j = s & 3;
            if (i < WC / 32 && (!EDGE || (i < cimax && j < cjmax))) acc[i][j] = mfma(fb[i], fa[j], acc[i][j]);
            if (NEXT) roll(s, an, bnx, 0, rl);
            if (DMA == 1 || DMA == 3) {
                if (s < 8) dma_a(dl, k + 2, dst, s);
                else dma_b(dl, k + 2, dst, s - 8);
            }
            if (DMA == 2) {
                if (s < 8) dma_a(dl, 0, dst, s);
                else dma_b(dl, 0, dst, s - 8);
            }
            if (DMA == 3 && s >= 8 && s < 13) param_dma<WC>(p, cm0, cn0, wm, wn, el, prm_lds, s - 8);
            if (DMA == 0 && !NEXT && s == 2) bias_to_f32(prm, el);  // the last step: its slots are free
            if (PASS >= 0 && PASS < O_PASSES) {
                oe_act<ACT>(y, glo, PASS, 16 + s);
                if (s == 4 || s == 5) oe_write(y, stg, PASS, 0, s - 4, el);      // block 0 (half 0's values)
                if ((s & 7) == 7) oe_write(y, stg, PASS, 1, s >> 3, el);         // block 1, each half when complete
            }
            __builtin_amdgcn_sched_barrier(0);
        }
    };
    using F = std::false_type;
    using T = std::true_type;

    // First tile: steps 0 and 1 into pairs 0 and 1.
    set_src(tm, tn);
    set_cur(tm, tn);
    {
        const DmaLane d = dma_lane(fresh_lane());
#pragma unroll
        for (int q = 0; q < 8; ++q) dma_a(d, 0, 0, q);
#pragma unroll
        for (int q = 0; q < 8; ++q) dma_b(d, 0, 0, q);
#pragma unroll
        for (int q = 0; q < 8; ++q) dma_a(d, 1, 1, q);
#pragma unroll
        for (int q = 0; q < 8; ++q) dma_b(d, 1, 1, q);
    }
    asm volatile("s_waitcnt vmcnt(16)" ::: "memory");  // step 0: step 1's 16 loads are newer
    __syncthreads();

#ifdef HN_GEMM_PHASE_STAMPS
    int stamp_tile = 0;
    auto stamp = [&](int ph) {
        if (blockIdx.x < STAMP_WGS && threadIdx.x == 0 && stamp_tile < STAMP_TILES)
            g_stamps[blockIdx.x][stamp_tile][ph] = __builtin_amdgcn_s_memtime();
    };
#else
    auto stamp = [](int) {};
#endif
    for (;;) {
        stamp(0);
        int ntm = 0, ntn = 0;
        const bool more = tile_of_slot(p, xcd, slot + stride, stride, ntm, ntn);
        // Slice (0, 0).
        {
            const uint8_t* const ab = smem + (2 * pair_of(0)) * R_BUF;
            const RdLane d = rd_lane(fresh_lane());
#pragma unroll
            for (int q = 0; q < 4; ++q) {
                if (q < WC / 32) read_b(ab + R_BUF, q, 0, d);
                read_a(ab, q, 0, d);
            }
        }
        const bool whole = cimax == WC / 32 && cjmax == 4;
        if (whole) {
            if (!pending) {
                // Nothing carried yet: the passes run on zeros, their stores
                // all out of range.
#pragma unroll
                for (int i = 0; i < 4; ++i)
#pragma unroll
                    for (int j = 0; j < O_JO; ++j)
#pragma unroll
                        for (int w = 0; w < 8; ++w) y[i][j][w] = 0u;
            }
            step(0, F{}, std::integral_constant<int, 0>{}, std::integral_constant<int, 3>{}, T{}, T{});
            step(1, F{}, std::integral_constant<int, 1>{}, std::integral_constant<int, 1>{}, T{}, F{});
            step(2, F{}, std::integral_constant<int, 2>{}, std::integral_constant<int, 1>{}, T{}, F{});
            step(3, F{}, std::integral_constant<int, 3>{}, std::integral_constant<int, 1>{}, T{}, F{});
            step(4, F{}, std::integral_constant<int, 4>{}, std::integral_constant<int, 1>{}, T{}, F{});
            stamp(1);
            static_assert(O_PASSES == 4, "the unrolled epilogue steps assume four passes");
            for (int k = O_PASSES + 1; k < KT - 2; ++k)
                step(k, F{}, std::integral_constant<int, -1>{}, std::integral_constant<int, 1>{}, T{}, F{});
            if (more) set_src(ntm, ntn);  // else step 0 of this tile again: harmless, in bounds
            step(KT - 2, F{}, std::integral_constant<int, -1>{}, std::integral_constant<int, 2>{}, T{}, F{});
            step(KT - 1, F{}, std::integral_constant<int, -1>{}, std::integral_constant<int, 0>{}, F{}, F{});
            stamp(2);
        } else {
            if (pending) oe_flush<ACT, WC>(p, y, stg, pwin, pimax, fresh_lane());
            step(0, T{}, std::integral_constant<int, -1>{}, std::integral_constant<int, 3>{}, T{}, T{});
            for (int k = 1; k < KT - 2; ++k)
                step(k, T{}, std::integral_constant<int, -1>{}, std::integral_constant<int, 1>{}, T{}, F{});
            if (more) set_src(ntm, ntn);
            step(KT - 2, T{}, std::integral_constant<int, -1>{}, std::integral_constant<int, 2>{}, T{}, F{});
            step(KT - 1, T{}, std::integral_constant<int, -1>{}, std::integral_constant<int, 0>{}, F{}, F{});
        }
        // Every wave is done reading the last step's pair.
        __syncthreads();
        stamp(3);
        if (more) {
            // The next tile's step 1 into the last step's pair.
            const int pr = pair_of(KT - 1);
            const DmaLane d = dma_lane(fresh_lane());
#pragma unroll
            for (int q = 0; q < 8; ++q) dma_a(d, 1, pr, q);
#pragma unroll
            for (int q = 0; q < 8; ++q) dma_b(d, 1, pr, q);
        }
        stamp(4);
        const __amdgpu_buffer_rsrc_t cwin = out_window(p, cm0 + wm * 128, cn0 + wn * WC, cimax);
        direct_passes<ACT, WC>(p, acc, prm, cwin, cimax, fresh_lane());
        stamp(5);
        convert_tile(acc, y, prm, fresh_lane());
        stamp(6);
        pwin = cwin;
        pimax = cimax;
        pending = true;
        if (!more) break;
        par = (KT + par) & 1;
        set_cur(ntm, ntn);
        slot += stride;
        // The next tile's step 0 landed: step 1's 16 loads are newer.
        asm volatile("s_waitcnt vmcnt(16)" ::: "memory");
        __syncthreads();
        stamp(7);
#ifdef HN_GEMM_PHASE_STAMPS
        ++stamp_tile;
#endif
    }
    oe_flush<ACT, WC>(p, y, stg, pwin, pimax, fresh_lane());
    // The last step's re-load of step 0 (no next tile) may still be landing.
    asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
    if (p.tail_M > p.M) {
        const int li = light_index(p, xcd, (int)(blockIdx.x >> 3), stride);
        const int64_t n0 = (int64_t)li * p.tail_cols;
        if (li < 0 || n0 >= p.N) return;
        __syncthreads();  // every wave is past the LDS of its last tile
        const int nc = (int)(p.N - n0 < p.tail_cols ? p.N - n0 : p.tail_cols);
        if (p.tail_M - p.M > 32) tail_wide<ACT, 2>(p, p.M, p.tail_M, n0, nc, smem);
        else tail_wide<ACT, 1>(p, p.M, p.tail_M, n0, nc, smem);
    }
}

// ---------------------------------------------------------------------------
// The last M % 256 <= TAIL_ROWS rows of a persistent row/column GEMM, [m0, M).
//
// As a 256-row tile of the persistent kernel such a stripe keeps the whole K
// loop of a full tile -- its DMAs, waits and barriers -- for a fraction of the
// MFMAs, and its K steps wait on their loads' latency: at the north star
// (M 10 800, 48 tail rows, 48 column tiles) an edge tile took about as long as
// a full one and the edge tiles put a ninth tile round on some workgroups
// (10 800 rows 362 us against 10 752 rows 317 us, same box).
//
// Here a workgroup owns 32 output columns of the stripe's JB 32-row blocks and
// splits K over its SK waves: wave w multiplies the 128-byte K steps w,
// w + SK, w + 2 SK, ... Each wave streams its steps through TAIL_STAGES
// private LDS stages (the A rows of the stripe, then the 32 B rows), filled
// by whole-line direct loads (dma_16B, 8 rows per 1 KB load) in the persistent
// kernel's swizzled row layout and read back as MFMA fragments (read_frag);
// no barrier is needed until the end. The waves' partial sums meet in LDS and
// are added in wave order, so the result is deterministic. The epilogue is
// the persistent kernel's: bf16(acc sa sb + bias), GELU-tanh of that bf16
// value, rounded to bf16; each thread stores 8 consecutive columns of one row
// (16 bytes); rows past M are loaded as the last row and not stored.
//
// BLOCKWISE (the decoder's 128 x 128 block scales, gemm_bw8_kernel's
// contract): a 128-byte K step is one scale block, and the stripe's rows and a
// workgroup's 32 columns lie in one 128-row and one 128-column scale block, so
// a wave adds each step's product times that block's factor
// f_k = sa[mb][k] sb[nb][k] (skipped when f_k = 0), and the epilogue is
// bf16(acc). The factors are read through the constant address space (scalar
// loads, outside the vector-memory counter the DMA waits count).
constexpr int TAIL_ROWS = 64;
constexpr int TAIL_COLS = 32;
constexpr int TAIL_STAGES = 3;
static_assert(O_MIN_KT >= 4, "every tail wave needs a K step (K / 128 >= O_MIN_KT, at most 4 waves)");

template <int JB>
constexpr int tail_stage_bytes() { return (32 * JB + 32) * BK; }
template <int SK, int JB>
constexpr int tail_smem_bytes() { return SK * TAIL_STAGES * tail_stage_bytes<JB>(); }

template <int MODE, int ACT, int SK, int JB>
__global__ __launch_bounds__(64 * SK) void gemm_tail_kernel(Params p, int64_t m0) {
    constexpr int AR = 32 * JB, NQ = (AR + 32) / 8, STG = tail_stage_bytes<JB>();
    static_assert(JB * 64 * 16 * 4 <= STG, "a wave's partial sums fit its stages");
    __shared__ __attribute__((aligned(16))) uint8_t smem[tail_smem_bytes<SK, JB>()];
    const int lane = threadIdx.x & 63;
    const int w = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int64_t n0 = (int64_t)blockIdx.x * TAIL_COLS;
    const int64_t K = p.K;
    uint8_t* const ws = smem + w * TAIL_STAGES * STG;
    const uint32_t ws_lds = lds_addr(ws);
    // Load q of a step fills stage rows 8 q .. 8 q + 7; lane l brings 16 bytes of
    // row 8 q + l / 8: the logical chunk that the swizzle puts at physical chunk l % 8.
    const uint8_t* src[NQ];
#pragma unroll
    for (int q = 0; q < NQ; ++q) {
        const TailSrc ts = tail_src(q, lane, AR, m0, p.M, n0, K);
        src[q] = (ts.a ? p.a : p.b) + ts.off;
    }
    const int KT = (int)(K / BK);
    const int T = tail_steps(KT, w, SK);  // this wave's steps: w + SK t, t < T (T >= 1)
    // Step t into stage st (tail_step: past the last step, step T - 1 again).
    auto issue = [&](int st, int t) {
        const int64_t off = (int64_t)tail_step(w, SK, t, T) * BK;
        const uint32_t base = ws_lds + st * STG;
        // The stage's fragment reads have landed before its refill is issued.
        asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
#pragma unroll
        for (int q = 0; q < NQ; ++q) dma_16B(src[q] + off, base + q * 1024);
    };
    f32x16 acc[JB];
#pragma unroll
    for (int j = 0; j < JB; ++j)
#pragma unroll
        for (int v = 0; v < 16; ++v) acc[j][v] = 0.0f;
    typedef const __attribute__((address_space(4))) float cfloat;
    cfloat* const sa_row = (cfloat*)p.sa + (m0 >> 7) * KT;  // BLOCKWISE: the stripe's scale row
    cfloat* const sb_row = (cfloat*)p.sb + (n0 >> 7) * KT;  // and the columns' one
#pragma unroll
    for (int d = 0; d < TAIL_STAGES; ++d) issue(d, d);
    int st = 0;
    for (int t = 0; t < T; ++t) {
        float f = 1.0f;
        if (MODE == BLOCKWISE) {
            const int k = w + SK * t;
            f = sa_row[k] * sb_row[k];
        }
        // Step t's loads are the oldest in flight: (TAIL_STAGES - 1) NQ later ones may stay.
        asm volatile("s_waitcnt vmcnt(%0)" ::"n"((TAIL_STAGES - 1) * NQ) : "memory");
        const uint8_t* const sb = ws + st * STG;
        if (MODE == ROWCOL) {
#pragma unroll
            for (int kh = 0; kh < 2; ++kh) {
                const i32x8 fb = read_frag(sb, AR + (lane & 31), kh, lane);
#pragma unroll
                for (int j = 0; j < JB; ++j)
                    acc[j] = mfma(fb, read_frag(sb, 32 * j + (lane & 31), kh, lane), acc[j]);
            }
        } else if (f != 0.0f) {
            f32x16 blk[JB];
#pragma unroll
            for (int j = 0; j < JB; ++j)
#pragma unroll
                for (int v = 0; v < 16; ++v) blk[j][v] = 0.0f;
#pragma unroll
            for (int kh = 0; kh < 2; ++kh) {
                const i32x8 fb = read_frag(sb, AR + (lane & 31), kh, lane);
#pragma unroll
                for (int j = 0; j < JB; ++j)
                    blk[j] = mfma(fb, read_frag(sb, 32 * j + (lane & 31), kh, lane), blk[j]);
            }
#pragma unroll
            for (int j = 0; j < JB; ++j)
#pragma unroll
                for (int v = 0; v < 16; ++v) acc[j][v] = fmaf(blk[j][v], f, acc[j][v]);
        }
        issue(st, t + TAIL_STAGES);
        st = st + 1 == TAIL_STAGES ? 0 : st + 1;
    }
    asm volatile("s_waitcnt vmcnt(0)" ::: "memory");  // the re-loads past the last step
    float* const part = reinterpret_cast<float*>(ws);  // [(block * 64 + lane) * 16 + register]
#pragma unroll
    for (int j = 0; j < JB; ++j)
#pragma unroll
        for (int q = 0; q < 4; ++q)
            *reinterpret_cast<float4*>(part + (j * 64 + lane) * 16 + 4 * q) =
                make_float4(acc[j][4 * q], acc[j][4 * q + 1], acc[j][4 * q + 2], acc[j][4 * q + 3]);
    __syncthreads();
    // Item it: row ml = it / 4 of the stripe, columns 8 g .. 8 g + 7 (g = it % 4).
    // acc[j][v] of lane l is out^T for column 8 (v / 4) + 4 (l / 32) + v % 4 and
    // row 32 j + l % 32, so column 8 g + 4 hh + b is register 4 g + b of lane
    // ml % 32 + 32 hh.
    for (int it = threadIdx.x; it < JB * 32 * 4; it += 64 * SK) {
        const int ml = it >> 2, g = it & 3;
        const int64_t m = m0 + ml;
        if (m >= p.M) continue;
        const int j = ml >> 5, rr = ml & 31;
        float y[8];
#pragma unroll
        for (int hh = 0; hh < 2; ++hh) {
            float4 s = make_float4(0.0f, 0.0f, 0.0f, 0.0f);
#pragma unroll
            for (int ww = 0; ww < SK; ++ww) {
                const float* const pw = reinterpret_cast<const float*>(smem + ww * TAIL_STAGES * STG);
                const float4 q = *reinterpret_cast<const float4*>(pw + (j * 64 + rr + 32 * hh) * 16 + 4 * g);
                s.x += q.x; s.y += q.y; s.z += q.z; s.w += q.w;
            }
            y[4 * hh] = s.x; y[4 * hh + 1] = s.y; y[4 * hh + 2] = s.z; y[4 * hh + 3] = s.w;
        }
        const int64_t n = n0 + 8 * g;
        if (MODE == BLOCKWISE) {
            *reinterpret_cast<uint4*>(p.out + m * p.ldc + n) =
                make_uint4(pack_bf16(y[0], y[1]), pack_bf16(y[2], y[3]), pack_bf16(y[4], y[5]), pack_bf16(y[6], y[7]));
            continue;
        }
        const float sam = p.sa[m];
        const float4 sb0 = *reinterpret_cast<const float4*>(p.sb + n);
        const float4 sb1 = *reinterpret_cast<const float4*>(p.sb + n + 4);
        const float sbv[8] = {sb0.x, sb0.y, sb0.z, sb0.w, sb1.x, sb1.y, sb1.z, sb1.w};
        float bv[8] = {};
        if (p.bias) {
            const uint2 b0 = *reinterpret_cast<const uint2*>(p.bias + n);
            const uint2 b1 = *reinterpret_cast<const uint2*>(p.bias + n + 4);
            const uint32_t bw[4] = {b0.x, b0.y, b1.x, b1.y};
#pragma unroll
            for (int c = 0; c < 4; ++c) {
                bv[2 * c] = bf16_bits_to_f32(bw[c] & 0xffffu);
                bv[2 * c + 1] = bf16_bits_to_f32(bw[c] >> 16);
            }
        }
        uint32_t o[4];
#pragma unroll
        for (int c = 0; c < 4; ++c) {
            const float v0 = fmaf(y[2 * c], sam * sbv[2 * c], bv[2 * c]);
            const float v1 = fmaf(y[2 * c + 1], sam * sbv[2 * c + 1], bv[2 * c + 1]);
            o[c] = pack_bf16(v0, v1);
            if (ACT == HN_ACT_GELU_TANH)
                o[c] = pack_bf16(gelu_tanh(__uint_as_float(o[c] << 16)),
                                 gelu_tanh(__uint_as_float(o[c] & 0xffff0000u)));
        }
        *reinterpret_cast<uint4*>(p.out + m * p.ldc + n) = make_uint4(o[0], o[1], o[2], o[3]);
    }
}

}  // namespace gemm
}  // namespace hn

using namespace hn;

static int gemm_launch(int mode, const void* a, const void* b, const float* sa, const float* sb,
                       const void* bias, void* out, int64_t M, int64_t N, int64_t K, int64_t ldc,
                       int act, void* stream, const char* who) {
    HN_REQUIRE(M >= 0 && N > 0 && K > 0, HN_E_ARG, "FP8 GEMM: invalid shape");
    HN_REQUIRE(N % 128 == 0 && K % 128 == 0, HN_E_ARG, "FP8 GEMM: N and K must be multiples of 128");
    HN_REQUIRE(K <= 128 * gemm::kMaxKT, HN_E_ARG, "FP8 GEMM: K must be <= 32768");
    HN_REQUIRE(ldc >= N && ldc % 8 == 0, HN_E_ARG, "FP8 GEMM: ldc must be >= N and a multiple of 8");
    // The persistent kernel's output windows address 128 rows of pitch with
    // 32-bit offsets.
    HN_REQUIRE(ldc <= (int64_t)1 << 22, HN_E_ARG, "FP8 GEMM: ldc must be <= 4194304");
    HN_REQUIRE(act == HN_ACT_NONE || act == HN_ACT_GELU_TANH, HN_E_ARG, "FP8 GEMM: unknown activation");
    HN_REQUIRE(aligned(a, 16) && aligned(b, 16) && aligned(out, 16) && aligned(sa, 4) &&
                   aligned(sb, mode == gemm::ROWCOL ? 16 : 4) && aligned(bias, 8),
               HN_E_ARG, "FP8 GEMM: misaligned pointer");
    if (M == 0) return HN_OK;
    HN_REQUIRE(a && b && sa && sb && out, HN_E_ARG, "FP8 GEMM: null pointer");
    if (const int rc = require_gfx950(who); rc != HN_OK) return rc;
    gemm::Params p{};
    p.a = (const uint8_t*)a; p.b = (const uint8_t*)b;
    p.sa = sa; p.sb = sb;
    p.bias = (const uint16_t*)bias;
    p.out = (uint16_t*)out;
    p.M = M; p.N = N; p.K = K; p.ldc = ldc; p.act = act;
    HN_REQUIRE((M + gemm::BM - 1) / gemm::BM * ((N + 191) / 192) <= 0x7fffffffLL, HN_E_ARG,
               "FP8 GEMM: too many tiles");
    const bool persistent = mode == gemm::ROWCOL && K / gemm::BK >= gemm::O_MIN_KT;
    // A last row stripe of at most TAIL_ROWS rows goes to gemm_tail_kernel (or,
    // in persistent launches, possibly to the light workgroups), and the tiles
    // cover only the rows above it: always in persistent launches; in
    // blockwise ones (one tile per workgroup, one workgroup per CU) when that
    // saves a whole round of tiles (the decoder's gate and up projections,
    // 10 800 x 4096 -> 12 288: 2064 tiles, 9 rounds, against 2016, 8) and K
    // has at least 4 scale blocks (a K step for each of up to 4 waves).
    const int64_t m_tail = M % gemm::BM;
    bool stripe = false;
    if (m_tail > 0 && m_tail <= gemm::TAIL_ROWS) {
        if (persistent) {
            stripe = true;
        } else if (mode == gemm::BLOCKWISE && K / gemm::BK >= 4) {
            const int64_t cus = device_cus(), tn = (N + gemm::BN - 1) / gemm::BN;
            const int64_t all = (M + gemm::BM - 1) / gemm::BM * tn, whole = M / gemm::BM * tn;
            stripe = (all + cus - 1) / cus > (whole + cus - 1) / cus;
        }
    }
    const int64_t Mt = stripe ? M - m_tail : M;
    const int64_t tm = (Mt + gemm::BM - 1) / gemm::BM;
    auto set_tiles = [&](int bn) {
        const gemm::TileCounts t = gemm::tile_counts(Mt, N, bn);
        p.bn = bn;
        p.tiles_m = t.tiles_m; p.tiles_n = t.tiles_n;
        p.tm_full = t.tm_full; p.tn_full = t.tn_full; p.m_tail = t.m_tail;
        p.tiles_full = t.tiles_full; p.tiles_part = t.tiles_part;
        p.per_xcd = mode == gemm::ROWCOL ? t.per_xcd : (int)((tm * t.tiles_n + 7) / 8);
    };
    set_tiles(gemm::BN);
    const dim3 grid((unsigned)(8 * (int64_t)p.per_xcd));
    // The tail stripe on a launch of its own, with the full M for its row
    // clamp and stores. K is split over 2 waves, or 4 when the stripe has
    // fewer 32-column groups than CUs.
    auto launch_tail = [&]() {
        gemm::Params pt = p;
        pt.M = M;
        pt.tail_M = 0;
        const dim3 tgrid((unsigned)(N / gemm::TAIL_COLS));
        const hipStream_t st = (hipStream_t)stream;
        const bool two = m_tail > 32, four = N / gemm::TAIL_COLS < device_cus(), gelu = act == HN_ACT_GELU_TANH;
        const dim3 tblock(four ? 256 : 128);
#define HN_TAIL(A, SK, JB) gemm::gemm_tail_kernel<gemm::ROWCOL, A, SK, JB><<<tgrid, tblock, 0, st>>>(pt, Mt)
#define HN_TAIL_BW(SK, JB) gemm::gemm_tail_kernel<gemm::BLOCKWISE, HN_ACT_NONE, SK, JB><<<tgrid, tblock, 0, st>>>(pt, Mt)
        if (mode == gemm::BLOCKWISE) {
            if (four) { if (two) HN_TAIL_BW(4, 2); else HN_TAIL_BW(4, 1); }
            else { if (two) HN_TAIL_BW(2, 2); else HN_TAIL_BW(2, 1); }
        } else if (gelu) {
            if (four) { if (two) HN_TAIL(HN_ACT_GELU_TANH, 4, 2); else HN_TAIL(HN_ACT_GELU_TANH, 4, 1); }
            else { if (two) HN_TAIL(HN_ACT_GELU_TANH, 2, 2); else HN_TAIL(HN_ACT_GELU_TANH, 2, 1); }
        } else {
            if (four) { if (two) HN_TAIL(HN_ACT_NONE, 4, 2); else HN_TAIL(HN_ACT_NONE, 4, 1); }
            else { if (two) HN_TAIL(HN_ACT_NONE, 2, 2); else HN_TAIL(HN_ACT_NONE, 2, 1); }
        }
#undef HN_TAIL
#undef HN_TAIL_BW
        return check_launch(who);
    };
    if (stripe && Mt == 0) return launch_tail();
    p.M = Mt;
    p.tail_M = Mt;
    if (persistent) {
        // Persistent: per XCD, min(queue length, CUs of the XCD) workgroups.
        // A launch of fewer 256-wide tiles than CUs is one round whatever
        // the tile; 192-wide tiles (three 32-column blocks per wave) do 3/4
        // of the work each and fill more CUs (config 1, 4096 x 3072: 192 ->
        // 256 tiles).
        const int cus = device_cus();
        const int per_xcd_cus = cus / 8 > 0 ? cus / 8 : 1;
        const int64_t t256 = tm * ((N + 255) / 256), t192 = tm * ((N + 191) / 192);
        if (t256 < cus && t192 > t256) {
            set_tiles(192);
            if (p.per_xcd > per_xcd_cus) set_tiles(gemm::BN);  // would need a second round
        }
        int wg_cap = per_xcd_cus;
#ifdef HN_GEMM_PHASE_STAMPS
        // Measurement build: HN_GEMM_WG_PER_XCD caps the workgroups per XCD
        // (the tile queues adapt; fewer CUs busy, same tiles).
        if (const char* e = getenv("HN_GEMM_WG_PER_XCD")) {
            const int v = atoi(e);
            if (v >= 1 && v < wg_cap) wg_cap = v;
        }
#endif
        const int S = p.per_xcd < wg_cap ? p.per_xcd : wg_cap;
        const dim3 pgrid((unsigned)(8 * S));
        const hipStream_t st = (hipStream_t)stream;
        if (Mt < M) {
            // The tail stripe rides on the light workgroups (tail_wide) when
            // every XCD has some, at least TAIL_WIDE_MIN_LIGHT in all, there
            // are no edge tiles, each light workgroup's share of the columns
            // fits one item and K is at most TAIL_WIDE_MAX_K; else it has a
            // launch of its own.
            bool every = false;
            const int nl = gemm::light_count(p, S, &every);
            const int64_t cols = nl > 0 ? (N / 32 + nl - 1) / nl * 32 : 0;
            if (p.tiles_part == 0 && every && nl >= gemm::TAIL_WIDE_MIN_LIGHT && cols <= gemm::TAIL_WIDE_COLS &&
                K <= gemm::TAIL_WIDE_MAX_K) {
                p.tail_M = M;
                p.tail_cols = (int)cols;
            } else if (const int rc = launch_tail(); rc != HN_OK) {
                return rc;
            }
        }
        if (p.bn == 192) {
            if (act == HN_ACT_GELU_TANH)
                gemm::gemm_rowcol_oe_kernel<HN_ACT_GELU_TANH, 96><<<pgrid, gemm::NT, 0, st>>>(p);
            else
                gemm::gemm_rowcol_oe_kernel<HN_ACT_NONE, 96><<<pgrid, gemm::NT, 0, st>>>(p);
        } else if (act == HN_ACT_GELU_TANH) {
            gemm::gemm_rowcol_oe_kernel<HN_ACT_GELU_TANH, 128><<<pgrid, gemm::NT, 0, st>>>(p);
        } else {
            gemm::gemm_rowcol_oe_kernel<HN_ACT_NONE, 128><<<pgrid, gemm::NT, 0, st>>>(p);
        }
    } else if (mode == gemm::ROWCOL) {
        gemm::gemm_rowcol_kernel<<<grid, gemm::NT, 0, (hipStream_t)stream>>>(p);
    } else {
        if (stripe) {
            if (const int rc = launch_tail(); rc != HN_OK) return rc;
        }
        gemm::gemm_bw8_kernel<<<grid, gemm::NT8, 0, (hipStream_t)stream>>>(p);
    }
    return check_launch(who);
}

extern "C" int hn_gemm_fp8_rowcol(const void* a, const void* b, const float* sa, const float* sb,
                                  const void* bias, void* out, int64_t M, int64_t N, int64_t K,
                                  int64_t ldc, int act, void* stream) {
    return gemm_launch(gemm::ROWCOL, a, b, sa, sb, bias, out, M, N, K, ldc, act, stream,
                       "hn_gemm_fp8_rowcol");
}

extern "C" int hn_gemm_fp8_blockwise(const void* a, const void* b, const float* sa,
                                     const float* sb, void* out, int64_t M, int64_t N, int64_t K,
                                     void* stream) {
    return gemm_launch(gemm::BLOCKWISE, a, b, sa, sb, nullptr, out, M, N, K, N, HN_ACT_NONE,
                       stream, "hn_gemm_fp8_blockwise");
}

#ifdef HN_GEMM_PHASE_STAMPS
// Measurement build only: copies the phase stamps (unsigned 64-bit,
// [16 workgroups][12 tiles][8 phases]) to host, or clears them (clear != 0).
extern "C" int hn_gemm_phase_stamps(void* host, int64_t bytes, int clear) {
    static const unsigned long long zeros[gemm::STAMP_WGS][gemm::STAMP_TILES][gemm::STAMP_PHASES] = {};
    HN_REQUIRE(bytes == (int64_t)sizeof(zeros), HN_E_ARG, "hn_gemm_phase_stamps: wrong size");
    const hipError_t e = clear ? hipMemcpyToSymbol(HIP_SYMBOL(gemm::g_stamps), zeros, sizeof(zeros))
                               : hipMemcpyFromSymbol(host, HIP_SYMBOL(gemm::g_stamps), sizeof(zeros));
    HN_REQUIRE(e == hipSuccess, HN_E_LAUNCH, "hn_gemm_phase_stamps: copy failed");
    return HN_OK;
}
#endif
