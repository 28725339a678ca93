// Operand-load geometry, tile queues and output-store geometry of the
// persistent FP8 GEMM (gemm_rowcol_oe_kernel), shared by the kernel and by
// the CPU checkers in tests/: the same functions compute every load's offset,
// every workgroup's tiles and every store's offset in both.
//
// Each of the 4 waves fills stage rows by its own index: 1 KB load q of wave
// w covers rows 64 w + 8 q + lane / 8 (q = 0..7), one 16-byte chunk per lane,
// with the 128-byte rows XOR-swizzled (physical chunk lane % 8 holds logical
// chunk swz_pos(row, lane % 8)). A wave loads those rows whatever rows it
// multiplies, so each offset is capped by the source tile's own extent.
#pragma once
#include <stdint.h>

#if defined(__HIPCC__)
#include <hip/hip_runtime.h>
#define HN_GEMM_HD __host__ __device__ __forceinline__
#else
#define HN_GEMM_HD inline
#endif

namespace hn {
namespace gemm {

// Physical 16-byte chunk of logical chunk `chunk` in stage row `row` (an involution).
HN_GEMM_HD int swz_pos(int row, int chunk) { return chunk ^ ((row >> 1) & 7); }

// Per-lane load geometry for wave `wave` and lane id `l`: its row in load 0,
// its byte offsets within the row for even and odd loads, and row * K.
struct DmaLane {
    int row;
    uint32_t chunk[2];
    uint32_t rowk;
};

HN_GEMM_HD DmaLane dma_lane_of(int wave, int l, int64_t K) {
    DmaLane d;
    d.row = wave * 64 + (l >> 3);
    d.chunk[0] = (uint32_t)swz_pos(d.row, l & 7) << 4;
    d.chunk[1] = (uint32_t)swz_pos(d.row + 8, l & 7) << 4;
    d.rowk = (uint32_t)d.row * (uint32_t)K;
    return d;
}

// Largest offset a load may take from its K step's source address (tile
// origin + 128 step): the last 16-byte chunk of the step's 128-byte window in
// the source tile's last row inside the operand, (rows - 1) K + 112.
HN_GEMM_HD uint32_t dma_limit(int64_t tile_rows, int64_t K) {
    return (uint32_t)((tile_rows - 1) * K + 112);
}

// Offset of load q: row K + chunk + 8 q K, capped at lim. A row r <= last
// keeps its exact offset (r K + chunk <= last K + 112 since chunk <= 112); a
// row past the operand's end starts at >= (last + 1) K >= last K + 128 and
// reads the last chunk of the last row's window instead (never used).
HN_GEMM_HD uint32_t dma_offset(const DmaLane& d, int q, int64_t K, uint32_t lim) {
    const uint32_t off = d.rowk + d.chunk[q & 1] + (uint32_t)(8 * q) * (uint32_t)K;
    return off < lim ? off : lim;
}


// ---------------------------------------------------------------------------
// Operand loads of the tail-stripe kernel (gemm_tail_kernel), also shared with
// the CPU checker. A wave's stage holds the stripe's ar = 32 JB A rows, then
// its workgroup's 32 B rows, 128 bytes of K each; load q of a K step fills
// stage rows 8 q .. 8 q + 7, lane l bringing row 8 q + l / 8's logical chunk
// swz_pos(row, l % 8). Its source is A row min(m0 + row, M - 1) (rows past M
// repeat the last row; their outputs are not stored) or B row n0 + row - ar;
// tail_src gives the byte offset at K step 0 from that operand's start (a K
// step adds 128).
struct TailSrc {
    bool a;
    int64_t off;
};

HN_GEMM_HD TailSrc tail_src(int q, int l, int ar, int64_t m0, int64_t M, int64_t n0, int64_t K) {
    const int row = 8 * q + (l >> 3);
    const int64_t chunk = (int64_t)swz_pos(row, l & 7) * 16;
    TailSrc t;
    t.a = row < ar;
    if (t.a) {
        const int64_t m = m0 + row;
        t.off = (m < M ? m : M - 1) * K + chunk;
    } else {
        t.off = (n0 + row - ar) * K + chunk;
    }
    return t;
}

// The wide form (tail_wide, run by a persistent launch's light workgroups):
// the stage holds the stripe's ar A rows, then B rows n0 .. n0 + nb - 1 for
// the workgroup's columns, rows past its last column nlast reading column
// nlast (never stored); otherwise as tail_src.
HN_GEMM_HD TailSrc tail_wide_src(int q, int l, int ar, int64_t m0, int64_t M, int64_t n0, int64_t nlast,
                                 int64_t K) {
    const int row = 8 * q + (l >> 3);
    const int64_t chunk = (int64_t)swz_pos(row, l & 7) * 16;
    TailSrc t;
    t.a = row < ar;
    if (t.a) {
        const int64_t m = m0 + row;
        t.off = (m < M ? m : M - 1) * K + chunk;
    } else {
        const int64_t n = n0 + row - ar;
        t.off = (n < nlast ? n : nlast) * K + chunk;
    }
    return t;
}

// K steps of a tail wave: wave w of SK takes steps w + SK t, t < T =
// tail_steps(KT, w, SK); loads issued past its last step repeat step T - 1
// (in bounds, never read), so every step issues the same loads.
HN_GEMM_HD int tail_steps(int KT, int w, int SK) { return (KT - w + SK - 1) / SK; }
HN_GEMM_HD int tail_step(int w, int SK, int t, int T) { return w + SK * (t < T ? t : T - 1); }

// ---------------------------------------------------------------------------
// Tile queues of the row/column kernels, also shared with the CPU checker
// (tests/gemm_tiles_check.cpp enumerates every workgroup's tiles through these
// functions).

constexpr int GROUP_M = 8;  // tile rows per group of a queue (L2 reuse of A and B panels)

HN_GEMM_HD int imin(int a, int b) { return a < b ? a : b; }

// Tile counts of an M x N output in 256-row, bn-column tiles: whole tiles
// first (tm_full x tn_full), then the edge tiles (the last row stripe if M %
// 256 != 0, then the last column stripe if N % bn != 0); per_xcd is the
// longest XCD queue (each class split evenly over the 8 XCDs).
struct TileCounts {
    int tiles_m, tiles_n, tm_full, tn_full, m_tail, tiles_full, tiles_part, per_xcd;
};

HN_GEMM_HD TileCounts tile_counts(int64_t M, int64_t N, int bn) {
    TileCounts t;
    t.tiles_m = (int)((M + 255) / 256);
    t.tiles_n = (int)((N + bn - 1) / bn);
    t.tm_full = (int)(M / 256);
    t.tn_full = (int)(N / bn);
    t.m_tail = (int)(M % 256 != 0);
    t.tiles_full = t.tm_full * t.tn_full;
    t.tiles_part = t.tiles_m * t.tiles_n - t.tiles_full;
    t.per_xcd = (t.tiles_full + 7) / 8 + (t.tiles_part + 7) / 8;
    return t;
}

// Queue entry i of XCD x -> tile. An XCD's queue holds its share of the full
// tiles, in groups of GROUP_M tile rows walking N (so the ~32 tiles it runs at
// once share A and B panels in its L2), followed by its share of the edge
// tiles. Edge tiles skip the MFMAs of blocks outside the matrix and run
// shorter (a 48-row edge tile about 0.45-0.65 of a full one: their DMAs,
// barriers and epilogue stay).
template <class Q>
HN_GEMM_HD bool tile_at(const Q& p, int x, int i, int& tm, int& tn) {
    const int F = p.tiles_full, P = p.tiles_part;
    const int fx = F / 8 + (x < F % 8 ? 1 : 0);
    if (i < fx) {
        const int f = x * (F / 8) + imin(x, F % 8) + i;
        const int per_group = GROUP_M * p.tn_full;
        const int first_m = (f / per_group) * GROUP_M;
        const int gm = imin(GROUP_M, p.tm_full - first_m);
        tm = first_m + (f % per_group) % gm;
        tn = (f % per_group) / gm;
        return true;
    }
    const int q = i - fx;
    if (q >= P / 8 + (x < P % 8 ? 1 : 0)) return false;
    int g = x * (P / 8) + imin(x, P % 8) + q;
    if (p.m_tail) {
        if (g < p.tiles_n) { tm = p.tm_full; tn = g; return true; }
        g -= p.tiles_n;
    }
    tm = g;
    tn = p.tn_full;
    return true;
}

// Persistent launches: workgroup s of XCD x's S runs the queue's full tiles
// s, s + S, s + 2 S, ... (round k: entry k S + s). Of the fx full tiles, the
// first r = fx % S workgroups ("heavy") get one more than the other L = S - r
// ("light"). The edge tiles go to the light workgroups only, dealt round-robin
// after their full tiles, whenever there are at most 2 L of them: a light
// workgroup then ends at most two edge tiles (about one full tile) after its
// last full one, where dealing them on round-robin across all workgroups
// would give heavy ones an edge tile on top of their extra full one.
// Measured against the plain order (same box): 10 800 x 3072 x 12 288 (43 x
// 12 tiles, 63 full and 1.5 edge tiles per XCD) 361.6 -> 347.5 us, the north
// star (252 full and 6 edge tiles per XCD, S = 32) 381 -> 378 us, which is
// still 4 % above 10 752 rows (no edge tiles): two 48-row edge tiles take
// longer than a full one. With more than 2 L edge tiles, they follow the
// plain round-robin order.
template <class Q>
HN_GEMM_HD bool tile_of_slot(const Q& p, int x, int i, int S, int& tm, int& tn) {
    const int F = p.tiles_full, P = p.tiles_part;
    const int fx = F / 8 + (x < F % 8 ? 1 : 0);
    const int px = P / 8 + (x < P % 8 ? 1 : 0);
    const int r = fx % S, L = r ? S - r : S;
    if (i < fx || px > 2 * L) return tile_at(p, x, i, tm, tn);
    const int s = i % S, k = i / S;
    if (s < r) return false;                   // heavy: no edge tiles
    const int q = (k - fx / S) * L + (s - r);  // this light workgroup's edge tile
    if (q >= px) return false;
    return tile_at(p, x, fx + q, tm, tn);
}

// A persistent launch without edge tiles can hand the tail stripe (the last
// M % 256 <= 64 rows) to its "light" workgroups: those with one full tile
// fewer, idle for the launch's last tile round. light_index numbers them
// across the XCDs (XCD by XCD, in slot order), -1 for the others;
// light_count is their number and says whether every XCD has some.
template <class Q>
HN_GEMM_HD int light_index(const Q& p, int x, int s, int S) {
    int before = 0;
    for (int xx = 0; xx < 8; ++xx) {
        const int r = (p.tiles_full / 8 + (xx < p.tiles_full % 8 ? 1 : 0)) % S;
        if (xx == x) return r > 0 && s >= r ? before + (s - r) : -1;
        before += r > 0 ? S - r : 0;
    }
    return -1;
}

template <class Q>
HN_GEMM_HD int light_count(const Q& p, int S, bool* every_xcd) {
    int n = 0;
    *every_xcd = true;
    for (int x = 0; x < 8; ++x) {
        const int r = (p.tiles_full / 8 + (x < p.tiles_full % 8 ? 1 : 0)) % S;
        if (r == 0) *every_xcd = false;
        else n += S - r;
    }
    return n;
}

// A wave's share of a tile: the 32-column blocks (imax) and 32-row blocks
// (jmax) that hold any output inside the M x N matrix -- what its MFMAs
// compute. A wave with 97..127 rows left has four row blocks, some of whose
// rows are past M: its stores rely on the output window below.
struct WaveExtent {
    int imax, jmax;
};

HN_GEMM_HD WaveExtent wave_extent(int64_t M, int64_t N, int64_t row0, int64_t col0, int wc) {
    const int64_t rows = M - row0, cols = N - col0;
    WaveExtent e;
    e.jmax = rows >= 128 ? 4 : (rows <= 0 ? 0 : (int)((rows + 31) >> 5));
    e.imax = cols >= wc ? wc / 32 : (cols <= 0 ? 0 : (int)(cols >> 5));
    return e;
}

// ---------------------------------------------------------------------------
// Output stores of the persistent kernel, also shared with the CPU checker
// (tests/gemm_tiles_check.cpp walks every store of every wave through these).
//
// A wave stores its 128 x wc sub-tile (first row m0w, first column n0w)
// through a raw buffer "window": base = element (m0w, n0w), size =
// out_window_bytes. A store's offset is bytes from the base (row * pitch +
// 2 * column, pitch = 2 ldc); the buffer's range check drops a store whose
// offset is at or past the size, i.e. every store to a row at or past M (a
// store never straddles a row, so never the size). The size is zero when no
// row or no column block is inside. Columns past N: with wc = 128 and N a
// multiple of 128 a wave's columns are all inside or none (imax 4 or 0);
// with wc = 96 each store tests its columns against imax (oe_store_on).

HN_GEMM_HD uint32_t mul24(uint32_t a, uint32_t b) {
#if defined(__HIP_DEVICE_COMPILE__)
    return __umul24(a, b);
#else
    return (uint32_t)((uint64_t)(a & 0xffffffu) * (uint64_t)(b & 0xffffffu));
#endif
}

HN_GEMM_HD int64_t out_window_bytes(int64_t M, int64_t ldc, int64_t m0w, int imax) {
    const int64_t rows = M - m0w;
    if (rows <= 0 || imax <= 0) return 0;
    return (rows > 128 ? 128 : rows) * ldc * 2;
}

// Carried store q (0..3) of pass P (0..3), 16 bytes read back from the
// staging area: row 32 (P / 2) + 8 q + lane / 8, columns 64 (P % 2) + 8 (lane
// % 8) + {0..7} of the sub-tile (stored during the next tile's first K steps
// or, before an edge tile and after the last tile, at once).
HN_GEMM_HD uint32_t oe_store_off(uint32_t pitch, int lane, int P, int q) {
    return mul24((uint32_t)(lane >> 3), pitch) + (uint32_t)((lane & 7) << 4) +
           (uint32_t)(32 * (P >> 1) + 8 * q) * pitch + (uint32_t)(128 * (P & 1));
}

HN_GEMM_HD bool oe_store_on(int wc, int imax, int P, int lane) {
    return wc == 128 || 64 * (P & 1) + 8 * (lane & 7) < 32 * imax;
}

// Row order of the MFMA fragment reads: lane l reads row oe_row(l % 32) of
// each 32-row block of both operands (bits 2 and 3 exchanged; an involution
// that maps each aligned group of 16 rows onto itself). The accumulator block
// then holds, for lane (h = l / 32, r = l % 32), output row oe_row(r) and
// columns 16 (v / 8) + 8 h + v % 8 for its values v = 0..15: eight
// consecutive columns per group of 8 values.
HN_GEMM_HD int oe_row(int r) { return (r & ~12) | ((r & 4) << 1) | ((r & 8) >> 1); }

// Direct store (pass P = 4..7, column block i = 2 (P % 2) + ii, half hv), 16
// bytes straight from the accumulator: row 32 (P / 2) + oe_row(lane % 32),
// columns 32 i + 16 hv + 8 (lane / 32) + {0..7} of the sub-tile.
HN_GEMM_HD uint32_t direct_store_off(uint32_t pitch, int lane, int P, int ii, int hv) {
    const int i = 2 * (P & 1) + ii;
    return mul24((uint32_t)oe_row(lane & 31), pitch) + (uint32_t)(32 * (P >> 1)) * pitch +
           (uint32_t)(2 * (32 * i + 16 * hv + 8 * (lane >> 5)));
}

HN_GEMM_HD bool direct_store_on(int wc, int imax, int i) { return 32 * i < wc && (wc == 128 || i < imax); }

}  // namespace gemm
}  // namespace hn
