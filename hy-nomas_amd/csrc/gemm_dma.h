// Operand-load geometry of the persistent FP8 GEMM (gemm_rowcol_oe_kernel),
// shared by the kernel and by the CPU bounds checker in tests/: the same
// functions compute every load's offset in both.
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

}  // namespace gemm
}  // namespace hn
