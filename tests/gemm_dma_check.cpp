// CPU bounds check of the persistent FP8 GEMM's operand loads, built from the
// kernel's own load geometry (hy-nomas_amd/csrc/gemm_dma.h): for an M x N x K
// problem with bn-column tiles, every load of every wave, of every tile and
// every K step, of both operands, is checked to stay inside its operand, and
// loads of rows inside a tile to keep their exact offset.
//
// usage: gemm_dma_check M N K bn [nocap]
//   nocap: leave the offsets uncapped (the checker must then find loads out
//          of bounds for a shape whose last tile is partial).
// Prints "loads=<n> out_of_bounds=<n> wrong_offset=<n>"; exit 0.
#include <stdint.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>

#include "../hy-nomas_amd/csrc/gemm_dma.h"

using namespace hn::gemm;

int main(int argc, char** argv) {
    if (argc < 5) {
        fprintf(stderr, "usage: %s M N K bn [nocap]\n", argv[0]);
        return 2;
    }
    const int64_t M = atoll(argv[1]), N = atoll(argv[2]), K = atoll(argv[3]), bn = atoll(argv[4]);
    const bool nocap = argc > 5 && strcmp(argv[5], "nocap") == 0;
    if (M <= 0 || N <= 0 || K <= 0 || K % 128 || (bn != 256 && bn != 192)) {
        fprintf(stderr, "bad shape\n");
        return 2;
    }
    long long loads = 0, oob = 0, wrong = 0;
    const int64_t extents[2] = {M, N}, tiles[2] = {256, bn};
    for (int operand = 0; operand < 2; ++operand) {
        const int64_t extent = extents[operand], tile = tiles[operand];
        for (int64_t t0 = 0; t0 < extent; t0 += tile) {
            const int64_t rows = extent - t0 < tile ? extent - t0 : tile;
            const uint32_t lim = nocap ? 0xffffffffu : dma_limit(rows, K);
            for (int wave = 0; wave < 4; ++wave)
                for (int lane = 0; lane < 64; ++lane) {
                    const DmaLane d = dma_lane_of(wave, lane, K);
                    for (int q = 0; q < 8; ++q) {
                        const uint32_t off = dma_offset(d, q, K, lim);
                        const int64_t r = d.row + 8 * q;
                        if (r < rows && off != (uint64_t)r * K + d.chunk[q & 1]) ++wrong;
                        for (int64_t step = 0; step < K / 128; ++step) {
                            const int64_t addr = t0 * K + step * 128 + (int64_t)off;
                            ++loads;
                            if (addr < 0 || addr + 16 > extent * K) ++oob;
                        }
                    }
                }
        }
    }
    printf("loads=%lld out_of_bounds=%lld wrong_offset=%lld\n", loads, oob, wrong);
    return 0;
}
