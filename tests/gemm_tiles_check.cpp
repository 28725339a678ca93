// CPU checker of the persistent FP8 GEMM's tile queues. It walks every
// workgroup of a launch through hy-nomas_amd/csrc/gemm_dma.h's tile_of_slot
// exactly as gemm_rowcol_oe_kernel does (workgroup `slot` of XCD x starts at
// queue entry slot and steps by S, the workgroups per XCD, until the first
// entry without a tile) and counts how often each output tile is produced.
// For every wave of every tile it also takes wave_extent (the same header)
// and, where the wave counts as inside, walks the stores its unchecked direct
// passes make -- rows 32 j + r (j = 2, 3; r < 32), columns 32 i + 8 vq + 4 h
// + e (i < wc / 32) of its sub-tile -- and counts those outside M x N; and it
// checks that the blocks below (imax, jmax) cover every output of the wave.
//
// Usage: gemm_tiles_check M N BN CUS
// Prints: tiles=<count> missing=<n> repeated=<n> max_full=<n> max_edge=<n>
//         max_load_x100=<100 * max over workgroups of full + edge / 2>
//         unchecked_outside=<stores> uncovered=<outputs> blocks_not_inside=<waves>
#include <cstdio>
#include <cstdlib>
#include <vector>

#include "../hy-nomas_amd/csrc/gemm_dma.h"

using namespace hn::gemm;

// The fields the queue functions read, filled the way the launch fills them.
struct Queue {
    int tiles_n, tm_full, tn_full, tiles_full, tiles_part, m_tail;
};

int main(int argc, char** argv) {
    if (argc != 5) {
        fprintf(stderr, "usage: %s M N BN CUS\n", argv[0]);
        return 2;
    }
    const long long M = atoll(argv[1]), N = atoll(argv[2]);
    const int bn = atoi(argv[3]), cus = atoi(argv[4]);
    const TileCounts t = tile_counts(M, N, bn);
    const Queue q{t.tiles_n, t.tm_full, t.tn_full, t.tiles_full, t.tiles_part, t.m_tail};
    const int per_xcd_cus = cus / 8 > 0 ? cus / 8 : 1;
    const int S = t.per_xcd < per_xcd_cus ? t.per_xcd : per_xcd_cus;  // the launch's grid / 8
    std::vector<int> hits((size_t)t.tiles_m * t.tiles_n, 0);
    int max_full = 0, max_edge = 0, max_load = 0, bad = 0;
    long long unchecked_outside = 0, uncovered = 0, blocks_not_inside = 0;
    const int wc = bn / 2;
    auto check_waves = [&](int tm, int tn) {
        for (int wm = 0; wm < 2; ++wm)
            for (int wn = 0; wn < 2; ++wn) {
                const long long row0 = (long long)tm * 256 + wm * 128, col0 = (long long)tn * bn + wn * wc;
                const WaveExtent e = wave_extent(M, N, row0, col0, wc);
                if (e.jmax == 4 && e.imax == wc / 32 && !e.inside) ++blocks_not_inside;
                for (int r = 0; r < 128; ++r)
                    for (int c = 0; c < wc; ++c) {
                        const bool valid = row0 + r < M && col0 + c < N;
                        if (valid && !(r / 32 < e.jmax && c / 32 < e.imax)) ++uncovered;
                    }
                if (!e.inside) continue;
                for (int j = 2; j < 4; ++j)
                    for (int r = 0; r < 32; ++r)
                        for (int i = 0; i < wc / 32; ++i)
                            for (int vq = 0; vq < 4; ++vq)
                                for (int h = 0; h < 2; ++h)
                                    for (int x = 0; x < 4; ++x) {
                                        const long long m = row0 + 32 * j + r;
                                        const long long n = col0 + 32 * i + 8 * vq + 4 * h + x;
                                        if (m >= M || n >= N) ++unchecked_outside;
                                    }
            }
    };
    for (int x = 0; x < 8; ++x)
        for (int slot = 0; slot < S; ++slot) {
            int full = 0, edge = 0, tm, tn;
            for (int i = slot; tile_of_slot(q, x, i, S, tm, tn); i += S) {
                if (tm < 0 || tm >= t.tiles_m || tn < 0 || tn >= t.tiles_n) {
                    ++bad;
                    break;
                }
                ++hits[(size_t)tm * t.tiles_n + tn];
                check_waves(tm, tn);
                if (tm < t.tm_full && tn < t.tn_full) ++full;
                else ++edge;
            }
            max_full = full > max_full ? full : max_full;
            max_edge = edge > max_edge ? edge : max_edge;
            const int load = 100 * full + 50 * edge;
            max_load = load > max_load ? load : max_load;
        }
    int missing = 0, repeated = 0;
    for (int h : hits) {
        missing += h == 0;
        repeated += h > 1;
    }
    printf("tiles=%zu missing=%d repeated=%d out_of_range=%d max_full=%d max_edge=%d max_load_x100=%d "
           "unchecked_outside=%lld uncovered=%lld blocks_not_inside=%lld\n",
           hits.size(), missing, repeated, bad, max_full, max_edge, max_load, unchecked_outside, uncovered,
           blocks_not_inside);
    return 0;
}
