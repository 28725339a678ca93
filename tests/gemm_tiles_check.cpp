// CPU checker of the persistent FP8 GEMM's tile queues. It walks every
// workgroup of a launch through hy-nomas_amd/csrc/gemm_dma.h's tile_of_slot
// exactly as gemm_rowcol_oe_kernel does (workgroup `slot` of XCD x starts at
// queue entry slot and steps by S, the workgroups per XCD, until the first
// entry without a tile) and counts how often each output tile is produced.
//
// Usage: gemm_tiles_check M N BN CUS
// Prints: tiles=<count> missing=<n> repeated=<n> max_full=<n> max_edge=<n>
//         max_load_x100=<100 * max over workgroups of full + edge / 2>
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
    for (int x = 0; x < 8; ++x)
        for (int slot = 0; slot < S; ++slot) {
            int full = 0, edge = 0, tm, tn;
            for (int i = slot; tile_of_slot(q, x, i, S, tm, tn); i += S) {
                if (tm < 0 || tm >= t.tiles_m || tn < 0 || tn >= t.tiles_n) {
                    ++bad;
                    break;
                }
                ++hits[(size_t)tm * t.tiles_n + tn];
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
    printf("tiles=%zu missing=%d repeated=%d out_of_range=%d max_full=%d max_edge=%d max_load_x100=%d\n",
           hits.size(), missing, repeated, bad, max_full, max_edge, max_load);
    return 0;
}
