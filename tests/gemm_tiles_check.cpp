// CPU checker of the persistent FP8 GEMM's tile queues and output stores. It
// walks every workgroup of a launch through hy-nomas_amd/csrc/gemm_dma.h's
// tile_of_slot exactly as gemm_rowcol_oe_kernel does (workgroup `slot` of XCD
// x starts at queue entry slot and steps by S, the workgroups per XCD, until
// the first entry without a tile) and counts how often each output tile is
// produced. With STORES = 1 it also walks every store the kernel makes for
// every tile -- per lane and wave 16 carried stores and 16 direct stores of
// 16 bytes, with the same header's offsets, predicates and output-window
// sizes -- and applies the buffer range check (a store whose offset is at or
// past the window's size is dropped): each output element inside M x N must
// be written exactly once, and no store may land outside M x N or outside its
// own wave's columns, or straddle the window's end. It also checks that each
// wave's MFMA blocks (wave_extent's imax, jmax) cover all its outputs.
//
// Usage: gemm_tiles_check M N BN CUS [LDC STORES]
// Prints: tiles=<count> missing=<n> repeated=<n> out_of_range=<n> max_full=<n>
//         max_edge=<n> max_load_x100=<100 * max over workgroups of full + edge / 2>
//         uncovered=<outputs> stores=<kept stores> dropped=<stores>
//         store_outside=<n> straddle=<n> unwritten=<elements> rewritten=<elements>
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
    if (argc != 5 && argc != 7) {
        fprintf(stderr, "usage: %s M N BN CUS [LDC STORES]\n", argv[0]);
        return 2;
    }
    const long long M = atoll(argv[1]), N = atoll(argv[2]);
    const int bn = atoi(argv[3]), cus = atoi(argv[4]);
    const long long ldc = argc == 7 ? atoll(argv[5]) : N;
    const bool walk_stores = argc == 7 && atoi(argv[6]) != 0;
    const TileCounts t = tile_counts(M, N, bn);
    const Queue q{t.tiles_n, t.tm_full, t.tn_full, t.tiles_full, t.tiles_part, t.m_tail};
    const int per_xcd_cus = cus / 8 > 0 ? cus / 8 : 1;
    const int S = t.per_xcd < per_xcd_cus ? t.per_xcd : per_xcd_cus;  // the launch's grid / 8
    std::vector<int> hits((size_t)t.tiles_m * t.tiles_n, 0);
    std::vector<unsigned char> writes(walk_stores ? (size_t)(M * N) : 0, 0);
    int max_full = 0, max_edge = 0, max_load = 0, bad = 0;
    long long uncovered = 0, kept = 0, dropped = 0, outside = 0, straddle = 0;
    const int wc = bn / 2;
    const uint32_t pitch = (uint32_t)(ldc * 2);
    // One store of `bytes` bytes at offset `off` of the window of the wave at
    // (row0, col0) whose size is `size`.
    auto store = [&](long long row0, long long col0, long long size, uint32_t off, int bytes) {
        if ((long long)off >= size) {
            ++dropped;
            return;
        }
        ++kept;
        if ((long long)off + bytes > size) ++straddle;
        const long long r = off / pitch, c = (off % pitch) / 2;
        for (int e = 0; e < bytes / 2; ++e) {
            const long long m = row0 + r, n = col0 + c + e;
            if (r >= 128 || c + e >= wc || m >= M || n >= N) {
                ++outside;
                continue;
            }
            unsigned char& w = writes[(size_t)(m * N + n)];
            w = w < 255 ? w + 1 : w;
        }
    };
    auto check_waves = [&](int tm, int tn) {
        for (int wm = 0; wm < 2; ++wm)
            for (int wn = 0; wn < 2; ++wn) {
                const long long row0 = (long long)tm * 256 + wm * 128, col0 = (long long)tn * bn + wn * wc;
                const WaveExtent e = wave_extent(M, N, row0, col0, wc);
                for (int r = 0; r < 128; ++r)
                    for (int c = 0; c < wc; ++c) {
                        const bool valid = row0 + r < M && col0 + c < N;
                        if (valid && !(r / 32 < e.jmax && c / 32 < e.imax)) ++uncovered;
                    }
                if (!walk_stores) continue;
                const long long size = out_window_bytes(M, ldc, row0, e.imax);
                for (int lane = 0; lane < 64; ++lane) {
                    for (int P = 0; P < 4; ++P)  // carried passes (or their flush)
                        for (int qq = 0; qq < 4; ++qq)
                            if (oe_store_on(wc, e.imax, P, lane))
                                store(row0, col0, size, oe_store_off(pitch, lane, P, qq), 16);
                    for (int P = 4; P < 8; ++P)  // direct passes
                        for (int ii = 0; ii < 2; ++ii)
                            for (int hv = 0; hv < 2; ++hv)
                                if (direct_store_on(wc, e.imax, 2 * (P & 1) + ii))
                                    store(row0, col0, size, direct_store_off(pitch, lane, P, ii, hv), 16);
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
    long long unwritten = 0, rewritten = 0;
    for (unsigned char w : writes) {
        unwritten += w == 0;
        rewritten += w > 1;
    }
    printf("tiles=%zu missing=%d repeated=%d out_of_range=%d max_full=%d max_edge=%d max_load_x100=%d "
           "uncovered=%lld stores=%lld dropped=%lld store_outside=%lld straddle=%lld unwritten=%lld "
           "rewritten=%lld\n",
           hits.size(), missing, repeated, bad, max_full, max_edge, max_load, uncovered, kept, dropped, outside,
           straddle, unwritten, rewritten);
    return 0;
}
