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
//
// usage: gemm_dma_check tail M N K SK JB
//   The tail-stripe kernel's loads (tail_src, tail_steps, tail_step) for the
//   stripe [M - M % 256, M) when M % 256 <= 64, else [0, M) (M <= 64): every
//   load of every workgroup (N / 32 of them), wave, lane and issued step
//   (the TAIL_STAGES = 3 re-loads past a wave's last step included), against
//   its operand's extent; the rows inside the stripe and the B rows at their
//   exact offsets; and each K step multiplied by exactly one wave.
// Prints "loads=<n> out_of_bounds=<n> wrong_offset=<n> step_cover_errors=<n>".
//
// usage: gemm_dma_check tailwide M N K CUS
//   The wide tail items the persistent kernel's light workgroups run
//   (tail_wide_src, light_index, light_count) for a launch over the rows
//   above the stripe [M - M % 256, M), with CUS / 8 workgroups per XCD (as
//   the launch takes them): every load of every light workgroup, wave, lane
//   and K step against its operand, the exact offsets of rows inside the
//   stripe and of B rows inside the item, the items covering [0, N) exactly
//   once, and each item on a workgroup with one full tile fewer than the
//   longest queue. fused=0 when the launch would not fuse the stripe.
// Prints "fused=<0|1> loads=<n> out_of_bounds=<n> wrong_offset=<n> column_cover_errors=<n>
//         not_light=<n> cols=<n>".
#include <stdint.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>

#include "../hy-nomas_amd/csrc/gemm_dma.h"

using namespace hn::gemm;

static int tail_main(int argc, char** argv) {
    if (argc != 7) {
        fprintf(stderr, "usage: %s tail M N K SK JB\n", argv[0]);
        return 2;
    }
    const int64_t M = atoll(argv[2]), N = atoll(argv[3]), K = atoll(argv[4]);
    const int SK = atoi(argv[5]), JB = atoi(argv[6]);
    if (M <= 0 || N <= 0 || N % 128 || K % 128 || K / 128 < SK || (JB != 1 && JB != 2)) {
        fprintf(stderr, "bad shape\n");
        return 2;
    }
    const int64_t m0 = M % 256 <= 64 && M >= 256 ? M - M % 256 : 0;
    const int ar = 32 * JB, nq = (ar + 32) / 8, KT = (int)(K / 128);
    long long loads = 0, oob = 0, wrong = 0, cover = 0;
    for (int64_t blk = 0; blk < N / 32; ++blk) {
        const int64_t n0 = blk * 32;
        int* hits = (int*)calloc((size_t)KT, sizeof(int));
        for (int w = 0; w < SK; ++w) {
            const int T = tail_steps(KT, w, SK);
            if (T < 1) ++cover;
            for (int t = 0; t < T; ++t) ++hits[tail_step(w, SK, t, T)];
            for (int lane = 0; lane < 64; ++lane)
                for (int q = 0; q < nq; ++q) {
                    const TailSrc ts = tail_src(q, lane, ar, m0, M, n0, K);
                    const int row = 8 * q + (lane >> 3);
                    const int64_t chunk = (int64_t)swz_pos(row, lane & 7) * 16;
                    if (ts.a && m0 + row < M && ts.off != (m0 + row) * K + chunk) ++wrong;
                    if (!ts.a && ts.off != (n0 + row - ar) * K + chunk) ++wrong;
                    const int64_t extent = ts.a ? M : N;
                    for (int t = 0; t < T + 3; ++t) {
                        const int64_t addr = ts.off + (int64_t)tail_step(w, SK, t, T) * 128;
                        ++loads;
                        if (addr < 0 || addr + 16 > extent * K) ++oob;
                    }
                }
        }
        for (int s = 0; s < KT; ++s) cover += hits[s] != 1;
        free(hits);
    }
    printf("loads=%lld out_of_bounds=%lld wrong_offset=%lld step_cover_errors=%lld\n", loads, oob, wrong, cover);
    return 0;
}

struct Queue {
    int tiles_n, tm_full, tn_full, tiles_full, tiles_part, m_tail;
};

static int tailwide_main(int argc, char** argv) {
    if (argc != 6) {
        fprintf(stderr, "usage: %s tailwide M N K CUS\n", argv[0]);
        return 2;
    }
    const int64_t M = atoll(argv[2]), N = atoll(argv[3]), K = atoll(argv[4]);
    const int cus = atoi(argv[5]);
    if (M <= 0 || N <= 0 || N % 128 || K % 128 || K / 128 < 2 || M % 256 == 0 || M % 256 > 64 || M < 256) {
        fprintf(stderr, "bad shape\n");
        return 2;
    }
    const int64_t Mt = M - M % 256;
    const TileCounts t = tile_counts(Mt, N, 256);
    const Queue q{t.tiles_n, t.tm_full, t.tn_full, t.tiles_full, t.tiles_part, t.m_tail};
    const int per_xcd_cus = cus / 8 > 0 ? cus / 8 : 1;
    const int S = t.per_xcd < per_xcd_cus ? t.per_xcd : per_xcd_cus;
    bool every = false;
    const int nl = light_count(q, S, &every);
    const int64_t cols = nl > 0 ? (N / 32 + nl - 1) / nl * 32 : 0;
    const bool fused = t.tiles_part == 0 && every && nl >= 16 && cols <= 384 && K <= 4096;
    long long loads = 0, oob = 0, wrong = 0, cover = 0, not_light = 0;
    if (fused) {
        const int ar = M % 256 > 32 ? 64 : 32, nq = (ar + 384) / 8, KT = (int)(K / 128);
        int* hits = (int*)calloc((size_t)N, sizeof(int));
        int longest = 0;
        for (int x = 0; x < 8; ++x)
            for (int s = 0; s < S; ++s) {
                int n = 0, tm, tn;
                for (int i = s; tile_of_slot(q, x, i, S, tm, tn); i += S) ++n;
                longest = n > longest ? n : longest;
            }
        for (int x = 0; x < 8; ++x)
            for (int s = 0; s < S; ++s) {
                const int li = light_index(q, x, s, S);
                if (li < 0) continue;
                int n = 0, tm, tn;
                for (int i = s; tile_of_slot(q, x, i, S, tm, tn); i += S) ++n;
                if (n != longest - 1) ++not_light;
                const int64_t n0 = (int64_t)li * cols;
                if (n0 >= N) continue;
                const int64_t nc = N - n0 < cols ? N - n0 : cols;
                for (int64_t c = n0; c < n0 + nc; ++c) ++hits[c];
                for (int w = 0; w < 4; ++w)
                    for (int lane = 0; lane < 64; ++lane)
                        for (int k = 0; k < nq / 4; ++k) {
                            const int qq = w + 4 * k;
                            const TailSrc ts = tail_wide_src(qq, lane, ar, Mt, M, n0, n0 + nc - 1, K);
                            const int row = 8 * qq + (lane >> 3);
                            const int64_t chunk = (int64_t)swz_pos(row, lane & 7) * 16;
                            if (ts.a && Mt + row < M && ts.off != (Mt + row) * K + chunk) ++wrong;
                            if (!ts.a && row - ar < nc && ts.off != (n0 + row - ar) * K + chunk) ++wrong;
                            const int64_t extent = ts.a ? M : N;
                            for (int st = 0; st < KT; ++st) {
                                const int64_t addr = ts.off + (int64_t)st * 128;
                                ++loads;
                                if (addr < 0 || addr + 16 > extent * K) ++oob;
                            }
                        }
            }
        for (int64_t c = 0; c < N; ++c) cover += hits[c] != 1;
        free(hits);
    }
    printf("fused=%d loads=%lld out_of_bounds=%lld wrong_offset=%lld column_cover_errors=%lld not_light=%lld "
           "cols=%lld\n", fused ? 1 : 0, loads, oob, wrong, cover, not_light, (long long)cols);
    return 0;
}

int main(int argc, char** argv) {
    if (argc > 1 && strcmp(argv[1], "tail") == 0) return tail_main(argc, argv);
    if (argc > 1 && strcmp(argv[1], "tailwide") == 0) return tailwide_main(argc, argv);
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
