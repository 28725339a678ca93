"""Tile queues and output stores of the persistent FP8 GEMM (CPU, no GPU needed).

`gemm_rowcol_oe_kernel` deals each XCD's queue over its workgroups with
`tile_of_slot` (`hy-nomas_amd/csrc/gemm_dma.h`): full tiles round-robin, then
the edge tiles to the workgroups with one full tile fewer. Its stores go
through per-wave buffer windows whose range check drops the rows past M, at
offsets from the same header. This test compiles that header into
`tests/gemm_tiles_check.cpp` with g++, walks every workgroup's tiles as the
kernel does, and checks that each output tile is produced exactly once -- a
persistent kernel that skipped or repeated a tile would leave output unwritten
or write it twice -- that every store the kernel makes either lands inside
M x N and its own wave's columns or is dropped by the window, writing each
output element exactly once, and that at the north-star and fc2 shapes no
workgroup runs a full tile plus an edge tile beyond the longest full-tile
queue."""
import subprocess
from pathlib import Path

import pytest

HERE = Path(__file__).resolve().parent


@pytest.fixture(scope="module")
def checker(tmp_path_factory):
    exe = tmp_path_factory.mktemp("tiles") / "gemm_tiles_check"
    subprocess.run(["g++", "-O2", "-std=c++17", "-Wall", "-Werror", str(HERE / "gemm_tiles_check.cpp"),
                    "-o", str(exe)], check=True)
    return exe


def _run(exe, M, N, bn, cus=256, ldc=None, stores=False):
    args = [str(exe), str(M), str(N), str(bn), str(cus)]
    if stores:
        args += [str(ldc or N), "1"]
    out = subprocess.run(args, check=True, capture_output=True, text=True).stdout
    return {k: int(v) for k, v in (kv.split("=") for kv in out.split())}


def _stores_ok(r):
    return (r["store_outside"] == 0 and r["straddle"] == 0 and r["unwritten"] == 0 and r["rewritten"] == 0
            and r["stores"] > 0)


@pytest.mark.parametrize("M,N,bn", [
    (10800, 12288, 256), (10800, 3072, 256), (10800, 9216, 256), (10800, 4096, 256), (10800, 12288 + 64, 256),
    (4096, 3072, 192), (132, 12288, 256), (132, 3072, 192), (4996, 3072, 256), (1, 128, 256),
    (300, 640, 256), (257, 257, 256), (10752, 12288, 256), (8192, 8192, 256), (5000, 7000, 256),
    (65536, 1024, 256), (100, 256, 192), (100, 256, 256), (227, 1024, 256), (97, 384, 192),
])
@pytest.mark.parametrize("cus", [256, 80])
def test_every_tile_exactly_once(checker, M, N, bn, cus):
    # the stores are walked once per shape, for the GEMM's N (a multiple of
    # 128; 257 and 7000 only exercise the queues)
    stores = cus == 256 and N % 128 == 0
    r = _run(checker, M, N, bn, cus, stores=stores)
    assert r["missing"] == 0 and r["repeated"] == 0 and r["out_of_range"] == 0, r
    if N % 128 == 0:
        # each wave's MFMA blocks cover all its outputs
        assert r["uncovered"] == 0, r
    if stores:
        assert _stores_ok(r), r


@pytest.mark.parametrize("M,N,bn", [(100, 256, 192), (227, 1024, 256), (10752 + 100, 3072, 256), (48, 640, 256)])
def test_rows_past_m_are_dropped_by_the_window(checker, M, N, bn):
    """Waves with fewer than 128 rows left (97..127 of them among these
    shapes: four row blocks, some rows past M) store whole 128-row sub-tiles;
    the window drops the stores past M and every output is still written
    once. Taking four row blocks for a whole sub-tile once let stores past row
    M through (a GPU memory fault at M = 100)."""
    r = _run(checker, M, N, bn, stores=True)
    assert r["dropped"] > 0 and _stores_ok(r), r


@pytest.mark.parametrize("M,N,bn,ldc", [(300, 640, 256, 648), (300, 384, 192, 392), (130, 256, 256, 1 << 22),
                                        (97, 384, 192, 1 << 22)])
def test_row_pitch_past_n(checker, M, N, bn, ldc):
    """ldc > N: the stores keep to the first N columns of each row, up to the
    largest pitch the GEMM accepts (2^22 columns, 128 rows of which still fit
    the 32-bit offsets)."""
    r = _run(checker, M, N, bn, ldc=ldc, stores=True)
    assert _stores_ok(r), r


def test_a_full_window_is_caught(tmp_path):
    """The checker sees stores past M: built with a window that always spans
    128 rows (the planted mistake, in the checker's CPU build only), the
    M = 100 shape reports stores outside the matrix."""
    exe = tmp_path / "gemm_tiles_check_planted"
    src = (HERE / "gemm_tiles_check.cpp").read_text().replace(
        "out_window_bytes(M, ldc, row0, e.imax)", "(e.imax > 0 && row0 < M ? 128 * ldc * 2 : 0)")
    assert "128 * ldc * 2" in src
    (tmp_path / "planted.cpp").write_text(src.replace('#include "../hy-nomas_amd/csrc/gemm_dma.h"',
                                                      f'#include "{HERE.parent}/hy-nomas_amd/csrc/gemm_dma.h"'))
    subprocess.run(["g++", "-O2", "-std=c++17", "-Wall", "-Werror", str(tmp_path / "planted.cpp"), "-o", str(exe)],
                   check=True)
    r = _run(exe, 100, 256, 256, stores=True)
    assert r["store_outside"] > 0, r


@pytest.mark.parametrize("M,N,full_rounds", [(10800, 12288, 8), (10800, 3072, 2), (10800, 9216, 6)])
def test_edge_tiles_go_to_the_shorter_queues(checker, M, N, full_rounds):
    # 10800 rows: a 48-row last tile row. The longest queue holds full_rounds
    # full tiles; the edge tiles (half-cost in this count) land on the
    # workgroups with one full tile fewer, so no queue exceeds full_rounds.
    r = _run(checker, M, N, 256)
    assert r["max_full"] == full_rounds and r["max_load_x100"] == 100 * full_rounds, r
