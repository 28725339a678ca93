"""Tile queues of the persistent FP8 GEMM (CPU, no GPU needed).

`gemm_rowcol_oe_kernel` deals each XCD's queue over its workgroups with
`tile_of_slot` (`hy-nomas_amd/csrc/gemm_dma.h`): full tiles round-robin, then
the edge tiles to the workgroups with one full tile fewer. This test compiles
that header into `tests/gemm_tiles_check.cpp` with g++, walks every
workgroup's tiles as the kernel does, and checks that each output tile is
produced exactly once -- a persistent kernel that skipped or repeated a tile
would leave output unwritten or write it twice -- and that at the north-star
and fc2 shapes no workgroup runs a full tile plus an edge tile beyond the
longest full-tile queue."""
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


def _run(exe, M, N, bn, cus=256):
    out = subprocess.run([str(exe), str(M), str(N), str(bn), str(cus)], check=True,
                         capture_output=True, text=True).stdout
    return {k: int(v) for k, v in (kv.split("=") for kv in out.split())}


@pytest.mark.parametrize("M,N,bn", [
    (10800, 12288, 256), (10800, 3072, 256), (10800, 9216, 256), (10800, 4096, 256), (10800, 12288 + 64, 256),
    (4096, 3072, 192), (132, 12288, 256), (132, 3072, 192), (4996, 3072, 256), (1, 128, 256),
    (300, 640, 256), (257, 257, 256), (10752, 12288, 256), (8192, 8192, 256), (5000, 7000, 256),
    (65536, 1024, 256), (100, 256, 192), (100, 256, 256), (227, 1024, 256), (97, 384, 192),
])
@pytest.mark.parametrize("cus", [256, 80])
def test_every_tile_exactly_once(checker, M, N, bn, cus):
    r = _run(checker, M, N, bn, cus)
    assert r["missing"] == 0 and r["repeated"] == 0 and r["out_of_range"] == 0, r
    # the unchecked direct stores of waves counted inside stay inside M x N,
    # and each wave's MFMA blocks cover all its outputs (for the N the GEMM
    # accepts, a multiple of 128; 257 only exercises the queues)
    assert r["unchecked_outside"] == 0, r
    if N % 128 == 0:
        assert r["uncovered"] == 0, r


@pytest.mark.parametrize("M,N,bn", [(100, 256, 192), (227, 1024, 256), (10752 + 100, 3072, 256)])
def test_four_row_blocks_need_not_be_inside(checker, M, N, bn):
    """A wave with 97..127 rows left has four row blocks but is not inside:
    taking the block count for insideness let the unchecked direct stores
    write past row M (a GPU memory fault at M = 100). These shapes hold such
    waves; the checker sees none of their stores outside the matrix."""
    r = _run(checker, M, N, bn)
    assert r["blocks_not_inside"] > 0 and r["unchecked_outside"] == 0, r


@pytest.mark.parametrize("M,N,full_rounds", [(10800, 12288, 8), (10800, 3072, 2), (10800, 9216, 6)])
def test_edge_tiles_go_to_the_shorter_queues(checker, M, N, full_rounds):
    # 10800 rows: a 48-row last tile row. The longest queue holds full_rounds
    # full tiles; the edge tiles (half-cost in this count) land on the
    # workgroups with one full tile fewer, so no queue exceeds full_rounds.
    r = _run(checker, M, N, 256)
    assert r["max_full"] == full_rounds and r["max_load_x100"] == 100 * full_rounds, r
