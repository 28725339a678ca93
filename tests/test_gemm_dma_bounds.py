"""Bounds of the persistent FP8 GEMM's operand loads (CPU, no GPU needed).

Each wave of `gemm_rowcol_oe_kernel` loads stage rows by its wave index,
whatever rows it multiplies, so every load's offset is capped by the source
tile's own extent. The offset and cap functions live in
`hy-nomas_amd/csrc/gemm_dma.h`, which the kernel includes; this test compiles
the same header into `tests/gemm_dma_check.cpp` with g++ and enumerates every
load of every tile and K step for shapes whose last tiles are partial (a last
row tile 129-191 rows deep, M = 132, is where an uncapped offset reads far
past A). A change to the cap in the header changes this test's verdict."""
import subprocess
from pathlib import Path

import pytest

HERE = Path(__file__).resolve().parent


@pytest.fixture(scope="module")
def checker(tmp_path_factory):
    exe = tmp_path_factory.mktemp("dma") / "gemm_dma_check"
    subprocess.run(["g++", "-O2", "-std=c++17", "-Wall", "-Werror", str(HERE / "gemm_dma_check.cpp"),
                    "-o", str(exe)], check=True)
    return exe


def _run(exe, M, N, K, bn, *extra):
    out = subprocess.run([str(exe), str(M), str(N), str(K), str(bn), *extra], check=True,
                         capture_output=True, text=True).stdout
    return {k: int(v) for k, v in (kv.split("=") for kv in out.split())}


@pytest.mark.parametrize("M,N,K,bn", [
    (132, 3072, 12288, 192), (132, 9216, 3072, 192), (4996, 4224, 1024, 256), (700, 1280, 1024, 192),
    (10800, 12288, 3072, 256), (1, 128, 896, 256), (1000, 640, 1280, 192), (255, 384, 896, 256),
])
def test_every_load_stays_inside_its_operand(checker, M, N, K, bn):
    r = _run(checker, M, N, K, bn)
    assert r["loads"] > 0 and r["out_of_bounds"] == 0 and r["wrong_offset"] == 0, r


def test_the_checker_sees_uncapped_loads(checker):
    # the same loads without the cap: a partial last tile reads past the operand
    r = _run(checker, 132, 3072, 12288, 192, "nocap")
    assert r["out_of_bounds"] > 0 and r["wrong_offset"] == 0, r


@pytest.mark.parametrize("M,N,K,SK,JB", [
    (10800, 12288, 3072, 2, 2), (10800, 3072, 12288, 4, 2), (257, 384, 1024, 2, 1), (288, 640, 896, 4, 1),
    (289, 512, 3072, 2, 2), (48, 1280, 3072, 4, 2), (1, 256, 4224, 4, 1), (64, 128, 896, 4, 2),
    (276, 8192, 4224, 2, 1), (576, 8192, 4352, 2, 2),
    # blockwise stripes: the decoder's gate/up, 4116 rows (K 512: one K step per wave), M <= 64
    (10800, 12288, 4096, 2, 2), (4116, 4096, 512, 4, 1), (48, 512, 1024, 4, 2), (33, 256, 4096, 4, 2),
])
def test_tail_stripe_loads_stay_inside(checker, M, N, K, SK, JB):
    """The tail-stripe kernel (the last M % 256 <= 64 rows): every load of
    every workgroup, wave and issued step -- the re-loads past a wave's last
    step included -- stays inside its operand, rows inside the stripe keep
    their exact offsets (rows past M repeat row M - 1), and the split of K
    over the waves multiplies each K step exactly once."""
    out = subprocess.run([str(checker), "tail", str(M), str(N), str(K), str(SK), str(JB)], check=True,
                         capture_output=True, text=True).stdout
    r = {k: int(v) for k, v in (kv.split("=") for kv in out.split())}
    assert r["loads"] > 0 and r["out_of_bounds"] == 0 and r["wrong_offset"] == 0, r
    assert r["step_cover_errors"] == 0, r


def test_tail_checker_catches_an_unclamped_row(tmp_path):
    """Planted in a CPU copy of the header only: without the clamp of A rows
    past M, the 48-row stripe of M = 10800 (two 32-row blocks) reads past A."""
    hdr = (HERE.parent / "hy-nomas_amd" / "csrc" / "gemm_dma.h").read_text()
    planted = hdr.replace("t.off = (m < M ? m : M - 1) * K + chunk;", "t.off = m * K + chunk;")
    assert planted != hdr
    (tmp_path / "gemm_dma.h").write_text(planted)
    src = (HERE / "gemm_dma_check.cpp").read_text().replace('#include "../hy-nomas_amd/csrc/gemm_dma.h"',
                                                             '#include "gemm_dma.h"')
    (tmp_path / "check.cpp").write_text(src)
    exe = tmp_path / "check"
    subprocess.run(["g++", "-O2", "-std=c++17", "-Wall", "-Werror", str(tmp_path / "check.cpp"), "-o", str(exe)],
                   check=True)
    out = subprocess.run([str(exe), "tail", "10800", "384", "3072", "2", "2"], check=True, capture_output=True,
                         text=True).stdout
    r = {k: int(v) for k, v in (kv.split("=") for kv in out.split())}
    assert r["out_of_bounds"] > 0, r


@pytest.mark.parametrize("M,N,K,cus,fused", [
    (10800, 12288, 3072, 256, 1),   # north star: 32 light workgroups, 384 columns each
    (10800, 9216, 3072, 256, 1),    # QKV: 24 light workgroups
    (10800, 3072, 12288, 256, 0),   # fc2 (K past 4096): the stripe keeps its own launch
    (10800, 3072, 3072, 256, 0),    # out-projection: 8 light workgroups, fewer than 16
    (10800, 4096, 4096, 256, 1),    # 12 light workgroups per XCD, 96 in all, K 4096
    (10800, 12288, 3072, 80, 1), (300, 384, 1024, 256, 0), (10752 + 33, 4096, 896, 256, 1),
    (10770, 2048, 1024, 256, 1),
    (10800, 12288 + 128, 3072, 256, 0),  # a column edge stripe: the stripe keeps its own launch
])
def test_tail_items_on_light_workgroups(checker, M, N, K, cus, fused):
    """The wide tail items the persistent kernel's light workgroups run after
    their last tile: every load in bounds, the stripe's rows and the item's B
    rows at their exact offsets, the items covering every column once, and
    every item on a workgroup with one full tile fewer than the longest
    queue."""
    out = subprocess.run([str(checker), "tailwide", str(M), str(N), str(K), str(cus)], check=True,
                         capture_output=True, text=True).stdout
    r = {k: int(v) for k, v in (kv.split("=") for kv in out.split())}
    assert r["fused"] == fused, r
    if fused:
        assert r["loads"] > 0 and r["out_of_bounds"] == 0 and r["wrong_offset"] == 0, r
        assert r["column_cover_errors"] == 0 and r["not_light"] == 0 and r["cols"] <= 384, r
