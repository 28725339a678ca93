"""Bounds of the persistent FP8 GEMM's operand loads (CPU, no GPU needed).

Each wave of `gemm_rowcol_oe_kernel` loads stage rows by its wave index
(rows 64 w + lane / 8 + 8 q), whatever rows it multiplies, so a load's
offset must be capped by the source tile's own extent. In `gemm_fp8.hip`
(`dma_off`, `set_src`) the offset from the K step's source address is
min(row K + chunk + 8 q K, (rows - 1) K + 112), with chunk the lane's
swizzled 16-byte chunk. This test enumerates every load of every tile at
the first and last K step and checks that it stays inside the operand, and
that rows inside it keep their exact offset. A last row tile between 129
and 191 rows deep (M = 132 in the DiT block test) is the case where a
missing cap reads far past A."""
import numpy as np
import pytest


def _swz_pos(row, chunk):
    return chunk ^ ((row >> 1) & 7)


def _loads_out_of_bounds(M, N, K, bn, lim_of=lambda rows, K: (rows - 1) * K + 112):
    wave = np.arange(4)[:, None, None]
    lane = np.arange(64)[None, :, None]
    q = np.arange(8)[None, None, :]
    row = wave * 64 + (lane >> 3)
    chunk = np.where(q & 1, _swz_pos(row + 8, lane & 7) << 4, _swz_pos(row, lane & 7) << 4)
    bad = 0
    for extent, tile in ((M, 256), (N, bn)):
        for t0 in range(0, extent, tile):
            rows = min(extent - t0, tile)
            off = np.minimum(row * K + chunk + 8 * q * K, lim_of(rows, K))
            inside = (row + 8 * q) < rows
            assert np.array_equal(off[inside], ((row + 8 * q) * K + chunk)[inside])
            for step in (0, K // 128 - 1):
                addr = t0 * K + step * 128 + off
                bad += int(addr.min() < 0 or (addr + 16).max() > extent * K)
    return bad


@pytest.mark.parametrize("M,N,K,bn", [
    (132, 3072, 12288, 192), (132, 9216, 3072, 192), (4996, 4224, 1024, 256), (700, 1280, 1024, 192),
    (10800, 12288, 3072, 256), (1, 128, 896, 256), (1000, 640, 1280, 192), (255, 384, 896, 256),
])
def test_every_load_stays_inside_its_operand(M, N, K, bn):
    assert _loads_out_of_bounds(M, N, K, bn) == 0


def test_the_check_catches_a_cap_past_the_step_window():
    # A cap of (rows K - 16) ignores the K step's 128-byte window offset.
    assert _loads_out_of_bounds(132, 3072, 12288, 192, lim_of=lambda rows, K: rows * K - 16) > 0
    assert _loads_out_of_bounds(132, 3072, 12288, 192, lim_of=lambda rows, K: 1 << 40) > 0
