"""The quantizers form x / s from the row's reciprocal plus one FMA correction
(hy-nomas_amd/csrc/quant.hip, struct Quot). This runs the exhaustive host
proof that the resulting codes equal those of the reference's IEEE fp32
division over the whole bf16 input domain (tests/fast_quotient_check.c), and
checks on small cases that the argument needs the correction."""
import subprocess
from pathlib import Path

import numpy as np
import pytest

from conftest import ROOT

SRC = Path(__file__).resolve().parent / "fast_quotient_check.c"


@pytest.fixture(scope="module")
def checker(tmp_path_factory):
    exe = tmp_path_factory.mktemp("fastquot") / "fast_quotient_check"
    subprocess.run(["gcc", "-O2", "-fopenmp", "-ffp-contract=off", "-fno-fast-math", "-o", str(exe),
                    str(SRC), str(ROOT / "oracle" / "fp8_oracle.c"), "-lm"], check=True)
    return exe


@pytest.mark.timeout(900)
def test_fast_quotient_codes_equal_ieee_division_exhaustively(checker):
    out = subprocess.run([str(checker)], capture_output=True, text=True, timeout=880)
    print(out.stdout)
    assert out.returncode == 0, out.stdout + out.stderr
    assert out.stdout.count(" 0 code mismatches") == 3


def test_plain_reciprocal_product_is_not_enough(O):
    """Without the FMA correction, fl(x * fl(1/s)) changes some codes, so the
    exhaustive check above is what licenses the kernels' three-operation form."""
    xbits = np.arange(0x3F80 + 1, dtype=np.uint32)          # every bf16 in [0, 1]
    x = O.bf16_bits_to_f32(xbits.astype(np.uint16))
    mismatches = 0
    for ab in range(0x3F80, 0x4000):                        # every bf16 amax in [1, 2)
        amax = O.bf16_bits_to_f32(np.array([ab], np.uint16))[0]
        s = np.float32(amax) / np.float32(448.0)
        r = np.float32(1.0) / s
        xs = x[x <= amax]
        mismatches += int((O.e4m3_encode((xs * r).astype(np.float32)) != O.e4m3_encode(xs / s)).sum())
    assert mismatches > 0
