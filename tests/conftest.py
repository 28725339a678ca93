import importlib
import sys
from pathlib import Path

import numpy as np
import pytest

ROOT = Path(__file__).resolve().parent.parent
if str(ROOT) not in sys.path:
    sys.path.insert(0, str(ROOT))

PKG = "hy-nomas_amd"


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (gfx950) GPU and the built HIP library")


def pytest_collection_modifyitems(config, items):
    try:
        import torch
        has_gpu = torch.cuda.is_available()
    except Exception:  # pragma: no cover
        has_gpu = False
    if has_gpu:
        return
    skip = pytest.mark.skip(reason="no GPU in this environment")
    for item in items:
        if "gpu" in item.keywords:
            item.add_marker(skip)


def pkg_module(name: str = ""):
    return importlib.import_module(PKG + ("." + name if name else ""))


@pytest.fixture(scope="session")
def O():
    from oracle import oracle
    oracle.lib()
    return oracle


@pytest.fixture(scope="session")
def dev():
    import torch
    return torch.device("cuda:0")


def bf16_bits(t):
    """Raw bits of a bf16 torch tensor as np.uint16."""
    import torch
    return t.detach().cpu().contiguous().view(torch.int16).numpy().view(np.uint16)


def u8(t):
    import torch
    return t.detach().cpu().contiguous().view(torch.uint8).numpy()


# Allowance for the error a kernel's result carries before its final bf16
# rounding, relative to |ref|: fp32 accumulation is far below it; the attention's
# fp16 probabilities (half-ulp relative 2^-11) perturb each normalised weight by
# at most about that much.
PRE_ROUNDING_REL = 2.0 ** -11


def bf16_half_ulp(x):
    """Half the spacing of the bf16 grid at |x|: 2^(e - 8) for |x| in
    [2^e, 2^(e+1)) (normal range; the subnormal spacing below 2^-126)."""
    a = np.maximum(np.abs(np.asarray(x, dtype=np.float64)), 2.0 ** -126)
    return np.exp2(np.floor(np.log2(a)) - 8)


def assert_close_bf16(got, ref, max_abs=2e-2, rel_l2=1e-2, what="", extra=None, ref_is_bf16=False):
    """The north-star float tolerance versus an fp32/fp64-accumulated reference:
    rel-L2 <= 1e-2, and elementwise
        |got - ref| <= max(2e-2, half_ulp_bf16(ref) + 2^-11 |ref|).
    The second term is the bf16 output's own rounding (half an ulp of the grid
    at |ref|) plus the pre-rounding allowance; it stays below 2e-2 for every
    |ref| < 8 (half ulp 2^-6 there) and only exceeds it from |ref| = 8 up,
    where one bf16 ulp is 0.0625.

    ref_is_bf16: the reference value is itself a bf16 result (the reference's
    own op sequence rounds to bf16, e.g. RMSNorm + RoPE or the residual add).
    Two correctly computed values then round nearly the same fp32 number and
    may sit one bf16 ulp apart: the second term becomes one full ulp at |ref|
    (2 half ulps) plus the allowance.

    `extra` (per element) adds a rounding allowance that the computed recipe
    itself carries (the caller states where it comes from)."""
    got = np.asarray(got, dtype=np.float64)
    ref = np.asarray(ref, dtype=np.float64)
    assert np.all(np.isfinite(got)), f"{what}: non-finite output"
    diff = np.abs(got - ref)
    ulps = 2.0 if ref_is_bf16 else 1.0
    bound = np.maximum(max_abs, ulps * bf16_half_ulp(ref) + PRE_ROUNDING_REL * np.abs(ref))
    if extra is not None:
        bound = bound + np.asarray(extra, dtype=np.float64)
    worst = float(np.max(diff / bound)) if got.size else 0.0
    err = float(np.max(diff)) if got.size else 0.0
    denom = float(np.linalg.norm(ref))
    rel = float(np.linalg.norm(got - ref) / denom) if denom > 0 else err
    if what:
        print(f"[close] {what}: max-abs {err:.3e} worst/bound {worst:.2f} rel-L2 {rel:.3e}", flush=True)
    assert worst <= 1.0 and rel <= rel_l2, (
        f"{what}: max-abs {err:.3e} (worst/bound {worst:.2f}) rel-L2 {rel:.3e}")
    return err, rel
