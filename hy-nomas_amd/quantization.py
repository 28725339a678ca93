"""Install the HIP FP8 GEMM behind the reference's extension seam.

Mirror of reactor/hy_nomas_quantization.py:8-40: the reference JIT-builds an
architecture-matched CUTLASS extension and then replaces
``cutlass_fp8.load_extension`` with ``lambda: extension``. Here the extension
is the prebuilt gfx950 library, whose ``gemm(a, b, sa, sb)`` has the same
contract, so the reference's CutlassFP8Linear, its custom op and its blockwise
quantizer run unchanged on MI355X once this is installed.
"""
from __future__ import annotations

from types import ModuleType


def extension():
    from .pixelumm_fp8 import load_extension
    return load_extension()


def install_fp8(cutlass_fp8_module: ModuleType) -> None:
    """Point ``cutlass_fp8_module.load_extension`` at the HIP extension."""
    ext = extension()
    cutlass_fp8_module.load_extension = lambda: ext
