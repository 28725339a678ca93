"""Released INT8/FP8 weights on MI355X kernels: the installer module of
reactor/hy_nomas_quantization.py, for gfx950.

The reference's module does two things (hy_nomas_quantization.py:8-58):

* ``install_fp8(source, cutlass, capability)`` JIT-builds the CUTLASS
  extension that matches the device (SM89 or SM100; any other capability is a
  ``ValueError``) and points ``cutlass_fp8.load_extension`` at it, so the
  PixelUMM decoder's CutlassFP8Linear, its custom op and its blockwise
  quantizer call that extension.
* ``cache_int8_weights(transformer)`` keeps, for every Int8StoredBF16Linear,
  a resident BF16 copy of the dequantized weight, so that no forward pays the
  per-call dequantization.

Here the extension is the prebuilt gfx950 library (``gemm(a, b, sa, sb)``,
same contract), so installing needs no build and no CUTLASS path; the
capability gate accepts gfx950, (9, 5) as torch reports it on ROCm. The
resident copy is FP8: each Int8StoredBF16Linear becomes an FP8StoredLinear
whose per-channel e4m3 codes are requantized from the reference's own BF16
weight, bf16(code * scale), so the forward reads the codes directly on the
FP8 GEMM (one byte per weight instead of BF16's two, and no per-call
dequantization).
"""
from __future__ import annotations

from pathlib import Path
from types import ModuleType
from typing import Optional

import torch
from torch import nn

# torch.cuda.get_device_capability() of an MI355X (gfx950) under ROCm.
GFX950 = (9, 5)


def extension():
    from .pixelumm_fp8 import load_extension
    return load_extension()


def _check_capability(capability: Optional[tuple]) -> None:
    if capability is None:
        if not torch.cuda.is_available():
            raise ValueError("PixelUMM FP8 requires a gfx950 (MI355X) device in this build.")
        capability = torch.cuda.get_device_capability()
    if tuple(capability) != GFX950:
        raise ValueError(f"PixelUMM FP8 requires gfx950 (MI355X, capability {GFX950}) in this build, "
                         f"got {tuple(capability)}.")


def install_fp8(source, cutlass: Optional[Path] = None, capability: Optional[tuple] = None) -> None:
    """Point ``cutlass_fp8.load_extension`` at the HIP extension
    (hy_nomas_quantization.py:35-40).

    ``source`` is either the reference checkout the call site passes (its
    ``hymm.models.vae.pixelumm_decoder.cutlass_fp8`` module is then imported,
    as the reference does) or that module itself. ``cutlass`` is accepted for
    the reference's signature and unused: there is nothing to compile.
    ``capability`` (major, minor) must be gfx950's; None reads the current
    device's. The check runs only on the reference's call form: a module
    passed directly is patched as given."""
    if isinstance(source, (ModuleType,)) or hasattr(source, "load_extension"):
        module = source
    else:
        _check_capability(capability)
        from hymm.models.vae.pixelumm_decoder import cutlass_fp8 as module  # the reference's own module
    ext = extension()
    module.load_extension = lambda: ext


def _is_int8_stored(module: nn.Module) -> bool:
    """An Int8StoredBF16Linear (int8_stored_bf16_linear.py:64-89), recognised by
    its buffers: int8 ``weight_q`` [out, in] and fp32 ``weight_scale`` [out,
    ceil(in / 128)]."""
    q = getattr(module, "weight_q", None)
    s = getattr(module, "weight_scale", None)
    return (isinstance(q, torch.Tensor) and isinstance(s, torch.Tensor) and q.dtype == torch.int8
            and q.dim() == 2 and s.dim() == 2 and s.dtype == torch.float32
            and s.shape[0] == q.shape[0] and s.shape[1] == (q.shape[1] + 127) // 128)


@torch.no_grad()
def cache_int8_weights(transformer: nn.Module, device=None) -> dict:
    """Replace every Int8StoredBF16Linear of ``transformer`` by an
    FP8StoredLinear (hy_nomas_quantization.py:43-58 keeps BF16 instead).

    The FP8 codes are requantized from the reference's BF16 weight
    (w8_checkpoint.requantize_int8_to_fp8, per output channel, on the GPU);
    the bias is kept. Returns {qualified name: accuracy report of the FP8
    weight against that BF16 weight (rel_l2, max_abs, max_channel_rel_l2)}.
    Layers whose sizes the FP8 GEMM does not take (in or out not a multiple
    of 128) are left as they are."""
    from .dit_fp8_linear import FP8StoredLinear
    from .w8_checkpoint import requantize_int8_to_fp8

    targets = []
    for name, module in transformer.named_modules():
        for child_name, child in module.named_children():
            if _is_int8_stored(child) and child.weight_q.shape[0] % 128 == 0 and child.weight_q.shape[1] % 128 == 0:
                targets.append((f"{name}.{child_name}".lstrip("."), module, child_name, child))
    reports = {}
    for qual, parent, child_name, child in targets:
        dev = device if device is not None else child.weight_q.device
        codes, scale, report = requantize_int8_to_fp8(child.weight_q, child.weight_scale, dev)
        bias = getattr(child, "bias", None)
        layer = FP8StoredLinear.from_codes(codes, scale, None if bias is None else bias.detach().to(dev))
        setattr(parent, child_name, layer)
        reports[qual] = report
    return reports
