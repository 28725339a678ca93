"""Blockwise-scaled FP8 linear on gfx950: the decoder's FP8 Linear surface.

Mirror of hymm/models/vae/pixelumm_decoder/cutlass_fp8.py:17-126 (and the
serialized-tensor check of prequantized.py:16-24) with the CUTLASS extension
replaced by the HIP one:

  * ``load_extension()`` returns an object whose ``gemm(a, b, sa, sb)`` keeps
    the native extension's contract (cutlass_fp8.cu:20-57): e4m3 [M,K] x
    e4m3 [N,K] with 128x128 fp32 block scales -> bf16 [M,N], RuntimeError on
    bad input. ``hy-nomas_amd/quantization.py`` installs it into the
    reference module through the same seam reactor uses
    (reactor/hy_nomas_quantization.py:35-40).
  * ``_quantize_blockwise`` / ``quantize_blockwise``: 128x128 block amax,
    ``clamp_min(1e-4) / 448``, e4m3 codes (cutlass_fp8.py:35-44), as a HIP kernel.
  * ``_linear``: opaque custom op quantize + gemm with a call counter (:47-57).
  * ``FP8Linear`` (also exported as ``CutlassFP8Linear``): buffers
    ``fp8_weight``/``fp8_scale``, ``from_quantized``, dtype-preserving
    ``_apply``, inference-only ``forward`` (:60-97).
  * ``enable_fp8`` replaces bias-free linears chosen by the caller (:100-121);
    ``execution_stats`` (:124-126).
"""
from __future__ import annotations

from collections import Counter
from functools import lru_cache

import torch
from torch import nn

from . import ops

_calls = Counter()


class HipFP8Extension:
    """Stand-in for the compiled CUTLASS module: one ``gemm`` entry point."""

    @staticmethod
    def gemm(a: torch.Tensor, b: torch.Tensor, sa: torch.Tensor, sb: torch.Tensor) -> torch.Tensor:
        if not (a.is_cuda and a.dim() == 2 and b.dim() == 2):
            raise RuntimeError("Expected CUDA matrices")
        for t in (b, sa, sb):
            if t.device != a.device:
                raise RuntimeError("Expected contiguous tensors on one device")
        return ops.gemm_fp8_blockwise(a, b, sa, sb)


@lru_cache(maxsize=1)
def load_extension() -> HipFP8Extension:
    from . import _lib
    _lib.load()
    return HipFP8Extension()


def _quantize_blockwise(x: torch.Tensor):
    if x.dim() != 2 or x.shape[1] % 128:
        raise ValueError("blockwise FP8 quantization expects [M, K] with K % 128 == 0")
    return ops.quantize_blockwise_fp8(x.to(torch.bfloat16) if x.dtype != torch.bfloat16 else x)


quantize_blockwise = _quantize_blockwise


@torch.library.custom_op("hy_nomas_amd::blockwise_linear", mutates_args=())
def _linear(x: torch.Tensor, weight: torch.Tensor, scale: torch.Tensor) -> torch.Tensor:
    q, s = quantize_blockwise(x)
    result = load_extension().gemm(q, weight, s, scale)
    _calls[(x.device.index, x.shape[0], x.shape[1], weight.shape[0])] += 1
    return result


@_linear.register_fake
def _linear_fake(x, weight, scale):
    return x.new_empty((x.shape[0], weight.shape[0]), dtype=torch.bfloat16)


def validate_serialized_tensors(weight, scale, expected_shape):
    """prequantized.py:16-24: dims % 128, e4m3/fp32, scales finite and > 0."""
    shape = tuple(expected_shape)
    if (len(shape) != 2 or any(d % 128 for d in shape)
            or weight.dtype != torch.float8_e4m3fn or tuple(weight.shape) != shape
            or scale.dtype != torch.float32
            or tuple(scale.shape) != tuple(d // 128 for d in shape)):
        raise ValueError("Invalid serialized FP8 weight/scale")
    if not torch.isfinite(scale).all() or not (scale > 0).all():
        raise ValueError("FP8 scales must be finite and positive")


class FP8Linear(nn.Module):
    def __init__(self, linear: nn.Linear):
        super().__init__()
        # One-time startup conversion, outside any timed region.
        q, s = _quantize_blockwise(linear.weight.detach())
        self.register_buffer("fp8_weight", q)
        self.register_buffer("fp8_scale", s)
        self.train(False)

    @classmethod
    def from_quantized(cls, weight, scale, expected_shape):
        """Install serialized buffers unchanged, without weight quantization."""
        validate_serialized_tensors(weight, scale, expected_shape)
        module = cls.__new__(cls)
        nn.Module.__init__(module)
        module.register_buffer("fp8_weight", weight.contiguous())
        module.register_buffer("fp8_scale", scale.contiguous())
        return module.eval()

    def _apply(self, fn, recurse=True):
        # Device/offload moves must preserve the serialized FP8 and FP32 dtypes.
        for name in ("fp8_weight", "fp8_scale"):
            tensor = self._buffers[name]
            target = fn(torch.empty(0, device=tensor.device, dtype=tensor.dtype))
            self._buffers[name] = tensor.to(device=target.device)
        return self

    def forward(self, x):
        if self.training or torch.is_grad_enabled():
            raise RuntimeError("FP8 linear supports eval + no_grad inference only")
        if x.dtype != torch.bfloat16:
            if not torch.is_autocast_enabled("cuda") or torch.get_autocast_dtype("cuda") != torch.bfloat16:
                raise TypeError("FP8 linear requires BF16 inputs or BF16 CUDA autocast")
            x = x.to(torch.bfloat16)
        y = _linear(x.reshape(-1, x.shape[-1]).contiguous(), self.fp8_weight, self.fp8_scale)
        return y.reshape(*x.shape[:-1], self.fp8_weight.shape[0])


CutlassFP8Linear = FP8Linear


@torch.no_grad()
def enable_fp8(model: nn.Module, names) -> int:
    """Replace the named bias-free nn.Linear submodules of ``model`` (validated
    first, then swapped, as enable_cutlass_fp8 does at cutlass_fp8.py:100-121)."""
    if model.training:
        raise ValueError("Expected an eval-mode model")
    targets = []
    for name in names:
        parent_name, _, leaf = name.rpartition(".")
        parent = model.get_submodule(parent_name) if parent_name else model
        linear = getattr(parent, leaf)
        if not isinstance(linear, nn.Linear) or linear.bias is not None:
            raise ValueError("Expected an unmodified bias-free linear")
        w = linear.weight
        if not w.is_cuda or w.dtype != torch.bfloat16 or any(d % 128 for d in w.shape):
            raise ValueError("Expected CUDA BF16 weights with dimensions divisible by 128")
        targets.append((parent, leaf))
    load_extension()
    for parent, leaf in targets:
        setattr(parent, leaf, FP8Linear(getattr(parent, leaf)))
    return len(targets)


def execution_stats():
    return [{"device": d, "M": m, "K": k, "N": n, "calls": count}
            for (d, m, k, n), count in sorted(_calls.items())]
