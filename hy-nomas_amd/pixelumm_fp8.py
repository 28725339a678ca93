"""The PixelUMM decoder's FP8 linear on gfx950, behind the reference's surface.

Contract kept from hymm/models/vae/pixelumm_decoder/cutlass_fp8.py:17-126 and
prequantized.py:16-24 (names, buffers, argument meaning, exception types):

  ================================  =======================================
  here                              role in the reference
  ================================  =======================================
  load_extension().gemm(a,b,sa,sb)  the native extension (cutlass_fp8.cu:20-57)
  quantize_blockwise                128 x 128 block activation quantizer (:35-44)
  _linear (custom op)               quantize + gemm, opaque to torch.compile (:47-57)
  FP8Linear / CutlassFP8Linear      module with fp8_weight / fp8_scale (:60-97)
  enable_fp8                        swap chosen bias-free linears (:100-121)
  execution_stats                   per-shape call counts (:124-126)
  validate_serialized_tensors       serialized weight/scale rules (prequantized.py:16-24)
  ================================  =======================================

The GEMM is the HIP blockwise kernel; ``quantization.install_fp8`` points the
reference module's ``load_extension`` at it, the seam reactor uses
(reactor/hy_nomas_quantization.py:35-40).
"""
from __future__ import annotations

from collections import Counter
from functools import lru_cache

import torch
from torch import nn

from . import ops

BLOCK = 128
_calls: Counter = Counter()   # (device index, M, K, N) -> calls


class HipFP8Extension:
    """What the reference's compiled extension module provides: ``gemm``."""

    @staticmethod
    def gemm(a: torch.Tensor, b: torch.Tensor, sa: torch.Tensor, sb: torch.Tensor) -> torch.Tensor:
        """bf16 [M, N] = sum over K blocks of (a_blk . b_blk^T) * sa * sb for e4m3
        a [M, K], b [N, K] and fp32 block scales; RuntimeError on bad input."""
        if not a.is_cuda or a.dim() != 2 or b.dim() != 2:
            raise RuntimeError("Expected CUDA matrices")
        if any(t.device != a.device for t in (b, sa, sb)):
            raise RuntimeError("Expected contiguous tensors on one device")
        return ops.gemm_fp8_blockwise(a, b, sa, sb)


@lru_cache(maxsize=1)
def load_extension() -> HipFP8Extension:
    """The extension object (loads libhynomas_fp8.so once; raises if absent)."""
    from . import _lib
    _lib.load()
    return HipFP8Extension()


def quantize_blockwise(x: torch.Tensor):
    """e4m3 codes [M, K] and fp32 scales [ceil(M/128), K/128] of x, per 128 x 128
    block: s = max(amax, 1e-4) / 448, code = e4m3(x / s), rows padded to 128."""
    if x.dim() != 2 or x.shape[1] % BLOCK:
        raise ValueError("blockwise FP8 quantization expects [M, K] with K % 128 == 0")
    return ops.quantize_blockwise_fp8(x if x.dtype == torch.bfloat16 else x.to(torch.bfloat16))


_quantize_blockwise = quantize_blockwise


@torch.library.custom_op("hy_nomas_amd::blockwise_linear", mutates_args=())
def _linear(x: torch.Tensor, weight: torch.Tensor, scale: torch.Tensor) -> torch.Tensor:
    codes, x_scale = quantize_blockwise(x)
    y = load_extension().gemm(codes, weight, x_scale, scale)
    _calls[(x.device.index, x.shape[0], x.shape[1], weight.shape[0])] += 1
    return y


@_linear.register_fake
def _linear_fake(x, weight, scale):
    return x.new_empty((x.shape[0], weight.shape[0]), dtype=torch.bfloat16)


SCALE_ROW_SPAN = 2.0 ** 60


def validate_serialized_tensors(weight: torch.Tensor, scale: torch.Tensor, expected_shape) -> None:
    """A serialized FP8 layer is valid when its [out, in] shape is the expected
    one with both dims multiples of 128, the codes are e4m3, and the scales are
    fp32 [out/128, in/128], finite and positive (ValueError otherwise)."""
    shape = tuple(expected_shape)
    geometry_ok = (len(shape) == 2 and all(d % BLOCK == 0 for d in shape)
                   and weight.dtype == torch.float8_e4m3fn and tuple(weight.shape) == shape
                   and scale.dtype == torch.float32
                   and tuple(scale.shape) == tuple(d // BLOCK for d in shape))
    if not geometry_ok:
        raise ValueError("Invalid serialized FP8 weight/scale")
    if not bool(torch.isfinite(scale).all()) or not bool((scale > 0).all()):
        raise ValueError("FP8 scales must be finite and positive")
    # The blockwise GEMM carries its accumulators in units of the current K
    # block's factor; a weight scale row spanning more than 2^60 could, with
    # the activation scales, push the rescale past fp32's range.
    row_span = scale.amax(dim=1) / scale.amin(dim=1)
    if bool((row_span > SCALE_ROW_SPAN).any()):
        raise ValueError("FP8 scales of one output block row span more than 2^60")


def _inference_input(module: nn.Module, x: torch.Tensor) -> torch.Tensor:
    """x as bf16, after the inference-only and dtype rules of the FP8 linear."""
    if module.training or torch.is_grad_enabled():
        raise RuntimeError("FP8 linear supports eval + no_grad inference only")
    if x.dtype == torch.bfloat16:
        return x
    bf16_autocast = (torch.is_autocast_enabled("cuda")
                     and torch.get_autocast_dtype("cuda") == torch.bfloat16)
    if not bf16_autocast:
        raise TypeError("FP8 linear requires BF16 inputs or BF16 CUDA autocast")
    return x.to(torch.bfloat16)


class FP8Linear(nn.Module):
    """A bias-free linear stored as e4m3 codes ``fp8_weight`` [out, in] and fp32
    128 x 128 block scales ``fp8_scale``; inference only."""

    def __init__(self, linear: nn.Linear):
        super().__init__()
        codes, scales = quantize_blockwise(linear.weight.detach())   # once, at conversion
        self.register_buffer("fp8_weight", codes)
        self.register_buffer("fp8_scale", scales)
        self.eval()

    @classmethod
    def from_quantized(cls, weight: torch.Tensor, scale: torch.Tensor, expected_shape) -> "FP8Linear":
        """A layer over already-serialized codes and scales (validated, then used
        as they are: no requantization)."""
        validate_serialized_tensors(weight, scale, expected_shape)
        layer = cls.__new__(cls)
        nn.Module.__init__(layer)
        layer.register_buffer("fp8_weight", weight.contiguous())
        layer.register_buffer("fp8_scale", scale.contiguous())
        return layer.eval()

    def _apply(self, fn, recurse=True):
        # .to(dtype) / .half() on the model must not convert the codes or the
        # scales: only the destination device is taken from fn, learnt from
        # an empty tensor of each buffer's own dtype.
        for key in ("fp8_weight", "fp8_scale"):
            buf = self._buffers[key]
            device = fn(buf.new_empty(0)).device
            self._buffers[key] = buf.to(device)
        return self

    def forward(self, x: torch.Tensor) -> torch.Tensor:
        x = _inference_input(self, x)
        lead, k = x.shape[:-1], x.shape[-1]
        y = _linear(x.reshape(-1, k).contiguous(), self.fp8_weight, self.fp8_scale)
        return y.reshape(*lead, self.fp8_weight.shape[0])


CutlassFP8Linear = FP8Linear


@torch.no_grad()
def enable_fp8(model: nn.Module, names) -> int:
    """Swap the named bias-free nn.Linear submodules of an eval-mode model for
    FP8Linear. Every target is checked (unmodified bias-free linear, CUDA bf16
    weight, dims multiples of 128) before any is swapped."""
    if model.training:
        raise ValueError("Expected an eval-mode model")

    def locate(path):
        owner_path, _, attr = path.rpartition(".")
        return (model.get_submodule(owner_path) if owner_path else model), attr

    plan = [locate(n) for n in names]
    for owner, attr in plan:
        layer = getattr(owner, attr)
        if not isinstance(layer, nn.Linear) or layer.bias is not None:
            raise ValueError("Expected an unmodified bias-free linear")
        w = layer.weight
        if not w.is_cuda or w.dtype != torch.bfloat16 or w.shape[0] % BLOCK or w.shape[1] % BLOCK:
            raise ValueError("Expected CUDA BF16 weights with dimensions divisible by 128")
    load_extension()
    for owner, attr in plan:
        setattr(owner, attr, FP8Linear(getattr(owner, attr)))
    return len(plan)


def execution_stats():
    """One record per (device, M, K, N) the FP8 linear ran with, and its count."""
    keys = ("device", "M", "K", "N")
    return [dict(zip(keys, key), calls=n) for key, n in sorted(_calls.items())]
