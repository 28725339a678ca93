"""FP8 stored DiT linear: per-output-channel e4m3 weights, per-token dynamic
e4m3 activations, one fused HIP GEMM with scales, bias and optional GELU-tanh.

Mirror of the reference's DiT quantized linear,
hymm/models/dit/modules/int8_stored_bf16_linear.py:46-100, whose W8A16 form
dequantizes to bf16 and calls F.linear. Here the weight stays FP8 and the
product runs on the gfx950 FP8 matrix cores:

  * ``quantize_weight(w)``  <- quantize_weight (:46-61): per output channel
    ``s = max(amax, 1e-4) / 448``, ``q = e4m3_rne(w / s)`` (the clamp rule of
    cutlass_fp8.py:39 over a 1 x K block).
  * ``FP8StoredLinear``     <- Int8StoredBF16Linear (:64-94): buffers
    ``weight_q`` / ``weight_scale``, ``dequant_weight()``, the same BF16 input
    contract (TypeError otherwise).
  * ``linear_weight(m)``    <- linear_weight (:97-100) for F.linear call sites.
  * ``fp8_linear(m, x, act)``: the fused call the FP8 block uses in place of
    ``F.linear(x, linear_weight(m), b)`` (nomas_compile_prepost.py:45-47,80-87).

The reference's compiled pre/post functions receive ``linear_weight(m)`` as a
plain tensor and call ``F.linear(x, w, b)`` on it (nomas_cpt.py:1356-1370,
1431-1441). For an FP8StoredLinear that tensor is an ``FP8Weight``: it reports
the bf16 [out, in] weight, turns ``F.linear`` into the fused FP8 custom op
(``hy_nomas_amd::linear_fp8``, opaque to torch.compile), and gives every other
operation the dequantized bf16 value the reference's dequant_weight() makes.
FP8StoredLinear.weight returns it too, so the reference's own unchanged
linear_weight (``module.weight`` for anything but its INT8 class) reaches the
FP8 GEMM without a call-site edit.
"""
from __future__ import annotations

import torch
import torch.nn as nn
import torch.nn.functional as F
from torch.utils._pytree import tree_map

from . import _lib as L
from . import ops


class FP8Weight(torch.Tensor):
    """A bf16 [out, in] weight held as e4m3 codes and fp32 per-row scales.

    ``F.linear(x, w, b)`` runs the per-token FP8 linear (activation quant +
    fused GEMM with the scales and bias); x must be bf16, like the FP8
    linear's forward. Any other operation on ``w`` sees
    bf16(code * scale), the value dequant_weight() returns.
    """

    @staticmethod
    def __new__(cls, codes: torch.Tensor, scale: torch.Tensor):
        return torch.Tensor._make_wrapper_subclass(cls, codes.shape, dtype=torch.bfloat16,
                                                   device=codes.device, requires_grad=False)

    def __init__(self, codes: torch.Tensor, scale: torch.Tensor):
        if codes.dtype != torch.float8_e4m3fn or codes.ndim != 2:
            raise TypeError("FP8Weight holds float8_e4m3fn [out, in] codes")
        if scale.dtype != torch.float32 or scale.numel() != codes.shape[0]:
            raise TypeError("FP8Weight needs one fp32 scale per output row")
        self.codes = codes
        self.scale = scale.reshape(-1)

    def __repr__(self):
        return f"FP8Weight(shape={tuple(self.shape)}, device={self.device})"

    def dequantize(self) -> torch.Tensor:
        return (self.codes.float() * self.scale[:, None]).to(torch.bfloat16)

    # torch.compile sees the two inner tensors (traceable wrapper subclass)
    def __tensor_flatten__(self):
        return ["codes", "scale"], None

    @staticmethod
    def __tensor_unflatten__(inner, meta, outer_size, outer_stride):
        return FP8Weight(inner["codes"], inner["scale"])

    @classmethod
    def __torch_function__(cls, func, types, args=(), kwargs=None):
        kwargs = kwargs or {}
        if func is F.linear:
            x = args[0] if args else kwargs["input"]
            w = args[1] if len(args) > 1 else kwargs["weight"]
            b = args[2] if len(args) > 2 else kwargs.get("bias")
            if isinstance(w, FP8Weight) and not isinstance(x, FP8Weight):
                return _linear_on_codes(x, w, b)
        with torch._C.DisableTorchFunctionSubclass():
            return func(*args, **kwargs)

    @classmethod
    def __torch_dispatch__(cls, func, types, args=(), kwargs=None):
        def value(t):
            return t.dequantize() if isinstance(t, FP8Weight) else t
        return func(*tree_map(value, args), **tree_map(value, kwargs or {}))


def _linear_on_codes(x: torch.Tensor, w: FP8Weight, bias) -> torch.Tensor:
    if x.dtype != torch.bfloat16:
        raise TypeError(f"FP8 stored Linear requires BF16 input, got {x.dtype}")
    if bias is not None:
        bias = bias.detach().to(torch.bfloat16)
    y = ops.linear_fp8(x.reshape(-1, x.shape[-1]), w.codes, w.scale, bias, L.HN_ACT_NONE)
    return y.reshape(*x.shape[:-1], w.shape[0])


def quantize_weight(weight: torch.Tensor) -> tuple[torch.Tensor, torch.Tensor]:
    """Per-output-channel FP8 quantization of a [out_features, in_features] weight."""
    if weight.ndim != 2 or not weight.is_floating_point():
        raise TypeError("Expected a floating-point [out_features, in_features] weight")
    if not torch.isfinite(weight).all():
        raise ValueError("Cannot quantize a weight containing NaN or Inf")
    q, s = ops.quantize_rows_fp8(weight.to(torch.bfloat16).contiguous(), L.HN_SCALE_CLAMP, 1e-4)
    return q, s


class FP8StoredLinear(nn.Module):
    """Stores e4m3 weights and fp32 per-channel scales; computes in FP8."""

    def __init__(self, original: nn.Linear):
        super().__init__()
        self.in_features = original.in_features
        self.out_features = original.out_features
        if self.in_features % 128 or self.out_features % 128:
            raise ValueError("FP8 linear needs in/out features divisible by 128")
        q, s = quantize_weight(original.weight.detach())
        self.register_buffer("weight_q", q)
        self.register_buffer("weight_scale", s)
        self.bias = original.bias

    @classmethod
    def from_codes(cls, weight_q: torch.Tensor, weight_scale: torch.Tensor,
                   bias: torch.Tensor | None = None) -> "FP8StoredLinear":
        """A layer from e4m3 codes [out, in] and fp32 per-channel scales [out]
        (e.g. requantized from a W8 checkpoint)."""
        out_f, in_f = weight_q.shape
        if weight_q.dtype != torch.float8_e4m3fn or weight_scale.dtype != torch.float32:
            raise TypeError("Expected float8_e4m3fn codes and float32 scales")
        if in_f % 128 or out_f % 128 or tuple(weight_scale.reshape(-1).shape) != (out_f,):
            raise ValueError("FP8 linear needs in/out features divisible by 128 and one scale per output")
        if not torch.isfinite(weight_scale).all() or not (weight_scale > 0).all():
            raise ValueError("FP8 scales must be finite and positive")
        m = cls.__new__(cls)
        nn.Module.__init__(m)
        m.in_features, m.out_features = in_f, out_f
        m.register_buffer("weight_q", weight_q)
        m.register_buffer("weight_scale", weight_scale.reshape(-1))
        m.bias = None if bias is None else nn.Parameter(bias.to(torch.bfloat16), requires_grad=False)
        return m

    def dequant_weight(self) -> torch.Tensor:
        return (self.weight_q.float() * self.weight_scale[:, None]).to(torch.bfloat16)

    @property
    def weight(self) -> FP8Weight:
        """The weight as the reference's call sites take it: F.linear with it
        runs the FP8 GEMM; anything else sees dequant_weight()."""
        return FP8Weight(self.weight_q, self.weight_scale)

    def forward(self, x: torch.Tensor, act: int = L.HN_ACT_NONE) -> torch.Tensor:
        if x.dtype != torch.bfloat16:
            if (x.device.type == "cuda" and torch.is_autocast_enabled("cuda")
                    and torch.get_autocast_dtype("cuda") == torch.bfloat16):
                x = x.to(torch.bfloat16)
            else:
                raise TypeError(f"FP8 stored Linear requires BF16 input, got {x.dtype}")
        bias = None if self.bias is None else self.bias.detach().to(torch.bfloat16)
        y = ops.linear_fp8(x.reshape(-1, x.shape[-1]), self.weight_q, self.weight_scale, bias, act)
        return y.reshape(*x.shape[:-1], self.out_features)


def fp8_linear_codes(module: "FP8StoredLinear", qx: torch.Tensor, sx: torch.Tensor,
                     gelu: bool = False) -> torch.Tensor:
    """The FP8 linear on activations already quantized per token (codes e4m3
    [M, in], scales fp32 [M]), e.g. by ops.ln_modulate_quantize_fp8."""
    bias = None if module.bias is None else module.bias.detach().to(torch.bfloat16)
    return ops.gemm_fp8_rowcol(qx, module.weight_q, sx, module.weight_scale, bias,
                               L.HN_ACT_GELU_TANH if gelu else L.HN_ACT_NONE)


def linear_weight(module: nn.Module) -> torch.Tensor:
    """The tensor the compiled pre/post functions pass to F.linear: the
    FP8Weight of an FP8StoredLinear, else the module's own weight."""
    return module.weight


def fp8_linear(module: nn.Module, x: torch.Tensor, gelu: bool = False) -> torch.Tensor:
    """Fused FP8 linear (+ GELU-tanh) for FP8StoredLinear; bf16 F.linear otherwise."""
    if isinstance(module, FP8StoredLinear):
        return module(x, L.HN_ACT_GELU_TANH if gelu else L.HN_ACT_NONE)
    y = F.linear(x, module.weight, module.bias)
    return F.gelu(y, approximate="tanh") if gelu else y


@torch.no_grad()
def convert_to_fp8(model: nn.Module, predicate=None) -> int:
    """Replace nn.Linear submodules (optionally filtered) with FP8StoredLinear."""
    targets = []
    for name, module in model.named_modules():
        for child_name, child in module.named_children():
            if isinstance(child, nn.Linear) and (predicate is None or predicate(f"{name}.{child_name}".lstrip("."), child)):
                targets.append((module, child_name, child))
    for parent, child_name, child in targets:
        setattr(parent, child_name, FP8StoredLinear(child))
    return len(targets)
