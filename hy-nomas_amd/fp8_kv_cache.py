"""FP8 (OCP e4m3) storage for segment-AR KV, written and read by HIP kernels.

Mirror of the reference's INT8 KV module
(hymm/models/dit/modules/int8_kv_cache.py:17-210) with the same functional
API, validation order and exceptions:

  * ``make_fp8_kv_block``   <- make_int8_kv_block      (:92-107)
  * ``is_fp8_kv_cache``     <- is_int8_kv_cache        (:110-111)
  * ``quantize_kv_into``    <- quantize_kv_into        (:125-158)
  * ``quantize_kv_pair_into`` <- quantize_kv_pair_into (:161-179)
  * ``dequantize_kv``       <- dequantize_kv           (:182-205)
  * ``kv_storage_bytes``    <- kv_storage_bytes        (:208-210)

Layout is the reference's: per layer a dict with ``k``/``v`` codes
[B, capacity, H, D] (token-major) and ``k_scale``/``v_scale`` fp32
[B, capacity, H, 1]. Each (batch, token, head) row gets
``s = amax > 0 ? amax / 448 : 1`` and ``code = e4m3_rne(x / s)`` (the
reference's ``peak / 127`` rule with the e4m3 range). ``make_int8_kv_block``
builds the reference's own INT8 cache; the same kernels then reproduce its
codes bit-exactly, so both formats are served by one path.

There is no CPU branch: the caches must live on the GPU.
"""
from __future__ import annotations

import torch

from . import ops
from .metrics import profiled

KV_KEYS = ("k", "v")
STORAGE_KEYS = ("k", "v", "k_scale", "v_scale")
FP8 = torch.float8_e4m3fn
CODE_DTYPES = (FP8, torch.int8)


def _make_block(batch, capacity, heads, dim, code_dtype, device, pin_memory):
    value_shape = (batch, capacity, heads, dim)
    scale_shape = (batch, capacity, heads, 1)
    return {
        "k": torch.empty(value_shape, device=device, dtype=code_dtype, pin_memory=pin_memory),
        "v": torch.empty(value_shape, device=device, dtype=code_dtype, pin_memory=pin_memory),
        "k_scale": torch.empty(scale_shape, device=device, dtype=torch.float32,
                               pin_memory=pin_memory),
        "v_scale": torch.empty(scale_shape, device=device, dtype=torch.float32,
                               pin_memory=pin_memory),
    }


def make_fp8_kv_block(batch: int, capacity: int, heads: int, dim: int, *,
                      device: torch.device | str, pin_memory: bool = False) -> dict:
    """Per-layer FP8 cache: e4m3 codes [B,cap,H,D] and fp32 scales [B,cap,H,1]."""
    return _make_block(batch, capacity, heads, dim, FP8, device, pin_memory)


def make_int8_kv_block(batch: int, capacity: int, heads: int, dim: int, *,
                       device: torch.device | str, pin_memory: bool = False) -> dict:
    """The reference's INT8 cache layout (int8_kv_cache.py:92-107)."""
    return _make_block(batch, capacity, heads, dim, torch.int8, device, pin_memory)


def is_fp8_kv_cache(cache: dict) -> bool:
    return cache["k"].dtype == FP8


def is_quantized_kv_cache(cache: dict) -> bool:
    return cache["k"].dtype in CODE_DTYPES


def _validate(cache: dict, key: str) -> None:
    if key not in KV_KEYS:
        raise ValueError(f"Invalid KV key: {key}")
    q = cache[key]
    scale = cache[f"{key}_scale"]
    if q.dtype not in CODE_DTYPES or scale.dtype != torch.float32:
        raise TypeError("FP8/INT8 KV data and FP32 scale are required")
    if scale.shape != (*q.shape[:-1], 1) or scale.device != q.device:
        raise ValueError("KV scale shape/device mismatch")


def quantize_kv_into(cache: dict, key: str, values: torch.Tensor, start: int, *,
                     assume_finite: bool = False) -> None:
    """Append BF16 values into quantized storage at token offset ``start``."""
    _validate(cache, key)
    q = cache[key]
    scale = cache[f"{key}_scale"]
    if values.ndim != 4 or values.dtype != torch.bfloat16:
        raise TypeError("KV quantization expects [B,L,H,D] BF16 values")
    batch, length, heads, dim = values.shape
    if (batch != q.shape[0] or heads != q.shape[2] or dim != q.shape[3]
            or start < 0 or start + length > q.shape[1]
            or values.device != q.device):
        raise ValueError("KV quantization shape, capacity, or device mismatch")
    if length == 0:
        return
    if not assume_finite and not bool(torch.isfinite(values).all()):
        raise ValueError("Cannot quantize non-finite KV values")
    ops.kv_quantize_(q, scale, values, start)


@profiled("fp8_encode")
def quantize_kv_pair_into(cache: dict, k: torch.Tensor, v: torch.Tensor, start: int) -> None:
    """Validate K and V before writing either persistent payload or scale."""
    if k.shape != v.shape or k.dtype != v.dtype or k.device != v.device:
        raise ValueError("K/V shapes, dtypes, and devices must match")
    for key, values in (("k", k), ("v", v)):
        _validate(cache, key)
        q = cache[key]
        if (values.ndim != 4 or values.dtype != torch.bfloat16
                or values.shape[0] != q.shape[0]
                or values.shape[2:] != q.shape[2:]
                or start < 0 or start + values.shape[1] > q.shape[1]
                or values.device != q.device):
            raise ValueError("KV pair shape, capacity, dtype, or device mismatch")
        if not bool(torch.isfinite(values).all()):
            raise ValueError("Cannot quantize non-finite KV values")
    if k.shape[1] == 0:
        return
    if (k.stride() == v.stride() and cache["k"].stride() == cache["v"].stride()
            and cache["k"].dtype == cache["v"].dtype
            and cache["k_scale"].stride() == cache["v_scale"].stride()):
        ops.kv_quantize_pair_(cache["k"], cache["v"], cache["k_scale"], cache["v_scale"],
                              k, v, start)
    else:
        quantize_kv_into(cache, "k", k, start, assume_finite=True)
        quantize_kv_into(cache, "v", v, start, assume_finite=True)


@profiled("fp8_decode")
def dequantize_kv(cache: dict, key: str, valid_len: int) -> torch.Tensor:
    """Decode only the valid prefix into a BF16 attention tensor."""
    _validate(cache, key)
    q = cache[key]
    if valid_len < 0 or valid_len > q.shape[1]:
        raise ValueError("Invalid KV valid length")
    return ops.kv_dequantize(q, cache[f"{key}_scale"], valid_len)


def kv_storage_bytes(cache: dict) -> int:
    keys = STORAGE_KEYS if is_quantized_kv_cache(cache) else KV_KEYS
    return sum(cache[key].numel() * cache[key].element_size() for key in keys)
