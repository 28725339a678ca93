"""Segment-AR KV storage in OCP e4m3 (or the reference's INT8 codes), written
and read by the HIP kernels of libhynomas_fp8.so.

Functional surface of the reference's INT8 KV module
(hymm/models/dit/modules/int8_kv_cache.py:92-210), with its layout, argument
order, exception types and messages:

  ==========================  ==================================  ===========
  here                        reference                           lines
  ==========================  ==================================  ===========
  make_fp8_kv_block           (FP8 form of make_int8_kv_block)    :92-107
  make_int8_kv_block          make_int8_kv_block                  :92-107
  is_fp8_kv_cache             (FP8 form of is_int8_kv_cache)      :110-111
  quantize_kv_into            quantize_kv_into                    :125-158
  quantize_kv_pair_into       quantize_kv_pair_into               :161-179
  dequantize_kv               dequantize_kv                       :182-205
  kv_storage_bytes            kv_storage_bytes                    :208-210
  ==========================  ==================================  ===========

Layout: a dict per layer. "k"/"v" hold one code byte per element,
[B, capacity, H, D], tokens major; "k_scale"/"v_scale" hold one fp32 per
(batch, token, head) row, [B, capacity, H, 1]. The e4m3 row rule is
s = amax / 448 (1 for an all-zero row) and code = e4m3_rne(x / s); an INT8
cache gets the reference's own codes (127 and round-half-away), bit for bit.

Finiteness is checked on the GPU: the kernels test every value before the
write and store nothing if one is NaN/Inf. By default the write then reads that
flag once and raises ValueError, as the reference does after its isfinite
checks; passing ``status`` (an int32 device tensor) leaves the flag there for
the caller to read later, with no host synchronisation in the write.
"""
from __future__ import annotations

from typing import Optional

import torch

from . import ops
from .metrics import profiled

KV_KEYS = ("k", "v")
STORAGE_KEYS = ("k", "v", "k_scale", "v_scale")
FP8 = torch.float8_e4m3fn
CODE_DTYPES = (FP8, torch.int8)

_NONFINITE = "Cannot quantize non-finite KV values"


def _allocate(batch, capacity, heads, dim, code_dtype, device, pin_memory) -> dict:
    geometry = {"k": (dim, code_dtype), "v": (dim, code_dtype),
                "k_scale": (1, torch.float32), "v_scale": (1, torch.float32)}
    return {name: torch.empty((batch, capacity, heads, last), dtype=dtype, device=device,
                              pin_memory=pin_memory)
            for name, (last, dtype) in geometry.items()}


def make_fp8_kv_block(batch: int, capacity: int, heads: int, dim: int, *,
                      device: torch.device | str, pin_memory: bool = False) -> dict:
    """Uninitialised storage for one layer: e4m3 codes and fp32 row scales."""
    return _allocate(batch, capacity, heads, dim, FP8, device, pin_memory)


def make_int8_kv_block(batch: int, capacity: int, heads: int, dim: int, *,
                       device: torch.device | str, pin_memory: bool = False) -> dict:
    """The same storage with INT8 codes: the reference's own cache format."""
    return _allocate(batch, capacity, heads, dim, torch.int8, device, pin_memory)


def is_fp8_kv_cache(cache: dict) -> bool:
    return cache["k"].dtype == FP8


def is_quantized_kv_cache(cache: dict) -> bool:
    return cache["k"].dtype in CODE_DTYPES


def _storage(cache: dict, key: str) -> tuple[torch.Tensor, torch.Tensor]:
    """The (codes, scales) pair named by key, after the storage checks."""
    if key not in KV_KEYS:
        raise ValueError(f"Invalid KV key: {key}")
    codes, scales = cache[key], cache[f"{key}_scale"]
    if codes.dtype not in CODE_DTYPES or scales.dtype != torch.float32:
        raise TypeError("FP8/INT8 KV data and FP32 scale are required")
    if scales.shape != (*codes.shape[:-1], 1) or scales.device != codes.device:
        raise ValueError("KV scale shape/device mismatch")
    return codes, scales


def _fits(codes: torch.Tensor, values: torch.Tensor, start: int) -> bool:
    """values [B, L, H, D] land in tokens [start, start + L) of codes' capacity."""
    return (values.shape[0] == codes.shape[0] and values.shape[2:] == codes.shape[2:]
            and 0 <= start and start + values.shape[1] <= codes.shape[1]
            and values.device == codes.device)


def _raise_if_flagged(status: torch.Tensor) -> None:
    if int(status[0].item()):
        raise ValueError(_NONFINITE)


def quantize_kv_into(cache: dict, key: str, values: torch.Tensor, start: int, *,
                     assume_finite: bool = False, status: Optional[torch.Tensor] = None) -> None:
    """Quantize bf16 values [B, L, H, D] into one storage tensor at tokens
    [start, start + L). Unless ``assume_finite``, NaN/Inf values are refused
    before anything is written (ValueError, or status[0] = 1 when a status
    tensor is given)."""
    codes, scales = _storage(cache, key)
    if values.ndim != 4 or values.dtype != torch.bfloat16:
        raise TypeError("KV quantization expects [B,L,H,D] BF16 values")
    if not _fits(codes, values, start):
        raise ValueError("KV quantization shape, capacity, or device mismatch")
    if values.shape[1] == 0:
        return
    if assume_finite:
        ops.kv_quantize_(codes, scales, values, start)
        return
    flag = status if status is not None else torch.empty(1, dtype=torch.int32, device=codes.device)
    ops.kv_quantize_(codes, scales, values, start, flag)
    if status is None:
        _raise_if_flagged(flag)


@profiled("fp8_encode")
def quantize_kv_pair_into(cache: dict, k: torch.Tensor, v: torch.Tensor, start: int, *,
                          status: Optional[torch.Tensor] = None) -> None:
    """Write one layer's K and V at tokens [start, start + L). Every check,
    the finiteness of both tensors included, passes before either tensor's
    codes or scales change."""
    if k.shape != v.shape or k.dtype != v.dtype or k.device != v.device:
        raise ValueError("K/V shapes, dtypes, and devices must match")
    for key, values in (("k", k), ("v", v)):
        codes, _ = _storage(cache, key)
        if values.ndim != 4 or values.dtype != torch.bfloat16 or not _fits(codes, values, start):
            raise ValueError("KV pair shape, capacity, dtype, or device mismatch")
    if k.shape[1] == 0:
        return
    if k.stride() != v.stride():
        k, v = k.contiguous(), v.contiguous()
    one_layout = (cache["k"].stride() == cache["v"].stride() and cache["k"].dtype == cache["v"].dtype
                  and cache["k_scale"].stride() == cache["v_scale"].stride())
    if one_layout:
        # one launch sequence: K and V validated together, then both written
        flag = status if status is not None else torch.empty(1, dtype=torch.int32, device=k.device)
        ops.kv_quantize_pair_(cache["k"], cache["v"], cache["k_scale"], cache["v_scale"], k, v,
                              start, flag)
        if status is None:
            _raise_if_flagged(flag)
        return
    # K and V storage laid out differently (never the case for blocks made
    # here): validate both on the host, then write each.
    finite = bool(torch.isfinite(k).all()) and bool(torch.isfinite(v).all())
    if status is not None:
        status.fill_(0 if finite else 1)
    if not finite:
        if status is None:
            raise ValueError(_NONFINITE)
        return
    ops.kv_quantize_(cache["k"], cache["k_scale"], k, start)
    ops.kv_quantize_(cache["v"], cache["v_scale"], v, start)


@profiled("fp8_decode")
def dequantize_kv(cache: dict, key: str, valid_len: int) -> torch.Tensor:
    """A new bf16 [B, valid_len, H, D] tensor holding bf16(code * scale) of
    the first valid_len tokens (the attention kernel never needs it; it reads
    the codes in place)."""
    codes, scales = _storage(cache, key)
    if valid_len < 0 or valid_len > codes.shape[1]:
        raise ValueError("Invalid KV valid length")
    return ops.kv_dequantize(codes, scales, valid_len)


def kv_storage_bytes(cache: dict) -> int:
    names = STORAGE_KEYS if is_quantized_kv_cache(cache) else KV_KEYS
    return sum(cache[n].numel() * cache[n].element_size() for n in names)
