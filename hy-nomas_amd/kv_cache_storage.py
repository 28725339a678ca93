"""Storage-format dispatch with the FP8 cache added.

Mirror of hymm/models/dit/modules/kv_cache_storage.py:6-23: ``cache_format``
now also reports "fp8" (e4m3 codes), ``quantization_mode`` accepts
``kv_cache_quantization: fp8``, and ``make_kv_block`` allocates the layer
cache the AR pipeline keeps per layer (causal_ar.py:584-620).
"""
from __future__ import annotations

import torch

MODES = ("none", "int8", "fp8", "qvg")


def cache_format(cache) -> str:
    mode = cache.get("storage_format")
    if mode is not None:
        return mode
    dtype = cache["k"].dtype
    if dtype == torch.int8:
        return "int8"
    if dtype == torch.float8_e4m3fn:
        return "fp8"
    return "none"


def cache_geometry(cache):
    return cache["k"].shape, cache["k"].device, cache["k"].dtype


def quantization_mode(inference) -> str:
    mode = getattr(inference, "kv_cache_quantization", "none")
    if mode not in MODES:
        raise ValueError("inference.kv_cache_quantization must be none, int8, fp8, or qvg")
    return mode


def make_kv_block(mode: str, batch: int, capacity: int, heads: int, dim: int, *, device,
                  dtype=torch.bfloat16) -> dict:
    from .fp8_kv_cache import make_fp8_kv_block, make_int8_kv_block
    if mode == "fp8":
        return make_fp8_kv_block(batch, capacity, heads, dim, device=device)
    if mode == "int8":
        return make_int8_kv_block(batch, capacity, heads, dim, device=device)
    if mode == "none":
        shape = (batch, capacity, heads, dim)
        return {"k": torch.empty(shape, device=device, dtype=dtype),
                "v": torch.empty(shape, device=device, dtype=dtype)}
    raise ValueError(f"unsupported KV cache mode for this build: {mode}")


def cache_storage_audit(cache) -> dict:
    keys = [k for k in ("k", "v", "k_scale", "v_scale") if k in cache]
    return {
        "storage_format": cache_format(cache),
        "gpu_storage_bytes": sum(cache[k].numel() * cache[k].element_size() for k in keys),
        "storage_dtypes": sorted({str(cache[k].dtype) for k in keys}),
        "transfer_bytes_scope": "KV payload only; excludes masks",
    }
