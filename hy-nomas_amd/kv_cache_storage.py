"""Storage-format dispatch with the FP8 cache added, and the binding that
makes the reference's AR pipeline choose, allocate and audit FP8 caches.

Mirror of hymm/models/dit/modules/kv_cache_storage.py:6-23,77-105:
``cache_format`` also reports "fp8" (e4m3 codes), ``quantization_mode``
accepts ``kv_cache_quantization: fp8``, ``make_kv_block`` allocates the layer
cache the AR pipeline keeps per layer (causal_ar.py:584-620), and
``cache_storage_audit`` returns the keys the pipeline reads at the end of a
generation (causal_ar.py:3365-3374): storage_format, gpu_storage_bytes,
storage_dtypes, codec_stats, peak_working_bytes, transfer_bytes_scope.

``install_fp8_kv_storage`` patches a loaded reference (the storage module, the
INT8 cache module and the pipeline class) so that the unchanged pipeline runs
on FP8 caches; ``uninstall`` restores every attribute it replaced.
"""
from __future__ import annotations

import threading
from types import ModuleType
from typing import Optional

import torch

MODES = ("none", "int8", "fp8", "qvg")
_INHERITED = object()
STORAGE_KEYS = ("k", "v", "k_scale", "v_scale")


def _is_fp8(cache) -> bool:
    return (isinstance(cache, dict) and cache.get("storage_format") in (None, "fp8")
            and isinstance(cache.get("k"), torch.Tensor)
            and cache["k"].dtype == torch.float8_e4m3fn)


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


def storage_bytes(tensors) -> int:
    """Bytes of the distinct storages behind ``tensors`` (views of one
    allocation count once, at the allocation's full size)."""
    seen = {}
    for t in tensors:
        s = t.untyped_storage()
        seen[(str(t.device), s.data_ptr(), s.nbytes())] = s.nbytes()
    return sum(seen.values())


def cache_storage_audit(cache) -> dict:
    """The per-layer audit row of kv_cache_storage.py:77-105 for a dense,
    INT8 or FP8 cache. ``codec_stats`` is the cache's "kv_codec_stats" dict
    (empty: the FP8 and INT8 codecs keep no working set beyond the storage),
    and ``peak_working_bytes`` is the larger of the storage bytes and a
    ``peak_working_bytes`` entry in it."""
    payload = [cache[k] for k in STORAGE_KEYS if k in cache]
    audit = {
        "storage_format": cache_format(cache),
        "gpu_storage_bytes": storage_bytes(payload),
        "storage_dtypes": sorted({str(t.dtype) for t in payload}),
        "codec_stats": dict(cache.get("kv_codec_stats", {})),
    }
    audit["peak_working_bytes"] = max(audit["gpu_storage_bytes"],
                                      audit["codec_stats"].get("peak_working_bytes", 0))
    audit["transfer_bytes_scope"] = "KV payload only; excludes masks"
    return audit


class FP8KVStorage:
    """Patches a loaded reference so its AR pipeline keeps FP8 caches.

    * ``storage_module`` (hymm/models/dit/modules/kv_cache_storage.py):
      ``quantization_mode`` returns "fp8" for ``kv_cache_quantization: fp8``
      (the pipeline reads it at causal_ar.py:357-361, and
      ``validate_kv_cache_config`` calls it); ``cache_format`` reports "fp8"
      for e4m3 caches; ``cache_storage_audit`` audits them. Every other
      config or cache goes to the module's own functions.
    * ``pipeline_cls`` (CPTCausalInferencePipeline) and ``int8_kv_module``
      (hymm/models/dit/modules/int8_kv_cache.py): ``_initialize_kv_cache``
      of a pipeline whose ``kv_storage_format`` is "fp8" runs the pipeline's
      own method down its quantized-storage branch (causal_ar.py:589-594),
      which imports ``make_int8_kv_block`` from ``int8_kv_module`` at the
      call; for that call the module attribute is ``make_fp8_kv_block``.
      The pipeline's own checks (head sharding, no CPU phase-swap offload for
      compressed storage) apply unchanged, the masks and counters it sets up
      are the ones it always sets up, and ``int8_kv_storage`` is False again
      on return, so the end-of-generation audit reads "int8_kv": False and
      "kv_storage_format": "fp8". The pipeline's own log line for that call
      names the quantized branch ("format=int8").

    The attention over an FP8 cache goes through ``FP8CacheAttention``
    (cache_attention.py), which also writes the cache on update passes;
    install both before the pipeline is constructed.
    """

    _lock = threading.Lock()

    def __init__(self, storage_module: ModuleType, *, pipeline_cls: Optional[type] = None,
                 int8_kv_module: Optional[ModuleType] = None):
        if (pipeline_cls is None) != (int8_kv_module is None):
            raise ValueError("pipeline_cls and int8_kv_module are installed together")
        self._saved: list[tuple[object, str, object]] = []
        self.stats = {"fp8_allocations": 0}
        mode0 = storage_module.quantization_mode
        format0 = storage_module.cache_format
        audit0 = storage_module.cache_storage_audit

        def quantization_mode_(inference):
            if getattr(inference, "kv_cache_quantization", "none") == "fp8":
                return "fp8"
            return mode0(inference)

        def cache_format_(cache):
            return "fp8" if _is_fp8(cache) else format0(cache)

        def cache_storage_audit_(cache):
            return cache_storage_audit(cache) if _is_fp8(cache) else audit0(cache)

        self._replace(storage_module, "quantization_mode", quantization_mode_)
        self._replace(storage_module, "cache_format", cache_format_)
        self._replace(storage_module, "cache_storage_audit", cache_storage_audit_)
        if pipeline_cls is not None:
            self._bind_pipeline(pipeline_cls, int8_kv_module)

    def _replace(self, owner, name: str, value) -> None:
        # a class keeps what its own __dict__ held (an inherited method leaves
        # nothing to restore: uninstall deletes the override)
        old = owner.__dict__.get(name, _INHERITED) if isinstance(owner, type) else getattr(owner, name)
        self._saved.append((owner, name, old))
        setattr(owner, name, value)

    def _bind_pipeline(self, pipeline_cls: type, int8_kv_module: ModuleType) -> None:
        from .fp8_kv_cache import make_fp8_kv_block
        init0 = pipeline_cls._initialize_kv_cache
        lock, stats = self._lock, self.stats

        def _initialize_kv_cache(pipe, batch_size, max_cache_tokens, dtype, device):
            if getattr(pipe, "kv_storage_format", None) != "fp8":
                return init0(pipe, batch_size, max_cache_tokens, dtype, device)
            with lock:
                make0 = int8_kv_module.make_int8_kv_block
                int8_kv_module.make_int8_kv_block = make_fp8_kv_block
                pipe.int8_kv_storage = True
                try:
                    result = init0(pipe, batch_size, max_cache_tokens, dtype, device)
                finally:
                    pipe.int8_kv_storage = False
                    int8_kv_module.make_int8_kv_block = make0
            stats["fp8_allocations"] += 1
            return result

        self._replace(pipeline_cls, "_initialize_kv_cache", _initialize_kv_cache)

    def uninstall(self) -> None:
        while self._saved:
            owner, name, value = self._saved.pop()
            if value is _INHERITED:
                delattr(owner, name)
            else:
                setattr(owner, name, value)


def install_fp8_kv_storage(storage_module: ModuleType, *, pipeline_cls: Optional[type] = None,
                           int8_kv_module: Optional[ModuleType] = None) -> FP8KVStorage:
    """Install ``FP8KVStorage`` on a loaded reference and return it."""
    return FP8KVStorage(storage_module, pipeline_cls=pipeline_cls, int8_kv_module=int8_kv_module)
