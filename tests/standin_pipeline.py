"""A stand-in for the parts of the reference's AR pipeline that pick, allocate,
grow and audit the KV cache, shaped like the code they stand for so the FP8
storage binding can be driven without the reference's dependencies:

  * ``storage``: hymm/models/dit/modules/kv_cache_storage.py -- the reference's
    rules: cache_format knows "int8"/"none", quantization_mode refuses "fp8"
    (:19-23), cache_storage_audit returns the per-layer row of :77-105.
  * ``int8_kv``: hymm/models/dit/modules/int8_kv_cache.py:92-107
    (make_int8_kv_block).
  * ``Pipeline``: CPTCausalInferencePipeline's __init__ storage choice
    (causal_ar.py:357-361), _initialize_kv_cache's allocation branches
    (:524-631, quantized blocks only when int8_kv_storage), the capacity
    growth loop (:632-690) and the end-of-generation audit (:3365-3374).

Each function reads the storage module's attributes at the call, as the
reference's function-local ``from ... import`` statements do.
"""
from __future__ import annotations

import types

import torch


def _storage_module() -> types.ModuleType:
    m = types.ModuleType("standin_kv_cache_storage")

    def cache_format(cache):
        mode = cache.get("storage_format")
        if mode is not None:
            return mode
        return "int8" if cache["k"].dtype == torch.int8 else "none"

    def cache_geometry(cache):
        return cache["k"].shape, cache["k"].device, cache["k"].dtype

    def quantization_mode(inference):
        mode = getattr(inference, "kv_cache_quantization", "none")
        if mode not in ("none", "int8", "qvg"):
            raise ValueError("inference.kv_cache_quantization must be none, int8, or qvg")
        return mode

    def validate_kv_cache_config(args):
        m.quantization_mode(args.inference)

    def cache_storage_audit(cache):
        tensors = [cache[k] for k in ("k", "v", "k_scale", "v_scale") if k in cache]
        row = {"storage_format": m.cache_format(cache),
               "gpu_storage_bytes": sum(t.untyped_storage().nbytes() for t in tensors),
               "storage_dtypes": sorted({str(t.dtype) for t in tensors}),
               "codec_stats": dict(cache.get("kv_codec_stats", {}))}
        row["peak_working_bytes"] = max(row["gpu_storage_bytes"],
                                        row["codec_stats"].get("peak_working_bytes", 0))
        row["transfer_bytes_scope"] = "KV payload only; excludes masks"
        return row

    for f in (cache_format, cache_geometry, quantization_mode, validate_kv_cache_config,
              cache_storage_audit):
        setattr(m, f.__name__, f)
    return m


def _int8_module() -> types.ModuleType:
    m = types.ModuleType("standin_int8_kv_cache")

    def make_int8_kv_block(batch, capacity, heads, dim, *, device, pin_memory=False):
        shape, scale = (batch, capacity, heads, dim), (batch, capacity, heads, 1)
        return {"k": torch.empty(shape, dtype=torch.int8, device=device),
                "v": torch.empty(shape, dtype=torch.int8, device=device),
                "k_scale": torch.empty(scale, dtype=torch.float32, device=device),
                "v_scale": torch.empty(scale, dtype=torch.float32, device=device)}

    m.make_int8_kv_block = make_int8_kv_block
    return m


def make_reference():
    """(storage module, int8 module, pipeline class), fresh for each test."""
    storage, int8_kv = _storage_module(), _int8_module()

    class Pipeline:
        def __init__(self, args, hidden_size=256, heads_num=2, num_double_blocks=3):
            self.args = args
            self.hidden_size, self.heads_num = hidden_size, heads_num
            self.num_double_blocks = num_double_blocks
            self.kv_cache = None
            storage.validate_kv_cache_config(args)
            self.kv_storage_format = storage.quantization_mode(args.inference)
            self.int8_kv_storage = self.kv_storage_format == "int8"
            self.qvg_kv_storage = self.kv_storage_format == "qvg"
            self.log = []

        def _initialize_kv_cache(self, batch_size, max_cache_tokens, dtype, device):
            head_dim = self.hidden_size // self.heads_num
            cpu_offload = bool(getattr(self.args.inference,
                                       "interactive_kv_cache_layerwise_cpu_offload", False))
            if cpu_offload and self.int8_kv_storage:
                raise ValueError("Compressed KV cannot use PhaseSwappedKVCache")
            if self.int8_kv_storage:
                make_int8_kv_block = int8_kv.make_int8_kv_block
                self.kv_cache = [make_int8_kv_block(batch_size, max_cache_tokens, self.heads_num,
                                                    head_dim, device=device)
                                 for _ in range(self.num_double_blocks)]
            else:
                shape = [batch_size, max_cache_tokens, self.heads_num, head_dim]
                self.kv_cache = [{"k": torch.empty(shape, dtype=dtype, device=device),
                                  "v": torch.empty(shape, dtype=dtype, device=device)}
                                 for _ in range(self.num_double_blocks)]
            self.cache_mask_list = [torch.zeros([batch_size, max_cache_tokens], dtype=torch.bool,
                                                device=device)
                                    for _ in range(self.num_double_blocks)]
            self.cache_valid_len = 0
            self.log.append(f"format={'int8' if self.int8_kv_storage else 'none'}")

        def _ensure_kv_cache_capacity(self, required_tokens):
            current = int(storage.cache_geometry(self.kv_cache[0])[0][1])
            if current >= required_tokens:
                return
            for cache in self.kv_cache:
                for key in ("k", "v", "k_scale", "v_scale"):
                    if key not in cache:
                        continue
                    old = cache[key]
                    grown = torch.empty([old.shape[0], required_tokens, *old.shape[2:]],
                                        dtype=old.dtype, device=old.device)
                    grown[:, :self.cache_valid_len].copy_(old[:, :self.cache_valid_len])
                    cache[key] = grown
            for i, old in enumerate(self.cache_mask_list):
                grown = torch.zeros([old.shape[0], required_tokens], dtype=old.dtype,
                                    device=old.device)
                grown[:, :self.cache_valid_len].copy_(old[:, :self.cache_valid_len])
                self.cache_mask_list[i] = grown

        def storage_audit(self):
            rows = [storage.cache_storage_audit(cache) for cache in self.kv_cache]
            return {"int8_kv": self.int8_kv_storage,
                    "kv_storage_format": rows[0]["storage_format"],
                    "gpu_kv_storage_bytes": sum(r["gpu_storage_bytes"] for r in rows),
                    "codec_stats": [r["codec_stats"] for r in rows],
                    "kv_storage_layers": rows,
                    "gpu_kv_peak_working_bytes_upper_bound": sum(r["peak_working_bytes"] for r in rows)}

    return storage, int8_kv, Pipeline


def args_for(mode: str, **inference):
    inf = types.SimpleNamespace(kv_cache_quantization=mode, **inference)
    return types.SimpleNamespace(inference=inf)
