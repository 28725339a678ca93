"""Attention over the FP8 (or INT8) KV cache without a decoded BF16 copy.

The reference decodes each layer's quantized history into a new BF16 tensor,
concatenates the current chunk and then runs Flex/FA3/SDPA
(hymm/models/dit/nomas_cpt.py:529-531,614-625,771-829). Here one HIP kernel
reads the codes in place (dequantizing tiles in registers/LDS) and appends the
current chunk's BF16 K/V as an unquantized tail.

  * ``chunk_attention``: the functional form -- queries of one chunk against
    cache tokens [0, kv_len) (+ optional tail), block-causal at chunk
    granularity (the BASELINE config-3 workload).
  * ``causal_attention_with_cache_mp``: the reference's cached-attention entry
    point (nomas_cpt.py:335-884) for quantized caches: same arguments, same
    cache write (validate K and V, then quantize at ``cache_valid_len``),
    same key set ([history | img (+ txt)]) and the same [B, L, H*D] outputs.
  * ``FP8CacheAttention``: installs itself over the native function by
    assignment and falls back to it for calls it does not cover, the pattern
    of reactor's CacheStaging (reactor/hy_nomas_cache.py:76-100,192-256).
"""
from __future__ import annotations

from typing import Optional

import torch

from . import ops
from .fp8_kv_cache import is_quantized_kv_cache, quantize_kv_pair_into
from .metrics import stage


def chunk_attention(q: torch.Tensor, kv_cache: dict, kv_len: int, *,
                    k_cur: Optional[torch.Tensor] = None, v_cur: Optional[torch.Tensor] = None,
                    q_pos0: int = 0, chunk_len: int = 0,
                    softmax_scale: Optional[float] = None) -> torch.Tensor:
    """softmax(q K^T * scale) V over cache tokens [0, kv_len) then k_cur/v_cur.

    q: bf16 [B, Lq, H, D]; kv_cache: {"k","v": e4m3/int8 [B,cap,H,D],
    "k_scale","v_scale": fp32 [B,cap,H,1]}. Query i sits at position
    q_pos0 + i, cache token t at t, tail token j at kv_len + j; with
    chunk_len > 0 a key is visible iff its chunk index is <= the query's.
    """
    if not is_quantized_kv_cache(kv_cache):
        raise TypeError("chunk_attention reads FP8/INT8 caches")
    if kv_len < 0 or kv_len > kv_cache["k"].shape[1]:
        raise ValueError("Invalid KV valid length")
    if q.ndim != 4 or q.shape[0] != kv_cache["k"].shape[0] or q.shape[2:] != kv_cache["k"].shape[2:]:
        raise ValueError("query / cache geometry mismatch")
    scale = -1.0 if softmax_scale is None else float(softmax_scale)
    return ops.attn_fp8kv(q, kv_cache["k"], kv_cache["v"], kv_cache["k_scale"],
                          kv_cache["v_scale"], kv_len, k_cur, v_cur, q_pos0, chunk_len, scale)


def _all_true(mask: Optional[torch.Tensor]) -> bool:
    return mask is None or mask.numel() == 0 or bool(mask.bool().all())


def eligible(q, k, v, kv_cache, cache_valid_len, text_mask=None, cache_mask=None,
             sparse_context=None, sp_metadata=None, intra_seg_vid_windows=None, **_) -> bool:
    """Calls this kernel covers: quantized cache, single GPU, dense attention,
    head dim 128, no padded keys (text padding / cache holes)."""
    img_q = q[0]
    if not isinstance(kv_cache, dict) or "k" not in kv_cache or not is_quantized_kv_cache(kv_cache):
        return False
    if sparse_context is not None or sp_metadata is not None or intra_seg_vid_windows:
        return False
    if "swa_capacity" in kv_cache or torch.is_grad_enabled():
        return False
    if img_q.shape[-1] != 128 or not img_q.is_cuda:
        return False
    if kv_cache["k"].shape[0] != img_q.shape[0]:
        return False
    if not _all_true(text_mask):
        return False
    if cache_mask is not None and cache_valid_len > 0 and not _all_true(cache_mask[:, :cache_valid_len]):
        return False
    return True


def causal_attention_with_cache_mp(q, k, v, kv_cache, cache_valid_len: int = 0,
                                   attn_mode: str = None, text_mask=None,
                                   update_cache: bool = False, cache_txt: bool = True,
                                   cache_mask=None, intra_seg_txt_offsets=None,
                                   intra_seg_vid_windows=None, tokens_per_frame: int = 0,
                                   seg_ar_attention_backend: str = "magi", sparse_context=None,
                                   sp_metadata=None, attention_metadata=None):
    """FP8/INT8-cache form of nomas_cpt.py:335-884 (dense, single GPU, unpadded keys).

    q, k, v: (img, txt) tuples of [B, L, H, D]. Returns (img_attn [B, L_img, H*D],
    txt_attn [B, L_txt, H*D]) in the inputs' dtypes.
    """
    img_q, txt_q = q
    img_k, txt_k = k
    img_v, txt_v = v
    img_dtype, txt_dtype = img_q.dtype, txt_q.dtype
    if torch.is_grad_enabled():
        raise ValueError("Compressed KV requires no-grad inference")
    if img_q.device != kv_cache["k"].device or txt_q.device != kv_cache["k"].device:
        raise RuntimeError("Current Q and KV cache must be on the same device")

    bf = torch.bfloat16
    img_q, txt_q, img_k, txt_k, img_v, txt_v = (t.to(bf) for t in (img_q, txt_q, img_k, txt_k, img_v, txt_v))
    cur_k = torch.cat([img_k, txt_k], dim=1)
    cur_v = torch.cat([img_v, txt_v], dim=1)
    cache_k, cache_v = (cur_k, cur_v) if cache_txt else (img_k, img_v)
    B = img_q.shape[0]
    txt_len = txt_k.shape[1]

    if update_cache:
        new_end = cache_valid_len + cache_k.shape[1]
        quantize_kv_pair_into(kv_cache, cache_k.detach(), cache_v.detach(), cache_valid_len)
        if cache_mask is not None:
            write_mask = torch.ones(B, cache_k.shape[1], dtype=torch.bool, device=img_k.device)
            if cache_txt and text_mask is not None:
                write_mask[:, img_k.shape[1]:] = text_mask.bool()
            cache_mask[:, cache_valid_len:new_end] = write_mask

    # Keys: [history (quantized, read in place) | current img (+ txt)], all BF16
    # for the current chunk exactly as the reference keeps them (nomas_cpt.py:614-625).
    if cache_txt or update_cache:
        tail_k, tail_v = cur_k, cur_v
    else:
        tail_k, tail_v = img_k, img_v
    q_full = torch.cat([img_q, txt_q], dim=1)
    with stage("cache_attention"):
        hidden = chunk_attention(q_full, kv_cache, cache_valid_len, k_cur=tail_k.contiguous(),
                                 v_cur=tail_v.contiguous())
    img_len = img_q.shape[1]
    img_attn = hidden[:, :img_len].to(img_dtype)
    txt_attn = hidden[:, img_len:].to(txt_dtype)
    if txt_len and text_mask is not None:
        txt_attn = txt_attn * text_mask.bool()[:, :, None, None].to(txt_attn.dtype)
    return (img_attn.reshape(B, img_len, -1), txt_attn.reshape(B, txt_attn.shape[1], -1))


class FP8CacheAttention:
    """Replace ``native.causal_attention_with_cache_mp`` by assignment; calls the
    kernel when ``eligible`` and the original function otherwise."""

    def __init__(self, native_module):
        self._native = native_module
        self._original = native_module.causal_attention_with_cache_mp
        self.stats = {"calls": 0, "fallbacks": 0}
        native_module.causal_attention_with_cache_mp = self

    def uninstall(self):
        self._native.causal_attention_with_cache_mp = self._original

    def __call__(self, q, k, v, kv_cache, cache_valid_len=0, *args, **kwargs):
        self.stats["calls"] += 1
        names = ("attn_mode", "text_mask", "update_cache", "cache_txt", "cache_mask",
                 "intra_seg_txt_offsets", "intra_seg_vid_windows", "tokens_per_frame",
                 "seg_ar_attention_backend", "sparse_context", "sp_metadata", "attention_metadata")
        bound = dict(zip(names, args))
        bound.update(kwargs)
        if eligible(q, k, v, kv_cache, cache_valid_len, **bound):
            return causal_attention_with_cache_mp(q, k, v, kv_cache, cache_valid_len, **bound)
        self.stats["fallbacks"] += 1
        return self._original(q, k, v, kv_cache, cache_valid_len, *args, **kwargs)
