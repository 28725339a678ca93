"""Attention over the FP8 (or INT8) KV cache without a decoded BF16 copy.

The reference decodes each layer's quantized history into a new BF16 tensor,
concatenates the current chunk and then runs Flex/FA3/SDPA
(hymm/models/dit/nomas_cpt.py:529-531,614-625,771-829). Here one HIP kernel
reads the codes in place (dequantizing tiles in LDS) and appends the current
chunk's BF16 K/V as an unquantized tail. Key validity (padded text, holes in
the cached history) is a per-key byte mask the kernel applies inside the
softmax, so nothing is gathered or compacted.

  * ``chunk_attention``: the functional form -- queries of one chunk against
    cache tokens [0, kv_len) (+ optional tail), block-causal at chunk
    granularity (the BASELINE config-3 workload), with optional key masks and
    a one-slot cache read by every query batch.
  * ``causal_attention_with_cache_mp``: the reference's cached-attention entry
    point (nomas_cpt.py:335-884) for quantized caches: same arguments, same
    cache write (validate K and V, then quantize at ``cache_valid_len``, then
    the cache_mask update), the same key set and key mask for each of the
    update / denoise x cache_txt cases, the same CFG history broadcast, zero
    rows for padded queries and the same [B, L, H*D] outputs.
  * ``FP8CacheAttention``: installs itself over the native function by
    assignment (the pattern of reactor's CacheStaging,
    reactor/hy_nomas_cache.py:76-100,192-256). Calls it does not cover go to
    the original function for INT8 caches, which the native code can decode;
    for FP8 caches, which it cannot read, they raise.
"""
from __future__ import annotations

from typing import Optional

import torch

from . import ops
from .fp8_kv_cache import is_fp8_kv_cache, is_quantized_kv_cache, quantize_kv_pair_into
from .metrics import stage


def chunk_attention(q: torch.Tensor, kv_cache: dict, kv_len: int, *,
                    k_cur: Optional[torch.Tensor] = None, v_cur: Optional[torch.Tensor] = None,
                    q_pos0: int = 0, chunk_len: int = 0,
                    softmax_scale: Optional[float] = None,
                    cache_valid: Optional[torch.Tensor] = None,
                    cur_valid: Optional[torch.Tensor] = None) -> torch.Tensor:
    """softmax(q K^T * scale) V over cache tokens [0, kv_len) then k_cur/v_cur.

    q: bf16 [B, Lq, H, D]; kv_cache: {"k","v": e4m3/int8 [B or 1, cap, H, D],
    "k_scale","v_scale": fp32 [B or 1, cap, H, 1]} (a one-slot cache is read by
    every query batch). Query i sits at position q_pos0 + i, cache token t at
    t, tail token j at kv_len + j; with chunk_len > 0 a key is visible iff its
    chunk index is <= the query's. cache_valid (bool [B or 1, >= kv_len]) and
    cur_valid (bool [B, >= Lc]) drop invalid keys; a query that sees no valid
    key gets a zero row.
    """
    if not is_quantized_kv_cache(kv_cache):
        raise TypeError("chunk_attention reads FP8/INT8 caches")
    if kv_len < 0 or kv_len > kv_cache["k"].shape[1]:
        raise ValueError("Invalid KV valid length")
    if (q.ndim != 4 or kv_cache["k"].shape[0] not in (q.shape[0], 1)
            or q.shape[2:] != kv_cache["k"].shape[2:]):
        raise ValueError("query / cache geometry mismatch")
    return ops.attn_fp8kv(q, kv_cache["k"], kv_cache["v"], kv_cache["k_scale"],
                          kv_cache["v_scale"], kv_len, k_cur, v_cur, q_pos0, chunk_len,
                          None if softmax_scale is None else float(softmax_scale),
                          cache_valid, cur_valid)


def _dense_sparse_context(sparse_context, kv_cache, update_cache):
    """The reference's dense cases of a sparse context (nomas_cpt.py:717-731):
    permanently dense first layers (counted in kv_cache["dense_layer_stats"])
    and dense warm-up reads. Returns (dense, note): dense is True when the call
    is plain dense attention; note records the dense-layer count afterwards."""
    if sparse_context is None:
        return True, None
    cfg = sparse_context["config"]
    if sparse_context["layer"] < int(cfg.get("dense_first_n_layers", 1)):
        def note():
            stats = kv_cache.setdefault("dense_layer_stats", {"denoise": 0, "write": 0})
            stats["write" if update_cache else "denoise"] += 1
        return True, note
    if sparse_context.get("dense", False):
        if update_cache:
            raise ValueError("Dense warmup reads cannot update sparse cache metadata")
        return True, None
    return False, None


def ineligible_reason(q, k, v, kv_cache, cache_valid_len, attn_mode=None, text_mask=None,
                      update_cache=False, cache_txt=True, cache_mask=None,
                      intra_seg_txt_offsets=None, intra_seg_vid_windows=None, tokens_per_frame=0,
                      seg_ar_attention_backend="magi", sparse_context=None, sp_metadata=None,
                      attention_metadata=None) -> Optional[str]:
    """Why the HIP path does not cover a call (None: it does). Needs no host
    sync: masks are applied inside the kernel, whatever their contents."""
    img_q = q[0]
    if not isinstance(kv_cache, dict) or "k" not in kv_cache or not is_quantized_kv_cache(kv_cache):
        return "the cache is not FP8/INT8 storage"
    if sp_metadata is not None:
        return "sequence-parallel metadata (multi-GPU) is out of scope"
    if "swa_capacity" in kv_cache:
        return "sliding-window caches are out of scope"
    if kv_cache.get("swa_sampling", "recent") != "recent":
        return "sampled-history caches are out of scope"
    if intra_seg_vid_windows and intra_seg_txt_offsets is not None and any(
            o is not None for o in intra_seg_txt_offsets) and cache_txt:
        return "intra-segment action masks are out of scope"
    if sparse_context is not None and not _dense_sparse_context(sparse_context, kv_cache, False)[0]:
        return "pooled sparse attention is out of scope"
    if torch.is_grad_enabled():
        return "autograd is enabled"
    if img_q.shape[-1] != 128:
        return "head dim must be 128"
    if not img_q.is_cuda:
        return "tensors are not on a GPU"
    if attn_mode not in (None, "flash3", "torch"):
        return f"attn_mode {attn_mode!r}"
    return None


def eligible(q, k, v, kv_cache, cache_valid_len, **kwargs) -> bool:
    return ineligible_reason(q, k, v, kv_cache, cache_valid_len, **kwargs) is None


def causal_attention_with_cache_mp(q, k, v, kv_cache, cache_valid_len: int = 0,
                                   attn_mode: str = None, text_mask=None,
                                   update_cache: bool = False, cache_txt: bool = True,
                                   cache_mask=None, intra_seg_txt_offsets=None,
                                   intra_seg_vid_windows=None, tokens_per_frame: int = 0,
                                   seg_ar_attention_backend: str = "magi", sparse_context=None,
                                   sp_metadata=None, attention_metadata=None):
    """FP8/INT8-cache form of nomas_cpt.py:335-884 on one GPU.

    q, k, v: (img, txt) tuples of [B, L, H, D]. Returns (img_attn [B, L_img, H*D],
    txt_attn [B, L_txt, H*D]) in the inputs' dtypes. The attended keys and
    their mask follow the reference's quantized-storage branch:

      =========================  ============================  ==========================
      call                       keys                          key mask
      =========================  ============================  ==========================
      update, cache_txt          history | img | txt           cache_mask[:, :total]
                                                               (all valid without one)
      update, not cache_txt      history | img | txt           history | img | text_mask
      denoise, cache_txt         history | img | txt           history | img | text_mask
      denoise, not cache_txt     history | img                 history | img
      =========================  ============================  ==========================

    where "history" is cache_mask[:, :cache_valid_len] (all valid without a
    mask). Query rows of padded text are zero, as the flash3/Flex paths leave
    them (nomas_cpt.py:782-829); attn_mode "torch" keeps SDPA's rows.
    """
    if seg_ar_attention_backend not in ("magi", "flex"):
        raise ValueError("Invalid seg_ar_attention_backend")
    img_q, txt_q = q
    img_k, txt_k = k
    img_v, txt_v = v
    img_dtype, txt_dtype = img_q.dtype, txt_q.dtype
    if torch.is_grad_enabled():
        raise ValueError("Compressed KV/SWA requires no-grad inference")
    if kv_cache["k"].dtype != kv_cache["v"].dtype:
        raise RuntimeError("KV cache K/V dtype mismatch")
    if kv_cache["k"].device != kv_cache["v"].device:
        raise RuntimeError("KV cache K/V device mismatch")
    if img_q.device != kv_cache["k"].device or txt_q.device != kv_cache["k"].device:
        raise RuntimeError("Current Q and KV cache must be on the same device")
    dense, note_dense = _dense_sparse_context(sparse_context, kv_cache, update_cache)
    if not dense:
        raise ValueError("pooled sparse attention is not supported on the FP8 path")

    bf = torch.bfloat16
    img_q, txt_q, img_k, txt_k, img_v, txt_v = (t.to(bf) for t in (img_q, txt_q, img_k, txt_k, img_v, txt_v))
    B = img_q.shape[0]
    img_len, txt_len = img_k.shape[1], txt_k.shape[1]
    dev = img_k.device
    cur_k = torch.cat([img_k, txt_k], dim=1)
    cur_v = torch.cat([img_v, txt_v], dim=1)
    cache_k, cache_v = (cur_k, cur_v) if cache_txt else (img_k, img_v)

    # One canonical history slot may serve the B current (CFG) branches, read
    # only (nomas_cpt.py:547-567).
    history_batch = kv_cache["k"].shape[0]
    if history_batch != B:
        if update_cache:
            raise ValueError(
                "KV-cache batch mismatch during update: "
                f"current={B}, cache={history_batch}. "
                "Read-only history broadcasting is supported, cache writes are not.")
        if history_batch != 1:
            raise ValueError(
                f"KV-cache batch mismatch: current={B}, cache={history_batch}; only a single "
                "canonical history slot can be broadcast.")

    txt_valid = None if text_mask is None else text_mask.bool()
    if txt_valid is not None and tuple(txt_valid.shape) != (B, txt_len):
        raise ValueError("text_mask must be [B, L_txt]")
    history_valid = None
    if cache_mask is not None and cache_valid_len > 0:
        history_valid = cache_mask[:, :cache_valid_len]

    if update_cache:
        new_end = cache_valid_len + cache_k.shape[1]
        quantize_kv_pair_into(kv_cache, cache_k.detach(), cache_v.detach(), cache_valid_len)
        if cache_mask is not None:
            write_mask = torch.ones(B, cache_k.shape[1], dtype=torch.bool, device=dev)
            if cache_txt and txt_valid is not None:
                write_mask[:, img_len:] = txt_valid
            cache_mask[:, cache_valid_len:new_end] = write_mask

    # Keys after the history: the current chunk's bf16 K/V (the reference keeps
    # them unquantized for their own attention, nomas_cpt.py:614-625).
    if cache_txt or update_cache:
        tail_k, tail_v = cur_k, cur_v
        if update_cache and cache_txt and cache_mask is None:
            tail_valid = None  # kv_mask is all ones here (nomas_cpt.py:657-662)
        elif txt_valid is None:
            tail_valid = None
        else:
            tail_valid = torch.cat([torch.ones(B, img_len, dtype=torch.bool, device=dev), txt_valid], 1)
    else:
        tail_k, tail_v, tail_valid = img_k, img_v, None

    q_full = torch.cat([img_q, txt_q], dim=1)
    with stage("cache_attention"):
        hidden = chunk_attention(q_full, kv_cache, cache_valid_len, k_cur=tail_k.contiguous(),
                                 v_cur=tail_v.contiguous(), cache_valid=history_valid,
                                 cur_valid=tail_valid)
    if note_dense is not None:
        note_dense()
    img_attn = hidden[:, :img_len].to(img_dtype)
    txt_attn = hidden[:, img_len:].to(txt_dtype)
    if txt_len and txt_valid is not None and attn_mode != "torch":
        txt_attn = txt_attn * txt_valid[:, :, None, None].to(txt_attn.dtype)
    return (img_attn.reshape(B, img_len, -1), txt_attn.reshape(B, txt_len, -1))


class FP8CacheAttention:
    """Replace ``native.causal_attention_with_cache_mp`` by assignment; calls
    the kernel for the calls it covers. Other calls go to the original function
    when the cache is INT8 (the native code decodes it) and raise when it is
    FP8 (the native code cannot read e4m3 storage)."""

    _NAMES = ("attn_mode", "text_mask", "update_cache", "cache_txt", "cache_mask",
              "intra_seg_txt_offsets", "intra_seg_vid_windows", "tokens_per_frame",
              "seg_ar_attention_backend", "sparse_context", "sp_metadata", "attention_metadata")

    def __init__(self, native_module):
        self._native = native_module
        self._original = native_module.causal_attention_with_cache_mp
        self.stats = {"calls": 0, "fallbacks": 0}
        native_module.causal_attention_with_cache_mp = self

    def uninstall(self):
        self._native.causal_attention_with_cache_mp = self._original

    def __call__(self, q, k, v, kv_cache, cache_valid_len=0, *args, **kwargs):
        bound = dict(zip(self._NAMES, args))
        bound.update(kwargs)
        reason = ineligible_reason(q, k, v, kv_cache, cache_valid_len, **bound)
        if reason is None:
            self.stats["calls"] += 1
            return causal_attention_with_cache_mp(q, k, v, kv_cache, cache_valid_len, **bound)
        if isinstance(kv_cache, dict) and "k" in kv_cache and is_fp8_kv_cache(kv_cache):
            raise RuntimeError(f"FP8 KV cache call not covered by the HIP path ({reason}); "
                               "the native function cannot read FP8 storage")
        self.stats["fallbacks"] += 1
        return self._original(q, k, v, kv_cache, cache_valid_len, *args, **kwargs)
