"""One DiT block forward with FP8 linears and the FP8 KV cache, and the
multi-block AR chunk step built from it (BASELINE configs 4 and 5).

Block math follows the reference's inference pre/post functions
(hymm/models/dit/modules/nomas_compile_prepost.py:14-99) for the image stream:
adaLN modulation from silu(vec); LayerNorm (eps 1e-6, no affine) + modulate,
fused with the per-token FP8 quantization of the QKV input into one kernel;
Q/K/V projection (fused into one 3072 -> 9216 FP8 GEMM); per-head RMSNorm
(fp32, eps 1e-6, weight); interleaved-pair RoPE in fp32 over (t, h, w) with
axes [16, 56, 56] and theta 256 (posemb_layers.py:191-260,401-453); cached
attention (FP8 cache history + this chunk's bf16 K/V); out-projection and
gated residual; LayerNorm + modulate (fused with fc1's input quantization as
above); FFN fc1 with GELU-tanh fused into the
GEMM epilogue, fc2; gated residual. With ``text=True`` the block also carries
the double-stream block's text stream (:37-38,55-63,90-98): its own adaLN
modulation from silu(vec_txt), LayerNorm + modulate + FP8 QKV, per-head
RMSNorm without RoPE, and the same out-projection / FFN structure; the two
streams meet in the cached attention, which attends [history | img | txt]
keys with the text and cache masks through cache_attention's form of the
reference's causal_attention_with_cache_mp (which also writes img + txt K/V
on update passes). The AR step follows
hymm/pipeline/causal_ar.py:2348-2432,2624-2645,2852: N denoising passes
without cache writes, one cache-write pass, then the valid length advances.
"""
from __future__ import annotations

import math

import torch
import torch.nn as nn
import torch.nn.functional as F

from . import ops
from .cache_attention import causal_attention_with_cache_mp, chunk_attention
from .dit_fp8_linear import FP8StoredLinear, fp8_linear, fp8_linear_codes
from .fp8_kv_cache import make_fp8_kv_block
from .metrics import stage


def rope_tables(frames: int, height: int, width: int, dims=(16, 56, 56), theta: float = 256.0,
                t_offset: int = 0, device=None):
    """cos/sin [frames*height*width, sum(dims)] fp32, interleaved (repeat_interleave(2))."""
    axes = [torch.arange(n, dtype=torch.float32, device=device) for n in (frames, height, width)]
    axes[0] = axes[0] + t_offset
    grid = torch.meshgrid(*axes, indexing="ij")
    cos, sin = [], []
    for d, g in zip(dims, grid):
        freqs = 1.0 / (theta ** (torch.arange(0, d, 2, device=device)[: d // 2].float() / d))
        ang = torch.outer(g.reshape(-1), freqs)
        cos.append(ang.cos().repeat_interleave(2, dim=1))
        sin.append(ang.sin().repeat_interleave(2, dim=1))
    return torch.cat(cos, dim=1), torch.cat(sin, dim=1)


def _modulate(x, shift, scale):
    return x * (1 + scale.unsqueeze(1)) + shift.unsqueeze(1)


class FP8DiTBlock(nn.Module):
    """One double-stream block at inference with FP8 linears: the image stream,
    and with ``text=True`` the text stream beside it."""

    def __init__(self, hidden: int = 3072, heads: int = 24, mlp_ratio: int = 4,
                 qk_eps: float = 1e-6, *, device=None, generator=None,
                 validate_kv_writes: bool = True, fuse_ln_quant: bool = True, text: bool = False):
        super().__init__()
        self.hidden, self.heads, self.head_dim = hidden, heads, hidden // heads
        self.qk_eps = qk_eps
        # The cache write is fused into the QK norm/RoPE kernel. True: the
        # values it would write are validated on the device first and nothing
        # is written if one is NaN/Inf (the reference's validate-before-write,
        # int8_kv_cache.py:161-179), flagged in a status word. False: unchecked.
        self.validate_kv_writes = validate_kv_writes
        # True: LayerNorm + modulate + the per-token FP8 quantization of the QKV
        # and fc1 inputs run as one kernel (ops.ln_modulate_quantize_fp8).
        self.fuse_ln_quant = fuse_ln_quant
        kw = dict(device=device, dtype=torch.bfloat16)

        def lin(i, o):
            m = nn.Linear(i, o, **kw)
            with torch.no_grad():
                m.weight.normal_(0.0, 0.02, generator=generator)
                m.bias.normal_(0.0, 0.02, generator=generator)
            return m

        self.mod = lin(hidden, 6 * hidden)  # tiny GEMV (M = batch), stays bf16
        self.qkv = FP8StoredLinear(lin(hidden, 3 * hidden))
        self.proj = FP8StoredLinear(lin(hidden, hidden))
        self.fc1 = FP8StoredLinear(lin(hidden, mlp_ratio * hidden))
        self.fc2 = FP8StoredLinear(lin(mlp_ratio * hidden, hidden))
        self.q_norm = nn.Parameter(torch.ones(self.head_dim, **kw))
        self.k_norm = nn.Parameter(torch.ones(self.head_dim, **kw))
        # text stream (made after the image stream's weights, so a seed gives
        # the same image weights with or without it)
        self.text = text
        if text:
            self.txt_mod = lin(hidden, 6 * hidden)
            self.txt_qkv = FP8StoredLinear(lin(hidden, 3 * hidden))
            self.txt_proj = FP8StoredLinear(lin(hidden, hidden))
            self.txt_fc1 = FP8StoredLinear(lin(hidden, mlp_ratio * hidden))
            self.txt_fc2 = FP8StoredLinear(lin(mlp_ratio * hidden, hidden))
            self.txt_q_norm = nn.Parameter(torch.ones(self.head_dim, **kw))
            self.txt_k_norm = nn.Parameter(torch.ones(self.head_dim, **kw))
        self._identity_rope = {}

    def _fused(self, linear) -> bool:
        return self.fuse_ln_quant and isinstance(linear, FP8StoredLinear)

    def _stream_qkv(self, x, vec, mod, qkv_linear):
        """adaLN parts from silu(vec), LayerNorm + modulate and the FP8 QKV
        projection of one stream: returns QKV [B, L, 3, H, D] and the parts."""
        B, L, C = x.shape
        H, D = self.heads, self.head_dim
        with stage("modulation"):
            parts = F.linear(F.silu(vec), mod.weight, mod.bias).chunk(6, dim=-1)
            if self._fused(qkv_linear):
                qx, sx = ops.ln_modulate_quantize_fp8(x, parts[0], parts[1], 1e-6)
            else:
                h = _modulate(F.layer_norm(x, (C,), eps=1e-6), parts[0], parts[1])
        with stage("qkv_fp8"):
            if self._fused(qkv_linear):
                qkv = fp8_linear_codes(qkv_linear, qx, sx).view(B, L, 3, H, D)
            else:
                qkv = fp8_linear(qkv_linear, h).view(B, L, 3, H, D)
        return qkv, parts

    def pre_attention(self, img, vec, cos, sin, kv_cache=None, cache_start: int = 0,
                      kv_status=None):
        """Image-stream half of nomas_compile_prepost.pre_attention (:29-72):
        adaLN parts, LayerNorm + modulate, fused FP8 QKV, then per-head RMSNorm
        and RoPE in one kernel, in place on the QKV output. Returns q, k, v
        [B, L, H, D] bf16 (views of that output) and the six modulation parts.
        With ``kv_cache`` given, the rotated K and V are also written into it at
        ``cache_start`` by the same kernel; with ``kv_status`` (int32 on the
        device) that write is validated first and skipped, status[0] = 1, if
        any value is NaN/Inf."""
        qkv, parts = self._stream_qkv(img, vec, self.mod, self.qkv)
        # select views (not unbind's multi-output views), so the in-place
        # norm/RoPE may modify them
        q, k, v = qkv.select(2, 0), qkv.select(2, 1), qkv.select(2, 2)
        with stage("qk_norm_rope"):
            if kv_cache is None:
                ops.qk_norm_rope_(q, k, v, self.q_norm, self.k_norm, cos, sin, self.qk_eps)
            else:
                ops.qk_norm_rope_kv_(q, k, v, self.q_norm, self.k_norm, cos, sin, self.qk_eps,
                                     kv_cache["k"], kv_cache["v"], kv_cache["k_scale"],
                                     kv_cache["v_scale"], cache_start, kv_status)
        return q, k, v, parts

    def pre_attention_txt(self, txt, vec_txt):
        """Text-stream half of pre_attention (:55-63): adaLN parts from
        silu(vec_txt), LayerNorm + modulate, fused FP8 QKV, per-head RMSNorm
        (the reference rotates only the image tokens). The norm runs in the
        image stream's kernel with cos = 1, sin = 0 tables, where the rotation
        returns its input: bf16(y * 1 + r * 0) = y."""
        if not self.text:
            raise ValueError("this block was built without the text stream (text=False)")
        qkv, parts = self._stream_qkv(txt, vec_txt, self.txt_mod, self.txt_qkv)
        q, k, v = qkv.select(2, 0), qkv.select(2, 1), qkv.select(2, 2)
        L = txt.shape[1]
        key = (L, txt.device)
        if key not in self._identity_rope:
            self._identity_rope[key] = (torch.ones(L, self.head_dim, dtype=torch.float32, device=txt.device),
                                        torch.zeros(L, self.head_dim, dtype=torch.float32, device=txt.device))
        cos, sin = self._identity_rope[key]
        with stage("qk_norm_rope"):
            ops.qk_norm_rope_(q, k, v, self.txt_q_norm, self.txt_k_norm, cos, sin, self.qk_eps)
        return q, k, v, parts

    def _post(self, x, attn, parts, proj, fc1, fc2):
        """nomas_compile_prepost.post_attention (:75-99) for one stream:
        out-projection and gated residual, LayerNorm + modulate, FFN with
        GELU-tanh fused into fc1's epilogue, gated residual."""
        B, L, C = x.shape
        with stage("post_fp8"):
            x = x + fp8_linear(proj, attn.reshape(B, L, C)) * parts[2].unsqueeze(1)
            if self._fused(fc1):
                qh, sh = ops.ln_modulate_quantize_fp8(x, parts[3], parts[4], 1e-6)
                h = fp8_linear_codes(fc1, qh, sh, gelu=True).view(B, L, -1)
            else:
                h = _modulate(F.layer_norm(x, (C,), eps=1e-6), parts[3], parts[4])
                h = fp8_linear(fc1, h, gelu=True)
            h = fp8_linear(fc2, h)
            x = x + h * parts[5].unsqueeze(1)
        return x

    def post_attention(self, img, attn, parts):
        """Image-stream half of nomas_compile_prepost.post_attention (:75-88)."""
        return self._post(img, attn, parts, self.proj, self.fc1, self.fc2)

    def post_attention_txt(self, txt, attn, parts):
        """Text-stream half of post_attention (:90-98)."""
        return self._post(txt, attn, parts, self.txt_proj, self.txt_fc1, self.txt_fc2)

    def forward(self, img, vec, cos, sin, kv_cache, cache_valid_len: int,
                update_cache: bool = False, kv_status=None, *, txt=None, vec_txt=None,
                text_mask=None, cache_mask=None, cache_txt: bool = True):
        """One block at inference. With ``update_cache`` this chunk's rotated K
        and V go into ``kv_cache`` at ``cache_valid_len``. When writes are
        validated and no ``kv_status`` is passed, a non-finite value raises
        ValueError here (one host read of the device flag); with one, the flag
        is left for the caller to read.

        With ``txt`` ([B, L_txt, C], text stream blocks only) the call follows
        the double-stream block (nomas_cpt.py:1293-1459): both streams' Q/K/V,
        then causal_attention_with_cache_mp over [history | img | txt] with
        ``text_mask`` (bool [B, L_txt]) and ``cache_mask`` (bool [B, cap], the
        history's validity, updated on writes), ``cache_txt`` as the
        reference's (the text keys are attended, and written on updates, on a
        segment's first chunk); returns (img, txt). Its cache write is the
        validated pair write (a non-finite value raises ValueError)."""
        if txt is not None:
            if kv_status is not None:
                raise ValueError("kv_status applies to the image-only path")
            q, k, v, parts = self.pre_attention(img, vec, cos, sin)
            tq, tk, tv, tparts = self.pre_attention_txt(txt, vec_txt)
            img_attn, txt_attn = causal_attention_with_cache_mp(
                (q, tq), (k, tk), (v, tv), kv_cache, cache_valid_len, "flash3", text_mask,
                update_cache, cache_txt, cache_mask)
            return self.post_attention(img, img_attn, parts), self.post_attention_txt(txt, txt_attn, tparts)
        status = None
        if update_cache and self.validate_kv_writes:
            status = kv_status if kv_status is not None else torch.empty(
                1, dtype=torch.int32, device=img.device)
        q, k, v, parts = self.pre_attention(img, vec, cos, sin, kv_cache if update_cache else None,
                                            cache_valid_len, status)
        if status is not None and kv_status is None and int(status[0].item()):
            raise ValueError("Cannot quantize non-finite KV values")
        with stage("cache_attention"):
            attn = chunk_attention(q, kv_cache, cache_valid_len, k_cur=k, v_cur=v)
        return self.post_attention(img, attn, parts)


class FP8ARModel(nn.Module):
    """A stack of FP8 blocks with one FP8 KV cache per block, stepped one chunk
    at a time: ``denoise_steps`` passes without cache writes, then one pass
    at t = 0 that writes this chunk's K/V, then the valid length advances.

    With ``text_len`` > 0 the blocks carry the text stream and every chunk
    opens a segment (the reference's cache_txt case): each pass takes the
    segment's text tokens [1, text_len, C] beside the image, attends
    [history | img | txt] under ``text_mask`` and the per-layer cache masks,
    and the write pass stores img + txt K/V, so the valid length advances by
    the image tokens plus ``text_len``."""

    def __init__(self, depth: int = 40, hidden: int = 3072, heads: int = 24,
                 latent_shape=(3, 45, 80), max_chunks: int = 17, *, device=None, seed: int = 0,
                 text_len: int = 0):
        super().__init__()
        g = torch.Generator(device=device).manual_seed(seed)
        self.text_len = int(text_len)
        self.blocks = nn.ModuleList(
            FP8DiTBlock(hidden, heads, device=device, generator=g, text=self.text_len > 0)
            for _ in range(depth))
        self.latent_shape = tuple(latent_shape)
        self.tokens_per_chunk = math.prod(latent_shape)
        self.write_tokens = self.tokens_per_chunk + self.text_len
        self.capacity = max_chunks * self.write_tokens
        self.heads, self.head_dim = heads, hidden // heads
        self.device = device
        self.caches = [make_fp8_kv_block(1, self.capacity, heads, self.head_dim, device=device)
                       for _ in range(depth)]
        # history validity per layer (padded text keys stay invalid)
        self.cache_masks = ([torch.zeros(1, self.capacity, dtype=torch.bool, device=device)
                             for _ in range(depth)] if self.text_len else None)
        # one device status word per layer for the validated cache writes
        self.kv_status = torch.zeros(depth, dtype=torch.int32, device=device)
        self.cache_valid_len = 0
        self.frames_done = 0

    @torch.no_grad()
    def forward_chunk(self, img, vec, update_cache: bool, txt=None, vec_txt=None, text_mask=None):
        t, h, w = self.latent_shape
        cos, sin = rope_tables(t, h, w, t_offset=self.frames_done, device=img.device)
        if self.text_len:
            if txt is None or txt.shape[1] != self.text_len:
                raise ValueError(f"this model takes {self.text_len} text tokens per chunk")
            vec_txt = vec if vec_txt is None else vec_txt
            for block, cache, mask in zip(self.blocks, self.caches, self.cache_masks):
                img, txt = block(img, vec, cos, sin, cache, self.cache_valid_len, update_cache,
                                 txt=txt, vec_txt=vec_txt, text_mask=text_mask, cache_mask=mask,
                                 cache_txt=True)
            return img
        for i, (block, cache) in enumerate(zip(self.blocks, self.caches)):
            img = block(img, vec, cos, sin, cache, self.cache_valid_len, update_cache,
                        kv_status=self.kv_status[i:i + 1] if update_cache else None)
        return img

    @torch.no_grad()
    def generate_chunk(self, noise, vecs_denoise, vec_write, sigmas, txt=None, vec_txt=None,
                       text_mask=None):
        """Euler flow updates over the denoising passes, then the cache write
        at t = 0 and the advance of the valid length (causal_ar.py:2348-2432,
        2624-2645,2852). A chunk that would not fit the cache is refused
        before any pass runs. In the write pass a layer whose K/V holds a
        NaN/Inf writes nothing; the valid length then stays where it was (rows
        that other layers wrote past it are never attended) and ValueError
        names the layers (with text: the first such layer raises)."""
        if self.cache_valid_len + self.write_tokens > self.capacity:
            raise ValueError(f"KV cache full: {self.cache_valid_len} + {self.write_tokens} tokens "
                             f"exceed the capacity {self.capacity}")
        if len(sigmas) != len(vecs_denoise) + 1:
            raise ValueError("sigmas must hold one more value than the denoising passes")
        x = noise
        for i, vec in enumerate(vecs_denoise):
            v_pred = self.forward_chunk(x, vec, False, txt, vec_txt, text_mask)
            x = x + (sigmas[i + 1] - sigmas[i]) * v_pred
        self.forward_chunk(x, vec_write, True, txt, vec_txt, text_mask)
        bad = torch.nonzero(self.kv_status).flatten().tolist()
        if bad:
            raise ValueError(f"Cannot quantize non-finite KV values (layers {bad})")
        self.cache_valid_len += self.write_tokens
        self.frames_done += self.latent_shape[0]
        return x
