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
GEMM epilogue, fc2; gated residual. The AR step follows
hymm/pipeline/causal_ar.py:2348-2432,2624-2645,2852: N denoising passes
without cache writes, one cache-write pass, then the valid length advances.
"""
from __future__ import annotations

import math

import torch
import torch.nn as nn
import torch.nn.functional as F

from . import ops
from .cache_attention import chunk_attention
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
    """Image stream of one double-stream block at inference, FP8 linears."""

    def __init__(self, hidden: int = 3072, heads: int = 24, mlp_ratio: int = 4,
                 qk_eps: float = 1e-6, *, device=None, generator=None,
                 validate_kv_writes: bool = True, fuse_ln_quant: bool = True):
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

    def _fused(self, linear) -> bool:
        return self.fuse_ln_quant and isinstance(linear, FP8StoredLinear)

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
        B, L, C = img.shape
        H, D = self.heads, self.head_dim
        with stage("modulation"):
            parts = F.linear(F.silu(vec), self.mod.weight, self.mod.bias).chunk(6, dim=-1)
            if self._fused(self.qkv):
                qx, sx = ops.ln_modulate_quantize_fp8(img, parts[0], parts[1], 1e-6)
            else:
                x = _modulate(F.layer_norm(img, (C,), eps=1e-6), parts[0], parts[1])
        with stage("qkv_fp8"):
            if self._fused(self.qkv):
                qkv = fp8_linear_codes(self.qkv, qx, sx).view(B, L, 3, H, D)
            else:
                qkv = fp8_linear(self.qkv, x).view(B, L, 3, H, D)
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

    def post_attention(self, img, attn, parts):
        """Image-stream half of nomas_compile_prepost.post_attention (:75-99):
        out-projection and gated residual, LayerNorm + modulate, FFN with
        GELU-tanh fused into fc1's epilogue, gated residual."""
        B, L, C = img.shape
        with stage("post_fp8"):
            img = img + fp8_linear(self.proj, attn.reshape(B, L, C)) * parts[2].unsqueeze(1)
            if self._fused(self.fc1):
                qh, sh = ops.ln_modulate_quantize_fp8(img, parts[3], parts[4], 1e-6)
                h = fp8_linear_codes(self.fc1, qh, sh, gelu=True).view(B, L, -1)
            else:
                h = _modulate(F.layer_norm(img, (C,), eps=1e-6), parts[3], parts[4])
                h = fp8_linear(self.fc1, h, gelu=True)
            h = fp8_linear(self.fc2, h)
            img = img + h * parts[5].unsqueeze(1)
        return img

    def forward(self, img, vec, cos, sin, kv_cache, cache_valid_len: int,
                update_cache: bool = False, kv_status=None):
        """One block at inference. With ``update_cache`` this chunk's rotated K
        and V go into ``kv_cache`` at ``cache_valid_len``. When writes are
        validated and no ``kv_status`` is passed, a non-finite value raises
        ValueError here (one host read of the device flag); with one, the flag
        is left for the caller to read."""
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
    at t = 0 that writes this chunk's K/V, then the valid length advances."""

    def __init__(self, depth: int = 40, hidden: int = 3072, heads: int = 24,
                 latent_shape=(3, 45, 80), max_chunks: int = 17, *, device=None, seed: int = 0):
        super().__init__()
        g = torch.Generator(device=device).manual_seed(seed)
        self.blocks = nn.ModuleList(
            FP8DiTBlock(hidden, heads, device=device, generator=g) for _ in range(depth))
        self.latent_shape = tuple(latent_shape)
        self.tokens_per_chunk = math.prod(latent_shape)
        self.capacity = max_chunks * self.tokens_per_chunk
        self.heads, self.head_dim = heads, hidden // heads
        self.device = device
        self.caches = [make_fp8_kv_block(1, self.capacity, heads, self.head_dim, device=device)
                       for _ in range(depth)]
        # one device status word per layer for the validated cache writes
        self.kv_status = torch.zeros(depth, dtype=torch.int32, device=device)
        self.cache_valid_len = 0
        self.frames_done = 0

    @torch.no_grad()
    def forward_chunk(self, img, vec, update_cache: bool):
        t, h, w = self.latent_shape
        cos, sin = rope_tables(t, h, w, t_offset=self.frames_done, device=img.device)
        for i, (block, cache) in enumerate(zip(self.blocks, self.caches)):
            img = block(img, vec, cos, sin, cache, self.cache_valid_len, update_cache,
                        kv_status=self.kv_status[i:i + 1] if update_cache else None)
        return img

    @torch.no_grad()
    def generate_chunk(self, noise, vecs_denoise, vec_write, sigmas):
        """Euler flow updates over the denoising passes, then the cache write
        at t = 0 and the advance of the valid length (causal_ar.py:2348-2432,
        2624-2645,2852). A chunk that would not fit the cache is refused
        before any pass runs. In the write pass a layer whose K/V holds a
        NaN/Inf writes nothing; the valid length then stays where it was (rows
        that other layers wrote past it are never attended) and ValueError
        names the layers."""
        if self.cache_valid_len + self.tokens_per_chunk > self.capacity:
            raise ValueError(f"KV cache full: {self.cache_valid_len} + {self.tokens_per_chunk} tokens "
                             f"exceed the capacity {self.capacity}")
        if len(sigmas) != len(vecs_denoise) + 1:
            raise ValueError("sigmas must hold one more value than the denoising passes")
        x = noise
        for i, vec in enumerate(vecs_denoise):
            v_pred = self.forward_chunk(x, vec, update_cache=False)
            x = x + (sigmas[i + 1] - sigmas[i]) * v_pred
        self.forward_chunk(x, vec_write, update_cache=True)
        bad = torch.nonzero(self.kv_status).flatten().tolist()
        if bad:
            raise ValueError(f"Cannot quantize non-finite KV values (layers {bad})")
        self.cache_valid_len += self.tokens_per_chunk
        self.frames_done += self.latent_shape[0]
        return x
