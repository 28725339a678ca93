"""torch.library custom ops over the C ABI of libhynomas_fp8.so.

Each op is opaque to torch.compile (a fake implementation gives shapes only),
launches on the current stream of the input's device, and raises on CPU
tensors: the FP8 path has no CPU fallback. The custom-op + register_fake
pattern is the one the reference uses for its FP8 GEMM
(hymm/models/vae/pixelumm_decoder/cutlass_fp8.py:47-57).
"""
from __future__ import annotations

import math
from typing import Optional

import torch

from . import _lib as L

FP8 = torch.float8_e4m3fn


def _gpu(*tensors) -> None:
    for t in tensors:
        if t is not None and not t.is_cuda:
            raise RuntimeError("hy-nomas_amd FP8 kernels need GPU tensors (there is no CPU path)")


def _stream(t: torch.Tensor) -> int:
    return torch.cuda.current_stream(t.device).cuda_stream


def _bytes(t: torch.Tensor) -> torch.Tensor:
    return t.view(torch.uint8) if t.dtype in (FP8, torch.int8) else t


# --------------------------------------------------------------------------
# quantizers

@torch.library.custom_op("hy_nomas_amd::quantize_rows_fp8", mutates_args=())
def quantize_rows_fp8(x: torch.Tensor, scale_mode: int = L.HN_SCALE_CLAMP,
                      amax_floor: float = 1e-4) -> tuple[torch.Tensor, torch.Tensor]:
    """Per-row e4m3 codes and fp32 scales of a bf16 [..., C] tensor."""
    _gpu(x)
    if x.dtype != torch.bfloat16:
        raise TypeError("quantize_rows_fp8 expects bf16 input")
    x2 = x.reshape(-1, x.shape[-1])
    if x2.stride(-1) != 1:
        x2 = x2.contiguous()
    q = torch.empty(x2.shape, dtype=FP8, device=x.device)
    s = torch.empty((x2.shape[0],), dtype=torch.float32, device=x.device)
    with torch.cuda.device(x.device):
        L.check(L.load().hn_quantize_rows_fp8(
            x2.data_ptr(), x2.shape[0], x2.shape[1], x2.stride(0), scale_mode, amax_floor,
            q.data_ptr(), s.data_ptr(), _stream(x)), "hn_quantize_rows_fp8")
    return q.view(x.shape), s.view(x.shape[:-1])


@quantize_rows_fp8.register_fake
def _(x, scale_mode=L.HN_SCALE_CLAMP, amax_floor=1e-4):
    return x.new_empty(x.shape, dtype=FP8), x.new_empty(x.shape[:-1], dtype=torch.float32)


@torch.library.custom_op("hy_nomas_amd::ln_modulate_quantize_fp8", mutates_args=())
def ln_modulate_quantize_fp8(x: torch.Tensor, shift: torch.Tensor, scale: torch.Tensor,
                             eps: float = 1e-6,
                             amax_floor: float = 1e-4) -> tuple[torch.Tensor, torch.Tensor]:
    """LayerNorm (no affine) + adaLN modulate + per-token e4m3 quantization of a
    bf16 [B, L, C] tensor in one pass: the codes and scales of
    quantize_rows_fp8(modulate(layer_norm(x), shift, scale)) with shift and
    scale bf16 [B, C] (nomas_compile_prepost.py:14-15,40-43,81-84). Returns
    codes [B*L, C] and fp32 scales [B*L]."""
    _gpu(x, shift, scale)
    if x.dtype != torch.bfloat16 or shift.dtype != torch.bfloat16 or scale.dtype != torch.bfloat16:
        raise TypeError("ln_modulate_quantize_fp8 expects bf16 tensors")
    if x.ndim != 3 or shift.shape != (x.shape[0], x.shape[2]) or scale.shape != shift.shape:
        raise ValueError("ln_modulate_quantize_fp8: x [B, L, C] with shift and scale [B, C]")
    x = x.contiguous()
    shift = shift.contiguous()
    scale = scale.contiguous()
    B, Lt, C = x.shape
    q = torch.empty((B * Lt, C), dtype=FP8, device=x.device)
    s = torch.empty((B * Lt,), dtype=torch.float32, device=x.device)
    with torch.cuda.device(x.device):
        L.check(L.load().hn_ln_mod_quantize_fp8(
            x.data_ptr(), B * Lt, C, max(Lt, 1), shift.data_ptr(), scale.data_ptr(), C, eps,
            amax_floor, q.data_ptr(), s.data_ptr(), _stream(x)), "hn_ln_mod_quantize_fp8")
    return q, s


@ln_modulate_quantize_fp8.register_fake
def _(x, shift, scale, eps=1e-6, amax_floor=1e-4):
    n = x.shape[0] * x.shape[1]
    return x.new_empty((n, x.shape[2]), dtype=FP8), x.new_empty((n,), dtype=torch.float32)


@torch.library.custom_op("hy_nomas_amd::quantize_blockwise_fp8", mutates_args=())
def quantize_blockwise_fp8(x: torch.Tensor) -> tuple[torch.Tensor, torch.Tensor]:
    """128x128 blockwise e4m3 codes [M,K] and scales [ceil(M/128), K/128]."""
    _gpu(x)
    if x.dtype != torch.bfloat16 or x.ndim != 2:
        raise TypeError("quantize_blockwise_fp8 expects a bf16 [M, K] matrix")
    x = x.contiguous()
    m, k = x.shape
    q = torch.empty((m, k), dtype=FP8, device=x.device)
    s = torch.empty(((m + 127) // 128, k // 128), dtype=torch.float32, device=x.device)
    with torch.cuda.device(x.device):
        L.check(L.load().hn_quantize_blockwise_fp8(x.data_ptr(), m, k, q.data_ptr(), s.data_ptr(),
                                                   _stream(x)), "hn_quantize_blockwise_fp8")
    return q, s


@quantize_blockwise_fp8.register_fake
def _(x):
    m, k = x.shape
    return (x.new_empty((m, k), dtype=FP8),
            x.new_empty(((m + 127) // 128, k // 128), dtype=torch.float32))


# --------------------------------------------------------------------------
# GEMMs

@torch.library.custom_op("hy_nomas_amd::gemm_fp8_rowcol", mutates_args=())
def gemm_fp8_rowcol(a: torch.Tensor, b: torch.Tensor, sa: torch.Tensor, sb: torch.Tensor,
                    bias: Optional[torch.Tensor] = None, act: int = L.HN_ACT_NONE) -> torch.Tensor:
    """act(a b^T * sa[m] * sb[n] + bias[n]) in bf16; a e4m3 [M,K], b e4m3 [N,K]."""
    _gpu(a, b, sa, sb, bias)
    if a.dtype != FP8 or b.dtype != FP8:
        raise TypeError("gemm_fp8_rowcol expects e4m3 operands")
    if sa.dtype != torch.float32 or sb.dtype != torch.float32:
        raise TypeError("gemm_fp8_rowcol expects fp32 scales")
    if bias is not None and bias.dtype != torch.bfloat16:
        raise TypeError("gemm_fp8_rowcol expects a bf16 bias")
    a = a.contiguous()
    b = b.contiguous()
    m, k = a.shape
    n = b.shape[0]
    if b.shape[1] != k or sa.numel() != m or sb.numel() != n or (bias is not None and bias.numel() != n):
        raise ValueError("gemm_fp8_rowcol shape mismatch")
    out = torch.empty((m, n), dtype=torch.bfloat16, device=a.device)
    with torch.cuda.device(a.device):
        L.check(L.load().hn_gemm_fp8_rowcol(
            a.data_ptr(), b.data_ptr(), sa.contiguous().data_ptr(), sb.contiguous().data_ptr(),
            None if bias is None else bias.contiguous().data_ptr(), out.data_ptr(),
            m, n, k, n, act, _stream(a)), "hn_gemm_fp8_rowcol")
    return out


@gemm_fp8_rowcol.register_fake
def _(a, b, sa, sb, bias=None, act=L.HN_ACT_NONE):
    return a.new_empty((a.shape[0], b.shape[0]), dtype=torch.bfloat16)


@torch.library.custom_op("hy_nomas_amd::gemm_fp8_blockwise", mutates_args=())
def gemm_fp8_blockwise(a: torch.Tensor, b: torch.Tensor, sa: torch.Tensor,
                       sb: torch.Tensor) -> torch.Tensor:
    """The reference extension's gemm(a, b, sa, sb) with 128x128 block scales."""
    _gpu(a, b, sa, sb)
    for t in (a, b, sa, sb):
        if not t.is_contiguous():
            raise RuntimeError("Expected contiguous tensors on one device")
    if a.dtype != FP8 or b.dtype != FP8:
        raise RuntimeError("Expected E4M3 FP8 inputs")
    if sa.dtype != torch.float32 or sb.dtype != torch.float32:
        raise RuntimeError("Expected FP32 scales")
    if a.dim() != 2 or b.dim() != 2:
        raise RuntimeError("Expected matrices")
    m, k = a.shape
    n = b.shape[0]
    if not (m > 0 and n > 0 and k > 0 and b.shape[1] == k and n % 128 == 0 and k % 128 == 0):
        raise RuntimeError("Invalid GEMM shape")
    if sa.dim() != 2 or tuple(sa.shape) != ((m + 127) // 128, k // 128):
        raise RuntimeError("Invalid activation scales")
    if sb.dim() != 2 or tuple(sb.shape) != (n // 128, k // 128):
        raise RuntimeError("Invalid weight scales")
    out = torch.empty((m, n), dtype=torch.bfloat16, device=a.device)
    with torch.cuda.device(a.device):
        L.check(L.load().hn_gemm_fp8_blockwise(a.data_ptr(), b.data_ptr(), sa.data_ptr(),
                                               sb.data_ptr(), out.data_ptr(), m, n, k,
                                               _stream(a)), "hn_gemm_fp8_blockwise")
    return out


@gemm_fp8_blockwise.register_fake
def _(a, b, sa, sb):
    return a.new_empty((a.shape[0], b.shape[0]), dtype=torch.bfloat16)


@torch.library.custom_op("hy_nomas_amd::linear_fp8", mutates_args=())
def linear_fp8(x: torch.Tensor, weight: torch.Tensor, weight_scale: torch.Tensor,
               bias: Optional[torch.Tensor] = None, act: int = L.HN_ACT_NONE) -> torch.Tensor:
    """Per-token dynamic e4m3 activation quant + per-channel-scaled FP8 GEMM.
    x bf16 [M, K] -> bf16 [M, N]."""
    qx, sx = quantize_rows_fp8(x, L.HN_SCALE_CLAMP, 1e-4)
    return gemm_fp8_rowcol(qx, weight, sx, weight_scale, bias, act)


@linear_fp8.register_fake
def _(x, weight, weight_scale, bias=None, act=L.HN_ACT_NONE):
    return x.new_empty((x.shape[0], weight.shape[0]), dtype=torch.bfloat16)


# --------------------------------------------------------------------------
# KV cache

def _kv_fmt(codes: torch.Tensor) -> int:
    if codes.dtype == FP8:
        return L.HN_KV_FP8
    if codes.dtype == torch.int8:
        return L.HN_KV_INT8
    raise TypeError("KV codes must be float8_e4m3fn or int8")


def _check_cache_write(codes: torch.Tensor, scale: torch.Tensor, values: torch.Tensor, start: int,
                       what: str) -> int:
    """Geometry of a KV write, checked on the host before any launch: codes
    [B, cap, H, D], fp32 scales [B, cap, H, 1], values [B, L, H, D] and
    0 <= start, start + L <= cap (int8_kv_cache.py:128-135). Returns cap."""
    if codes.ndim != 4 or values.ndim != 4:
        raise ValueError(f"{what}: cache and values must be [B, L, H, D]")
    B, cap, H, D = codes.shape
    if scale.dtype != torch.float32 or tuple(scale.shape) != (B, cap, H, 1):
        raise ValueError(f"{what}: scale must be fp32 [B, cap, H, 1] matching the codes")
    if values.shape[0] != B or values.shape[2] != H or values.shape[3] != D:
        raise ValueError(f"{what}: values [B, L, H, D] do not match the cache's B, H, D")
    if start < 0 or start + values.shape[1] > cap:
        raise ValueError(f"{what}: tokens [{start}, {start + values.shape[1]}) exceed the cache capacity {cap}")
    return cap


def _status_ptr(status: Optional[torch.Tensor]):
    """Device pointer of a KV-write status word (int32, one element), or None."""
    if status is None:
        return None
    if status.dtype != torch.int32 or status.numel() < 1:
        raise TypeError("status must be an int32 tensor of at least one element")
    return status.data_ptr()


# The three cache writers below mutate an optional status word; torch's
# custom-op wrapper finds mutated arguments by position, so each op is
# registered with every argument required and called through a wrapper that
# passes them all.

def kv_quantize_pair_(k_codes, v_codes, k_scale, v_scale, k, v, start: int, status=None) -> None:
    """Quantize bf16 K/V [B,L,H,D] into the caches at token offset ``start``
    (see _kv_quantize_pair_op)."""
    _kv_quantize_pair_op(k_codes, v_codes, k_scale, v_scale, k, v, start, status)


def kv_quantize_(codes, scale, x, start: int, status=None) -> None:
    """Quantize bf16 values [B,L,H,D] into one cache tensor (see _kv_quantize_op)."""
    _kv_quantize_op(codes, scale, x, start, status)


@torch.library.custom_op("hy_nomas_amd::kv_quantize_pair_",
                         mutates_args=("k_codes", "v_codes", "k_scale", "v_scale", "status"))
def _kv_quantize_pair_op(k_codes: torch.Tensor, v_codes: torch.Tensor, k_scale: torch.Tensor,
                         v_scale: torch.Tensor, k: torch.Tensor, v: torch.Tensor,
                         start: int, status: Optional[torch.Tensor]) -> None:
    """Quantize bf16 K/V [B,L,H,D] into the caches at token offset ``start``.

    With ``status`` (int32 on the device), K and V are validated on the device
    first: status[0] becomes 1 and nothing is written if any value is NaN/Inf,
    else 0. No host synchronisation. None: the caller guarantees finite values."""
    fmt = _kv_fmt(k_codes)
    if v_codes.dtype != k_codes.dtype or k.stride() != v.stride() or k.shape != v.shape:
        raise ValueError("K/V caches and values must share dtype and layout")
    if (k_codes.stride() != v_codes.stride() or k_scale.stride() != v_scale.stride()
            or k_codes.shape != v_codes.shape or k_scale.shape != v_scale.shape):
        raise ValueError("K/V caches must share layout")
    cap = _check_cache_write(k_codes, k_scale, k, start, "kv_quantize_pair_")
    sp = _status_ptr(status)
    _gpu(k_codes, v_codes, k_scale, v_scale, k, v, status)
    B, Lt, H, D = k.shape
    with torch.cuda.device(k.device):
        L.check(L.load().hn_kv_quantize_pair(
            fmt, k.data_ptr(), v.data_ptr(), L.strides(k), B, Lt, H, D,
            k_codes.data_ptr(), v_codes.data_ptr(), L.strides(k_codes),
            k_scale.data_ptr(), v_scale.data_ptr(), L.strides(k_scale), cap, start, sp, _stream(k)),
            "hn_kv_quantize_pair")


@_kv_quantize_pair_op.register_fake
def _(k_codes, v_codes, k_scale, v_scale, k, v, start, status):
    return None


@torch.library.custom_op("hy_nomas_amd::kv_quantize_", mutates_args=("codes", "scale", "status"))
def _kv_quantize_op(codes: torch.Tensor, scale: torch.Tensor, x: torch.Tensor, start: int,
                    status: Optional[torch.Tensor]) -> None:
    """Quantize bf16 values [B,L,H,D] into one cache tensor at ``start``
    (``status`` as in _kv_quantize_pair_op)."""
    fmt = _kv_fmt(codes)
    cap = _check_cache_write(codes, scale, x, start, "kv_quantize_")
    sp = _status_ptr(status)
    _gpu(codes, scale, x, status)
    B, Lt, H, D = x.shape
    with torch.cuda.device(x.device):
        L.check(L.load().hn_kv_quantize(
            fmt, x.data_ptr(), L.strides(x), B, Lt, H, D, codes.data_ptr(), L.strides(codes),
            scale.data_ptr(), L.strides(scale), cap, start, sp, _stream(x)), "hn_kv_quantize")


@_kv_quantize_op.register_fake
def _(codes, scale, x, start, status):
    return None


@torch.library.custom_op("hy_nomas_amd::kv_dequantize", mutates_args=())
def kv_dequantize(codes: torch.Tensor, scale: torch.Tensor, valid_len: int) -> torch.Tensor:
    """bf16(code * scale) for tokens [0, valid_len): a new [B, valid_len, H, D] tensor."""
    _gpu(codes, scale)
    fmt = _kv_fmt(codes)
    B, _, H, D = codes.shape
    y = torch.empty((B, valid_len, H, D), dtype=torch.bfloat16, device=codes.device)
    if valid_len == 0:
        return y
    with torch.cuda.device(codes.device):
        L.check(L.load().hn_kv_dequantize(
            fmt, codes.data_ptr(), L.strides(codes), scale.data_ptr(), L.strides(scale),
            B, valid_len, H, D, y.data_ptr(), L.strides(y), _stream(codes)), "hn_kv_dequantize")
    return y


@kv_dequantize.register_fake
def _(codes, scale, valid_len):
    B, _, H, D = codes.shape
    return codes.new_empty((B, valid_len, H, D), dtype=torch.bfloat16)


# --------------------------------------------------------------------------
# fused QK RMSNorm + RoPE (+ KV cache write)

def _qk_launch(q, k, v, q_weight, k_weight, cos, sin, eps, cache, start, status=None):
    if not (q.dtype == k.dtype == v.dtype == torch.bfloat16):
        raise TypeError("qk_norm_rope expects bf16 q, k, v")
    if q.stride() != k.stride() or q.stride() != v.stride() or q.shape != k.shape or q.shape != v.shape:
        raise ValueError("q, k and v must share shape and strides")
    B, Lt, H, D = q.shape
    cos = cos.reshape(-1, D)
    sin = sin.reshape(-1, D)
    if cos.dtype != torch.float32 or sin.dtype != torch.float32 or cos.shape[0] < Lt or cos.stride() != sin.stride():
        raise ValueError("cos/sin must be fp32 [L, D] tables with one layout")
    qw = q_weight.to(torch.bfloat16).contiguous()
    kw = k_weight.to(torch.bfloat16).contiguous()
    if cache:
        k_codes, v_codes, k_scale, v_scale = cache
        fmt = _kv_fmt(k_codes)
        if (v_codes.dtype != k_codes.dtype or k_codes.stride() != v_codes.stride()
                or k_scale.stride() != v_scale.stride() or k_codes.shape != v_codes.shape
                or k_scale.shape != v_scale.shape):
            raise ValueError("K/V caches must share dtype and layout")
        cap = _check_cache_write(k_codes, k_scale, k, start, "qk_norm_rope_kv_")
        cargs = (k_codes.data_ptr(), v_codes.data_ptr(), L.strides(k_codes), k_scale.data_ptr(),
                 v_scale.data_ptr(), L.strides(k_scale), cap, start, _status_ptr(status))
    else:
        fmt = L.HN_KV_FP8
        cargs = (None, None, None, None, None, None, 0, start, None)
    _gpu(q, k, v, q_weight, k_weight, cos, sin, status, *(cache or ()))
    with torch.cuda.device(q.device):
        L.check(L.load().hn_qk_norm_rope_kv(
            fmt, q.data_ptr(), k.data_ptr(), v.data_ptr(), L.strides(q), B, Lt, H, D,
            qw.data_ptr(), kw.data_ptr(), cos.data_ptr(), sin.data_ptr(), cos.stride(0), eps,
            *cargs, _stream(q)), "hn_qk_norm_rope_kv")


@torch.library.custom_op("hy_nomas_amd::qk_norm_rope_", mutates_args=("q", "k"))
def qk_norm_rope_(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor, q_weight: torch.Tensor,
                  k_weight: torch.Tensor, cos: torch.Tensor, sin: torch.Tensor, eps: float) -> None:
    """In place: q, k <- RoPE(RMSNorm(q)), RoPE(RMSNorm(k)) for bf16 [B, L, H, 128]
    views sharing strides (v is only checked for layout)."""
    _qk_launch(q, k, v, q_weight, k_weight, cos, sin, eps, None, 0)


@qk_norm_rope_.register_fake
def _(q, k, v, q_weight, k_weight, cos, sin, eps):
    return None


def qk_norm_rope_kv_(q, k, v, q_weight, k_weight, cos, sin, eps: float, k_codes, v_codes, k_scale,
                     v_scale, start: int, status=None) -> None:
    """qk_norm_rope_, and the rotated k and v written into the KV caches at
    token offset ``start`` by the same kernel. With ``status`` (int32 on the
    device) the values to be written are validated on the device first:
    status[0] becomes 1 and the cache is left untouched if any is NaN/Inf."""
    _qk_norm_rope_kv_op(q, k, v, q_weight, k_weight, cos, sin, eps, k_codes, v_codes, k_scale, v_scale,
                        start, status)


@torch.library.custom_op("hy_nomas_amd::qk_norm_rope_kv_",
                         mutates_args=("q", "k", "k_codes", "v_codes", "k_scale", "v_scale", "status"))
def _qk_norm_rope_kv_op(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor, q_weight: torch.Tensor,
                        k_weight: torch.Tensor, cos: torch.Tensor, sin: torch.Tensor, eps: float,
                        k_codes: torch.Tensor, v_codes: torch.Tensor, k_scale: torch.Tensor,
                        v_scale: torch.Tensor, start: int, status: Optional[torch.Tensor]) -> None:
    _qk_launch(q, k, v, q_weight, k_weight, cos, sin, eps, (k_codes, v_codes, k_scale, v_scale), start,
               status)


@_qk_norm_rope_kv_op.register_fake
def _(q, k, v, q_weight, k_weight, cos, sin, eps, k_codes, v_codes, k_scale, v_scale, start, status):
    return None


# --------------------------------------------------------------------------
# attention

def _valid_bytes(mask: Optional[torch.Tensor], rows: int, cols: int, what: str):
    """A key-validity mask as (uint8 view, batch stride): bool or uint8 [rows or
    1, >= cols] with contiguous tokens; a batch of 1 is read by every row."""
    if mask is None:
        return None, 0
    if mask.dtype not in (torch.bool, torch.uint8) or mask.ndim != 2:
        raise TypeError(f"attn_fp8kv: {what} must be a bool [B, L] mask")
    if mask.shape[0] not in (rows, 1) or mask.shape[1] < cols:
        raise ValueError(f"attn_fp8kv: {what} must cover [{rows}, {cols}]")
    if cols and mask.stride(1) != 1:
        mask = mask.contiguous()
    stride = 0 if mask.shape[0] == 1 else mask.stride(0)
    return mask.view(torch.uint8), stride


@torch.library.custom_op("hy_nomas_amd::attn_fp8kv", mutates_args=())
def attn_fp8kv(q: torch.Tensor, k_codes: torch.Tensor, v_codes: torch.Tensor,
               k_scale: torch.Tensor, v_scale: torch.Tensor, kv_len: int,
               k_cur: Optional[torch.Tensor] = None, v_cur: Optional[torch.Tensor] = None,
               q_pos0: int = 0, chunk_len: int = 0,
               softmax_scale: Optional[float] = None,
               cache_valid: Optional[torch.Tensor] = None,
               cur_valid: Optional[torch.Tensor] = None) -> torch.Tensor:
    """Chunk attention of q [B,Lq,H,D] over cache tokens [0, kv_len) then the
    optional bf16 tail k_cur/v_cur [B,Lc,H,D]; see hn_attn_fp8kv for the mask.

    The cache may hold B slots or one slot that every query batch reads (the
    read-only CFG broadcast). cache_valid (bool [B or 1, >= kv_len]) and
    cur_valid (bool [B, >= Lc]) exclude invalid keys."""
    if q.dtype != torch.bfloat16:
        raise TypeError("attn_fp8kv expects bf16 queries")
    fmt = _kv_fmt(k_codes)
    if q.ndim != 4:
        raise ValueError("attn_fp8kv: q must be [B, Lq, H, D]")
    B, Lq, H, D = q.shape
    if k_codes.ndim != 4 or k_codes.shape[2:] != (H, D) or k_codes.shape[0] not in (B, 1):
        raise ValueError("attn_fp8kv: cache [B or 1, cap, H, D] does not match q")
    if (v_codes.dtype != k_codes.dtype or v_codes.shape != k_codes.shape
            or v_codes.stride() != k_codes.stride()):
        raise ValueError("attn_fp8kv: K and V codes must share dtype, shape and strides")
    cap = k_codes.shape[1]
    if (k_scale.dtype != torch.float32 or v_scale.dtype != torch.float32
            or tuple(k_scale.shape) != (*k_codes.shape[:3], 1) or v_scale.shape != k_scale.shape
            or v_scale.stride() != k_scale.stride()):
        raise ValueError("attn_fp8kv: K and V scales must be fp32 [B, cap, H, 1] with one layout")
    if not 0 <= kv_len <= cap:
        raise ValueError(f"attn_fp8kv: kv_len {kv_len} outside the cache capacity {cap}")
    if softmax_scale is None:
        softmax_scale = D ** -0.5
    if not (softmax_scale > 0 and math.isfinite(softmax_scale)):
        raise ValueError("attn_fp8kv: softmax_scale must be finite and positive")
    if k_codes.shape[0] != B:  # one history slot read by every query batch
        k_codes, v_codes = k_codes.expand(B, -1, -1, -1), v_codes.expand(B, -1, -1, -1)
        k_scale, v_scale = k_scale.expand(B, -1, -1, -1), v_scale.expand(B, -1, -1, -1)
    cur_len = 0 if k_cur is None else k_cur.shape[1]
    if k_cur is not None and (k_cur.ndim != 4 or k_cur.shape[0] != B or k_cur.shape[2:] != (H, D)):
        raise ValueError("attn_fp8kv: k_cur must be [B, Lc, H, D] matching q")
    if cur_len and (v_cur is None or v_cur.shape != k_cur.shape or k_cur.stride() != v_cur.stride()
                    or k_cur.dtype != torch.bfloat16 or v_cur.dtype != torch.bfloat16):
        raise ValueError("k_cur/v_cur must be matching bf16 tensors")
    kvb, kvs = _valid_bytes(cache_valid if kv_len else None, B, kv_len, "cache_valid")
    uvb, uvs = _valid_bytes(cur_valid if cur_len else None, B, cur_len, "cur_valid")
    _gpu(q, k_codes, v_codes, k_scale, v_scale, k_cur, v_cur, kvb, uvb)
    out = torch.empty((B, Lq, H, D), dtype=torch.bfloat16, device=q.device)
    with torch.cuda.device(q.device):
        lib = L.load()
        ws_bytes = lib.hn_attn_fp8kv_workspace_size(B, Lq, H, D, kv_len, cur_len)
        ws = torch.empty((ws_bytes,), dtype=torch.uint8, device=q.device) if ws_bytes else None
        L.check(lib.hn_attn_fp8kv(
            fmt, q.data_ptr(), L.strides(q), B, Lq, H, D,
            k_codes.data_ptr(), v_codes.data_ptr(), L.strides(k_codes),
            k_scale.data_ptr(), v_scale.data_ptr(), L.strides(k_scale), cap, kv_len,
            L.ptr(kvb), kvs,
            None if not cur_len else k_cur.data_ptr(), None if not cur_len else v_cur.data_ptr(),
            L.strides(k_cur) if cur_len else None, cur_len, L.ptr(uvb), uvs, q_pos0, chunk_len,
            float(softmax_scale), out.data_ptr(), L.strides(out),
            None if ws is None else ws.data_ptr(), ws_bytes, _stream(q)), "hn_attn_fp8kv")
    return out


@attn_fp8kv.register_fake
def _(q, k_codes, v_codes, k_scale, v_scale, kv_len, k_cur=None, v_cur=None, q_pos0=0,
      chunk_len=0, softmax_scale=None, cache_valid=None, cur_valid=None):
    return torch.empty_like(q)
