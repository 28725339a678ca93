"""CPU oracle for the FP8 quantized inference path -- TEST INFRASTRUCTURE ONLY.

Only ``tests/``, ``__graft_entry__.smoke()`` and ``bench.py``'s ``cpu_baseline``
leg may import this module, and only as the checker. The product library never
imports, links or calls anything under ``oracle/``.

Byte/integer work (the e4m3 codec and every quantizer) is the C restatement in
``fp8_oracle.c`` (built by ``oracle/Makefile`` into ``liboracle.so``). The
floating-point references (dequantize-then-matmul, block-causal attention) are
numpy in float64.

Reference recipes followed (file:line in the upstream repository):
  * per-token / per-channel FP8 quant  hymm/models/vae/pixelumm_decoder/cutlass_fp8.py:35-41
    (same recipe, 1 x K blocks instead of 128 x 128)
  * blockwise 128x128 FP8 quant        hymm/models/vae/pixelumm_decoder/cutlass_fp8.py:35-41
  * KV quantize-on-write               hymm/models/dit/modules/int8_kv_cache.py:125-158
    (FP8: 448 and an e4m3 RNE cast in place of 127 and round-half-away)
  * KV decode                          hymm/models/dit/modules/int8_kv_cache.py:182-205
  * W8 weight quant (INT8-compat)      hymm/models/dit/modules/int8_stored_bf16_linear.py:46-61
  * dequantize-then-matmul             hymm/models/dit/modules/int8_stored_bf16_linear.py:82-94
  * LayerNorm + adaLN modulate         hymm/models/dit/modules/nomas_compile_prepost.py:14-15,40-43,81-84
  * blockwise GEMM contract            hymm/models/vae/pixelumm_decoder/csrc/cutlass_fp8.cu:20-57
  * cached attention semantics         hymm/models/dit/nomas_cpt.py:464-685,771-781 and
                                       hymm/models/dit/modules/attention/range_attention.py:212-239

Bit patterns: bf16 tensors travel as ``np.uint16`` arrays of their raw bits.
"""
from __future__ import annotations

import ctypes
import os
import subprocess
from pathlib import Path

import numpy as np

HERE = Path(__file__).resolve().parent
LIB_PATH = HERE / "liboracle.so"

SCALE_CLAMP = 0      # s = max(amax, floor) / 448          (cutlass_fp8.py:39)
SCALE_ZERO_ONE = 1   # s = amax > 0 ? amax / 448 : 1       (int8_kv_cache.py:44,152)
LINEAR_AMAX_FLOOR = np.float32(1e-4)

KV_FP8 = 0
KV_INT8 = 1

_lib = None


def build() -> Path:
    """Compile liboracle.so with the committed Makefile (gcc only)."""
    subprocess.run(["make", "-s", "-C", str(HERE), "liboracle.so"], check=True)
    return LIB_PATH


def lib():
    global _lib
    if _lib is None:
        if not LIB_PATH.exists():
            build()
        L = ctypes.CDLL(str(LIB_PATH))
        P = ctypes.c_void_p
        I64 = ctypes.c_int64
        L.hn_oracle_e4m3_encode.restype = ctypes.c_uint8
        L.hn_oracle_e4m3_encode.argtypes = [ctypes.c_float]
        L.hn_oracle_e4m3_decode.restype = ctypes.c_float
        L.hn_oracle_e4m3_decode.argtypes = [ctypes.c_uint8]
        L.hn_oracle_e4m3_encode_f32.argtypes = [P, I64, P]
        L.hn_oracle_e4m3_decode_n.argtypes = [P, I64, P]
        L.hn_oracle_e4m3_range_mismatches.restype = I64
        L.hn_oracle_e4m3_range_mismatches.argtypes = [ctypes.c_uint32, I64, P, P]
        L.hn_oracle_quantize_rows_fp8.argtypes = [P, I64, I64, I64, ctypes.c_int,
                                                  ctypes.c_float, P, P]
        L.hn_oracle_quantize_blockwise_fp8.argtypes = [P, I64, I64, P, P]
        L.hn_oracle_kv_quantize.argtypes = [P, I64, I64, I64, I64, P, P, P, P, P,
                                            I64, ctypes.c_int]
        L.hn_oracle_quantize_weight_int8.argtypes = [P, I64, I64, P, P]
        _lib = L
    return _lib


def _ptr(a: np.ndarray):
    return a.ctypes.data_as(ctypes.c_void_p)


# --------------------------------------------------------------------------
# bf16 <-> f32 bit helpers (RNE), the conversion torch's .to(bfloat16) performs.

def bf16_bits_to_f32(u16: np.ndarray) -> np.ndarray:
    return (np.asarray(u16, dtype=np.uint16).astype(np.uint32) << 16).view(np.float32)


def f32_to_bf16_bits(f: np.ndarray) -> np.ndarray:
    u = np.ascontiguousarray(f, dtype=np.float32).view(np.uint32).astype(np.uint64)
    nan = np.isnan(np.asarray(f, dtype=np.float32))
    rounded = ((u + 0x7FFF + ((u >> 16) & 1)) >> 16).astype(np.uint16)
    return np.where(nan, np.uint16(0x7FC0), rounded).astype(np.uint16)


# --------------------------------------------------------------------------
# e4m3 codec

def e4m3_encode(x: np.ndarray) -> np.ndarray:
    x = np.ascontiguousarray(x, dtype=np.float32)
    out = np.empty(x.shape, dtype=np.uint8)
    lib().hn_oracle_e4m3_encode_f32(_ptr(x), x.size, _ptr(out))
    return out


def e4m3_range_mismatches(first: int, codes: np.ndarray):
    """(count, first index) of codes[i] != e4m3 encode of the fp32 bit pattern
    first + i (first index -1 when every code agrees)."""
    codes = np.ascontiguousarray(codes, dtype=np.uint8)
    where = ctypes.c_int64(-1)
    bad = lib().hn_oracle_e4m3_range_mismatches(first, codes.size, _ptr(codes), ctypes.byref(where))
    return int(bad), int(where.value)


def e4m3_decode(q: np.ndarray) -> np.ndarray:
    q = np.ascontiguousarray(q, dtype=np.uint8)
    out = np.empty(q.shape, dtype=np.float32)
    lib().hn_oracle_e4m3_decode_n(_ptr(q), q.size, _ptr(out))
    return out


def int8_decode(q: np.ndarray) -> np.ndarray:
    return np.asarray(q, dtype=np.uint8).view(np.int8).astype(np.float32)


# --------------------------------------------------------------------------
# quantizers

def quantize_rows_fp8(x_bits: np.ndarray, mode: int = SCALE_CLAMP,
                      floor: float = float(LINEAR_AMAX_FLOOR)):
    """Per-row (per-token / per-output-channel) FP8: returns (codes u8 [R,C], scale f32 [R])."""
    x_bits = np.ascontiguousarray(x_bits, dtype=np.uint16)
    rows, cols = x_bits.shape
    q = np.empty((rows, cols), dtype=np.uint8)
    s = np.empty((rows,), dtype=np.float32)
    lib().hn_oracle_quantize_rows_fp8(_ptr(x_bits), rows, cols, cols, mode,
                                      ctypes.c_float(floor), _ptr(q), _ptr(s))
    return q, s


def ln_modulate_bf16(x_bits: np.ndarray, shift_bits: np.ndarray, scale_bits: np.ndarray,
                     eps: float = 1e-6, rows_per_batch: int | None = None) -> np.ndarray:
    """LayerNorm (no affine) + adaLN modulate of bf16 rows, as bf16 bits:
    y = bf16(F.layer_norm(x, eps)), o = bf16(bf16(y * bf16(1 + scale)) + shift)
    (nomas_compile_prepost.py:14-15,40-43,81-84: bf16 tensor ops, each
    rounding once, round to nearest even). Row r uses shift / scale row
    r // rows_per_batch ([B, C]).

    The fp32 mean and variance restate the GPU kernel's fixed summation order
    (hn_ln_mod_quantize_fp8): lane l of 64 adds its values in storage order
    (8-value chunks l, l + 64, ...), then the lanes combine by xor butterfly;
    mean = sum * fp32(1 / C), var = sum((x - mean)^2) * fp32(1 / C), rstd =
    1 / sqrt(var + eps), every step one correctly rounded fp32 operation
    (numpy float32). Pinned against a float64 LayerNorm and torch's CPU
    F.layer_norm (at most one bf16 ulp apart, at rounding boundaries) in
    tests/test_oracle.py."""
    x_bits = np.ascontiguousarray(x_bits, dtype=np.uint16)
    rows, cols = x_bits.shape
    if cols % 8:
        raise ValueError("cols must be a multiple of 8")
    rpb = rows if rows_per_batch is None else int(rows_per_batch)
    x = bf16_bits_to_f32(x_bits)
    nch = cols // 8
    lanes = np.arange(64)

    def wave_sum(vals):  # vals float32 [rows, nch, 8] -> float32 [rows]
        part = np.zeros((rows, 64), dtype=np.float32)
        for c0 in range(0, nch, 64):
            cnt = min(64, nch - c0)
            for k in range(8):
                part[:, :cnt] = part[:, :cnt] + vals[:, c0:c0 + cnt, k]
        off = 32
        while off:
            part = part + part[:, lanes ^ off]
            off >>= 1
        return part[:, 0]

    inv_cols = np.float32(1.0) / np.float32(cols)
    xc = x.reshape(rows, nch, 8)
    # rows holding Inf or NaN give NaN (inf - inf), as the kernel's fp32 ops do
    with np.errstate(invalid="ignore", over="ignore"):
        mean = (wave_sum(xc) * inv_cols).astype(np.float32)
        d = (xc - mean[:, None, None]).astype(np.float32)
        var = (wave_sum((d * d).astype(np.float32)) * inv_cols).astype(np.float32)
        rstd = (np.float32(1.0) / np.sqrt((var + np.float32(eps)).astype(np.float32))).astype(np.float32)
        y = bf16_bits_to_f32(f32_to_bf16_bits((d * rstd[:, None, None]).astype(np.float32).reshape(rows, cols)))
    b = np.arange(rows) // rpb
    sc = bf16_bits_to_f32(np.asarray(scale_bits, dtype=np.uint16))[b]
    sh = bf16_bits_to_f32(np.asarray(shift_bits, dtype=np.uint16))[b]
    a = bf16_bits_to_f32(f32_to_bf16_bits((np.float32(1.0) + sc).astype(np.float32)))
    m = bf16_bits_to_f32(f32_to_bf16_bits((y * a).astype(np.float32)))
    return f32_to_bf16_bits((m + sh).astype(np.float32))


def ln_modulate_quantize_fp8(x_bits, shift_bits, scale_bits, eps: float = 1e-6,
                             rows_per_batch: int | None = None):
    """ln_modulate_bf16 followed by the per-token FP8 quantizer (SCALE_CLAMP,
    floor 1e-4): the fused hn_ln_mod_quantize_fp8 (codes u8 [R, C], scale f32 [R])."""
    return quantize_rows_fp8(ln_modulate_bf16(x_bits, shift_bits, scale_bits, eps, rows_per_batch))


def quantize_blockwise_fp8(x_bits: np.ndarray):
    """128x128 blockwise FP8: returns (codes u8 [M,K], scale f32 [ceil(M/128), K/128])."""
    x_bits = np.ascontiguousarray(x_bits, dtype=np.uint16)
    m, k = x_bits.shape
    if k % 128:
        raise ValueError("K must be a multiple of 128")
    q = np.empty((m, k), dtype=np.uint8)
    s = np.empty(((m + 127) // 128, k // 128), dtype=np.float32)
    lib().hn_oracle_quantize_blockwise_fp8(_ptr(x_bits), m, k, _ptr(q), _ptr(s))
    return q, s


def kv_quantize_into(x_bits: np.ndarray, cache_q: np.ndarray, cache_s: np.ndarray,
                     start: int, fmt: int = KV_FP8) -> None:
    """Write values [B,L,H,D] into cache_q [B,cap,H,D] / cache_s [B,cap,H,1] at token ``start``."""
    if cache_q.dtype != np.uint8 or cache_s.dtype != np.float32:
        raise TypeError("cache_q must be uint8 and cache_s float32")
    B, L, H, D = x_bits.shape
    if start < 0 or start + L > cache_q.shape[1]:
        raise ValueError("capacity")
    x_bits = np.asarray(x_bits, dtype=np.uint16)
    xs = np.array([st // 2 for st in x_bits.strides], dtype=np.int64)
    qs = np.array([st for st in cache_q.strides], dtype=np.int64)
    ss = np.array([st // 4 for st in cache_s.strides[:3]], dtype=np.int64)
    lib().hn_oracle_kv_quantize(_ptr(x_bits), B, L, H, D, _ptr(xs), _ptr(cache_q),
                                _ptr(qs), _ptr(cache_s), _ptr(ss), start, fmt)


def kv_quantize(x_bits: np.ndarray, fmt: int = KV_FP8):
    """Convenience form: returns (codes u8 [B,L,H,D], scale f32 [B,L,H,1])."""
    B, L, H, D = x_bits.shape
    q = np.zeros((B, L, H, D), dtype=np.uint8)
    s = np.zeros((B, L, H, 1), dtype=np.float32)
    kv_quantize_into(x_bits, q, s, 0, fmt)
    return q, s


def kv_dequantize(q: np.ndarray, s: np.ndarray, fmt: int = KV_FP8) -> np.ndarray:
    """int8_kv_cache.py:203-204: y = bf16(q_f32 * s). Returns bf16 bits."""
    vals = e4m3_decode(q) if fmt == KV_FP8 else int8_decode(q)
    return f32_to_bf16_bits(vals * np.asarray(s, dtype=np.float32))


def quantize_weight_int8(w: np.ndarray):
    w = np.ascontiguousarray(w, dtype=np.float32)
    n, k = w.shape
    q = np.empty((n, k), dtype=np.int8)
    s = np.empty((n, (k + 127) // 128), dtype=np.float32)
    lib().hn_oracle_quantize_weight_int8(_ptr(w), n, k, _ptr(q), _ptr(s))
    return q, s


# --------------------------------------------------------------------------
# floating-point references (float64)

def gelu_tanh(x: np.ndarray) -> np.ndarray:
    """torch.nn.functional.gelu(approximate='tanh') in float64."""
    x = np.asarray(x, dtype=np.float64)
    return 0.5 * x * (1.0 + np.tanh(np.sqrt(2.0 / np.pi) * (x + 0.044715 * x ** 3)))


def linear_reference(qx, sx, qw, sw, bias=None, gelu=False) -> np.ndarray:
    """Dequantize-then-matmul (int8_stored_bf16_linear.py:82-94 structure, FP8 codes):
    Y = (q_x * s_x[m]) @ (q_w * s_w[n])^T + b, accumulated in float64."""
    a = e4m3_decode(qx).astype(np.float64) * np.asarray(sx, np.float64).reshape(-1, 1)
    w = e4m3_decode(qw).astype(np.float64) * np.asarray(sw, np.float64).reshape(-1, 1)
    y = a @ w.T
    if bias is not None:
        y = y + np.asarray(bias, dtype=np.float64).reshape(1, -1)
    return gelu_tanh(y) if gelu else y


def blockwise_gemm_reference(qa, sa, qb, sb) -> np.ndarray:
    """test_pixelumm_decoder_optimizations.py:204-219: dequant(qa,sa) @ dequant(qb,sb).T."""
    m, k = qa.shape
    n = qb.shape[0]
    a = e4m3_decode(qa).astype(np.float64) * np.repeat(np.repeat(
        np.asarray(sa, np.float64), 128, 0), 128, 1)[:m, :k]
    b = e4m3_decode(qb).astype(np.float64) * np.repeat(np.repeat(
        np.asarray(sb, np.float64), 128, 0), 128, 1)[:n, :k]
    return a @ b.T


def block_causal_visible(q_pos: np.ndarray, k_pos: np.ndarray, chunk_len: int) -> np.ndarray:
    """Chunk-granular block-causal visibility: key visible iff chunk(k) <= chunk(q).
    chunk_len <= 0 means full attention (the cached path of nomas_cpt.py:464-685)."""
    q_pos = np.asarray(q_pos, dtype=np.int64)
    k_pos = np.asarray(k_pos, dtype=np.int64)
    if chunk_len <= 0:
        return np.ones((q_pos.size, k_pos.size), dtype=bool)
    return (k_pos[None, :] // chunk_len) <= (q_pos[:, None] // chunk_len)


def attention_reference(q, k, v, visible=None, key_valid=None, scale=None) -> np.ndarray:
    """softmax(q k^T * scale) v in float64 for one batch slot.
    q [Lq,H,D], k/v [Lk,H,D] (real values, e.g. dequantized cache), visible [Lq,Lk]
    bool, key_valid [Lk] bool. Query rows with no visible key return zeros (the
    masked-row convention of range_attention.py:212-239)."""
    q = np.asarray(q)
    Lq, H, D = q.shape
    Lk = k.shape[0]
    if scale is None:
        scale = D ** -0.5
    mask = np.ones((Lq, Lk), dtype=bool) if visible is None else np.asarray(visible, bool)
    if key_valid is not None:
        mask = mask & np.asarray(key_valid, bool)[None, :]
    out = np.zeros((Lq, H, D), dtype=np.float64)
    any_vis = mask.any(axis=1)
    for h in range(H):
        kh = np.ascontiguousarray(k[:, h, :], dtype=np.float64)
        vh = np.ascontiguousarray(v[:, h, :], dtype=np.float64)
        s = (np.asarray(q[:, h, :], np.float64) @ kh.T) * scale
        s = np.where(mask, s, -np.inf)
        m = np.max(np.where(any_vis[:, None], s, 0.0), axis=1, keepdims=True)
        m = np.where(np.isfinite(m), m, 0.0)
        p = np.where(mask, np.exp(s - m), 0.0)
        denom = p.sum(axis=1, keepdims=True)
        denom = np.where(denom > 0, denom, 1.0)
        out[:, h, :] = (p / denom) @ vh
    return out
