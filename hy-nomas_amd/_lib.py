"""ctypes binding of libhynomas_fp8.so (the C ABI declared in include/hynomas_fp8.h).

There is no fallback: if the library is missing, or a call is made for tensors
that are not on a GPU, the call raises. Argument errors detected by the
library come back as RuntimeError carrying hn_last_error().
"""
from __future__ import annotations

import ctypes
import threading
from pathlib import Path

LIB_PATH = Path(__file__).resolve().parent / "libhynomas_fp8.so"

HN_OK = 0
HN_E_ARG = -1
HN_E_LAUNCH = -2
HN_E_DEVICE = -3
ABI_VERSION = 4
HN_SCALE_CLAMP = 0
HN_SCALE_ZERO_ONE = 1
HN_KV_FP8 = 0
HN_KV_INT8 = 1
HN_ACT_NONE = 0
HN_ACT_GELU_TANH = 1

_P = ctypes.c_void_p
_I64 = ctypes.c_int64
_I = ctypes.c_int
_F = ctypes.c_float
_PI64 = ctypes.POINTER(ctypes.c_int64)

# name -> argtypes, in the order of include/hynomas_fp8.h
SIGNATURES = {
    "hn_last_error": [],
    "hn_abi_version": [],
    "hn_quantize_rows_fp8": [_P, _I64, _I64, _I64, _I, _F, _P, _P, _P],
    "hn_quantize_blockwise_fp8": [_P, _I64, _I64, _P, _P, _P],
    "hn_ln_mod_quantize_fp8": [_P, _I64, _I64, _I64, _P, _P, _I64, _F, _F, _P, _P, _P],
    "hn_kv_quantize": [_I, _P, _PI64, _I64, _I64, _I64, _I64, _P, _PI64, _P, _PI64, _I64, _I64,
                       _P, _P],
    "hn_kv_quantize_pair": [_I, _P, _P, _PI64, _I64, _I64, _I64, _I64, _P, _P, _PI64, _P, _P,
                            _PI64, _I64, _I64, _P, _P],
    "hn_kv_dequantize": [_I, _P, _PI64, _P, _PI64, _I64, _I64, _I64, _I64, _P, _PI64, _P],
    "hn_gemm_fp8_rowcol": [_P, _P, _P, _P, _P, _P, _I64, _I64, _I64, _I64, _I, _P],
    "hn_gemm_fp8_blockwise": [_P, _P, _P, _P, _P, _I64, _I64, _I64, _P],
    "hn_attn_fp8kv": [_I, _P, _PI64, _I64, _I64, _I64, _I64, _P, _P, _PI64, _P, _P, _PI64,
                      _I64, _I64, _P, _I64, _P, _P, _PI64, _I64, _P, _I64, _I64, _I64, _F, _P,
                      _PI64, _P, _I64, _P],
    "hn_attn_fp8kv_workspace_size": [_I64, _I64, _I64, _I64, _I64, _I64],
    "hn_attn_fp8kv_noalloc": [_I, _P, _PI64, _I64, _I64, _I64, _I64, _P, _P, _PI64, _P, _P, _PI64,
                              _I64, _I64, _P, _I64, _P, _P, _PI64, _I64, _P, _I64, _I64, _I64, _F,
                              _P, _PI64, _P],
    "hn_attn_fp8kv_noalloc_scratch_bytes": [],
    "hn_qk_norm_rope_kv": [_I, _P, _P, _P, _PI64, _I64, _I64, _I64, _I64, _P, _P, _P, _P, _I64, _F,
                           _P, _P, _PI64, _P, _P, _PI64, _I64, _I64, _P, _P],
    "hn_e4m3_encode_range": [ctypes.c_uint32, _I64, _P, _P],
}
RESTYPES = {"hn_last_error": ctypes.c_char_p, "hn_attn_fp8kv_workspace_size": _I64,
            "hn_attn_fp8kv_noalloc_scratch_bytes": _I64}

_lib = None
_lock = threading.Lock()


def load(path: Path | str | None = None) -> ctypes.CDLL:
    """Load (once) and return the library with argtypes set. Raises if absent."""
    global _lib
    with _lock:
        if _lib is not None:
            return _lib
        p = Path(path) if path is not None else LIB_PATH
        if not p.exists():
            raise RuntimeError(
                f"{p.name} is not built: run `python -c 'import __graft_entry__ as g; g.build()'` "
                "(there is no CPU fallback for the FP8 kernels)")
        lib = ctypes.CDLL(str(p))
        for name, args in SIGNATURES.items():
            fn = getattr(lib, name)
            fn.argtypes = args
            fn.restype = RESTYPES.get(name, _I)
        if lib.hn_abi_version() != ABI_VERSION:
            raise RuntimeError(f"{p.name} has ABI version {lib.hn_abi_version()}, this binding expects "
                               f"{ABI_VERSION}: rebuild the library")
        _lib = lib
        return lib


def check(rc: int, what: str) -> None:
    if rc != HN_OK:
        msg = load().hn_last_error().decode(errors="replace")
        raise RuntimeError(f"{what} failed ({rc}): {msg}")


def strides(t) -> ctypes.Array:
    """Element strides of a tensor as an int64[ndim] C array."""
    st = t.stride()
    return (ctypes.c_int64 * len(st))(*st)


def ptr(t) -> int | None:
    return None if t is None else t.data_ptr()
