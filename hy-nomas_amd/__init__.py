"""hy-nomas_amd: the FP8 quantized inference hot path of Hy-Nomas, MI355X-native.

Host side in Python over one C-ABI HIP library (libhynomas_fp8.so, built from
csrc/ for gfx950). Modules mirror the reference surfaces they replace:

  pixelumm_fp8      <- hymm/models/vae/pixelumm_decoder/cutlass_fp8.py (blockwise FP8 linear)
  dit_fp8_linear    <- hymm/models/dit/modules/int8_stored_bf16_linear.py (DiT linear)
  fp8_kv_cache      <- hymm/models/dit/modules/int8_kv_cache.py (KV quantize/decode)
  kv_cache_storage  <- hymm/models/dit/modules/kv_cache_storage.py (format dispatch)
  cache_attention   <- nomas_cpt.causal_attention_with_cache_mp + reactor CacheStaging
  quantization      <- reactor/hy_nomas_quantization.py (install seam)
  dit_block         <- nomas_compile_prepost.pre/post_attention + the AR chunk loop
  ops               torch custom ops over the C ABI; _lib the ctypes binding
"""
from . import _lib, ops  # noqa: F401

__all__ = ["ops"]
__version__ = "0.1.0"
