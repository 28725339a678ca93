"""C ABI and host-side boundary checks that need no GPU: every symbol the
header declares is exported, argument errors are reported before any launch,
and the Python mirror validates like the reference."""
import ctypes
import re
from pathlib import Path

import pytest
import torch

from conftest import ROOT, pkg_module

HEADER = ROOT / "include" / "hynomas_fp8.h"


def _declared():
    text = HEADER.read_text()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(hn_[a-z0-9_]+)\s*\(", text)))


@pytest.fixture(scope="module")
def lib():
    return pkg_module("_lib").load()


def test_every_declared_symbol_is_exported(lib):
    names = _declared()
    assert len(names) >= 10
    for n in names:
        assert hasattr(lib, n), f"{n} declared in {HEADER.name} but not exported"
    assert set(names) == set(pkg_module("_lib").SIGNATURES), "ctypes table out of sync with header"


def test_abi_version(lib):
    assert lib.hn_abi_version() == 4 == pkg_module("_lib").ABI_VERSION


def _err(lib):
    return lib.hn_last_error().decode()


def test_argument_errors_are_reported_without_a_launch(lib):
    L = pkg_module("_lib")
    assert lib.hn_quantize_rows_fp8(None, 4, 7, 7, 0, 1e-4, None, None, None) == -1
    assert "multiple of 8" in _err(lib)
    assert lib.hn_quantize_blockwise_fp8(None, 4, 100, None, None, None) == -1
    assert "multiple of 128" in _err(lib)
    st = (ctypes.c_int64 * 4)(128, 128, 128, 1)
    assert lib.hn_kv_quantize(0, None, st, 1, 1, 1, 64, None, st, None, st, 8, 0, None, None) == -1
    assert "head dim 128" in _err(lib)
    assert lib.hn_kv_quantize(7, None, st, 1, 1, 1, 128, None, st, None, st, 8, 0, None, None) == -1
    assert lib.hn_gemm_fp8_rowcol(None, None, None, None, None, None, 16, 100, 128, 100, 0, None) == -1
    assert "multiples of 128" in _err(lib)
    assert lib.hn_gemm_fp8_rowcol(None, None, None, None, None, None, 16, 128, 128, 128, 9, None) == -1
    assert "activation" in _err(lib)
    assert lib.hn_gemm_fp8_blockwise(None, None, None, None, None, 16, 128, 96, None) == -1
    assert lib.hn_attn_fp8kv(0, None, st, 1, 1, 1, 64, None, None, st, None, None, st, 0, 0, None, 0,
                             None, None, None, 0, None, 0, 0, 0, 1.0, None, st, None, 0, None) == -1
    assert "head dim" in _err(lib)
    assert lib.hn_attn_fp8kv_workspace_size(1, 128, 24, 64, 1000, 0) == 0   # bad head dim
    assert lib.hn_qk_norm_rope_kv(0, None, None, None, st, 1, 4, 2, 64, None, None, None, None, 128,
                                  1e-6, None, None, None, None, None, None, 0, 0, None, None) == -1
    assert "head dim" in _err(lib)
    assert lib.hn_qk_norm_rope_kv(3, None, None, None, st, 1, 4, 2, 128, None, None, None, None, 128,
                                  1e-6, None, None, None, None, None, None, 0, 0, None, None) == -1
    assert "format" in _err(lib)
    assert lib.hn_quantize_rows_fp8(None, 4, 16392, 16392, 0, 1e-4, None, None, None) == -1
    assert "16384" in _err(lib)
    # fused LayerNorm + modulate + quant: width, modulation layout, eps
    lnq = lib.hn_ln_mod_quantize_fp8
    assert lnq(None, 4, 100, 4, None, None, 100, 1e-6, 1e-4, None, None, None) == -1
    assert "multiple of 8" in _err(lib)
    assert lnq(None, 4, 8200, 4, None, None, 8200, 1e-6, 1e-4, None, None, None) == -1
    assert "8192" in _err(lib)
    assert lnq(None, 4, 128, 0, None, None, 128, 1e-6, 1e-4, None, None, None) == -1
    assert "rows_per_batch" in _err(lib)
    assert lnq(None, 4, 128, 4, None, None, 64, 1e-6, 1e-4, None, None, None) == -1
    assert "stride" in _err(lib)
    assert lnq(None, 4, 128, 4, None, None, 128, -1.0, 1e-4, None, None, None) == -1
    assert "eps" in _err(lib)
    # zero-size work is a no-op that needs no pointers
    assert lnq(None, 0, 128, 1, None, None, 128, 1e-6, 1e-4, None, None, None) == L.HN_OK
    assert lib.hn_quantize_rows_fp8(None, 0, 8, 8, 0, 1e-4, None, None, None) == L.HN_OK
    assert lib.hn_gemm_fp8_rowcol(None, None, None, None, None, None, 0, 128, 128, 128, 0, None) == L.HN_OK


# Fake, 256-byte-aligned device addresses: every call below is refused on the
# host before anything touches them.
_A = 0x10000


def test_capacity_and_scale_refusals(lib):
    """Writes past the cache capacity and invalid attention arguments are
    refused by the C ABI itself (int8_kv_cache.py:128-135; cutlass_fp8.cu:21-34)."""
    st = (ctypes.c_int64 * 4)(128, 128, 128, 1)
    ss = (ctypes.c_int64 * 3)(1, 1, 1)
    # L = 4 tokens at start 6 of an 8-token cache
    for start, cap in ((6, 8), (0, 3), (9, 8)):
        assert lib.hn_kv_quantize(0, _A, st, 1, 4, 1, 128, _A, st, _A, ss, cap, start, None, None) == -1
        assert "capacity" in _err(lib)
        assert lib.hn_kv_quantize_pair(0, _A, _A, st, 1, 4, 1, 128, _A, _A, st, _A, _A, ss, cap, start,
                                       None, None) == -1
        assert "capacity" in _err(lib)
        assert lib.hn_qk_norm_rope_kv(0, _A, _A, _A, st, 1, 4, 1, 128, _A, _A, _A, _A, 128, 1e-6,
                                      _A, _A, st, _A, _A, ss, cap, start, None, None) == -1
        assert "capacity" in _err(lib)
    # a status word needs a cache write
    assert lib.hn_qk_norm_rope_kv(0, _A, _A, _A, st, 1, 4, 1, 128, _A, _A, _A, _A, 128, 1e-6,
                                  None, None, None, None, None, None, 0, 0, _A, None) == -1
    assert "status" in _err(lib)

    def attn(kv_len=8, cap=8, scale=0.1, cvs=0):
        return lib.hn_attn_fp8kv(0, _A, st, 1, 4, 1, 128, _A, _A, st, _A, _A, ss, cap, kv_len, None, cvs,
                                 None, None, None, 0, None, 0, 0, 0, scale, _A, st, None, 0, None)
    assert attn(kv_len=9) == -1 and "capacity" in _err(lib)
    for bad in (0.0, -0.5, float("nan"), float("inf")):
        assert attn(scale=bad) == -1 and "softmax_scale" in _err(lib)
    assert attn(cvs=-1) == -1 and "stride" in _err(lib)


@pytest.mark.skipif(torch.cuda.is_available(), reason="checks the refusal on a machine without a GPU")
def test_no_gfx950_device_is_refused(lib):
    """A call with valid arguments and work to do returns HN_E_DEVICE when no
    gfx950 is present, before any launch (here: no GPU at all)."""
    L = pkg_module("_lib")
    assert lib.hn_quantize_rows_fp8(_A, 4, 8, 8, 0, 1e-4, _A, _A, None) == L.HN_E_DEVICE
    assert "device" in _err(lib)
    assert lib.hn_gemm_fp8_rowcol(_A, _A, _A, _A, None, _A, 16, 128, 128, 128, 0, None) == L.HN_E_DEVICE
    st = (ctypes.c_int64 * 4)(128, 128, 128, 1)
    ss = (ctypes.c_int64 * 3)(1, 1, 1)
    assert lib.hn_kv_quantize_pair(0, _A, _A, st, 1, 4, 1, 128, _A, _A, st, _A, _A, ss, 8, 0,
                                   None, None) == L.HN_E_DEVICE
    assert lib.hn_attn_fp8kv(0, _A, st, 1, 4, 1, 128, _A, _A, st, _A, _A, ss, 8, 8, None, 0, None, None,
                             None, 0, None, 0, 0, 0, 0.1, _A, st, None, 0, None) == L.HN_E_DEVICE


def test_ops_check_geometry_before_any_launch():
    """The custom ops check cache geometry and capacity on the host, before the
    GPU-tensor check (so CPU tensors exercise them) and before any launch."""
    ops = pkg_module("ops")
    kvc = pkg_module("fp8_kv_cache")
    cache = kvc.make_fp8_kv_block(1, 8, 2, 128, device="cpu")
    vals = torch.zeros(1, 4, 2, 128, dtype=torch.bfloat16)
    c = (cache["k"], cache["v"], cache["k_scale"], cache["v_scale"])
    with pytest.raises(ValueError, match="capacity"):
        ops.kv_quantize_pair_(*c, vals, vals, 5)
    with pytest.raises(ValueError, match="capacity"):
        ops.kv_quantize_(cache["k"], cache["k_scale"], vals, -1)
    with pytest.raises(ValueError, match="B, H, D"):
        ops.kv_quantize_(cache["k"], cache["k_scale"], torch.zeros(1, 4, 3, 128, dtype=torch.bfloat16), 0)
    with pytest.raises(ValueError, match="scale"):
        ops.kv_quantize_(cache["k"], cache["k_scale"][:, :4], vals, 0)
    qkv = torch.zeros(1, 4, 3, 2, 128, dtype=torch.bfloat16)
    q, k, v = qkv.select(2, 0), qkv.select(2, 1), qkv.select(2, 2)
    w = torch.ones(128, dtype=torch.bfloat16)
    cs = torch.zeros(4, 128)
    with pytest.raises(ValueError, match="capacity"):
        ops.qk_norm_rope_kv_(q, k, v, w, w, cs, cs, 1e-6, *c, 6)
    small = kvc.make_fp8_kv_block(1, 8, 1, 128, device="cpu")
    with pytest.raises(ValueError, match="B, H, D"):
        ops.qk_norm_rope_kv_(q, k, v, w, w, cs, cs, 1e-6, small["k"], small["v"], small["k_scale"],
                             small["v_scale"], 0)
    # attention: capacity, scale, K/V layout, tail geometry
    qa = torch.zeros(1, 4, 2, 128, dtype=torch.bfloat16)
    with pytest.raises(ValueError, match="capacity"):
        ops.attn_fp8kv(qa, *c, 9)
    with pytest.raises(ValueError, match="softmax_scale"):
        ops.attn_fp8kv(qa, *c, 8, softmax_scale=0.0)
    with pytest.raises(ValueError, match="share dtype, shape and strides"):
        ops.attn_fp8kv(qa, cache["k"], cache["v"][:, :4], cache["k_scale"], cache["v_scale"], 4)
    with pytest.raises(ValueError, match="scales"):
        ops.attn_fp8kv(qa, cache["k"], cache["v"], cache["k_scale"], cache["v_scale"][:, :4], 4)
    with pytest.raises(ValueError, match="k_cur"):
        ops.attn_fp8kv(qa, *c, 8, torch.zeros(1, 4, 3, 128, dtype=torch.bfloat16),
                       torch.zeros(1, 4, 3, 128, dtype=torch.bfloat16))
    with pytest.raises(ValueError, match="cache_valid"):
        ops.attn_fp8kv(qa, *c, 8, cache_valid=torch.ones(1, 7, dtype=torch.bool))
    two = torch.zeros(2, 4, 2, 128, dtype=torch.bfloat16)
    three = kvc.make_fp8_kv_block(3, 8, 2, 128, device="cpu")
    with pytest.raises(ValueError, match="does not match q"):
        ops.attn_fp8kv(two, three["k"], three["v"], three["k_scale"], three["v_scale"], 4)
    # a one-slot cache is accepted for any query batch (read-only broadcast):
    # it gets as far as the GPU-tensor check
    with pytest.raises(RuntimeError, match="GPU"):
        ops.attn_fp8kv(two, *c, 8)


def test_ar_model_refuses_a_chunk_past_capacity():
    """FP8ARModel.generate_chunk checks cache_valid_len + the tokens a chunk
    writes (image, plus text with the text stream) <= capacity before running
    any pass."""
    dit = pkg_module("dit_block")
    m = dit.FP8ARModel.__new__(dit.FP8ARModel)
    m.cache_valid_len, m.tokens_per_chunk, m.write_tokens, m.capacity = 20, 10, 10, 25
    with pytest.raises(ValueError, match="capacity"):
        m.generate_chunk(None, [None], None, [1.0, 0.0])
    m.cache_valid_len, m.write_tokens = 10, 16          # 10 image + 6 text tokens
    with pytest.raises(ValueError, match="capacity"):
        m.generate_chunk(None, [None], None, [1.0, 0.0])


def test_ops_refuse_cpu_tensors():
    ops = pkg_module("ops")
    x = torch.zeros(4, 128, dtype=torch.bfloat16)
    with pytest.raises(RuntimeError, match="GPU"):
        ops.quantize_rows_fp8(x)
    with pytest.raises(RuntimeError, match="GPU"):
        ops.linear_fp8(x, torch.zeros(128, 128, dtype=torch.float8_e4m3fn), torch.ones(128))


def test_kv_api_validates_before_writing():
    kvc = pkg_module("fp8_kv_cache")
    cache = kvc.make_fp8_kv_block(1, 8, 2, 128, device="cpu")
    assert cache["k"].dtype == torch.float8_e4m3fn and cache["k_scale"].shape == (1, 8, 2, 1)
    assert kvc.is_fp8_kv_cache(cache) and kvc.kv_storage_bytes(cache) == 2 * 8 * 2 * 128 + 2 * 8 * 2 * 4
    good = torch.zeros(1, 4, 2, 128, dtype=torch.bfloat16)
    # (the finiteness check runs on the GPU: tests/test_gpu_quant.py)
    with pytest.raises(RuntimeError, match="GPU"):
        kvc.quantize_kv_pair_into(cache, good, good, 0)
    with pytest.raises(ValueError, match="capacity"):
        kvc.quantize_kv_pair_into(cache, good, good, 6)
    with pytest.raises(ValueError, match="must match"):
        kvc.quantize_kv_pair_into(cache, good, good[:, :3], 0)
    with pytest.raises(TypeError):
        kvc.quantize_kv_into(cache, "k", good.float(), 0)
    with pytest.raises(ValueError, match="Invalid KV key"):
        kvc.quantize_kv_into(cache, "q", good, 0)
    with pytest.raises(ValueError, match="valid length"):
        kvc.dequantize_kv(cache, "k", 9)
    i8 = kvc.make_int8_kv_block(1, 8, 2, 128, device="cpu")
    assert i8["k"].dtype == torch.int8 and kvc.is_quantized_kv_cache(i8)


def test_storage_format_dispatch():
    st = pkg_module("kv_cache_storage")
    kvc = pkg_module("fp8_kv_cache")
    assert st.cache_format(kvc.make_fp8_kv_block(1, 2, 1, 128, device="cpu")) == "fp8"
    assert st.cache_format(kvc.make_int8_kv_block(1, 2, 1, 128, device="cpu")) == "int8"
    assert st.cache_format({"k": torch.zeros(1, 2, 1, 128, dtype=torch.bfloat16)}) == "none"

    class Inf:
        kv_cache_quantization = "fp8"
    assert st.quantization_mode(Inf) == "fp8"
    Inf.kv_cache_quantization = "int4"
    with pytest.raises(ValueError):
        st.quantization_mode(Inf)
    audit = st.cache_storage_audit(kvc.make_fp8_kv_block(1, 4, 2, 128, device="cpu"))
    assert audit["gpu_storage_bytes"] == 2 * 4 * 2 * 128 + 2 * 4 * 2 * 4


def test_serialized_fp8_validation_and_dtype_preserving_apply():
    pf = pkg_module("pixelumm_fp8")
    w = torch.zeros(256, 128, dtype=torch.float8_e4m3fn)
    s = torch.ones(2, 1, dtype=torch.float32)
    m = pf.FP8Linear.from_quantized(w, s, (256, 128))
    m.to(dtype=torch.bfloat16)
    assert m.fp8_weight.dtype == torch.float8_e4m3fn and m.fp8_scale.dtype == torch.float32
    assert pf.CutlassFP8Linear is pf.FP8Linear
    with pytest.raises(ValueError):
        pf.FP8Linear.from_quantized(w, s, (256, 100))
    with pytest.raises(ValueError, match="positive"):
        pf.FP8Linear.from_quantized(w, torch.zeros(2, 1), (256, 128))
    # a scale row spanning more than 2^60 is refused: the blockwise GEMM's
    # carried rescale f_prev / f must stay inside fp32
    w2 = torch.zeros(128, 384, dtype=torch.float8_e4m3fn)
    pf.validate_serialized_tensors(w2, torch.tensor([[1.0, 2.0 ** 60, 1.0]]), (128, 384))  # span 2^60
    with pytest.raises(ValueError, match="2\\^60"):
        pf.validate_serialized_tensors(w2, torch.tensor([[0.5, 2.0 ** 60, 1.0]]), (128, 384))  # 2^61
    m.train()
    with pytest.raises(RuntimeError, match="inference"):
        m(torch.zeros(4, 128, dtype=torch.bfloat16))
