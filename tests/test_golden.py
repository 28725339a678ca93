"""The committed fixtures (tests/golden/fp8_path_golden.npz, written by
tests/golden/make_golden.py from torch restatements of the reference recipes)
against the oracle (CPU) and against the HIP kernels (GPU). Codes and scales
must match bit for bit; float outputs within the north-star tolerance."""
from pathlib import Path

import numpy as np
import pytest
import torch

from conftest import assert_close_bf16, pkg_module, u8

G = np.load(Path(__file__).resolve().parent / "golden" / "fp8_path_golden.npz")


def _bf16(bits, device):
    return torch.from_numpy(np.ascontiguousarray(bits).view(np.int16)).view(torch.bfloat16).to(device)


def _f32(bits):
    return (bits.astype(np.uint32) << 16).view(np.float32)


# ------------------------------------------------------------------ oracle (CPU)

def test_oracle_row_quant_matches_golden(O):
    q, s = O.quantize_rows_fp8(G["rows_x"], O.SCALE_CLAMP)
    assert np.array_equal(q, G["rows_q"]) and np.array_equal(s, G["rows_s"])
    q, s = O.quantize_rows_fp8(G["rows_x"], O.SCALE_ZERO_ONE)
    assert np.array_equal(q, G["rows_q_zero_one"]) and np.array_equal(s, G["rows_s_zero_one"])


def test_oracle_blockwise_quant_matches_golden(O):
    q, s = O.quantize_blockwise_fp8(G["block_x"])
    assert np.array_equal(q, G["block_q"]) and np.array_equal(s, G["block_s"])


def test_oracle_kv_quant_matches_golden(O):
    q, s = O.kv_quantize(G["kv_x"], O.KV_FP8)
    assert np.array_equal(q, G["kv_q_fp8"]) and np.array_equal(s, G["kv_s_fp8"])
    q, s = O.kv_quantize(G["kv_x"], O.KV_INT8)
    assert np.array_equal(q.view(np.int8), G["kv_q_int8"]) and np.array_equal(s, G["kv_s_int8"])


def test_oracle_linear_matches_golden(O):
    qx, sx = O.quantize_rows_fp8(G["lin_x"], O.SCALE_CLAMP)
    qw, sw = O.quantize_rows_fp8(G["lin_w"], O.SCALE_CLAMP)
    assert np.array_equal(qw, G["lin_qw"]) and np.array_equal(sw, G["lin_sw"])
    b = _f32(G["lin_b"])
    for gelu, key in ((False, "lin_y"), (True, "lin_y_gelu")):
        y = O.linear_reference(qx, sx, qw, sw, b, gelu=gelu)
        np.testing.assert_allclose(y, G[key], rtol=1e-6, atol=1e-7)


def test_oracle_attention_matches_golden(O):
    H, D, kv_len, chunk, q0, Lq = (int(v) for v in G["att_meta"])
    k = O.e4m3_decode(G["att_kq"][0]) * G["att_ks"][0]
    v = O.e4m3_decode(G["att_vq"][0]) * G["att_vs"][0]
    vis = O.block_causal_visible(np.arange(q0, q0 + Lq), np.arange(kv_len), chunk)
    o = O.attention_reference(_f32(G["att_q"][0]), k, v, visible=vis)
    np.testing.assert_allclose(o, G["att_o"], rtol=1e-5, atol=1e-6)


# ------------------------------------------------------------------ HIP kernels (GPU)

@pytest.mark.gpu
def test_gpu_quantizers_match_golden(dev):
    print("case golden quantizers", flush=True)
    ops = pkg_module("ops")
    L = pkg_module("_lib")
    x = _bf16(G["rows_x"], dev)
    q, s = ops.quantize_rows_fp8(x, L.HN_SCALE_CLAMP, 1e-4)
    assert np.array_equal(u8(q), G["rows_q"]) and np.array_equal(s.cpu().numpy(), G["rows_s"])
    q, s = ops.quantize_rows_fp8(x, L.HN_SCALE_ZERO_ONE, 0.0)
    assert np.array_equal(u8(q), G["rows_q_zero_one"])
    assert np.array_equal(s.cpu().numpy(), G["rows_s_zero_one"])
    q, s = ops.quantize_blockwise_fp8(_bf16(G["block_x"], dev))
    assert np.array_equal(u8(q), G["block_q"]) and np.array_equal(s.cpu().numpy(), G["block_s"])


@pytest.mark.gpu
@pytest.mark.parametrize("fmt", ["fp8", "int8"])
def test_gpu_kv_write_matches_golden(dev, fmt):
    print(f"case golden kv write {fmt}", flush=True)
    kvc = pkg_module("fp8_kv_cache")
    x = _bf16(G["kv_x"], dev)
    B, Lt, H, D = x.shape
    make = kvc.make_fp8_kv_block if fmt == "fp8" else kvc.make_int8_kv_block
    cache = make(B, Lt + 3, H, D, device=dev)
    for t in cache.values():                      # the cache is allocated uninitialised
        t.view(torch.uint8).zero_()
    kvc.quantize_kv_pair_into(cache, x, x, 2)
    codes = u8(cache["k"][:, 2:2 + Lt])
    want_q = G["kv_q_fp8"] if fmt == "fp8" else G["kv_q_int8"].view(np.uint8)
    want_s = G["kv_s_fp8"] if fmt == "fp8" else G["kv_s_int8"]
    assert np.array_equal(codes, want_q) and np.array_equal(u8(cache["v"][:, 2:2 + Lt]), want_q)
    assert np.array_equal(cache["k_scale"][:, 2:2 + Lt].cpu().numpy(), want_s)
    assert not u8(cache["k"][:, :2]).any() and not u8(cache["k"][:, 2 + Lt:]).any()


@pytest.mark.gpu
@pytest.mark.parametrize("gelu", [False, True])
def test_gpu_linear_matches_golden(dev, gelu):
    print(f"case golden linear gelu={gelu}", flush=True)
    ops = pkg_module("ops")
    L = pkg_module("_lib")
    dl = pkg_module("dit_fp8_linear")
    qw, sw = dl.quantize_weight(_bf16(G["lin_w"], dev))
    assert np.array_equal(u8(qw), G["lin_qw"]) and np.array_equal(sw.cpu().numpy().reshape(-1), G["lin_sw"])
    y = ops.linear_fp8(_bf16(G["lin_x"], dev), qw, sw.reshape(-1), _bf16(G["lin_b"], dev),
                       L.HN_ACT_GELU_TANH if gelu else L.HN_ACT_NONE)
    assert_close_bf16(y.float().cpu().numpy(), G["lin_y_gelu" if gelu else "lin_y"], what="golden linear")


@pytest.mark.gpu
def test_gpu_chunk_attention_matches_golden(dev):
    print("case golden chunk attention", flush=True)
    ca = pkg_module("cache_attention")
    kvc = pkg_module("fp8_kv_cache")
    H, D, kv_len, chunk, q0, Lq = (int(v) for v in G["att_meta"])
    cache = kvc.make_fp8_kv_block(1, kv_len, H, D, device=dev)
    cache["k"].view(torch.uint8).copy_(torch.from_numpy(G["att_kq"]))
    cache["v"].view(torch.uint8).copy_(torch.from_numpy(G["att_vq"]))
    cache["k_scale"].copy_(torch.from_numpy(G["att_ks"]))
    cache["v_scale"].copy_(torch.from_numpy(G["att_vs"]))
    out = ca.chunk_attention(_bf16(G["att_q"], dev), cache, kv_len, q_pos0=q0, chunk_len=chunk)
    assert_close_bf16(out[0].float().cpu().numpy(), G["att_o"], what="golden attention")
