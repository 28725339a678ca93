"""hn_attn_fp8kv_noalloc (split-key scratch in a library-held device array)
against hn_attn_fp8kv (caller workspace), both through the C ABI: identical
outputs on two calls in a row, the second smaller; and the scratch size
against every split launch the planner makes."""
import pytest
import torch

from conftest import pkg_module

pytestmark = pytest.mark.gpu


def _cache(dev, L, H, seed):
    kvc = pkg_module("fp8_kv_cache")
    g = torch.Generator(device=dev).manual_seed(seed)
    cache = kvc.make_fp8_kv_block(1, L, H, 128, device=dev)
    gain = torch.empty(H, device=dev).uniform_(0.5, 4.0, generator=g)
    k = (torch.randn(1, L, H, 128, device=dev, generator=g) * gain[None, None, :, None]).to(torch.bfloat16)
    v = (torch.randn(1, L, H, 128, device=dev, generator=g) * gain[None, None, :, None]).to(torch.bfloat16)
    kvc.quantize_kv_pair_into(cache, k, v, 0)
    return cache


def _args(q, cache, kv_len, out, valid=None):
    L = pkg_module("_lib")
    B, Lq, H, D = q.shape
    vb = None if valid is None else valid.view(torch.uint8)
    return (L.HN_KV_FP8, q.data_ptr(), L.strides(q), B, Lq, H, D,
            cache["k"].data_ptr(), cache["v"].data_ptr(), L.strides(cache["k"]),
            cache["k_scale"].data_ptr(), cache["v_scale"].data_ptr(), L.strides(cache["k_scale"]),
            cache["k"].shape[1], kv_len, None if vb is None else vb.data_ptr(),
            0 if vb is None else vb.stride(0),
            None, None, None, 0, None, 0, 0, 0, D ** -0.5, out.data_ptr(), L.strides(out))


def _both(dev, q, cache, kv_len, valid=None):
    """Outputs of the workspace entry point and of the no-alloc one."""
    L = pkg_module("_lib")
    lib = L.load()
    B, Lq, H, D = q.shape
    stream = torch.cuda.current_stream().cuda_stream
    ws_bytes = lib.hn_attn_fp8kv_workspace_size(B, Lq, H, D, kv_len, 0)
    assert 0 < ws_bytes <= lib.hn_attn_fp8kv_noalloc_scratch_bytes()   # the scratch is used
    ws = torch.empty(ws_bytes, dtype=torch.uint8, device=dev)
    ref = torch.empty_like(q)
    got = torch.full_like(q, float("nan"))
    L.check(lib.hn_attn_fp8kv(*_args(q, cache, kv_len, ref, valid), ws.data_ptr(), ws_bytes, stream),
            "hn_attn_fp8kv")
    L.check(lib.hn_attn_fp8kv_noalloc(*_args(q, cache, kv_len, got, valid), stream),
            "hn_attn_fp8kv_noalloc")
    torch.cuda.synchronize()
    return ref, got


def test_noalloc_matches_workspace_entry_point_twice(dev):
    print("case noalloc: decode-style, then a smaller masked call", flush=True)
    g = torch.Generator(device=dev).manual_seed(5)
    # 1: decode-style Lq 128 over 86400 keys, 24 heads (split keys, ~33 MB of partials)
    cache = _cache(dev, 86400, 24, 1)
    q = torch.randn(1, 128, 24, 128, device=dev, generator=g).to(torch.bfloat16)
    ref, got = _both(dev, q, cache, 86400)
    assert torch.equal(got, ref)
    del cache
    # 2: a smaller call right after (fewer heads, queries and keys, with a key
    # mask): the scratch keeps the first call's partials, which must not leak in
    cache = _cache(dev, 20000, 8, 2)
    q = torch.randn(1, 64, 8, 128, device=dev, generator=g).to(torch.bfloat16)
    valid = torch.rand(1, 20000, device=dev, generator=g) > 0.25
    ref, got = _both(dev, q, cache, 20000, valid)
    assert torch.equal(got, ref)
    assert torch.isfinite(got.float()).all()


def test_noalloc_scratch_covers_every_split_launch(dev):
    """The scratch holds any call's split-key partials on this device: a split
    launch keeps at most 2 workgroups per CU (128 query rows of 128 + 2 fp32
    each), so no shape reaches hn_attn_fp8kv_noalloc's refusal on 256 CUs. The
    sweep checks the workspace sizes the planner asks for against the scratch."""
    lib = pkg_module("_lib").load()
    cap = lib.hn_attn_fp8kv_noalloc_scratch_bytes()
    cus = torch.cuda.get_device_properties(dev).multi_processor_count
    assert cap == 40 << 20 and 2 * cus * 128 * 130 * 4 <= cap
    worst = 0
    for B in (1, 2, 3):
        for H in (1, 2, 8, 24, 64):
            for Lq in (1, 48, 100, 128, 200, 256, 1000, 10800):
                for kv in (4096, 86400, 172800):
                    worst = max(worst, lib.hn_attn_fp8kv_workspace_size(B, Lq, H, 128, kv, 0))
    assert 0 < worst <= 2 * cus * 128 * 130 * 4
