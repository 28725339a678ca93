"""GPU parity of the FP8-KV chunk attention against the oracle's float64
softmax(Q K^T / sqrt(D)) V over the K, V the reference attends over: the
cache decoded to bf16(code * scale). Bar: the north star's, max-abs 2e-2 and
rel-L2 1e-2, with the elementwise bound max(2e-2, 1.5 * 2^-8 |ref|) of
conftest.assert_close_bf16 (the bf16 output's own rounding). The kernel
multiplies fp16 probabilities (relative rounding 2^-11) into V, which that
bound covers without an extra allowance."""
import types

import numpy as np
import pytest
import torch

from conftest import assert_close_bf16, bf16_bits, pkg_module, u8

pytestmark = pytest.mark.gpu


def _check(O, got, q, k, v, what, **kw):
    """got vs the float64 oracle on the same K/V and mask."""
    ref = O.attention_reference(q, k, v, **kw)
    if got.ndim == 2:
        ref = ref.reshape(got.shape)
    assert_close_bf16(got, ref, what=what)


def _cache_from_chunks(dev, n_chunks, chunk, H, D, seed, fmt="fp8", capacity=None):
    """Config-2 generator per chunk: N(0,1) x per-head gain U(0.5, 4), written
    chunk by chunk with the KV write kernel."""
    kvc = pkg_module("fp8_kv_cache")
    make = kvc.make_fp8_kv_block if fmt == "fp8" else kvc.make_int8_kv_block
    cap = capacity or n_chunks * chunk
    cache = make(1, cap, H, D, device=dev)
    for c in range(n_chunks):
        g = torch.Generator(device=dev).manual_seed(seed + c)
        gain = torch.empty(H, device=dev).uniform_(0.5, 4.0, generator=g)
        k = (torch.randn(1, chunk, H, D, device=dev, generator=g) * gain[None, None, :, None]).to(torch.bfloat16)
        v = (torch.randn(1, chunk, H, D, device=dev, generator=g) * gain[None, None, :, None]).to(torch.bfloat16)
        kvc.quantize_kv_pair_into(cache, k, v, c * chunk)
    return cache


def _dequant(O, cache, n, fmt="fp8"):
    """The K/V the reference attends over: bf16(code * scale), the decode of
    int8_kv_cache.py:88,204 feeding the attention at nomas_cpt.py:530-531."""
    f = O.KV_FP8 if fmt == "fp8" else O.KV_INT8
    k = O.bf16_bits_to_f32(O.kv_dequantize(u8(cache["k"][0, :n]), cache["k_scale"][0, :n].cpu().numpy(), f))
    v = O.bf16_bits_to_f32(O.kv_dequantize(u8(cache["v"][0, :n]), cache["v_scale"][0, :n].cpu().numpy(), f))
    return k, v


def _q(dev, Lq, H, D, seed):
    g = torch.Generator(device=dev).manual_seed(seed)
    return torch.randn(1, Lq, H, D, device=dev, generator=g).to(torch.bfloat16)


@pytest.mark.parametrize("Lq,n_chunks,chunk,q_chunk0,fmt", [
    (200, 3, 150, 1, "fp8"),       # Q spans chunks 1-2: partial tiles + the causal triangle
    (128, 2, 128, 1, "fp8"),       # tile-aligned, Q is the last chunk: dense
    (37, 4, 37, 3, "fp8"),         # tiny ragged chunk
    (300, 3, 100, 0, "int8"),      # INT8-compat cache, Q over chunks 0-2
])
def test_chunk_attention_small(O, dev, Lq, n_chunks, chunk, q_chunk0, fmt):
    print(f"case attn Lq={Lq} chunks={n_chunks}x{chunk} q0={q_chunk0} {fmt}", flush=True)
    ca = pkg_module("cache_attention")
    H, D = 3, 128
    cache = _cache_from_chunks(dev, n_chunks, chunk, H, D, 100 + Lq, fmt)
    kv_len = n_chunks * chunk
    q = _q(dev, Lq, H, D, Lq)
    q_pos0 = q_chunk0 * chunk
    out = ca.chunk_attention(q, cache, kv_len, q_pos0=q_pos0, chunk_len=chunk)
    kh, vh = _dequant(O, cache, kv_len, fmt)
    vis = O.block_causal_visible(np.arange(q_pos0, q_pos0 + Lq), np.arange(kv_len), chunk)
    _check(O, out[0].float().cpu().numpy(), O.bf16_bits_to_f32(bf16_bits(q[0])), kh, vh, "chunk attention",
           visible=vis)


def test_chunk_attention_with_bf16_tail(O, dev):
    """Denoising-pass form: FP8 history + the current chunk's bf16 K/V, full visibility."""
    ca = pkg_module("cache_attention")
    H, D, chunk = 2, 128, 160
    cache = _cache_from_chunks(dev, 2, chunk, H, D, 7)
    g = torch.Generator(device=dev).manual_seed(9)
    kc = (torch.randn(1, chunk, H, D, device=dev, generator=g) * 2).to(torch.bfloat16)
    vc = (torch.randn(1, chunk, H, D, device=dev, generator=g) * 2).to(torch.bfloat16)
    q = _q(dev, chunk, H, D, 3)
    out = ca.chunk_attention(q, cache, 2 * chunk, k_cur=kc, v_cur=vc)
    kh, vh = _dequant(O, cache, 2 * chunk)
    kall = np.concatenate([kh, O.bf16_bits_to_f32(bf16_bits(kc[0]))], 0)
    vall = np.concatenate([vh, O.bf16_bits_to_f32(bf16_bits(vc[0]))], 0)
    _check(O, out[0].float().cpu().numpy(), O.bf16_bits_to_f32(bf16_bits(q[0])), kall, vall, "attention + tail")
    # tail only (empty cache prefix)
    out2 = ca.chunk_attention(q, cache, 0, k_cur=kc, v_cur=vc)
    _check(O, out2[0].float().cpu().numpy(), O.bf16_bits_to_f32(bf16_bits(q[0])), kall[2 * chunk:],
           vall[2 * chunk:], "tail only")


def test_chunk_attention_config3_sampled_rows(O, dev):
    """Q [1, 10800, 24, 128] of the last chunk over an 8-chunk
    (86400-token) FP8 cache, scale 1/sqrt(128). 96 query rows checked, all heads."""
    print("case attn config3", flush=True)
    ca = pkg_module("cache_attention")
    H, D, chunk, n = 24, 128, 10800, 8
    cache = _cache_from_chunks(dev, n, chunk, H, D, 1000)
    q = _q(dev, chunk, H, D, 77)
    kv_len = n * chunk
    out = ca.chunk_attention(q, cache, kv_len, q_pos0=(n - 1) * chunk, chunk_len=chunk)
    torch.cuda.synchronize()
    assert torch.isfinite(out.float()).all()
    rows = np.concatenate([np.arange(0, 32), np.arange(5400, 5432), np.arange(10768, 10800)])
    kh, vh = _dequant(O, cache, kv_len)
    _check(O, out[0, rows].float().cpu().numpy(), O.bf16_bits_to_f32(bf16_bits(q[0, rows])), kh, vh, "config 3")


def test_chunk_attention_two_chunk_queries_triangle(O, dev):
    """Multi-chunk Q at config-3 geometry (2 chunks of 10800 over 3 cached chunks):
    rows on both sides of the chunk boundary."""
    ca = pkg_module("cache_attention")
    H, D, chunk = 2, 128, 10800
    cache = _cache_from_chunks(dev, 3, chunk, H, D, 55)
    q = _q(dev, 2 * chunk, H, D, 5)
    out = ca.chunk_attention(q, cache, 3 * chunk, q_pos0=chunk, chunk_len=chunk)
    rows = np.concatenate([np.arange(10780, 10820), np.arange(21560, 21600)])
    kh, vh = _dequant(O, cache, 3 * chunk)
    vis = O.block_causal_visible(chunk + rows, np.arange(3 * chunk), chunk)
    _check(O, out[0, rows].float().cpu().numpy(), O.bf16_bits_to_f32(bf16_bits(q[0, rows])), kh, vh, "triangle",
           visible=vis)


# The 8-wave workgroup shape (256 queries) takes the whole 256-query tiles of a
# launch once they fill every CU (B H floor(Lq / 256) >= 256 on MI355X); rows
# past the last whole tile go to the 4-wave shape in a second launch.

@pytest.mark.parametrize("fmt", ["fp8", "int8"])
def test_eight_wave_tiles_causal_triangle(O, dev, fmt):
    """H 128 x 2 whole tiles: every row on the 8-wave shape. Q covers chunks 1-3
    of a 4-chunk cache, so tiles straddle chunk boundaries (per-element mask)."""
    print(f"case attn 8-wave triangle {fmt}", flush=True)
    ca = pkg_module("cache_attention")
    H, D, chunk, n, Lq, q_pos0 = 128, 128, 200, 4, 512, 200
    cache = _cache_from_chunks(dev, n, chunk, H, D, 600, fmt)
    kv_len = n * chunk
    q = _q(dev, Lq, H, D, 61)
    out = ca.chunk_attention(q, cache, kv_len, q_pos0=q_pos0, chunk_len=chunk)
    kh, vh = _dequant(O, cache, kv_len, fmt)
    vis = O.block_causal_visible(np.arange(q_pos0, q_pos0 + Lq), np.arange(kv_len), chunk)
    _check(O, out[0].float().cpu().numpy(), O.bf16_bits_to_f32(bf16_bits(q[0])), kh, vh, "8-wave triangle",
           visible=vis)


def test_eight_wave_tiles_with_bf16_tail(O, dev):
    """Denoising-pass form on the 8-wave shape: 2 FP8 chunks + the current
    chunk's bf16 K/V (tail tiles copied into LDS by 512 threads)."""
    print("case attn 8-wave tail", flush=True)
    ca = pkg_module("cache_attention")
    H, D, chunk = 64, 128, 1024
    cache = _cache_from_chunks(dev, 2, chunk, H, D, 21)
    g = torch.Generator(device=dev).manual_seed(22)
    kc = (torch.randn(1, chunk, H, D, device=dev, generator=g) * 2).to(torch.bfloat16)
    vc = (torch.randn(1, chunk, H, D, device=dev, generator=g) * 2).to(torch.bfloat16)
    q = _q(dev, chunk, H, D, 23)
    out = ca.chunk_attention(q, cache, 2 * chunk, k_cur=kc, v_cur=vc)
    rows = np.arange(0, chunk, 3)
    kh, vh = _dequant(O, cache, 2 * chunk)
    kall = np.concatenate([kh, O.bf16_bits_to_f32(bf16_bits(kc[0]))], 0)
    vall = np.concatenate([vh, O.bf16_bits_to_f32(bf16_bits(vc[0]))], 0)
    _check(O, out[0, rows].float().cpu().numpy(), O.bf16_bits_to_f32(bf16_bits(q[0, rows])), kall, vall,
           "8-wave + tail")


def test_eight_wave_tiles_with_split_remainder(O, dev):
    """Lq 1100 = 4 whole 256-query tiles + 76 rows, H 64, 16384 keys: rows < 1024
    on the 8-wave shape, the last 76 on the 4-wave shape with the key range
    split (workspace + combine, offset into the output)."""
    print("case attn 8-wave + split remainder", flush=True)
    lib = pkg_module("_lib").load()
    H, D, chunk, n, Lq = 64, 128, 4096, 4, 1100
    kv_len = n * chunk
    ws = lib.hn_attn_fp8kv_workspace_size(1, Lq, H, D, kv_len, 0)
    assert 0 < ws <= 16 * H * (Lq - 1024) * (D + 2) * 4   # only the remainder rows are split
    ca = pkg_module("cache_attention")
    cache = _cache_from_chunks(dev, n, chunk, H, D, 31)
    q = _q(dev, Lq, H, D, 32)
    out = ca.chunk_attention(q, cache, kv_len, q_pos0=(n - 1) * chunk, chunk_len=chunk)
    rows = np.concatenate([np.arange(0, 16), np.arange(1000, 1100)])
    kh, vh = _dequant(O, cache, kv_len)
    _check(O, out[0, rows].float().cpu().numpy(), O.bf16_bits_to_f32(bf16_bits(q[0, rows])), kh, vh,
           "8-wave + split remainder")


@pytest.mark.parametrize("kv_len,cur_len", [(64, 0), (100, 0), (130, 0), (0, 40), (64, 100), (130, 70)])
def test_eight_wave_short_key_ranges(O, dev, kv_len, cur_len):
    """The 8-wave shape (H 128 x 2 whole tiles, every row on it) over 1-4 key
    tiles: ranges shorter than its three K/V stages, partial last tiles, and
    FP8 cache tiles followed by bf16 tail tiles; every key visible."""
    print(f"case attn 8-wave short kv={kv_len} cur={cur_len}", flush=True)
    ca = pkg_module("cache_attention")
    kvc = pkg_module("fp8_kv_cache")
    H, D, Lq = 128, 128, 512
    if kv_len:
        cache = _cache_from_chunks(dev, 1, kv_len, H, D, 40 + kv_len)
    else:
        cache = kvc.make_fp8_kv_block(1, 64, H, D, device=dev)
        for buf in cache.values():
            buf.view(torch.uint8).zero_()
    q = _q(dev, Lq, H, D, 41)
    kh, vh = _dequant(O, cache, kv_len)
    if cur_len:
        g = torch.Generator(device=dev).manual_seed(42)
        kc = (torch.randn(1, cur_len, H, D, device=dev, generator=g) * 2).to(torch.bfloat16)
        vc = (torch.randn(1, cur_len, H, D, device=dev, generator=g) * 2).to(torch.bfloat16)
        out = ca.chunk_attention(q, cache, kv_len, k_cur=kc, v_cur=vc)
        kh = np.concatenate([kh, O.bf16_bits_to_f32(bf16_bits(kc[0]))], 0)
        vh = np.concatenate([vh, O.bf16_bits_to_f32(bf16_bits(vc[0]))], 0)
    else:
        out = ca.chunk_attention(q, cache, kv_len)
    rows = np.arange(0, Lq, 3)
    _check(O, out[0, rows].float().cpu().numpy(), O.bf16_bits_to_f32(bf16_bits(q[0, rows])), kh, vh,
           "8-wave short range")


@pytest.mark.parametrize("Lq,kv_len,H", [(128, 86400, 24), (100, 20000, 4), (1, 5000, 2)])
def test_split_kv_decode_style(O, dev, Lq, kv_len, H):
    """Few queries over a long cache: the key range is split across workgroups
    (workspace + combine); rows checked against the oracle."""
    print(f"case split-kv Lq={Lq} kv={kv_len} H={H}", flush=True)
    lib = pkg_module("_lib").load()
    assert lib.hn_attn_fp8kv_workspace_size(1, Lq, H, 128, kv_len, 0) > 0
    ca = pkg_module("cache_attention")
    chunk = kv_len // 8 if kv_len % 8 == 0 else kv_len
    n = kv_len // chunk
    cache = _cache_from_chunks(dev, n, chunk, H, 128, 300 + Lq)
    q = _q(dev, Lq, H, 128, 11)
    out = ca.chunk_attention(q, cache, kv_len)
    rows = np.arange(0, Lq, max(1, Lq // 16))
    kh, vh = _dequant(O, cache, kv_len)
    _check(O, out[0, rows].float().cpu().numpy(), O.bf16_bits_to_f32(bf16_bits(q[0, rows])), kh, vh, "split-kv")


def test_attention_invariants(dev):
    """Constant V -> O = V; no visible key -> zeros."""
    kvc = pkg_module("fp8_kv_cache")
    ca = pkg_module("cache_attention")
    H, D, L = 2, 128, 300
    cache = kvc.make_fp8_kv_block(1, L, H, D, device=dev)
    k = torch.randn(1, L, H, D, device=dev).to(torch.bfloat16)
    vrow = torch.randn(1, 1, H, D, device=dev).to(torch.bfloat16)
    kvc.quantize_kv_pair_into(cache, k, vrow.expand(1, L, H, D).contiguous(), 0)
    q = torch.randn(1, 50, H, D, device=dev).to(torch.bfloat16)
    out = ca.chunk_attention(q, cache, L)
    vdq = kvc.dequantize_kv(cache, "v", 1)
    assert torch.allclose(out.float(), vdq.float().expand(1, 50, H, D), atol=2e-2, rtol=0)
    empty = ca.chunk_attention(q, cache, 0)
    assert (empty == 0).all()


def test_attention_is_deterministic(dev):
    ca = pkg_module("cache_attention")
    cache = _cache_from_chunks(dev, 2, 500, 4, 128, 3)
    q = _q(dev, 500, 4, 128, 1)
    a = ca.chunk_attention(q, cache, 1000, q_pos0=500, chunk_len=500)
    b = ca.chunk_attention(q, cache, 1000, q_pos0=500, chunk_len=500)
    assert torch.equal(a, b)


def test_causal_attention_with_cache_mp_matches_reference_semantics(O, dev):
    """The cached-attention entry point (update and denoise passes) against the
    reference composition [decoded history | current img + txt] (nomas_cpt.py:614-625)."""
    ca = pkg_module("cache_attention")
    kvc = pkg_module("fp8_kv_cache")
    H, D, Li, Lt = 2, 128, 96, 16
    cache = kvc.make_fp8_kv_block(1, 400, H, D, device=dev)
    mask = torch.zeros(1, 400, dtype=torch.bool, device=dev)
    valid = 0
    g = torch.Generator(device=dev).manual_seed(4)

    def rnd(L):
        return torch.randn(1, L, H, D, device=dev, generator=g).to(torch.bfloat16)

    for step, update in enumerate([True, False, True]):
        q, k, v = (rnd(Li), rnd(Lt)), (rnd(Li), rnd(Lt)), (rnd(Li), rnd(Lt))
        hist_k, hist_v = _dequant(O, cache, valid)
        with torch.no_grad():
            img, txt = ca.causal_attention_with_cache_mp(q, k, v, cache, valid, "flash3", None,
                                                         update, True, mask)
        cur_k = np.concatenate([O.bf16_bits_to_f32(bf16_bits(t[0])) for t in k], 0)
        cur_v = np.concatenate([O.bf16_bits_to_f32(bf16_bits(t[0])) for t in v], 0)
        kall = np.concatenate([hist_k, cur_k], 0)
        vall = np.concatenate([hist_v, cur_v], 0)
        qall = np.concatenate([O.bf16_bits_to_f32(bf16_bits(t[0])) for t in q], 0)
        got = torch.cat([img[0], txt[0]], 0).float().cpu().numpy()
        assert img.shape == (1, Li, H * D) and txt.shape == (1, Lt, H * D)
        _check(O, got, qall, kall, vall, f"cached attention step {step}")
        if update:
            assert mask[0, valid:valid + Li + Lt].all()
            valid += Li + Lt


# ---------------------------------------------------------------------------
# Key validity (padded text, holes in the cached history) and the read-only
# history broadcast of CFG branches.

def _tail(dev, B, L, H, seed, gain=2.0):
    g = torch.Generator(device=dev).manual_seed(seed)
    k = (torch.randn(B, L, H, 128, device=dev, generator=g) * gain).to(torch.bfloat16)
    v = (torch.randn(B, L, H, 128, device=dev, generator=g) * gain).to(torch.bfloat16)
    return k, v


@pytest.mark.parametrize("H,Lq,chunk,n,cur,fmt", [
    (3, 200, 300, 2, 90, "fp8"),       # 4-wave shape
    (128, 512, 300, 2, 90, "fp8"),     # 8-wave shape (H 128 x 2 whole 256-query tiles)
    (3, 150, 200, 3, 0, "int8"),       # INT8 cache, no tail
    (4, 100, 5000, 4, 40, "fp8"),      # few queries, long cache: split key ranges + combine
])
def test_key_validity_masks(O, dev, H, Lq, chunk, n, cur, fmt):
    """cache_valid holes (random, plus one wholly masked tile) and padded tail
    keys drop out of the softmax; checked against the oracle with key_valid."""
    print(f"case attn masks H={H} Lq={Lq} kv={n}x{chunk} cur={cur} {fmt}", flush=True)
    ca = pkg_module("cache_attention")
    D = 128
    cache = _cache_from_chunks(dev, n, chunk, H, D, 900 + H, fmt)
    kv_len = n * chunk
    g = torch.Generator(device=dev).manual_seed(3)
    cache_valid = torch.rand(1, kv_len + 17, generator=g, device=dev) > 0.3   # longer than kv_len
    cache_valid[0, 64:128] = False
    q = _q(dev, Lq, H, D, 5)
    kh, vh = _dequant(O, cache, kv_len, fmt)
    key_valid = cache_valid[0, :kv_len].cpu().numpy()
    if cur:
        kc, vc = _tail(dev, 1, cur, H, 6)
        cur_valid = torch.ones(1, cur, dtype=torch.bool, device=dev)
        cur_valid[0, cur - 20:] = False
        out = ca.chunk_attention(q, cache, kv_len, k_cur=kc, v_cur=vc, cache_valid=cache_valid,
                                 cur_valid=cur_valid)
        kh = np.concatenate([kh, O.bf16_bits_to_f32(bf16_bits(kc[0]))], 0)
        vh = np.concatenate([vh, O.bf16_bits_to_f32(bf16_bits(vc[0]))], 0)
        key_valid = np.concatenate([key_valid, cur_valid[0].cpu().numpy()])
    else:
        out = ca.chunk_attention(q, cache, kv_len, cache_valid=cache_valid)
    rows = np.arange(0, Lq, 3)
    _check(O, out[0, rows].float().cpu().numpy(), O.bf16_bits_to_f32(bf16_bits(q[0, rows])), kh, vh,
           "key masks", key_valid=key_valid)


def test_masks_with_block_causal_chunks(O, dev):
    """Key masks together with the chunk-granular causal mask (Q over chunks 1-2)."""
    ca = pkg_module("cache_attention")
    H, D, chunk = 2, 128, 150
    cache = _cache_from_chunks(dev, 3, chunk, H, D, 31)
    kv_len = 3 * chunk
    valid = torch.ones(1, kv_len, dtype=torch.bool, device=dev)
    valid[0, 10:40] = False
    valid[0, 200:260] = False
    q = _q(dev, 2 * chunk, H, D, 8)
    out = ca.chunk_attention(q, cache, kv_len, q_pos0=chunk, chunk_len=chunk, cache_valid=valid)
    kh, vh = _dequant(O, cache, kv_len)
    vis = O.block_causal_visible(np.arange(chunk, 3 * chunk), np.arange(kv_len), chunk)
    _check(O, out[0].float().cpu().numpy(), O.bf16_bits_to_f32(bf16_bits(q[0])), kh, vh,
           "masks + block-causal", visible=vis, key_valid=valid[0].cpu().numpy())


@pytest.mark.parametrize("H,Lq", [(3, 100), (128, 512)])
def test_fully_masked_rows_are_zero(dev, H, Lq):
    """A query that sees no valid key gets a zero row (range_attention.py:212-239)."""
    ca = pkg_module("cache_attention")
    cache = _cache_from_chunks(dev, 1, 300, H, 128, 4)
    q = _q(dev, Lq, H, 128, 2)
    none = torch.zeros(1, 300, dtype=torch.bool, device=dev)
    out = ca.chunk_attention(q, cache, 300, cache_valid=none)
    assert (out == 0).all()
    kc, vc = _tail(dev, 1, 64, H, 9)
    out = ca.chunk_attention(q, cache, 300, k_cur=kc, v_cur=vc, cache_valid=none,
                             cur_valid=torch.zeros(1, 64, dtype=torch.bool, device=dev))
    assert (out == 0).all()


@pytest.mark.parametrize("H,Lq", [(2, 120), (64, 512)])
def test_cfg_history_broadcast(O, dev, H, Lq):
    """One canonical history slot read by B = 2 query batches (nomas_cpt.py:547-567),
    with a batch-1 history mask and per-batch tail masks."""
    print(f"case attn cfg broadcast H={H} Lq={Lq}", flush=True)
    ca = pkg_module("cache_attention")
    D, kv_len, cur, B = 128, 700, 80, 2
    cache = _cache_from_chunks(dev, 1, kv_len, H, D, 12)
    hist_valid = torch.ones(1, kv_len, dtype=torch.bool, device=dev)
    hist_valid[0, 300:380] = False
    kc, vc = _tail(dev, B, cur, H, 13)
    cur_valid = torch.ones(B, cur, dtype=torch.bool, device=dev)
    cur_valid[1, 50:] = False
    g = torch.Generator(device=dev).manual_seed(14)
    q = torch.randn(B, Lq, H, D, device=dev, generator=g).to(torch.bfloat16)
    out = ca.chunk_attention(q, cache, kv_len, k_cur=kc, v_cur=vc, cache_valid=hist_valid,
                             cur_valid=cur_valid)
    kh, vh = _dequant(O, cache, kv_len)
    rows = np.arange(0, Lq, 4)
    for b in range(B):
        kall = np.concatenate([kh, O.bf16_bits_to_f32(bf16_bits(kc[b]))], 0)
        vall = np.concatenate([vh, O.bf16_bits_to_f32(bf16_bits(vc[b]))], 0)
        kv = np.concatenate([hist_valid[0].cpu().numpy(), cur_valid[b].cpu().numpy()])
        _check(O, out[b, rows].float().cpu().numpy(), O.bf16_bits_to_f32(bf16_bits(q[b, rows])), kall,
               vall, f"CFG broadcast batch {b}", key_valid=kv)


# ---------------------------------------------------------------------------
# The attention seam: FP8CacheAttention installed over a stand-in of the
# reference's module, driven through update and denoise passes with padded
# text, against a restatement of the reference's key and mask composition for
# quantized storage (nomas_cpt.py:464-685, attended at :782-829).

def _reference_cached_attention(O, q, k, v, hist, hist_mask, text_mask, update, cache_txt,
                                cache_mask_given, attn_mode="flash3"):
    """float64 outputs [B, Li + Lt, H, D] of nomas_cpt.causal_attention_with_cache_mp
    for an INT8/FP8 cache whose decoded history is hist = (K, V) [Lh, H, D]
    (one slot, shared by every batch) with validity hist_mask [Lh]."""
    img_q, txt_q = (O.bf16_bits_to_f32(bf16_bits(t)) for t in q)
    img_k, txt_k = (O.bf16_bits_to_f32(bf16_bits(t)) for t in k)
    img_v, txt_v = (O.bf16_bits_to_f32(bf16_bits(t)) for t in v)
    B, Li = img_q.shape[:2]
    Lt = txt_q.shape[1]
    txt_mask = np.ones((B, Lt), bool) if text_mask is None else text_mask.cpu().numpy().astype(bool)
    outs = []
    for b in range(B):
        keys = [hist[0], img_k[b]]
        vals = [hist[1], img_v[b]]
        if cache_txt or update:               # history | cur (img + txt)
            keys.append(txt_k[b])
            vals.append(txt_v[b])
        hmask = hist_mask if cache_mask_given else np.ones(hist[0].shape[0], bool)
        if update and cache_txt:
            # kv_mask = cache_mask[:, :total] after the write, or all ones without one
            kv = (np.concatenate([hmask, np.ones(Li, bool), txt_mask[b]]) if cache_mask_given
                  else np.ones(hist[0].shape[0] + Li + Lt, bool))
        elif update:
            kv = np.concatenate([hmask, np.ones(Li, bool), txt_mask[b]])
        elif cache_txt:
            kv = np.concatenate([hmask, np.ones(Li, bool), txt_mask[b]])
        else:
            kv = np.concatenate([hmask, np.ones(Li, bool)])
        qf = np.concatenate([img_q[b], txt_q[b]], 0)
        o = O.attention_reference(qf, np.concatenate(keys, 0), np.concatenate(vals, 0), key_valid=kv)
        if attn_mode != "torch":
            o[Li:][~txt_mask[b]] = 0.0        # padded query rows stay zero
        outs.append(o)
    return np.stack(outs)


def _stand_in_native():
    calls = []

    def native(*args, **kwargs):
        calls.append(args)
        return "native"
    return types.SimpleNamespace(causal_attention_with_cache_mp=native), calls


@pytest.mark.parametrize("fmt", ["fp8", "int8"])
def test_installed_seam_update_and_denoise_with_padded_text(O, dev, fmt):
    print(f"case attn seam {fmt}", flush=True)
    ca = pkg_module("cache_attention")
    kvc = pkg_module("fp8_kv_cache")
    native, calls = _stand_in_native()
    hook = ca.FP8CacheAttention(native)
    assert native.causal_attention_with_cache_mp is hook
    H, D, Li, Lt, cap = 2, 128, 96, 24, 1000
    make = kvc.make_fp8_kv_block if fmt == "fp8" else kvc.make_int8_kv_block
    cache = make(1, cap, H, D, device=dev)
    cache_mask = torch.zeros(1, cap, dtype=torch.bool, device=dev)
    g = torch.Generator(device=dev).manual_seed(21)

    def rnd(B, L):
        return torch.randn(B, L, H, D, device=dev, generator=g).to(torch.bfloat16)

    text_mask = torch.ones(1, Lt, dtype=torch.bool, device=dev)
    text_mask[0, Lt - 7:] = False
    valid = 0
    # (update, cache_txt): a segment's first chunk (write img + txt, then
    # denoise the next chunk with its text), then a later chunk of the
    # segment (write img only, denoise without text)
    for step, (update, cache_txt) in enumerate([(True, True), (False, True), (True, False),
                                                (False, False), (True, True)]):
        q, k, v = (rnd(1, Li), rnd(1, Lt)), (rnd(1, Li), rnd(1, Lt)), (rnd(1, Li), rnd(1, Lt))
        hist = _dequant(O, cache, valid, fmt)
        hist_mask = cache_mask[0, :valid].cpu().numpy()
        ref = _reference_cached_attention(O, q, k, v, hist, hist_mask, text_mask, update, cache_txt, True)
        with torch.no_grad():
            img, txt = native.causal_attention_with_cache_mp(q, k, v, cache, valid, "flash3", text_mask,
                                                             update, cache_txt, cache_mask)
        assert img.shape == (1, Li, H * D) and txt.shape == (1, Lt, H * D)
        got = torch.cat([img[0], txt[0]], 0).float().cpu().numpy().reshape(Li + Lt, H, D)
        assert_close_bf16(got, ref[0], what=f"seam step {step}")
        assert (txt[0].reshape(Lt, H, D)[Lt - 7:] == 0).all(), "padded query rows must be zero"
        if update:
            n = Li + (Lt if cache_txt else 0)
            want = np.concatenate([np.ones(Li, bool), text_mask[0].cpu().numpy()]) if cache_txt else np.ones(Li, bool)
            assert np.array_equal(cache_mask[0, valid:valid + n].cpu().numpy(), want)
            valid += n
    assert not calls and hook.stats["calls"] == 5 and hook.stats["fallbacks"] == 0
    hook.uninstall()
    assert native.causal_attention_with_cache_mp is not hook


def test_installed_seam_cfg_broadcast_and_no_mask_quirk(O, dev):
    """Denoise passes of B = 2 CFG branches over one history slot (with
    per-branch text masks), and a write without a cache_mask, where the
    reference attends every current key, padded text included."""
    ca = pkg_module("cache_attention")
    kvc = pkg_module("fp8_kv_cache")
    native, calls = _stand_in_native()
    hook = ca.FP8CacheAttention(native)
    H, D, Li, Lt = 2, 128, 64, 32
    cache = kvc.make_fp8_kv_block(1, 600, H, D, device=dev)
    g = torch.Generator(device=dev).manual_seed(33)

    def rnd(B, L):
        return torch.randn(B, L, H, D, device=dev, generator=g).to(torch.bfloat16)

    tm1 = torch.ones(1, Lt, dtype=torch.bool, device=dev)
    tm1[0, 20:] = False
    q, k, v = (rnd(1, Li), rnd(1, Lt)), (rnd(1, Li), rnd(1, Lt)), (rnd(1, Li), rnd(1, Lt))
    ref = _reference_cached_attention(O, q, k, v, _dequant(O, cache, 0), np.ones(0, bool), tm1, True,
                                      True, False)
    with torch.no_grad():
        img, txt = native.causal_attention_with_cache_mp(q, k, v, cache, 0, "flash3", tm1, True, True, None)
    got = torch.cat([img[0], txt[0]], 0).float().cpu().numpy().reshape(Li + Lt, H, D)
    assert_close_bf16(got, ref[0], what="write without cache_mask")
    valid = Li + Lt
    tm2 = torch.ones(2, Lt, dtype=torch.bool, device=dev)
    tm2[0, 25:] = False
    tm2[1, 10:] = False
    cmask = torch.ones(1, 600, dtype=torch.bool, device=dev)
    cmask[0, Li + 20:valid] = False
    q, k, v = (rnd(2, Li), rnd(2, Lt)), (rnd(2, Li), rnd(2, Lt)), (rnd(2, Li), rnd(2, Lt))
    ref = _reference_cached_attention(O, q, k, v, _dequant(O, cache, valid), cmask[0, :valid].cpu().numpy(),
                                      tm2, False, True, True)
    with torch.no_grad():
        img, txt = native.causal_attention_with_cache_mp(q, k, v, cache, valid, "flash3", tm2, False, True,
                                                         cmask)
    got = torch.cat([img, txt], 1).float().cpu().numpy().reshape(2, Li + Lt, H, D)
    for b in range(2):
        assert_close_bf16(got[b], ref[b], what=f"CFG branch {b}")
    # a write cannot broadcast (one history slot, two branches)
    with pytest.raises(ValueError, match="batch mismatch during update"):
        with torch.no_grad():
            native.causal_attention_with_cache_mp(q, k, v, cache, valid, "flash3", tm2, True, True, cmask)
    assert not calls
    hook.uninstall()


def test_installed_seam_fallback_rules(dev):
    """Calls outside the HIP path: an INT8 cache goes to the native function
    (which decodes INT8); an FP8 cache raises (the native code cannot read it)."""
    ca = pkg_module("cache_attention")
    kvc = pkg_module("fp8_kv_cache")
    native, calls = _stand_in_native()
    hook = ca.FP8CacheAttention(native)
    H, D = 2, 128
    q = (torch.zeros(1, 8, H, D, dtype=torch.bfloat16, device=dev),
         torch.zeros(1, 4, H, D, dtype=torch.bfloat16, device=dev))
    sparse = {"config": {"dense_first_n_layers": 1}, "layer": 5}
    i8 = kvc.make_int8_kv_block(1, 64, H, D, device=dev)
    with torch.no_grad():
        assert native.causal_attention_with_cache_mp(q, q, q, i8, 0, "flash3", None, False, True, None,
                                                     None, None, 0, "magi", sparse) == "native"
    assert len(calls) == 1 and hook.stats["fallbacks"] == 1
    f8 = kvc.make_fp8_kv_block(1, 64, H, D, device=dev)
    with pytest.raises(RuntimeError, match="FP8 KV cache call not covered"):
        with torch.no_grad():
            native.causal_attention_with_cache_mp(q, q, q, f8, 0, "flash3", None, False, True, None,
                                                  None, None, 0, "magi", sparse)
    # a permanently dense first layer of a sparse context is plain attention
    dense = {"config": {"dense_first_n_layers": 2}, "layer": 0}
    with torch.no_grad():
        native.causal_attention_with_cache_mp(q, q, q, f8, 0, "flash3", None, False, True, None,
                                              None, None, 0, "magi", dense)
    assert f8["dense_layer_stats"] == {"denoise": 1, "write": 0}
    hook.uninstall()


def test_installed_seam_torch_mode_keeps_padded_query_rows(O, dev):
    """attn_mode "torch": the reference's SDPA branch (nomas_cpt.py:771-781)
    passes kv_mask as the attention mask for quantized storage and does not
    zero padded query rows, so a padded text query keeps its attention over
    the valid keys."""
    ca = pkg_module("cache_attention")
    kvc = pkg_module("fp8_kv_cache")
    native, calls = _stand_in_native()
    hook = ca.FP8CacheAttention(native)
    H, D, Li, Lt = 2, 128, 80, 24
    cache = _cache_from_chunks(dev, 2, 100, H, D, seed=41, capacity=600)
    valid = 200
    cmask = torch.ones(1, 600, dtype=torch.bool, device=dev)
    cmask[0, 130:150] = False
    g = torch.Generator(device=dev).manual_seed(42)

    def rnd(B, L):
        return torch.randn(B, L, H, D, device=dev, generator=g).to(torch.bfloat16)

    tm = torch.ones(1, Lt, dtype=torch.bool, device=dev)
    tm[0, 15:] = False
    for update, cache_txt in ((False, True), (True, False)):
        q, k, v = (rnd(1, Li), rnd(1, Lt)), (rnd(1, Li), rnd(1, Lt)), (rnd(1, Li), rnd(1, Lt))
        ref = _reference_cached_attention(O, q, k, v, _dequant(O, cache, valid),
                                          cmask[0, :valid].cpu().numpy(), tm, update, cache_txt, True,
                                          attn_mode="torch")
        with torch.no_grad():
            img, txt = native.causal_attention_with_cache_mp(q, k, v, cache, valid, "torch", tm, update,
                                                             cache_txt, cmask)
        got = torch.cat([img[0], txt[0]], 0).float().cpu().numpy().reshape(Li + Lt, H, D)
        assert_close_bf16(got, ref[0], what=f"torch mode update={update}")
        assert (txt[0].reshape(Lt, H, D)[15:].abs().sum() > 0), "padded rows keep SDPA's values"
        if update:
            valid += Li
    assert not calls
    hook.uninstall()


def test_pipeline_fp8_storage_write_and_audit(O, dev):
    """The stand-in AR pipeline (tests/standin_pipeline.py) with the FP8
    storage binding and the attention seam installed: it selects
    kv_cache_quantization fp8, allocates FP8 blocks on the GPU, writes a
    chunk through an update pass (codes and scales bit-exact), grows its
    capacity, and audits its caches with the keys causal_ar.py:3365-3374
    reads."""
    from standin_pipeline import args_for, make_reference
    st = pkg_module("kv_cache_storage")
    ca = pkg_module("cache_attention")
    storage, int8_kv, Pipeline = make_reference()
    native, calls = _stand_in_native()
    store_hook = st.install_fp8_kv_storage(storage, pipeline_cls=Pipeline, int8_kv_module=int8_kv)
    attn_hook = ca.FP8CacheAttention(native)
    try:
        H, D, Li, Lt = 2, 128, 96, 32
        pipe = Pipeline(args_for("fp8"), hidden_size=H * D, heads_num=H, num_double_blocks=2)
        pipe._initialize_kv_cache(1, Li + Lt, torch.bfloat16, dev)
        g = torch.Generator(device=dev).manual_seed(5)

        def rnd(L, s):
            return (torch.randn(1, L, H, D, device=dev, generator=g) * s).to(torch.bfloat16)

        tm = torch.ones(1, Lt, dtype=torch.bool, device=dev)
        tm[0, 28:] = False
        for layer, cache in enumerate(pipe.kv_cache):
            q, k, v = (rnd(Li, 1), rnd(Lt, 1)), (rnd(Li, 2), rnd(Lt, 2)), (rnd(Li, 3), rnd(Lt, 3))
            with torch.no_grad():
                native.causal_attention_with_cache_mp(q, k, v, cache, pipe.cache_valid_len, "flash3", tm,
                                                      True, True, pipe.cache_mask_list[layer])
            for name, cur in (("k", k), ("v", v)):
                x = torch.cat(cur, 1)
                qo, so = O.kv_quantize(bf16_bits(x))
                assert np.array_equal(u8(cache[name][:, :Li + Lt]), qo), f"layer {layer} {name} codes"
                assert np.array_equal(cache[name + "_scale"][:, :Li + Lt].cpu().numpy().view(np.uint32),
                                      so.view(np.uint32)), f"layer {layer} {name} scales"
            want = np.concatenate([np.ones(Li, bool), tm[0].cpu().numpy()])
            assert np.array_equal(pipe.cache_mask_list[layer][0].cpu().numpy(), want)
        pipe.cache_valid_len += Li + Lt
        before = [u8(c["k"]).copy() for c in pipe.kv_cache]
        pipe._ensure_kv_cache_capacity(400)
        for c, b in zip(pipe.kv_cache, before):
            assert c["k"].dtype == torch.float8_e4m3fn and c["k"].shape[1] == 400
            assert np.array_equal(u8(c["k"][:, :Li + Lt]), b)
        audit = pipe.storage_audit()
        assert audit["kv_storage_format"] == "fp8" and audit["int8_kv"] is False
        per_layer = 2 * 400 * H * D + 2 * 400 * H * 4
        assert audit["gpu_kv_storage_bytes"] == 2 * per_layer
        assert audit["gpu_kv_peak_working_bytes_upper_bound"] == 2 * per_layer
        assert audit["codec_stats"] == [{}, {}]
        assert not calls and attn_hook.stats["calls"] == 2
    finally:
        attn_hook.uninstall()
        store_hook.uninstall()


def test_v_beyond_fp16_range_enters_as_65504(O, dev):
    """The documented range of the PV product: V is held as fp16, converted
    toward zero, so cached or tail V values past 65504 in magnitude enter as
    +-65504 (include/hynomas_fp8.h, hn_attn_fp8kv); everything else is the
    reference's bf16 value. Checked against the oracle with V clipped there,
    and shown to differ from attention over the unclipped values."""
    kvc = pkg_module("fp8_kv_cache")
    ca = pkg_module("cache_attention")
    H, D, n, Lc, Lq = 2, 128, 64, 40, 32
    g = torch.Generator(device=dev).manual_seed(77)
    k = torch.randn(1, n, H, D, device=dev, generator=g).to(torch.bfloat16)
    v = torch.randn(1, n, H, D, device=dev, generator=g)
    v[0, 5, 0, :8] = 1.0e5                       # a cached row holding values past fp16's range
    v[0, 9, 1, 3] = -9.0e4
    cache = kvc.make_fp8_kv_block(1, n, H, D, device=dev)
    kvc.quantize_kv_pair_into(cache, k, v.to(torch.bfloat16), 0)
    kc = torch.randn(1, Lc, H, D, device=dev, generator=g).to(torch.bfloat16)
    vc = torch.randn(1, Lc, H, D, device=dev, generator=g)
    vc[0, 3, :, 10:20] = 7.0e4                   # and tail values
    vc = vc.to(torch.bfloat16)
    q = (torch.randn(1, Lq, H, D, device=dev, generator=g) * 3).to(torch.bfloat16)
    out = ca.chunk_attention(q, cache, n, k_cur=kc, v_cur=vc)
    kh, vh = _dequant(O, cache, n)
    kall = np.concatenate([kh, O.bf16_bits_to_f32(bf16_bits(kc[0]))], 0)
    vall = np.concatenate([vh, O.bf16_bits_to_f32(bf16_bits(vc[0]))], 0)
    assert np.abs(vall).max() > 65504.0
    qf = O.bf16_bits_to_f32(bf16_bits(q[0]))
    got = out[0].float().cpu().numpy()
    ref = O.attention_reference(qf, kall, np.clip(vall, -65504.0, 65504.0))
    assert_close_bf16(got, ref, what="V clipped at 65504")
    unclipped = O.attention_reference(qf, kall, vall)
    assert np.abs(unclipped - got).max() > 1.0


@pytest.mark.parametrize("B,H,Lq,n_chunks,chunk,cur,holes", [
    (2, 128, 300, 2, 512, 64, True),    # 8-wave rows 0-255 + split 4-wave rows 256-299, masks, tail
    (1, 24, 128, 16, 512, 0, False),    # decode style: key splits and the merge kernel
    (1, 3, 37, 3, 100, 37, False),      # small 4-wave launch with a tail
])
def test_attention_writes_nothing_outside_out(dev, B, H, Lq, n_chunks, chunk, cur, holes):
    """The output written into a view of a larger buffer (64 guard rows past
    Lq and one guard head per row): the view equals the contiguous result of
    the same call and every guard element keeps its fill, for each launch
    shape (8-wave tiles with the split remainder, key splits with the merge,
    the plain 4-wave launch)."""
    print(f"case attn guard band B={B} H={H} Lq={Lq} keys={n_chunks}x{chunk} cur={cur}", flush=True)
    ops, L = pkg_module("ops"), pkg_module("_lib")
    D = 128
    cache = _cache_from_chunks(dev, n_chunks, chunk, H, D, 900 + Lq)
    kv_len = n_chunks * chunk
    g = torch.Generator(device=dev).manual_seed(Lq + H)
    q = torch.randn(B, Lq, H, D, device=dev, generator=g).to(torch.bfloat16)
    k_cur = v_cur = None
    if cur:
        k_cur = torch.randn(B, cur, H, D, device=dev, generator=g).to(torch.bfloat16)
        v_cur = torch.randn(B, cur, H, D, device=dev, generator=g).to(torch.bfloat16)
    cache_valid = None
    if holes:
        cache_valid = torch.rand(B, kv_len, device=dev, generator=g) > 0.1
    ref = ops.attn_fp8kv(q, cache["k"], cache["v"], cache["k_scale"], cache["v_scale"], kv_len,
                         k_cur, v_cur, 0, 0, None, cache_valid, None)
    buf = torch.full((B, Lq + 64, H + 1, D), 5.0, dtype=torch.bfloat16, device=dev)
    out = buf[:, :Lq, :H, :]
    kc, vc = cache["k"].expand(B, -1, -1, -1), cache["v"].expand(B, -1, -1, -1)
    ksc, vsc = cache["k_scale"].expand(B, -1, -1, -1), cache["v_scale"].expand(B, -1, -1, -1)
    kvb = None if cache_valid is None else cache_valid.to(torch.uint8).contiguous()
    lib = L.load()
    ws_bytes = lib.hn_attn_fp8kv_workspace_size(B, Lq, H, D, kv_len, cur)
    ws = torch.empty((ws_bytes,), dtype=torch.uint8, device=dev) if ws_bytes else None
    L.check(lib.hn_attn_fp8kv(
        L.HN_KV_FP8, q.data_ptr(), L.strides(q), B, Lq, H, D,
        kc.data_ptr(), vc.data_ptr(), L.strides(kc), ksc.data_ptr(), vsc.data_ptr(), L.strides(ksc),
        cache["k"].shape[1], kv_len, L.ptr(kvb), 0 if kvb is None else kvb.stride(0),
        None if not cur else k_cur.data_ptr(), None if not cur else v_cur.data_ptr(),
        L.strides(k_cur) if cur else None, cur, None, 0, 0, 0, float(D) ** -0.5,
        out.data_ptr(), L.strides(out), None if ws is None else ws.data_ptr(), ws_bytes,
        torch.cuda.current_stream().cuda_stream), "hn_attn_fp8kv")
    assert torch.equal(out, ref)
    assert bool((buf[:, Lq:] == 5.0).all()) and bool((buf[:, :, H:] == 5.0).all())
