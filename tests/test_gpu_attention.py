"""GPU parity of the FP8-KV chunk attention against the oracle's float64
softmax(Q K^T / sqrt(D)) V over the K, V the reference attends over: the
cache decoded to bf16(code * scale). Bar: max-abs 2e-2 and rel-L2 1e-2.

Like the reference's flash attention, the kernel multiplies probabilities
rounded to bf16 into V (|bf16(p) - p| <= 2^-8 p), so an output element may
differ from the exact-softmax oracle by up to 2^-8 * sum_k p_k |v_k| / l. The
elementwise bound adds that term, computed by the oracle from the same softmax
weights applied to |V| (P_ROUND * envelope); the rel-L2 bar is unchanged."""
import numpy as np
import pytest
import torch

from conftest import assert_close_bf16, bf16_bits, pkg_module, u8

pytestmark = pytest.mark.gpu

P_ROUND = 2.0 ** -8   # relative rounding of a probability to bf16


def _check(O, got, q, k, v, what, **kw):
    """got vs the oracle, with the bf16-probability allowance described above."""
    ref = O.attention_reference(q, k, v, **kw)
    env = O.attention_reference(q, k, np.abs(v), **kw)
    if got.ndim == 2:
        ref, env = ref.reshape(got.shape), env.reshape(got.shape)
    assert_close_bf16(got, ref, what=what, extra=P_ROUND * env)


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
