"""Fused QK RMSNorm + RoPE (+ KV cache write), hn_qk_norm_rope_kv, against a
CPU restatement of the reference's op sequence
(hymm/models/dit/modules/nomas_compile_prepost.py:18-27,49-54) on the same
bf16 inputs, and its cache write against the oracle applied to the kernel's
own rotated K and to V.

The kernel rounds at the reference's points (bf16 after the normalisation,
after the weight, after RoPE); the only arithmetic it does not order the same
way is the fp32 sum of squares (a 16-lane tree instead of the CPU's vector
loop), which can move the fp32 inverse RMS by an ulp and so flip the bf16
rounding of a normalised value y by one ulp. RoPE then carries that step,
times |cos| + |sin| <= sqrt 2, into the outputs of that row, even where
y0 cos - y1 sin nearly cancels and the output itself is tiny. Bar: in each
row, |got - ref| <= 2 ulp_bf16(max |y| of the row) (the carried step plus the
output's own rounding), and at least 99% of the elements bit-identical. The
cache codes and scales are bit-exact."""
import numpy as np
import pytest
import torch

from conftest import bf16_bits, pkg_module, u8

pytestmark = pytest.mark.gpu


def _ref_norm_rope(x, w, cos, sin, eps):
    """The reference's per-head RMSNorm then interleaved-pair RoPE, bf16 in/out (CPU)."""
    y = x.float()
    y = y * torch.rsqrt(y.pow(2).mean(-1, keepdim=True) + eps)
    y = y.to(x.dtype) * w
    real, imag = y.float().reshape(*y.shape[:-1], -1, 2).unbind(-1)
    rot = torch.stack((-imag, real), dim=-1).flatten(3)
    L, D = x.shape[1], x.shape[-1]
    out = (y.float() * cos.view(1, L, 1, D) + rot * sin.view(1, L, 1, D)).to(x.dtype)
    return out, y.float().abs().amax(-1, keepdim=True)


def _ordered(bits):
    """bf16 bit patterns -> integers ordered like the values (one step = one ulp)."""
    b = bits.astype(np.int32)
    return np.where(b & 0x8000, 0x8000 - b, b)


def _check_close(got, ref, what):
    want, ymax = ref
    d = np.abs(_ordered(bf16_bits(got)) - _ordered(bf16_bits(want)))
    exact = float((d == 0).mean())
    g, w = got.float().numpy(), want.float().numpy()
    ulp = 2.0 ** (np.floor(np.log2(np.maximum(ymax.numpy(), 2.0 ** -100))) - 7)
    ratio = np.abs(g - w) / (2 * ulp)
    print(f"{what}: max ulp diff {int(d.max())}, max error / bound {ratio.max():.2f}, "
          f"bit-identical {exact:.4%}", flush=True)
    assert ratio.max() <= 1.0 and exact >= 0.99, what


def _inputs(dev, B, L, H, seed, layout="qkv"):
    g = torch.Generator().manual_seed(seed)
    D = 128
    qkv = (torch.randn(B, L, 3, H, D, generator=g) * 2).to(torch.bfloat16)
    qkv[0, 0, :, 0] = 0.0                                  # all-zero rows: rsqrt(eps) branch
    qkv[0, 1, :, 1] *= 300.0                               # large rows
    qw = (1 + 0.1 * torch.randn(D, generator=g)).to(torch.bfloat16)
    kw = (1 + 0.1 * torch.randn(D, generator=g)).to(torch.bfloat16)
    db = pkg_module("dit_block")
    cos, sin = db.rope_tables(1, 1, L, t_offset=3)        # fp32 [L, 128], CPU
    return qkv, qw, kw, cos, sin


@pytest.mark.parametrize("B,L,H", [(1, 7, 2), (2, 37, 3), (1, 600, 24)])
def test_qk_norm_rope_matches_reference(dev, B, L, H):
    print(f"case qk_norm_rope B={B} L={L} H={H}", flush=True)
    ops = pkg_module("ops")
    qkv, qw, kw, cos, sin = _inputs(dev, B, L, H, 100 + L)
    g = qkv.to(dev)
    q, k, v = g.unbind(2)                                 # strided views of the fused QKV output
    ops.qk_norm_rope_(q, k, v, qw.to(dev), kw.to(dev), cos.to(dev), sin.to(dev), 1e-6)
    torch.cuda.synchronize()
    _check_close(q.cpu(), _ref_norm_rope(qkv[:, :, 0], qw, cos, sin, 1e-6), "q")
    _check_close(k.cpu(), _ref_norm_rope(qkv[:, :, 1], kw, cos, sin, 1e-6), "k")
    assert torch.equal(v.cpu(), qkv[:, :, 2])              # v untouched


@pytest.mark.parametrize("fmt", ["fp8", "int8"])
def test_fused_cache_write_is_the_kv_write_of_the_rotated_k(O, dev, fmt):
    print(f"case qk_norm_rope cache {fmt}", flush=True)
    ops = pkg_module("ops")
    kvc = pkg_module("fp8_kv_cache")
    B, L, H = 2, 45, 4
    qkv, qw, kw, cos, sin = _inputs(dev, B, L, H, 7)
    g = qkv.to(dev)
    q, k, v = g.unbind(2)
    make = kvc.make_fp8_kv_block if fmt == "fp8" else kvc.make_int8_kv_block
    cache = make(B, 3 * L, H, 128, device=dev)
    for buf in cache.values():
        buf.view(torch.uint8).zero_()
    ops.qk_norm_rope_kv_(q, k, v, qw.to(dev), kw.to(dev), cos.to(dev), sin.to(dev), 1e-6,
                         cache["k"], cache["v"], cache["k_scale"], cache["v_scale"], L)
    torch.cuda.synchronize()
    f = O.KV_FP8 if fmt == "fp8" else O.KV_INT8
    for name, x in (("k", k), ("v", v)):
        qo, so = O.kv_quantize(bf16_bits(x), f)
        assert np.array_equal(u8(cache[name])[:, L:2 * L], qo), name
        assert np.array_equal(cache[name + "_scale"][:, L:2 * L].cpu().numpy().view(np.uint32),
                              so.view(np.uint32)), name
        assert not u8(cache[name])[:, :L].any() and not u8(cache[name])[:, 2 * L:].any()


def test_block_fused_and_validated_cache_writes_agree(dev):
    """The DiT block's two write paths (validate then write, or fused into the
    norm/RoPE kernel) produce the same cache bytes and the same output."""
    print("case block write paths", flush=True)
    db = pkg_module("dit_block")
    kvc = pkg_module("fp8_kv_cache")
    hidden, heads, (t, h, w) = 256, 2, (1, 4, 9)
    L = t * h * w
    outs, caches = [], []
    for validate in (True, False):
        g = torch.Generator(device=dev).manual_seed(5)
        blk = db.FP8DiTBlock(hidden, heads, device=dev, generator=g, validate_kv_writes=validate)
        cache = kvc.make_fp8_kv_block(1, 2 * L, heads, 128, device=dev)
        for buf in cache.values():
            buf.view(torch.uint8).zero_()
        img = torch.randn(1, L, hidden, device=dev, generator=g).to(torch.bfloat16)
        vec = torch.randn(1, hidden, device=dev, generator=g).to(torch.bfloat16)
        cos, sin = db.rope_tables(t, h, w, device=dev)
        with torch.no_grad():
            outs.append(blk(img, vec, cos, sin, cache, 0, update_cache=True))
        caches.append(cache)
    assert torch.equal(outs[0], outs[1])
    for key in ("k", "v", "k_scale", "v_scale"):
        assert torch.equal(caches[0][key].view(torch.uint8), caches[1][key].view(torch.uint8)), key


@pytest.mark.parametrize("where", ["k", "v"])
def test_fused_cache_write_validated_on_device(dev, where):
    """With a status word, the fused kernel's cache write is checked first on
    the device: a NaN in k (or an Inf in v) leaves every cache byte unchanged
    and sets the flag, while q and k are still rotated in place exactly as
    without the cache write; finite values give flag 0 and the unchecked
    write's bytes."""
    print(f"case qk status {where}", flush=True)
    ops = pkg_module("ops")
    kvc = pkg_module("fp8_kv_cache")
    db = pkg_module("dit_block")
    B, L, H, D = 1, 36, 2, 128
    g = torch.Generator(device=dev).manual_seed(41)
    qkv = torch.randn(B, L, 3, H, D, device=dev, generator=g).to(torch.bfloat16)
    w = (1 + 0.1 * torch.randn(D, device=dev, generator=g)).to(torch.bfloat16)
    cos, sin = db.rope_tables(1, 4, 9, device=dev)

    def run(x, status):
        x = x.clone()
        q, k, v = x.select(2, 0), x.select(2, 1), x.select(2, 2)
        cache = kvc.make_fp8_kv_block(B, 2 * L, H, D, device=dev)
        for buf in cache.values():
            buf.view(torch.uint8).fill_(0x33)
        ops.qk_norm_rope_kv_(q, k, v, w, w, cos, sin, 1e-6, cache["k"], cache["v"], cache["k_scale"],
                             cache["v_scale"], L // 2, status)
        return x, cache

    good_x, good_cache = run(qkv, None)
    status = torch.full((1,), 9, dtype=torch.int32, device=dev)
    x2, cache2 = run(qkv, status)
    assert int(status.item()) == 0
    assert torch.equal(x2, good_x)
    for name in good_cache:
        assert torch.equal(cache2[name].view(torch.uint8), good_cache[name].view(torch.uint8)), name
    bad = qkv.clone()
    if where == "k":
        bad[0, 7, 1, 1, 3] = float("nan")
    else:
        bad[0, 30, 2, 0, 100] = float("inf")
    ref_x, _ = run(bad, None)
    x3, cache3 = run(bad, status)
    assert int(status.item()) == 1
    for name, buf in cache3.items():
        assert (buf.view(torch.uint8) == 0x33).all(), f"{name} was written"
    assert torch.equal(x3.view(torch.int16), ref_x.view(torch.int16))   # q/k rotated regardless


def test_qk_norm_rope_argument_errors(dev):
    ops = pkg_module("ops")
    x = torch.zeros(1, 4, 3, 2, 128, dtype=torch.bfloat16, device=dev)
    q, k, v = x.unbind(2)
    w = torch.ones(128, dtype=torch.bfloat16, device=dev)
    cs = torch.zeros(4, 128, device=dev)
    with pytest.raises(ValueError):
        ops.qk_norm_rope_(q, k.contiguous(), v, w, w, cs, cs, 1e-6)   # strides differ
    with pytest.raises(ValueError):
        ops.qk_norm_rope_(q, k, v, w, w, cs[:2], cs[:2], 1e-6)        # table too short
