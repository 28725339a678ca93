"""GPU parity of the quantizers: codes and scales bit-exact against the C oracle."""
import numpy as np
import pytest
import torch

from conftest import bf16_bits, pkg_module, u8

pytestmark = pytest.mark.gpu


def _gen(shape, seed, scale=1.0):
    g = torch.Generator().manual_seed(seed)
    return (torch.randn(*shape, generator=g) * scale).to(torch.bfloat16)


@pytest.mark.parametrize("rows,cols", [(1, 8), (7, 3072), (300, 2048), (64, 12288), (5, 16384), (33, 136)])
@pytest.mark.parametrize("mode", [0, 1])
def test_rows_fp8_bit_exact(O, dev, rows, cols, mode):
    print(f"case rows_fp8 {rows}x{cols} mode={mode}", flush=True)
    ops = pkg_module("ops")
    x = _gen((rows, cols), rows * 31 + cols, 3.0)
    x[::3, : cols // 2] *= 1e-3
    if rows > 2:
        x[1] = 0
    q, s = ops.quantize_rows_fp8(x.to(dev), mode, 1e-4)
    qo, so = O.quantize_rows_fp8(bf16_bits(x), mode)
    assert np.array_equal(u8(q), qo)
    assert np.array_equal(s.cpu().numpy().view(np.uint32), so.view(np.uint32))


def test_rows_fp8_special_values(O, dev):
    print("case rows_fp8 special values", flush=True)
    ops = pkg_module("ops")
    bits = np.zeros((6, 64), np.uint16)
    bits[0, :] = 0x0001                      # bf16 subnormals
    bits[1, ::2] = 0x8003
    bits[2, 5] = 0x3F80                      # single non-zero (1.0)
    bits[3, :] = np.arange(64, dtype=np.uint16) * 0x0101   # mixed patterns, finite
    bits[3] &= 0x7F7F
    bits[4, :] = 0x43E0                      # 448 everywhere
    bits[5, :] = 0x0000                      # zero row
    x = torch.from_numpy(bits.view(np.int16).copy()).view(torch.bfloat16)
    for mode in (0, 1):
        q, s = ops.quantize_rows_fp8(x.to(dev), mode, 1e-4)
        qo, so = O.quantize_rows_fp8(bits, mode)
        assert np.array_equal(u8(q), qo)
        assert np.array_equal(s.cpu().numpy().view(np.uint32), so.view(np.uint32))


def _edge_rows(cols):
    """Rows around the quantizers' quotient paths: signed zeros and bf16
    subnormals under a normal row maximum; row maxima just above and just below
    the point (s = 2^-100) where the kernels switch to the IEEE division;
    negative zero rows; and extreme-range rows (1e38 next to tiny values)."""
    rng = np.random.default_rng(17)
    rows = []
    r = (rng.integers(0, 0x3F80, cols) | (rng.integers(0, 2, cols) << 15)).astype(np.uint16)
    r[:8] = [0x3F80, 0x8000, 0x0000, 0x8001, 0x0001, 0x807F, 0x0080, 0xBF80]
    rows.append(r)
    for top in (0x1200, 0x1210, 0x11F0, 0x1180, 0x0F00):   # 2^-91 (s ~ 2^-99.8) .. 2^-97
        r = (rng.integers(0, top + 1, cols) | (rng.integers(0, 2, cols) << 15)).astype(np.uint16)
        r[0] = top
        rows.append(r)
    rows.append(np.full(cols, 0x8000, np.uint16))            # all -0.0
    r = (rng.integers(0, 0x7F7F, cols) | (rng.integers(0, 2, cols) << 15)).astype(np.uint16)
    r[0] = 0x7F7F                                             # bf16 max with every magnitude below it
    rows.append(r)
    # peak 127: the INT8 scale is exactly 1, so x / s sits on the half-away
    # ties and on the +-127 clamp (int8_kv_cache.py:150-157); -0 keeps code 0
    ties = np.array([0.5, 1.5, 2.5, 3.5, 63.5, 125.5, 126.5, 127.0, 126.0, 0.25, 0.75, 1.0],
                    np.float32)
    vals = np.concatenate([ties, -ties, [-0.0, 0.0]]).astype(np.float32)
    r = (rng.integers(0, 0x42FE, cols) | (rng.integers(0, 2, cols) << 15)).astype(np.uint16)
    r[:vals.size] = (vals.view(np.uint32) >> 16).astype(np.uint16)
    rows.append(r)
    return np.stack(rows)


def test_rows_fp8_quotient_edge_rows(O, dev):
    print("case rows_fp8 quotient edge rows", flush=True)
    ops = pkg_module("ops")
    bits = _edge_rows(1024)
    x = torch.from_numpy(bits.view(np.int16).copy()).view(torch.bfloat16)
    for mode in (0, 1):
        q, s = ops.quantize_rows_fp8(x.to(dev), mode, 1e-4)
        qo, so = O.quantize_rows_fp8(bits, mode)
        assert np.array_equal(u8(q), qo), f"mode {mode} codes"
        assert np.array_equal(s.cpu().numpy().view(np.uint32), so.view(np.uint32))


@pytest.mark.parametrize("fmt", ["fp8", "int8"])
def test_kv_quantize_quotient_edge_rows(O, dev, fmt):
    print(f"case kv quotient edge rows {fmt}", flush=True)
    kvc = pkg_module("fp8_kv_cache")
    bits = _edge_rows(128)                                    # one (token, head) row each
    n = bits.shape[0]
    x = torch.from_numpy(bits.view(np.int16).copy()).view(torch.bfloat16).reshape(1, n, 1, 128)
    make = kvc.make_fp8_kv_block if fmt == "fp8" else kvc.make_int8_kv_block
    cache = make(1, n, 1, 128, device=dev)
    kvc.quantize_kv_pair_into(cache, x.to(dev), x.to(dev), 0)
    qo, so = O.kv_quantize(bits.reshape(1, n, 1, 128), O.KV_FP8 if fmt == "fp8" else O.KV_INT8)
    assert np.array_equal(u8(cache["k"]), qo) and np.array_equal(u8(cache["v"]), qo)
    assert np.array_equal(cache["k_scale"].cpu().numpy().view(np.uint32), so.view(np.uint32))


@pytest.mark.parametrize("width,lo,hi", [(512, 128, 384), (12288, 1024, 7176)])
def test_rows_fp8_strided_input(O, dev, width, lo, hi):
    """A column window of wider rows (16-byte aligned start): one wave per row
    for 256 columns, one workgroup per row for 6152 (> 4096)."""
    ops = pkg_module("ops")
    x = _gen((64, width), 11)
    view = x.to(dev)[:, lo:hi]               # row stride `width`
    q, s = ops.quantize_rows_fp8(view, 0, 1e-4)
    qo, so = O.quantize_rows_fp8(bf16_bits(x[:, lo:hi]))
    assert np.array_equal(u8(q), qo) and np.array_equal(s.cpu().numpy(), so)


@pytest.mark.parametrize("m,k", [(1, 128), (129, 256), (300, 384), (4096, 3072), (4097, 128)])
def test_blockwise_fp8_bit_exact(O, dev, m, k):
    print(f"case blockwise {m}x{k}", flush=True)
    ops = pkg_module("ops")
    x = _gen((m, k), m + k)
    if k > 128:
        x[:, 128:256] *= 20
    q, s = ops.quantize_blockwise_fp8(x.to(dev))
    qo, so = O.quantize_blockwise_fp8(bf16_bits(x))
    assert np.array_equal(u8(q), qo)
    assert np.array_equal(s.cpu().numpy(), so)


def _kv_inputs(B, H, L, D, seed):
    g = torch.Generator().manual_seed(seed)
    gain = torch.empty(H).uniform_(0.5, 4.0, generator=g)
    x = torch.randn(B, H, L, D, generator=g) * gain[None, :, None, None]
    return x.to(torch.bfloat16)                 # [B, H, L, D] memory (config-2 layout)


@pytest.mark.parametrize("fmt", ["fp8", "int8"])
def test_kv_quantize_config2_full_size_bit_exact(O, dev, fmt):
    """K, V [1, 24, 10800, 128] written at chunk slot 2 of a
    3-chunk cache; every code and scale compared."""
    print(f"case kv config2 {fmt}", flush=True)
    kvc = pkg_module("fp8_kv_cache")
    B, H, L, D = 1, 24, 10800, 128
    k = _kv_inputs(B, H, L, D, 1)
    v = _kv_inputs(B, H, L, D, 2)
    make = kvc.make_fp8_kv_block if fmt == "fp8" else kvc.make_int8_kv_block
    cache = make(B, 3 * L, H, D, device=dev)
    for t in cache.values():
        t.view(torch.uint8).fill_(0xAB)
    kd, vd = k.to(dev).transpose(1, 2), v.to(dev).transpose(1, 2)   # [B, L, H, D] views
    kvc.quantize_kv_pair_into(cache, kd, vd, 2 * L)
    torch.cuda.synchronize()
    f = O.KV_FP8 if fmt == "fp8" else O.KV_INT8
    for name, x in (("k", k), ("v", v)):
        qo, so = O.kv_quantize(np.transpose(bf16_bits(x), (0, 2, 1, 3)), f)
        got = u8(cache[name])
        assert np.array_equal(got[:, 2 * L:], qo), f"{name} codes"
        assert (got[:, :2 * L] == 0xAB).all(), f"{name}: bytes before `start` were touched"
        gs = cache[name + "_scale"].cpu().numpy()
        assert np.array_equal(gs[:, 2 * L:].view(np.uint32), so.view(np.uint32)), f"{name} scales"


@pytest.mark.parametrize("fmt", ["fp8", "int8"])
def test_kv_dequantize_matches_oracle(O, dev, fmt):
    kvc = pkg_module("fp8_kv_cache")
    B, H, L, D = 2, 3, 70, 128
    make = kvc.make_fp8_kv_block if fmt == "fp8" else kvc.make_int8_kv_block
    cache = make(B, 100, H, D, device=dev)
    k = _kv_inputs(B, H, L, D, 5).transpose(1, 2).contiguous()
    kvc.quantize_kv_pair_into(cache, k.to(dev), k.to(dev), 0)
    y = kvc.dequantize_kv(cache, "k", 65)
    f = O.KV_FP8 if fmt == "fp8" else O.KV_INT8
    ref = O.kv_dequantize(u8(cache["k"])[:, :65], cache["k_scale"].cpu().numpy()[:, :65], f)
    assert np.array_equal(bf16_bits(y), ref)
    assert kvc.dequantize_kv(cache, "v", 0).shape == (B, 0, H, D)


@pytest.mark.parametrize("bad", [float("inf"), float("nan"), -float("inf")])
def test_kv_write_rejects_non_finite_before_writing(O, dev, bad):
    """The finiteness check runs on the GPU before the write: with a NaN/Inf
    in V, neither K nor V (codes or scales) changes. Without a status tensor
    the call raises ValueError as the reference does; with one it sets the
    flag and returns without a host synchronisation."""
    kvc = pkg_module("fp8_kv_cache")
    cache = kvc.make_fp8_kv_block(1, 16, 2, 128, device=dev)
    for buf in cache.values():
        buf.view(torch.uint8).fill_(7)
    k = torch.randn(1, 4, 2, 128, device=dev).to(torch.bfloat16)
    v = k.clone()
    v[0, 2, 1, 9] = bad
    with pytest.raises(ValueError, match="non-finite"):
        kvc.quantize_kv_pair_into(cache, k, v, 3)
    for name, buf in cache.items():
        assert (buf.view(torch.uint8) == 7).all(), f"{name} was written"
    status = torch.full((1,), 5, dtype=torch.int32, device=dev)
    kvc.quantize_kv_pair_into(cache, v, k, 3, status=status)      # non-finite in K this time
    assert int(status.item()) == 1
    for name, buf in cache.items():
        assert (buf.view(torch.uint8) == 7).all(), f"{name} was written (deferred mode)"
    with pytest.raises(ValueError, match="non-finite"):
        kvc.quantize_kv_into(cache, "v", v, 0)
    assert (u8(cache["v"]) == 7).all()
    # finite values: status 0 and the usual bit-exact codes
    kvc.quantize_kv_pair_into(cache, k, k, 3, status=status)
    assert int(status.item()) == 0
    qo, so = O.kv_quantize(bf16_bits(k))
    assert np.array_equal(u8(cache["k"])[:, 3:7], qo) and np.array_equal(u8(cache["v"])[:, 3:7], qo)
    assert np.array_equal(cache["k_scale"][:, 3:7].cpu().numpy().view(np.uint32), so.view(np.uint32))
    assert (u8(cache["k"])[:, :3] == 7).all() and (u8(cache["k"])[:, 7:] == 7).all()


def test_kv_write_twice_is_deterministic(dev):
    kvc = pkg_module("fp8_kv_cache")
    x = _kv_inputs(1, 4, 500, 128, 9).transpose(1, 2).contiguous().to(dev)
    a = kvc.make_fp8_kv_block(1, 500, 4, 128, device=dev)
    b = kvc.make_fp8_kv_block(1, 500, 4, 128, device=dev)
    kvc.quantize_kv_pair_into(a, x, x, 0)
    kvc.quantize_kv_pair_into(b, x, x, 0)
    assert torch.equal(a["k"].view(torch.uint8), b["k"].view(torch.uint8))
    assert torch.equal(a["v_scale"], b["v_scale"])


# LayerNorm + adaLN modulate + per-token FP8 quant, fused (the block's path into
# its QKV and fc1 linears).

def _ln_inputs(dev, B, L, C, seed):
    g = torch.Generator(device=dev).manual_seed(seed)
    x = (torch.randn(B, L, C, device=dev, generator=g) * 3 + 0.5).to(torch.bfloat16)
    sh = (torch.randn(B, C, device=dev, generator=g) * 0.5).to(torch.bfloat16)
    sc = (torch.randn(B, C, device=dev, generator=g) * 0.5).to(torch.bfloat16)
    return x, sh, sc


@pytest.mark.parametrize("B,L,C", [(1, 300, 3072), (2, 130, 640), (1, 5, 8), (1, 10800, 3072)])
def test_ln_modulate_quantize_bit_exact(O, dev, B, L, C):
    """Codes and scales equal the oracle's (its LayerNorm restates the kernel's fp32
    summation order; the modulate and the quantizer are the reference recipes)."""
    print(f"case ln-mod-quant {B}x{L}x{C}", flush=True)
    ops = pkg_module("ops")
    x, sh, sc = _ln_inputs(dev, B, L, C, B * L + C)
    q, s = ops.ln_modulate_quantize_fp8(x, sh, sc, 1e-6)
    qo, so = O.ln_modulate_quantize_fp8(bf16_bits(x.reshape(B * L, C)), bf16_bits(sh), bf16_bits(sc), 1e-6,
                                        rows_per_batch=L)
    assert np.array_equal(u8(q), qo)
    assert np.array_equal(s.cpu().numpy(), so)


def test_ln_modulate_quantize_matches_unfused_torch_path(dev):
    """Against F.layer_norm + the bf16 modulate ops + quantize_rows_fp8 on the GPU
    (torch's own LayerNorm summation): codes agree except where a LayerNorm output
    sits on a bf16 rounding boundary."""
    ops = pkg_module("ops")
    B, L, C = 1, 2048, 3072
    x, sh, sc = _ln_inputs(dev, B, L, C, 5)
    q, s = ops.ln_modulate_quantize_fp8(x, sh, sc, 1e-6)
    y = torch.nn.functional.layer_norm(x, (C,), eps=1e-6)
    mod = y * (1 + sc.unsqueeze(1)) + sh.unsqueeze(1)
    qr, sr = ops.quantize_rows_fp8(mod.reshape(B * L, C))
    agree = (u8(q) == u8(qr)).mean()
    print(f"[ln fused vs F.layer_norm path] codes identical: {agree:.6f} "
          f"({int((u8(q) != u8(qr)).sum())} of {q.numel()} differ)", flush=True)
    assert agree >= 0.999, agree
    assert torch.allclose(s, sr, rtol=2 ** -7, atol=0)


def test_ln_modulate_quantize_rejects_bad_shapes(dev):
    ops = pkg_module("ops")
    x, sh, sc = _ln_inputs(dev, 1, 4, 64, 1)
    with pytest.raises(ValueError):
        ops.ln_modulate_quantize_fp8(x, sh[:, :32], sc, 1e-6)
    with pytest.raises(TypeError):
        ops.ln_modulate_quantize_fp8(x.float(), sh, sc, 1e-6)


def _codes_match(got, want):
    """Codes equal, except that a NaN code (0x7F | sign) matches either sign:
    the sign of a NaN after a division is not reproducible across devices."""
    nan = (want & 0x7F) == 0x7F
    return np.array_equal(got[~nan], want[~nan]) and ((got[nan] & 0x7F) == 0x7F).all()


@pytest.mark.parametrize("cols", [3072, 12288])
def test_quantizers_non_finite_rows(O, dev, cols):
    """NaN in a row makes its scale NaN and every code a NaN code (torch's amax
    propagates NaN; clamp_min keeps it); an infinite row max gives scale inf.
    Per-token quant in both scale modes (one wave per row for 3072 columns,
    one workgroup per row for 12288), blockwise quant, and the fused LayerNorm
    + modulate + quant, against the oracle."""
    print(f"case non-finite rows cols={cols}", flush=True)
    ops = pkg_module("ops")
    x = _gen((24, cols), 5, 2.0)
    x[3, 17] = float("nan")
    x[7, :] = float("nan")
    x[11, 40] = float("inf")
    x[15, 41] = -float("inf")
    bits = bf16_bits(x)
    for mode in (0, 1):
        q, s = ops.quantize_rows_fp8(x.to(dev), mode, 1e-4)
        qo, so = O.quantize_rows_fp8(bits, mode)
        assert np.array_equal(s.cpu().numpy(), so, equal_nan=True), mode
        assert _codes_match(u8(q), qo), mode
    if cols % 128 == 0:
        xb = torch.cat([x, _gen((104, cols), 6, 2.0)])          # 128 rows: one block row
        q, s = ops.quantize_blockwise_fp8(xb.to(dev))
        qo, so = O.quantize_blockwise_fp8(bf16_bits(xb))
        assert np.isnan(so).any() and np.array_equal(s.cpu().numpy(), so, equal_nan=True)
        assert _codes_match(u8(q), qo)
    if cols <= 8192:
        sh = (torch.randn(1, cols) * 0.5).to(torch.bfloat16)
        sc = (torch.randn(1, cols) * 0.5).to(torch.bfloat16)
        q, s = ops.ln_modulate_quantize_fp8(x.view(1, 24, cols).to(dev), sh.to(dev), sc.to(dev), 1e-6)
        qo, so = O.ln_modulate_quantize_fp8(bits, bf16_bits(sh), bf16_bits(sc), 1e-6, rows_per_batch=24)
        assert np.isnan(so[[3, 7, 11, 15]]).all()
        assert np.array_equal(s.cpu().numpy(), so, equal_nan=True)
        assert _codes_match(u8(q), qo)


def test_hardware_e4m3_conversion_matches_oracle_over_quantizer_range(O, dev):
    """The quantizers encode with gfx950's v_cvt_pk_fp8_f32 (e4m3_encode4 in
    csrc/hn_common.h). Every quotient they produce is finite with
    |x / s| <= 448 (1 + 2^-23) < 448.5, so the conversion is checked against
    the oracle's RNE encoder over every fp32 bit pattern with |x| <= 448.5,
    both signs (2 x 1.14e9 inputs): no code may differ."""
    from concurrent.futures import ThreadPoolExecutor
    L = pkg_module("_lib")
    lib = L.load()
    last = 0x43E04000                       # 448.5
    assert np.array([last], np.uint32).view(np.float32)[0] == 448.5
    chunk = 1 << 27
    buf = torch.empty(chunk, dtype=torch.uint8, device=dev)
    stream = torch.cuda.current_stream(dev).cuda_stream
    pool = ThreadPoolExecutor(8)            # the oracle call releases the GIL
    checked = 0
    for sign in (0, 0x80000000):
        start = 0
        while start <= last:
            n = min(chunk, (last + 1 - start + 3) // 4 * 4)
            L.check(lib.hn_e4m3_encode_range(sign | start, n, buf.data_ptr(), stream),
                    "hn_e4m3_encode_range")
            codes = buf[:n].cpu().numpy()
            cuts = [n * i // 8 for i in range(9)]
            jobs = [pool.submit(O.e4m3_range_mismatches, sign | (start + lo), codes[lo:hi])
                    for lo, hi in zip(cuts, cuts[1:])]
            for lo, j in zip(cuts, jobs):
                bad, where = j.result()
                assert bad == 0, (f"{bad} codes differ from the oracle; first at fp32 bits "
                                  f"{sign | (start + lo + where):#010x}")
            checked += n
            start += n
    pool.shutdown()
    print(f"[e4m3] {checked} fp32 inputs, hardware conversion == oracle", flush=True)
    assert checked >= 2 * (last + 1)


@pytest.mark.parametrize("cols", [640, 3072, 12288])
def test_quantizers_write_nothing_past_their_outputs(dev, cols):
    """Each quantizer writes into buffers 16 rows longer than its output (and,
    for the blockwise scales, one block row longer), pre-filled: the output
    part equals the op's own result and every guard byte keeps its fill. The
    narrow (one wave per row), wide (one workgroup per row), fused LayerNorm
    and blockwise paths."""
    print(f"case quant guard band cols={cols}", flush=True)
    ops, L = pkg_module("ops"), pkg_module("_lib")
    lib = L.load()
    st = torch.cuda.current_stream().cuda_stream
    rows = 300
    g = torch.Generator(device=dev).manual_seed(cols)
    x = (torch.randn(rows, cols, device=dev, generator=g) * 2).to(torch.bfloat16)

    def guarded(shape, dtype, fill):
        t = torch.empty(shape, dtype=dtype, device=dev)
        t.view(torch.uint8).fill_(fill)
        return t

    # per-token rows
    q = guarded((rows + 16, cols), torch.uint8, 0xAB)
    s = guarded((rows + 16,), torch.float32, 0xCD)
    L.check(lib.hn_quantize_rows_fp8(x.data_ptr(), rows, cols, cols, L.HN_SCALE_CLAMP, 1e-4,
                                     q.data_ptr(), s.data_ptr(), st), "rows")
    qr, sr = ops.quantize_rows_fp8(x)
    assert torch.equal(q[:rows], qr.view(torch.uint8)) and torch.equal(s[:rows], sr)
    assert bool((q[rows:] == 0xAB).all()) and bool((s[rows:].view(torch.uint8) == 0xCD).all())
    # fused LayerNorm + modulate (widths up to 8192)
    if cols <= 8192:
        sh = (torch.randn(1, cols, device=dev, generator=g) * 0.5).to(torch.bfloat16)
        sc = (torch.randn(1, cols, device=dev, generator=g) * 0.5).to(torch.bfloat16)
        q = guarded((rows + 16, cols), torch.uint8, 0xAB)
        s = guarded((rows + 16,), torch.float32, 0xCD)
        L.check(lib.hn_ln_mod_quantize_fp8(x.data_ptr(), rows, cols, rows, sh.data_ptr(), sc.data_ptr(),
                                           cols, 1e-6, 1e-4, q.data_ptr(), s.data_ptr(), st), "ln")
        qr, sr = ops.ln_modulate_quantize_fp8(x.view(1, rows, cols), sh, sc, 1e-6)
        assert torch.equal(q[:rows], qr.view(rows, cols).view(torch.uint8))
        assert torch.equal(s[:rows], sr.view(rows))
        assert bool((q[rows:] == 0xAB).all()) and bool((s[rows:].view(torch.uint8) == 0xCD).all())
    # blockwise 128 x 128 (300 rows: the last block row is 44 deep)
    nb = (rows + 127) // 128
    q = guarded((rows + 16, cols), torch.uint8, 0xAB)
    s = guarded((nb + 1, cols // 128), torch.float32, 0xCD)
    L.check(lib.hn_quantize_blockwise_fp8(x.data_ptr(), rows, cols, q.data_ptr(), s.data_ptr(), st), "bw")
    qr, sr = ops.quantize_blockwise_fp8(x)
    assert torch.equal(q[:rows], qr.view(torch.uint8)) and torch.equal(s[:nb], sr)
    assert bool((q[rows:] == 0xAB).all()) and bool((s[nb:].view(torch.uint8) == 0xCD).all())


@pytest.mark.parametrize("fmt", ["fp8", "int8"])
def test_kv_write_touches_only_its_slot(dev, fmt):
    """A write of 30 tokens at start 40 of a 100-token cache (B 2): codes and
    scales of tokens [0, 40) and [70, 100) keep their fill."""
    kvc = pkg_module("fp8_kv_cache")
    make = kvc.make_fp8_kv_block if fmt == "fp8" else kvc.make_int8_kv_block
    cache = make(2, 100, 3, 128, device=dev)
    for t in cache.values():
        t.view(torch.uint8).fill_(0x5A)
    g = torch.Generator(device=dev).manual_seed(3)
    k = (torch.randn(2, 30, 3, 128, device=dev, generator=g) * 2).to(torch.bfloat16)
    v = (torch.randn(2, 30, 3, 128, device=dev, generator=g) * 2).to(torch.bfloat16)
    kvc.quantize_kv_pair_into(cache, k, v, 40)
    for name, t in cache.items():
        b = t.view(torch.uint8)
        assert bool((b[:, :40] == 0x5A).all()) and bool((b[:, 70:] == 0x5A).all()), name
        assert not bool((b[:, 40:70] == 0x5A).all()), name
