"""W8 checkpoint ingest (hy-nomas_amd/w8_checkpoint.py): the reference's three
on-disk layouts (int8_stored_bf16_linear.py:13-18,121-306), their validation,
the reference's dequantized weight, and -- on the GPU -- requantization to
per-channel FP8 and loading into FP8StoredLinear modules.

Checkpoints are synthesized the way the reference's offline converter writes
them: INT8 codes from the reference's quantize_weight recipe (the oracle's
restatement, pinned against torch in test_oracle.py), bf16 for other tensors."""
import json

import numpy as np
import pytest
import torch
import torch.nn as nn
from safetensors.torch import save_file

from conftest import assert_close_bf16, bf16_bits, pkg_module, u8


class Tiny(nn.Module):
    def __init__(self):
        super().__init__()
        self.a = nn.Linear(256, 128)
        self.norm = nn.LayerNorm(128)
        self.b = nn.Linear(128, 256, bias=False)


LAYERS = {"a": [128, 256], "b": [256, 128]}


def _tensors(O):
    g = torch.Generator().manual_seed(3)
    t = {}
    for name, (n, k) in LAYERS.items():
        w = (torch.randn(n, k, generator=g) * 0.05).to(torch.bfloat16).float()
        q, s = O.quantize_weight_int8(w.numpy())
        t[name + ".weight_q"] = torch.from_numpy(q)
        t[name + ".weight_scale"] = torch.from_numpy(s)
    t["a.bias"] = (torch.randn(128, generator=g) * 0.01).to(torch.bfloat16)
    t["norm.weight"] = torch.ones(128, dtype=torch.bfloat16)
    t["norm.bias"] = torch.zeros(128, dtype=torch.bfloat16)
    return t


def _nomas_meta(**over):
    meta = {"format": "nomas-int8-bf16-single-v1", "group_size": "128",
            "quantization": "symmetric_int8_absmax", "compute_dtype": "bfloat16",
            "rounding": "half_away_from_zero", "model_type": "tiny", "layers": json.dumps(LAYERS)}
    meta.update(over)
    return meta


def _write_nomas(path, tensors, **over):
    save_file(tensors, str(path), metadata=_nomas_meta(**over))
    return path


def _write_embedded(W, path, tensors, tamper=None):
    sums = {k: W.tensor_sha256(v) for k, v in tensors.items()}
    if tamper:
        sums[tamper] = "0" * 64
    manifest = {"format": W.FORMAT, "group_size": 128, "model_type": "tiny", "layers": LAYERS,
                "tensor_sha256": sums}
    save_file(tensors, str(path), metadata={W.SINGLE_FILE_MANIFEST: json.dumps(manifest)})
    return path


def _write_dir(W, root, tensors):
    root.mkdir()
    keys = sorted(tensors)
    shards = []
    for i, part in enumerate((keys[: len(keys) // 2], keys[len(keys) // 2:])):
        name = f"shard{i}.safetensors"
        save_file({k: tensors[k] for k in part}, str(root / name))
        shards.append({"file": name, "bytes": (root / name).stat().st_size,
                       "sha256": W._sha256_file(root / name)})
    (root / W.MANIFEST).write_text(json.dumps({"format": W.FORMAT, "group_size": 128,
                                               "model_type": "tiny", "layers": LAYERS, "shards": shards}))
    return root


@pytest.fixture(scope="module")
def W():
    return pkg_module("w8_checkpoint")


def test_all_three_layouts_validate(O, W, tmp_path):
    t = _tensors(O)
    for ckpt in (_write_nomas(tmp_path / "n.safetensors", t),
                 _write_embedded(W, tmp_path / "e.safetensors", t),
                 _write_dir(W, tmp_path / "d", t)):
        manifest, files, _ = W.read_w8_manifest(ckpt, "tiny")
        assert manifest["layers"] == LAYERS and files


def test_header_and_shape_errors(O, W, tmp_path):
    t = _tensors(O)
    with pytest.raises(ValueError, match="rounding"):
        W.read_w8_manifest(_write_nomas(tmp_path / "r.safetensors", t, rounding="nearest_even"))
    with pytest.raises(ValueError, match="model_type"):
        W.read_w8_manifest(_write_nomas(tmp_path / "m.safetensors", t), "other")
    with pytest.raises(ValueError, match="layers do not match"):
        W.read_w8_manifest(_write_nomas(tmp_path / "l.safetensors", t, layers=json.dumps({"a": [128, 256]})))
    bad = dict(t)
    bad["a.weight_scale"] = torch.ones(128, 3)
    with pytest.raises(ValueError, match="shape/dtype"):
        W.read_w8_manifest(_write_nomas(tmp_path / "s.safetensors", bad))
    save_file(t, str(tmp_path / "plain.safetensors"))
    with pytest.raises(ValueError, match="missing supported"):
        W.read_w8_manifest(tmp_path / "plain.safetensors")


def test_checksums_are_enforced(O, W, tmp_path):
    t = _tensors(O)
    path = _write_embedded(W, tmp_path / "e.safetensors", t, tamper="a.weight_q")
    with pytest.raises(ValueError, match="checksum mismatch"):
        W.load_w8_as_fp8(Tiny, "tiny", path, "cpu")     # fails before any GPU work
    root = _write_dir(W, tmp_path / "d", t)
    shard = root / "shard0.safetensors"
    raw = bytearray(shard.read_bytes())
    raw[-1] ^= 0xFF
    shard.write_bytes(bytes(raw))
    with pytest.raises(ValueError, match="checksum mismatch"):
        W.read_w8_manifest(root, "tiny")


def test_dequantized_weight_is_the_reference_formula(O, W):
    t = _tensors(O)
    q, s = t["a.weight_q"], t["a.weight_scale"]
    w = W.dequantize_int8_weight(q, s)
    ref = O.f32_to_bf16_bits(q.numpy().astype(np.float32) * np.repeat(s.numpy(), 128, axis=1)[:, :256])
    assert np.array_equal(bf16_bits(w), ref)


@pytest.mark.gpu
@pytest.mark.parametrize("layout", ["nomas", "embedded", "dir"])
def test_load_w8_as_fp8(O, W, dev, tmp_path, layout):
    print(f"case w8 load {layout}", flush=True)
    t = _tensors(O)
    ckpt = {"nomas": lambda: _write_nomas(tmp_path / "n.safetensors", t),
            "embedded": lambda: _write_embedded(W, tmp_path / "e.safetensors", t),
            "dir": lambda: _write_dir(W, tmp_path / "d", t)}[layout]()
    model, reports = W.load_w8_as_fp8(Tiny, "tiny", ckpt, dev)
    dl = pkg_module("dit_fp8_linear")
    for name in LAYERS:
        m = getattr(model, name)
        assert isinstance(m, dl.FP8StoredLinear)
        w_bits = bf16_bits(W.dequantize_int8_weight(t[name + ".weight_q"], t[name + ".weight_scale"]))
        qo, so = O.quantize_rows_fp8(w_bits, O.SCALE_CLAMP)
        assert np.array_equal(u8(m.weight_q), qo) and np.array_equal(m.weight_scale.cpu().numpy(), so)
        print(f"{name}: {reports[name]}", flush=True)
        assert reports[name]["rel_l2"] < 0.05 and reports[name]["max_channel_rel_l2"] < 0.08
    assert torch.equal(model.norm.weight.cpu(), t["norm.weight"])
    x = torch.randn(40, 256, device=dev).to(torch.bfloat16)
    y = model.a(x)
    qx, sx = O.quantize_rows_fp8(bf16_bits(x))
    ref = O.linear_reference(qx, sx, u8(model.a.weight_q), model.a.weight_scale.cpu().numpy(),
                             O.bf16_bits_to_f32(bf16_bits(t["a.bias"])))
    assert_close_bf16(y.float().cpu().numpy(), ref, what="W8-loaded FP8 linear")


def test_directory_layout_checks_layer_tensors(O, W, tmp_path):
    """The directory layout's layer tensors get the same geometry check as the
    single files (int8 [out, in] codes, fp32 [out, ceil(in/128)] scales), and
    a missing one is a ValueError -- all before any GPU work."""
    t = _tensors(O)
    cases = {
        "uint8 codes": dict(t, **{"a.weight_q": t["a.weight_q"].view(torch.uint8)}),
        "float codes": dict(t, **{"b.weight_q": t["b.weight_q"].float()}),
        "scale shape": dict(t, **{"a.weight_scale": torch.ones(128, 3)}),
    }
    for i, (what, bad) in enumerate(cases.items()):
        root = _write_dir(W, tmp_path / f"d{i}", bad)
        with pytest.raises(ValueError, match="shape/dtype"):
            W.load_w8_as_fp8(Tiny, "tiny", root, "cpu")
    missing = {k: v for k, v in t.items() if k != "b.weight_scale"}
    root = _write_dir(W, tmp_path / "dm", missing)
    with pytest.raises(ValueError, match="weight_scale"):
        W.load_w8_as_fp8(Tiny, "tiny", root, "cpu")


class TinyRope(Tiny):
    """Tiny with a table the checkpoint omits (a non-persistent buffer, like the
    reference's camera RoPE tables) and the method that rebuilds it."""

    def __init__(self):
        super().__init__()
        self.register_buffer("freqs", torch.arange(16, dtype=torch.float32), persistent=False)

    def rebuild_derived_buffers(self):
        self.freqs = torch.arange(16, dtype=torch.float32) * 0.5


class TinyRopeNoRebuild(Tiny):
    def __init__(self):
        super().__init__()
        self.register_buffer("freqs", torch.arange(16, dtype=torch.float32), persistent=False)


@pytest.mark.gpu
def test_load_w8_rebuilds_derived_buffers(O, W, dev, tmp_path):
    t = _tensors(O)
    ckpt = _write_nomas(tmp_path / "n.safetensors", t)
    model, _ = W.load_w8_as_fp8(TinyRope, "tiny", ckpt, dev)
    assert model.freqs.device.type == "cuda" and torch.equal(model.freqs.cpu(), torch.arange(16) * 0.5)
    with pytest.raises(ValueError, match="Unmaterialized model buffers"):
        W.load_w8_as_fp8(TinyRopeNoRebuild, "tiny", ckpt, dev)
    model, _ = W.load_w8_as_fp8(TinyRopeNoRebuild, "tiny", ckpt, dev,
                                rebuild_buffers=lambda m: setattr(m, "freqs", torch.ones(16)))
    assert torch.equal(model.freqs.cpu(), torch.ones(16))


class _Proj(nn.Module):
    def __init__(self, names, dims):
        super().__init__()
        for n, (o, i) in zip(names, dims):
            setattr(self, n, nn.Linear(i, o, bias=False))


class _Layer(nn.Module):
    def __init__(self, h, f):
        super().__init__()
        self.mlp = _Proj(("gate_proj", "up_proj", "down_proj"), ((f, h), (f, h), (h, f)))
        self.attn = _Proj(("q_proj", "o_proj"), ((h, h), (h, h)))
        self.norm = nn.LayerNorm(h)


class _Decoder(nn.Module):
    """Stand-in for the PixelUMM decoder's layer structure (model.py:43-53)."""

    def __init__(self, n=2, h=256, f=512):
        super().__init__()
        self.layers = nn.ModuleList(_Layer(h, f) for _ in range(n))


def _pixelumm_file(W, dev, dec):
    pf = pkg_module("pixelumm_fp8")
    g = torch.Generator(device=dev).manual_seed(9)
    state, names = {}, []
    for i, layer in enumerate(dec.layers):
        for p in W.PIXELUMM_PROJECTIONS:
            lin = layer.get_submodule(p)
            w = (torch.randn(lin.weight.shape, device=dev, generator=g) * 0.05).to(torch.bfloat16)
            q, s = pf.quantize_blockwise(w)
            state[f"layers.{i}.{p}.fp8_weight"], state[f"layers.{i}.{p}.fp8_scale"] = q, s
            names.append(f"decoder.layers.{i}.{p}.weight")
        state[f"layers.{i}.norm.weight"] = torch.ones(256, dtype=torch.bfloat16, device=dev)
    meta = dict(W.PIXELUMM_HEADER, quantized_source_keys=json.dumps(names), quantized_layers=str(len(names)))
    return state, meta


@pytest.mark.gpu
def test_install_serialized_fp8(O, W, dev):
    """PixelUMM FP8 single-file install (prequantized.py:27-65) on a stand-in
    decoder: the serialized codes and scales are used as they are, the layers
    compute the blockwise FP8 linear, and each rule refuses a broken input."""
    print("case pixelumm install", flush=True)
    pf = pkg_module("pixelumm_fp8")
    dec = _Decoder().to(dev).to(torch.bfloat16).eval()
    state, meta = _pixelumm_file(W, dev, dec)
    assert W.install_serialized_fp8(dec, state, meta, "cutlass") == 10
    assert dec._prequantized_fp8 and dec._prequantized_fp8_layers == 10
    assert dec._prequantized_fp8_backend == "cutlass"
    up = dec.layers[1].mlp.up_proj
    assert isinstance(up, pf.FP8Linear) and up.fp8_weight is state["layers.1.mlp.up_proj.fp8_weight"]
    x = torch.randn(300, 256, device=dev).to(torch.bfloat16)
    with torch.no_grad():
        y = up(x)
    qa, sa = pf.quantize_blockwise(x)
    ref = O.blockwise_gemm_reference(u8(qa), sa.cpu().numpy(), u8(up.fp8_weight), up.fp8_scale.cpu().numpy())
    got = y.float().cpu().numpy()
    rel = float(np.linalg.norm(got - ref) / np.linalg.norm(ref))
    assert rel < 0.004, rel          # the reference harness's bound
    # refusals
    fresh = lambda: _Decoder().to(dev).to(torch.bfloat16).eval()
    with pytest.raises(ValueError, match="metadata"):
        W.install_serialized_fp8(fresh(), state, dict(meta, block_size="64"))
    short = json.dumps(json.loads(meta["quantized_source_keys"])[:-1])
    with pytest.raises(ValueError, match="manifest"):
        W.install_serialized_fp8(fresh(), state, dict(meta, quantized_source_keys=short))
    with pytest.raises(ValueError, match="backend"):
        W.install_serialized_fp8(fresh(), state, meta, "deepgemm")
    biased = fresh()
    biased.layers[0].attn.q_proj = nn.Linear(256, 256).to(dev).to(torch.bfloat16)
    with pytest.raises(ValueError, match="bias-free"):
        W.install_serialized_fp8(biased, state, meta)
    with pytest.raises(ValueError, match="BF16"):
        W.install_serialized_fp8(fresh(), dict(state, **{"layers.0.norm.weight": torch.ones(256, device=dev)}), meta)
    bad_scale = dict(state, **{"layers.0.mlp.gate_proj.fp8_scale": -state["layers.0.mlp.gate_proj.fp8_scale"]})
    with pytest.raises(ValueError, match="positive"):
        W.install_serialized_fp8(fresh(), bad_scale, meta)
    # a refusal found past the first layers (the last layer's scale, the bf16
    # sweep) leaves every projection an nn.Linear and sets no attribute
    last = "layers.1.attn.o_proj.fp8_scale"
    for broken in (dict(state, **{last: -state[last]}),
                   dict(state, **{"layers.1.norm.weight": torch.ones(256, device=dev)})):
        d = fresh()
        with pytest.raises(ValueError):
            W.install_serialized_fp8(d, broken, meta)
        assert all(type(d.get_submodule(f"layers.{i}.{p}")) is nn.Linear
                   for i in range(2) for p in W.PIXELUMM_PROJECTIONS)
        assert not hasattr(d, "_prequantized_fp8")


class _Int8Stored(nn.Module):
    """Stand-in for the reference's Int8StoredBF16Linear
    (int8_stored_bf16_linear.py:64-89): int8 weight_q, fp32 group scales, bias."""

    def __init__(self, q, s, bias=None):
        super().__init__()
        self.register_buffer("weight_q", q)
        self.register_buffer("weight_scale", s)
        self.bias = bias


class _Int8Model(nn.Module):
    def __init__(self, t):
        super().__init__()
        self.a = _Int8Stored(t["a.weight_q"], t["a.weight_scale"], nn.Parameter(t["a.bias"], requires_grad=False))
        self.inner = nn.Sequential(_Int8Stored(t["b.weight_q"], t["b.weight_scale"]), nn.LayerNorm(256))
        # not a multiple of 128: left in place
        self.odd = _Int8Stored(torch.zeros(100, 256, dtype=torch.int8), torch.ones(100, 2))


def test_cache_int8_weights_recognises_only_int8_stored_layers(O):
    """The installer's resident-weight cache (hy_nomas_quantization.py:43-58)
    touches nothing in a model without INT8-stored layers."""
    qz = pkg_module("quantization")
    plain = nn.Sequential(nn.Linear(128, 128), nn.LayerNorm(128))
    assert qz.cache_int8_weights(plain) == {}
    assert isinstance(plain[0], nn.Linear)
    t = _tensors(O)
    assert qz._is_int8_stored(_Int8Stored(t["a.weight_q"], t["a.weight_scale"]))
    assert not qz._is_int8_stored(_Int8Stored(t["a.weight_q"].float(), t["a.weight_scale"]))
    assert not qz._is_int8_stored(_Int8Stored(t["a.weight_q"], t["a.weight_scale"][:, :1]))


def test_install_fp8_reference_call_form(monkeypatch):
    """install_fp8(source, cutlass, capability) as the reference's call site
    makes it (hy_nomas_quantization.py:35-40): gfx950's capability patches the
    reference's cutlass_fp8 module, any other raises ValueError first."""
    import sys
    import types
    from pathlib import Path
    qz = pkg_module("quantization")
    with pytest.raises(ValueError, match="gfx950"):
        qz.install_fp8(Path("/nonexistent/reference"), Path("/nonexistent/cutlass"), (10, 0))
    with pytest.raises(ValueError, match="gfx950"):
        qz.install_fp8(Path("/nonexistent/reference"), None, (8, 9))
    names = ["hymm", "hymm.models", "hymm.models.vae", "hymm.models.vae.pixelumm_decoder",
             "hymm.models.vae.pixelumm_decoder.cutlass_fp8"]
    mods = [types.ModuleType(n) for n in names]
    for parent, child, n in zip(mods, mods[1:], names[1:]):
        setattr(parent, n.rsplit(".", 1)[1], child)
    for n, m in zip(names, mods):
        monkeypatch.setitem(sys.modules, n, m)
    target = mods[-1]
    target.load_extension = lambda: "cutlass build"
    qz.install_fp8(Path("/nonexistent/reference"), None, qz.GFX950)
    assert type(target.load_extension()).__name__ == "HipFP8Extension"


@pytest.mark.gpu
def test_cache_int8_weights_makes_fp8_resident_layers(O, W, dev):
    """Every INT8-stored layer becomes an FP8StoredLinear whose codes are the
    per-channel e4m3 requantization of the reference's bf16 weight (bit-exact
    with the oracle), with its bias; the forward is the FP8 linear."""
    print("case cache_int8_weights", flush=True)
    qz = pkg_module("quantization")
    dl = pkg_module("dit_fp8_linear")
    t = _tensors(O)
    model = _Int8Model({k: v.to(dev) for k, v in t.items()}).to(dev)
    reports = qz.cache_int8_weights(model)
    assert sorted(reports) == ["a", "inner.0"]
    assert isinstance(model.a, dl.FP8StoredLinear) and isinstance(model.inner[0], dl.FP8StoredLinear)
    assert isinstance(model.odd, _Int8Stored)
    for name, m in (("a", model.a), ("b", model.inner[0])):
        w_bits = bf16_bits(W.dequantize_int8_weight(t[name + ".weight_q"], t[name + ".weight_scale"]))
        qo, so = O.quantize_rows_fp8(w_bits, O.SCALE_CLAMP)
        assert np.array_equal(u8(m.weight_q), qo) and np.array_equal(m.weight_scale.cpu().numpy(), so)
    assert reports["a"]["rel_l2"] < 0.05
    x = torch.randn(40, 256, device=dev).to(torch.bfloat16)
    with torch.no_grad():
        y = model.a(x)
    qx, sx = O.quantize_rows_fp8(bf16_bits(x))
    ref = O.linear_reference(qx, sx, u8(model.a.weight_q), model.a.weight_scale.cpu().numpy(),
                             O.bf16_bits_to_f32(bf16_bits(t["a.bias"])))
    assert_close_bf16(y.float().cpu().numpy(), ref, what="cached INT8 layer as FP8 linear")
