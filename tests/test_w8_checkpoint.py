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
