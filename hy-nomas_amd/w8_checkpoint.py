"""On-disk quantized weight formats into the FP8 path.

Ingests the reference's W8 DiT checkpoints -- INT8 codes per output channel x
128-wide input group with fp32 scales -- and the PixelUMM FP8 single-file
format, validating them the way the reference loader does
(hymm/models/dit/modules/int8_stored_bf16_linear.py:13-18,121-306 and
hymm/models/vae/pixelumm_decoder/prequantized.py:6-65):

  * ``read_w8_manifest``      <- _read_single_file_manifest / _read_manifest:
    the single-file "nomas-int8-bf16-single-v1" header, the embedded
    "nomas-dit-w8-bf16-v1" manifest (per-tensor sha256) and the manifest
    directory (sha256 per shard).
  * ``dequantize_int8_weight`` <- Int8StoredBF16Linear.dequant_weight (:82-88):
    W = bf16(q * repeat(scale, 128)), the weight the reference computes with.
  * ``requantize_int8_to_fp8``: that W -> per-output-channel e4m3 codes and
    fp32 scales (max(amax, 1e-4) / 448, the row quantizer on the GPU), plus an
    accuracy report of the FP8 weight against W.
  * ``load_w8_as_fp8``        <- load_w8_bf16_model (:247-306): builds the model
    on the meta device, swaps every listed Linear for an FP8StoredLinear from
    the requantized codes, loads the other tensors strictly, checks scales,
    finiteness and checksums.
  * ``install_serialized_fp8`` <- prequantized.install_serialized_fp8 (:29-65).

Files are read with safetensors only (no pickle).
"""
from __future__ import annotations

import hashlib
import json
from pathlib import Path

import torch
import torch.nn as nn
from safetensors import safe_open
from safetensors.torch import load_file

from . import _lib as L
from . import ops
from .dit_fp8_linear import FP8StoredLinear

FORMAT = "nomas-dit-w8-bf16-v1"
GROUP_SIZE = 128
MANIFEST = "w8_bf16_manifest.json"
SINGLE_FILE_MANIFEST = "w8_bf16_manifest"
NOMAS_SINGLE_FILE_FORMAT = "nomas-int8-bf16-single-v1"
PIXELUMM_FORMAT = "pixelumm_fp8_bf16_single_v1"


def _sha256_file(path: Path) -> str:
    digest = hashlib.sha256()
    with path.open("rb") as handle:
        for chunk in iter(lambda: handle.read(8 << 20), b""):
            digest.update(chunk)
    return digest.hexdigest()


def tensor_sha256(tensor: torch.Tensor) -> str:
    """sha256 of a tensor's exact CPU bytes (bf16 and int8 storage included)."""
    raw = tensor.detach().cpu().contiguous().reshape(-1).view(torch.uint8).numpy()
    return hashlib.sha256(memoryview(raw)).hexdigest()


def _is_hex64(s) -> bool:
    return isinstance(s, str) and len(s) == 64 and all(c in "0123456789abcdef" for c in s)


def _check_layers(layers, reader_keys, reader):
    if not isinstance(layers, dict) or not layers:
        raise ValueError("W8 checkpoint metadata requires nonempty layers")
    for name, shape in layers.items():
        if (not isinstance(name, str) or not name or not isinstance(shape, list) or len(shape) != 2
                or any(type(d) is not int or d <= 0 for d in shape)):
            raise ValueError(f"Invalid W8 layer name/shape: {name!r}")
    for suffix in (".weight_q", ".weight_scale"):
        if {k[: -len(suffix)] for k in reader_keys if k.endswith(suffix)} != set(layers):
            raise ValueError(f"W8 layers do not match {suffix} tensor keys")
    for name, (out_f, in_f) in layers.items():
        for suffix, shape, dtype in ((".weight_q", [out_f, in_f], "I8"),
                                     (".weight_scale", [out_f, (in_f + GROUP_SIZE - 1) // GROUP_SIZE], "F32")):
            sl = reader.get_slice(name + suffix)
            if list(sl.get_shape()) != shape or sl.get_dtype() != dtype:
                raise ValueError(f"W8 tensor shape/dtype mismatch: {name + suffix}")


def read_single_file_manifest(path, model_type=None) -> dict:
    """Validate the header of a single-file W8 checkpoint (either format)."""
    with safe_open(str(path), framework="pt", device="cpu") as reader:
        meta = reader.metadata() or {}
        keys = set(reader.keys())
        if SINGLE_FILE_MANIFEST not in meta:
            if meta.get("format") != NOMAS_SINGLE_FILE_FORMAT:
                raise ValueError("Single-file W8 checkpoint is missing supported embedded metadata")
            for key, expected in (("group_size", str(GROUP_SIZE)),
                                  ("quantization", "symmetric_int8_absmax"),
                                  ("compute_dtype", "bfloat16"),
                                  ("rounding", "half_away_from_zero")):
                if meta.get(key) != expected:
                    raise ValueError(f"NOMAS INT8 checkpoint requires {key}={expected}")
            declared = meta.get("model_type")
            if not isinstance(declared, str) or not declared.strip():
                raise ValueError("NOMAS INT8 checkpoint requires model_type metadata")
            if model_type is not None and declared != model_type:
                raise ValueError("NOMAS INT8 model_type does not match configuration")
            try:
                layers = json.loads(meta.get("layers", ""))
            except (TypeError, ValueError) as exc:
                raise ValueError("NOMAS INT8 layers metadata must be a JSON object") from exc
            _check_layers(layers, keys, reader)
            return {"format": NOMAS_SINGLE_FILE_FORMAT, "group_size": GROUP_SIZE,
                    "model_type": declared, "layers": layers}
        manifest = json.loads(meta[SINGLE_FILE_MANIFEST])
        if (not isinstance(manifest, dict) or manifest.get("format") != FORMAT
                or manifest.get("group_size") != GROUP_SIZE
                or not isinstance(manifest.get("model_type"), str)):
            raise ValueError("Unsupported single-file W8/BF16 metadata")
        if model_type is not None and manifest["model_type"] != model_type:
            raise ValueError("W8/BF16 model_type does not match configuration")
        checksums = manifest.get("tensor_sha256")
        if not isinstance(checksums, dict) or set(checksums) != keys:
            raise ValueError("Single-file W8 tensor checksum keys do not match file tensors")
        if not all(_is_hex64(c) for c in checksums.values()):
            raise ValueError("Invalid single-file W8 tensor checksum")
        _check_layers(manifest.get("layers"), keys, reader)
        return manifest


def read_manifest_dir(root, model_type) -> dict:
    """Validate a W8 manifest directory: format, shards inside the directory,
    byte counts and sha256 of every shard."""
    root = Path(root).resolve()
    manifest = json.loads((root / MANIFEST).read_text())
    if manifest.get("format") != FORMAT or manifest.get("group_size") != GROUP_SIZE:
        raise ValueError("Unsupported W8/BF16 manifest format or group_size")
    if manifest.get("model_type") != model_type:
        raise ValueError("W8/BF16 model_type does not match configuration")
    layers, shards = manifest.get("layers"), manifest.get("shards")
    if not isinstance(layers, dict) or not layers or not isinstance(shards, list) or not shards:
        raise ValueError("Manifest requires nonempty layers and shards")
    seen = set()
    for shard in shards:
        if not isinstance(shard, dict):
            raise ValueError("Invalid shard record")
        name = shard.get("file")
        if not isinstance(name, str) or Path(name).name != name or not name.endswith(".safetensors"):
            raise ValueError("Unsafe W8/BF16 shard path")
        path = (root / name).resolve()
        if not path.is_relative_to(root) or name in seen:
            raise ValueError("Duplicate or escaping W8/BF16 shard path")
        seen.add(name)
        if type(shard.get("bytes")) is not int or shard["bytes"] <= 0 or not _is_hex64(shard.get("sha256")):
            raise ValueError("Invalid shard byte count or checksum")
        if path.stat().st_size != shard["bytes"] or _sha256_file(path) != shard["sha256"]:
            raise ValueError(f"W8/BF16 shard checksum mismatch: {name}")
    return manifest


def read_w8_manifest(checkpoint, model_type=None):
    """(manifest, files, per-tensor checksums or None) for a file or a directory."""
    path = Path(checkpoint).expanduser().resolve()
    if path.is_file():
        manifest = read_single_file_manifest(path, model_type)
        return manifest, [path], manifest.get("tensor_sha256")
    manifest = read_manifest_dir(path, model_type)
    return manifest, [path / s["file"] for s in manifest["shards"]], None


def dequantize_int8_weight(weight_q: torch.Tensor, weight_scale: torch.Tensor) -> torch.Tensor:
    """The reference's dequantized weight: bf16(q_f32 * repeat(scale, 128)) [N, K]."""
    n, k = weight_q.shape
    scale = weight_scale.float().repeat_interleave(GROUP_SIZE, dim=1)[:, :k]
    return (weight_q.float() * scale).to(torch.bfloat16)


@torch.no_grad()
def requantize_int8_to_fp8(weight_q: torch.Tensor, weight_scale: torch.Tensor, device):
    """INT8 (per channel x 128 group) -> FP8 per-output-channel, on the GPU.

    Returns (codes e4m3 [N, K], scales fp32 [N], report). The FP8 weight is
    quantized from the reference's own bf16 weight, so its codes are those of
    quantize_weight applied to that weight; the report compares the FP8
    weight with it: rel-L2, max-abs and max per-channel rel-L2."""
    w = dequantize_int8_weight(weight_q.to(device), weight_scale.to(device))
    codes, scale = ops.quantize_rows_fp8(w, L.HN_SCALE_CLAMP, 1e-4)
    w32 = w.float()
    err = codes.float() * scale[:, None] - w32
    norm = torch.linalg.vector_norm(w32)
    per_ch = torch.linalg.vector_norm(err, dim=1) / torch.linalg.vector_norm(w32, dim=1).clamp_min(1e-30)
    report = {"rel_l2": float(torch.linalg.vector_norm(err) / norm) if norm > 0 else 0.0,
              "max_abs": float(err.abs().max()),
              "max_channel_rel_l2": float(per_ch.max())}
    return codes, scale, report


def load_w8_as_fp8(model_factory, model_type, checkpoint, device) -> tuple[nn.Module, dict]:
    """Load a W8 checkpoint with every listed Linear as an FP8StoredLinear.

    Mirrors load_w8_bf16_model: the model is built on the meta device, listed
    layers must match the model's Linear names and shapes, every other tensor
    is loaded strictly (bf16 allowed for floating tensors), scales must be
    finite and positive, floating tensors finite, and per-tensor checksums
    are verified when the file carries them. Returns (model, {layer: report})."""
    manifest, files, checksums = read_w8_manifest(checkpoint, model_type)
    with torch.device("meta"):
        model = model_factory()
    if any(not t.is_meta for t in model.parameters()):
        raise ValueError("W8/BF16 model_factory must construct parameters on meta")
    linears = {name: list(m.weight.shape) for name, m in model.named_modules() if isinstance(m, nn.Linear)}
    if any(name not in linears or shape != linears[name] for name, shape in manifest["layers"].items()):
        raise ValueError("W8/BF16 layer names/shapes do not match model Linear modules")
    tensors = {}
    for f in files:
        for key, t in load_file(str(f), device="cpu").items():
            if key in tensors:
                raise ValueError(f"Duplicate W8/BF16 tensor: {key}")
            if checksums is not None and tensor_sha256(t) != checksums[key]:
                raise ValueError(f"Single-file W8 tensor checksum mismatch: {key}")
            if t.is_floating_point() and not torch.isfinite(t).all():
                raise ValueError(f"Nonfinite W8/BF16 tensor: {key}")
            tensors[key] = t
    reports = {}
    for name in manifest["layers"]:
        q, s = tensors.pop(name + ".weight_q"), tensors.pop(name + ".weight_scale")
        if not torch.all(s > 0):
            raise ValueError(f"Invalid quantization scales: {name}.weight_scale")
        codes, scale, reports[name] = requantize_int8_to_fp8(q, s, device)
        original = model.get_submodule(name)
        bias = tensors.pop(name + ".bias", None)
        if (bias is None) != (original.bias is None):
            raise ValueError(f"W8/BF16 bias presence mismatch: {name}")
        module = FP8StoredLinear.from_codes(codes, scale, None if bias is None else bias.to(device))
        parent, _, leaf = name.rpartition(".")
        setattr(model.get_submodule(parent) if parent else model, leaf, module)
    expected = {k: v for k, v in model.state_dict().items() if v.is_meta}
    unexpected = set(tensors) - set(expected)
    if unexpected:
        raise ValueError(f"Unexpected W8/BF16 tensors: {sorted(unexpected)[:5]}")
    missing = set(expected) - set(tensors)
    if missing:
        raise ValueError(f"Missing W8/BF16 tensors: {sorted(missing)[:5]}")
    for key, t in tensors.items():
        want = expected[key]
        ok_dtype = t.dtype == want.dtype or (want.dtype.is_floating_point and t.dtype == torch.bfloat16)
        if tuple(t.shape) != tuple(want.shape) or not ok_dtype:
            raise ValueError(f"W8/BF16 tensor shape/dtype mismatch: {key}")
    model.load_state_dict({k: t.to(device) for k, t in tensors.items()}, strict=False, assign=True)
    model.eval().requires_grad_(False)
    return model, reports


def is_prequantized_pixelumm(path) -> bool:
    with safe_open(str(path), framework="pt", device="cpu") as handle:
        return (handle.metadata() or {}).get("format") == PIXELUMM_FORMAT


def install_serialized_fp8(decoder: nn.Module, state: dict, metadata: dict) -> int:
    """Install FP8 linears from a PixelUMM FP8/BF16 single-file state: the
    decoder's five MLP/attention projections per layer, validated like the
    reference (metadata, complete layer manifest, bias-free targets,
    serialized tensor shapes/scales, bf16 for everything else)."""
    from .pixelumm_fp8 import FP8Linear
    if (metadata.get("format") != PIXELUMM_FORMAT or metadata.get("block_size") != "128"
            or metadata.get("weight_dtype") != "float8_e4m3fn"
            or metadata.get("scale_dtype") != "float32"):
        raise ValueError("Unsupported PixelUMM FP8 checkpoint metadata")
    targets = [f"layers.{i}.{name}" for i in range(len(decoder.layers))
               for name in ("mlp.gate_proj", "mlp.up_proj", "mlp.down_proj", "attn.q_proj", "attn.o_proj")]
    declared = json.loads(metadata.get("quantized_source_keys", "[]"))
    expected = {"decoder." + name + ".weight" for name in targets}
    if (set(declared) != expected or len(declared) != len(expected)
            or int(metadata.get("quantized_layers", -1)) != len(targets)):
        raise ValueError("Incomplete or incompatible PixelUMM FP8 layer manifest")
    for name in targets:
        linear = decoder.get_submodule(name)
        if not isinstance(linear, nn.Linear) or linear.bias is not None:
            raise ValueError("Expected a bias-free PixelUMM linear: " + name)
        module = FP8Linear.from_quantized(state[name + ".fp8_weight"], state[name + ".fp8_scale"],
                                          linear.weight.shape)
        parent, _, leaf = name.rpartition(".")
        setattr(decoder.get_submodule(parent), leaf, module)
    for key, tensor in state.items():
        if not key.endswith((".fp8_weight", ".fp8_scale")) and tensor.dtype != torch.bfloat16:
            raise ValueError("Expected BF16 unquantized tensor: " + key)
    return len(targets)
