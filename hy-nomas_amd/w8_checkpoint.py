"""On-disk quantized weight formats, read into the FP8 path.

Two families of files are accepted, with the checks the reference's loaders
apply (hymm/models/dit/modules/int8_stored_bf16_linear.py:13-18,121-306 and
hymm/models/vae/pixelumm_decoder/prequantized.py:6-65):

* **W8 DiT checkpoints**: per layer, INT8 codes ``<layer>.weight_q`` [out, in]
  and fp32 scales ``<layer>.weight_scale`` [out, ceil(in / 128)] (one per
  output row and 128-wide input group), every other tensor bf16 (or the
  model's own dtype). Three layouts hold them -- a single file with the
  "nomas-int8-bf16-single-v1" header, a single file with an embedded
  "nomas-dit-w8-bf16-v1" manifest and per-tensor sha256, or a manifest
  directory of sha256-checked shards. ``load_w8_as_fp8`` dequantizes each
  layer to the reference's bf16 weight and requantizes it per output
  channel to e4m3 on the GPU, with an accuracy report.
* **PixelUMM FP8 single files** ("pixelumm_fp8_bf16_single_v1"): e4m3
  128 x 128-block weights for the decoder's projections, installed as they
  are by ``install_serialized_fp8``.

The rules live in the tables below (header values, tensor geometry, shard
records); one checker applies them to every layout. Files are read with
safetensors only (no pickle).
"""
from __future__ import annotations

import hashlib
import json
from pathlib import Path
from typing import Callable, Optional

import torch
import torch.nn as nn
from safetensors import safe_open
from safetensors.torch import load_file

from . import _lib as L
from . import ops
from .dit_fp8_linear import FP8StoredLinear

GROUP_SIZE = 128
FORMAT = "nomas-dit-w8-bf16-v1"                     # manifest format (embedded or directory)
MANIFEST = "w8_bf16_manifest.json"                  # directory layout: manifest file name
SINGLE_FILE_MANIFEST = "w8_bf16_manifest"           # single file: metadata key of the manifest
NOMAS_SINGLE_FILE_FORMAT = "nomas-int8-bf16-single-v1"
PIXELUMM_FORMAT = "pixelumm_fp8_bf16_single_v1"

# Header values a "nomas-int8-bf16-single-v1" file must carry.
NOMAS_HEADER = {
    "group_size": str(GROUP_SIZE),
    "quantization": "symmetric_int8_absmax",
    "compute_dtype": "bfloat16",
    "rounding": "half_away_from_zero",
}

# Per quantized layer of shape [out, in]: tensor suffix -> (shape, safetensors
# dtype tag, torch dtype).
def _layer_tensors(out_f: int, in_f: int) -> dict:
    groups = (in_f + GROUP_SIZE - 1) // GROUP_SIZE
    return {".weight_q": ([out_f, in_f], "I8", torch.int8),
            ".weight_scale": ([out_f, groups], "F32", torch.float32)}


# PixelUMM FP8 single file: required metadata and the projections quantized in
# every decoder layer.
PIXELUMM_HEADER = {
    "format": PIXELUMM_FORMAT,
    "block_size": "128",
    "weight_dtype": "float8_e4m3fn",
    "scale_dtype": "float32",
}
PIXELUMM_PROJECTIONS = ("mlp.gate_proj", "mlp.up_proj", "mlp.down_proj", "attn.q_proj", "attn.o_proj")
PIXELUMM_BACKENDS = ("hip", "cutlass")   # "cutlass": the reference's name for this GEMM's role


# ---------------------------------------------------------------------------
# checksums

def _sha256_file(path: Path) -> str:
    h = hashlib.sha256()
    with path.open("rb") as f:
        while block := f.read(8 << 20):
            h.update(block)
    return h.hexdigest()


def tensor_sha256(tensor: torch.Tensor) -> str:
    """sha256 of a tensor's storage bytes on the CPU (what the embedded
    manifest records per tensor, bf16 and int8 alike)."""
    data = tensor.detach().cpu().contiguous().reshape(-1).view(torch.uint8).numpy()
    return hashlib.sha256(memoryview(data)).hexdigest()


def _hex_digest(value) -> bool:
    return isinstance(value, str) and len(value) == 64 and set(value) <= set("0123456789abcdef")


# ---------------------------------------------------------------------------
# manifest checks

def _check_layer_table(layers, what: str) -> dict:
    if not isinstance(layers, dict) or not layers:
        raise ValueError(f"{what} requires nonempty layers")
    for name, shape in layers.items():
        ok = (isinstance(name, str) and name and isinstance(shape, list) and len(shape) == 2
              and all(type(d) is int and d > 0 for d in shape))
        if not ok:
            raise ValueError(f"Invalid W8 layer name/shape: {name!r}")
    return layers


def _check_layer_tensors(layers: dict, keys, describe: Callable[[str], Optional[tuple]]) -> None:
    """Each listed layer has exactly its two tensors, of the table's shape and
    dtype; ``describe(key)`` gives (shape list, safetensors dtype tag) or None
    when the key is absent."""
    keys = set(keys)
    for suffix in (".weight_q", ".weight_scale"):
        if {k[: -len(suffix)] for k in keys if k.endswith(suffix)} != set(layers):
            raise ValueError(f"W8 layers do not match {suffix} tensor keys")
    for name, (out_f, in_f) in layers.items():
        for suffix, (shape, tag, _) in _layer_tensors(out_f, in_f).items():
            found = describe(name + suffix)
            if found is None:
                raise ValueError(f"Missing W8 tensor: {name + suffix}")
            if list(found[0]) != shape or found[1] != tag:
                raise ValueError(f"W8 tensor shape/dtype mismatch: {name + suffix}")


_TAG = {torch.int8: "I8", torch.float32: "F32", torch.bfloat16: "BF16", torch.float16: "F16",
        torch.uint8: "U8", torch.int32: "I32", torch.int64: "I64"}


def read_single_file_manifest(path, model_type=None) -> dict:
    """The manifest of a single-file W8 checkpoint, validated from its header
    and tensor index only (no payload read)."""
    with safe_open(str(path), framework="pt", device="cpu") as reader:
        meta = reader.metadata() or {}
        keys = set(reader.keys())

        def describe(key):
            if key not in keys:
                return None
            sl = reader.get_slice(key)
            return list(sl.get_shape()), sl.get_dtype()

        if SINGLE_FILE_MANIFEST in meta:
            # embedded manifest: always checksum-validated, whatever else the header says
            manifest = json.loads(meta[SINGLE_FILE_MANIFEST])
            if (not isinstance(manifest, dict) or manifest.get("format") != FORMAT
                    or manifest.get("group_size") != GROUP_SIZE
                    or not isinstance(manifest.get("model_type"), str)):
                raise ValueError("Unsupported single-file W8/BF16 metadata")
            if model_type is not None and manifest["model_type"] != model_type:
                raise ValueError("W8/BF16 model_type does not match configuration")
            sums = manifest.get("tensor_sha256")
            if not isinstance(sums, dict) or set(sums) != keys:
                raise ValueError("Single-file W8 tensor checksum keys do not match file tensors")
            if not all(_hex_digest(v) for v in sums.values()):
                raise ValueError("Invalid single-file W8 tensor checksum")
            _check_layer_tensors(_check_layer_table(manifest.get("layers"), "Single-file W8 metadata"),
                                 keys, describe)
            return manifest
        if meta.get("format") != NOMAS_SINGLE_FILE_FORMAT:
            raise ValueError("Single-file W8 checkpoint is missing supported embedded metadata")
        for key, want in NOMAS_HEADER.items():
            if meta.get(key) != want:
                raise ValueError(f"NOMAS INT8 checkpoint requires {key}={want}")
        declared = meta.get("model_type")
        if not isinstance(declared, str) or not declared.strip():
            raise ValueError("NOMAS INT8 checkpoint requires model_type metadata")
        if model_type is not None and declared != model_type:
            raise ValueError("NOMAS INT8 model_type does not match configuration")
        try:
            layers = json.loads(meta.get("layers", ""))
        except (TypeError, ValueError) as exc:
            raise ValueError("NOMAS INT8 layers metadata must be a JSON object") from exc
        _check_layer_tensors(_check_layer_table(layers, "NOMAS INT8 metadata"), keys, describe)
        return {"format": NOMAS_SINGLE_FILE_FORMAT, "group_size": GROUP_SIZE,
                "model_type": declared, "layers": layers}


def _check_shard(root: Path, shard, seen: set) -> Path:
    if not isinstance(shard, dict):
        raise ValueError("Invalid shard record")
    name = shard.get("file")
    if not isinstance(name, str) or Path(name).name != name or not name.endswith(".safetensors"):
        raise ValueError("Unsafe W8/BF16 shard path")
    path = (root / name).resolve()
    if name in seen or not path.is_relative_to(root):
        raise ValueError("Duplicate or escaping W8/BF16 shard path")
    seen.add(name)
    size, digest = shard.get("bytes"), shard.get("sha256")
    if type(size) is not int or size <= 0 or not _hex_digest(digest):
        raise ValueError("Invalid shard byte count or checksum")
    if path.stat().st_size != size or _sha256_file(path) != digest:
        raise ValueError(f"W8/BF16 shard checksum mismatch: {name}")
    return path


def read_manifest_dir(root, model_type) -> dict:
    """The manifest of a W8 directory: format, shard paths confined to the
    directory, byte count and sha256 of every shard. The layer tensors'
    geometry is checked when the shards are read (load_w8_as_fp8)."""
    root = Path(root).resolve()
    manifest = json.loads((root / MANIFEST).read_text())
    if manifest.get("format") != FORMAT or manifest.get("group_size") != GROUP_SIZE:
        raise ValueError("Unsupported W8/BF16 manifest format or group_size")
    if manifest.get("model_type") != model_type:
        raise ValueError("W8/BF16 model_type does not match configuration")
    layers, shards = manifest.get("layers"), manifest.get("shards")
    if not isinstance(layers, dict) or not layers or not isinstance(shards, list) or not shards:
        raise ValueError("Manifest requires nonempty layers and shards")
    _check_layer_table(layers, "W8 manifest")
    seen: set = set()
    for shard in shards:
        _check_shard(root, shard, seen)
    return manifest


def read_w8_manifest(checkpoint, model_type=None):
    """(manifest, files, per-tensor checksums or None) of a file or directory."""
    path = Path(checkpoint).expanduser().resolve()
    if path.is_file():
        manifest = read_single_file_manifest(path, model_type)
        return manifest, [path], manifest.get("tensor_sha256")
    manifest = read_manifest_dir(path, model_type)
    return manifest, [path / s["file"] for s in manifest["shards"]], None


# ---------------------------------------------------------------------------
# INT8 -> FP8

def dequantize_int8_weight(weight_q: torch.Tensor, weight_scale: torch.Tensor) -> torch.Tensor:
    """The weight the reference computes with: bf16(code * scale of its
    128-wide input group), [out, in] (int8_stored_bf16_linear.py:82-88)."""
    out_f, in_f = weight_q.shape
    per_column = weight_scale.float().repeat_interleave(GROUP_SIZE, dim=1)[:, :in_f]
    return (weight_q.float() * per_column).to(torch.bfloat16)


@torch.no_grad()
def requantize_int8_to_fp8(weight_q: torch.Tensor, weight_scale: torch.Tensor, device):
    """Per-output-channel e4m3 codes and fp32 scales of the reference's bf16
    weight, quantized on the GPU (s = max(amax, 1e-4) / 448), with a report
    of the FP8 weight against that bf16 weight: rel-L2, max-abs and the
    largest per-channel rel-L2."""
    w = dequantize_int8_weight(weight_q.to(device), weight_scale.to(device))
    codes, scale = ops.quantize_rows_fp8(w, L.HN_SCALE_CLAMP, 1e-4)
    ref = w.float()
    err = codes.float() * scale[:, None] - ref
    total = torch.linalg.vector_norm(ref)
    per_row = torch.linalg.vector_norm(err, dim=1) / torch.linalg.vector_norm(ref, dim=1).clamp_min(1e-30)
    report = {"rel_l2": float(torch.linalg.vector_norm(err) / total) if total > 0 else 0.0,
              "max_abs": float(err.abs().max()),
              "max_channel_rel_l2": float(per_row.max())}
    return codes, scale, report


def _rebuild_derived_buffers(model: nn.Module, rebuild: Optional[Callable[[nn.Module], None]]) -> None:
    """Buffers a checkpoint leaves out (non-persistent tables such as RoPE
    frequencies) are rebuilt after loading: by ``rebuild(model)`` if given,
    and by every module's own ``rebuild_derived_buffers()`` method. Any buffer
    still on the meta device afterwards is an error (the reference's
    _restore_derived_buffers, int8_stored_bf16_linear.py:232-244)."""
    if rebuild is not None:
        rebuild(model)
    for module in model.modules():
        hook = getattr(module, "rebuild_derived_buffers", None)
        if callable(hook) and any(b.is_meta for b in module.buffers(recurse=False)):
            hook()
    still_meta = [name for name, buf in model.named_buffers() if buf.is_meta]
    if still_meta:
        raise ValueError(f"Unmaterialized model buffers: {still_meta[:5]}")


def load_w8_as_fp8(model_factory, model_type, checkpoint, device,
                   rebuild_buffers: Optional[Callable[[nn.Module], None]] = None) -> tuple[nn.Module, dict]:
    """Load a W8 checkpoint with every listed Linear as an FP8StoredLinear.

    The model is built on the meta device; the listed layers must be its
    Linear modules with matching shapes. Every file is validated before any
    GPU work (checksums, layer tensor geometry, finite values, positive
    scales); the other tensors load strictly (bf16 accepted for floating
    tensors); omitted non-persistent buffers are rebuilt. Returns (model,
    {layer: requantization report})."""
    manifest, files, checksums = read_w8_manifest(checkpoint, model_type)
    with torch.device("meta"):
        model = model_factory()
    if any(not p.is_meta for p in model.parameters()):
        raise ValueError("W8/BF16 model_factory must construct parameters on meta")
    linear_shapes = {n: list(m.weight.shape) for n, m in model.named_modules() if isinstance(m, nn.Linear)}
    layers = manifest["layers"]
    if any(linear_shapes.get(n) != shape for n, shape in layers.items()):
        raise ValueError("W8/BF16 layer names/shapes do not match model Linear modules")

    tensors: dict = {}
    for f in files:
        for key, t in load_file(str(f), device="cpu").items():
            if key in tensors:
                raise ValueError(f"Duplicate W8/BF16 tensor: {key}")
            if checksums is not None and tensor_sha256(t) != checksums[key]:
                raise ValueError(f"Single-file W8 tensor checksum mismatch: {key}")
            if t.is_floating_point() and not bool(torch.isfinite(t).all()):
                raise ValueError(f"Nonfinite W8/BF16 tensor: {key}")
            tensors[key] = t
    # the same geometry check for every layout (the directory's shards are
    # only now read)
    _check_layer_tensors(layers, tensors.keys(),
                         lambda k: None if k not in tensors else (list(tensors[k].shape),
                                                                  _TAG.get(tensors[k].dtype, "?")))
    for name in layers:
        if not bool((tensors[name + ".weight_scale"] > 0).all()):
            raise ValueError(f"Invalid quantization scales: {name}.weight_scale")

    reports = {}
    for name in layers:
        codes, scale, reports[name] = requantize_int8_to_fp8(
            tensors.pop(name + ".weight_q"), tensors.pop(name + ".weight_scale"), device)
        original = model.get_submodule(name)
        bias = tensors.pop(name + ".bias", None)
        if (bias is None) != (original.bias is None):
            raise ValueError(f"W8/BF16 bias presence mismatch: {name}")
        layer = FP8StoredLinear.from_codes(codes, scale, None if bias is None else bias.to(device))
        owner, _, attr = name.rpartition(".")
        setattr(model.get_submodule(owner) if owner else model, attr, layer)

    expected = {k: v for k, v in model.state_dict().items() if v.is_meta}
    extra, absent = set(tensors) - set(expected), set(expected) - set(tensors)
    if extra:
        raise ValueError(f"Unexpected W8/BF16 tensors: {sorted(extra)[:5]}")
    if absent:
        raise ValueError(f"Missing W8/BF16 tensors: {sorted(absent)[:5]}")
    for key, t in tensors.items():
        want = expected[key]
        dtype_ok = t.dtype == want.dtype or (want.dtype.is_floating_point and t.dtype == torch.bfloat16)
        if tuple(t.shape) != tuple(want.shape) or not dtype_ok:
            raise ValueError(f"W8/BF16 tensor shape/dtype mismatch: {key}")
    model.load_state_dict({k: t.to(device) for k, t in tensors.items()}, strict=False, assign=True)
    _rebuild_derived_buffers(model, rebuild_buffers)
    model.to(device)
    model.eval().requires_grad_(False)
    return model, reports


# ---------------------------------------------------------------------------
# PixelUMM FP8 single files

def is_prequantized_pixelumm(path) -> bool:
    with safe_open(str(path), framework="pt", device="cpu") as reader:
        return (reader.metadata() or {}).get("format") == PIXELUMM_FORMAT


def install_serialized_fp8(decoder: nn.Module, state: dict, metadata: dict, backend: str = "hip") -> int:
    """Put the serialized e4m3 weights of a PixelUMM FP8 file into the
    decoder's projections (PIXELUMM_PROJECTIONS of every layer) as FP8Linear
    modules, unchanged. The metadata must match PIXELUMM_HEADER and declare
    exactly those layers; every target must be a bias-free nn.Linear whose
    serialized tensors pass validate_serialized_tensors; every other tensor of
    the state must be bf16. Returns the number of layers installed.

    The rules and their messages are the reference's
    (pixelumm_decoder/prequantized.py:27-65), checked in the same order; here
    every rule is checked, and every FP8Linear built, before the first layer
    is replaced, so a refused file leaves the decoder as it was."""
    if backend not in PIXELUMM_BACKENDS:
        raise ValueError("Unsupported serialized PixelUMM FP8 backend: " + str(backend))
    if any(metadata.get(k) != v for k, v in PIXELUMM_HEADER.items()):
        raise ValueError("Unsupported PixelUMM FP8 checkpoint metadata")
    paths = [f"layers.{i}.{p}" for i in range(len(decoder.layers)) for p in PIXELUMM_PROJECTIONS]
    _check_pixelumm_manifest(metadata, paths)
    plan = [(path, _serialized_fp8_linear(decoder, state, path)) for path in paths]
    stray = next((k for k, t in state.items()
                  if not k.endswith((".fp8_weight", ".fp8_scale")) and t.dtype != torch.bfloat16), None)
    if stray is not None:
        raise ValueError("Expected BF16 unquantized tensor: " + stray)
    for path, module in plan:
        owner, _, attr = path.rpartition(".")
        setattr(decoder.get_submodule(owner), attr, module)
    decoder._prequantized_fp8_backend = backend
    decoder._prequantized_fp8 = True
    decoder._prequantized_fp8_layers = len(plan)
    return len(plan)


def _check_pixelumm_manifest(metadata: dict, paths: list) -> None:
    """The file's manifest names exactly the decoder's projection weights."""
    declared = json.loads(metadata.get("quantized_source_keys", "[]"))
    wanted = {f"decoder.{t}.weight" for t in paths}
    if (len(declared) != len(wanted) or set(declared) != wanted
            or int(metadata.get("quantized_layers", -1)) != len(paths)):
        raise ValueError("Incomplete or incompatible PixelUMM FP8 layer manifest")


def _serialized_fp8_linear(decoder: nn.Module, state: dict, path: str):
    """The FP8Linear that replaces the bias-free nn.Linear at `path`, built
    from its serialized codes and block scales (validated by from_quantized)."""
    from .pixelumm_fp8 import FP8Linear
    layer = decoder.get_submodule(path)
    if not isinstance(layer, nn.Linear) or layer.bias is not None:
        raise ValueError("Expected a bias-free PixelUMM linear: " + path)
    return FP8Linear.from_quantized(state[path + ".fp8_weight"], state[path + ".fp8_scale"], layer.weight.shape)
