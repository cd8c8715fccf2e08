"""A layer's resident weights as the reference's fixture pairs: the gate matrix, the router biases and the
shared expert, each an .npz archive with a manifest.json beside it (src/vesper/gate.py:22-99,
src/vesper/router.py:129-171, src/vesper/shared.py:20-138).

Formats (the reference's, so a fixture written by either side loads in the other):

* gate: kind "gate_projection_fixture", tensor {name "layers.<l>.ffn.gate.weight", dtype BF16, shape
  [experts, hidden], bytes, sha256}; archive member weight.npy, uint16 BF16 bits, finite.
* router: kind "router_bias_fixture", config (the routing configuration) and inference_config_sha256 equal to
  the model's; tensors bias and bias_vl {tensor "layers.<l>.ffn.gate.<name>", dtype F32, shape [experts],
  bytes, sha256}; archive members bias.npy / bias_vl.npy, float32, finite.
* shared: kind "shared_expert_fp8", swiglu_limit; six tensors "<p>_weight" [rows, width] F8_E4M3 and
  "<p>_scale" [rows/32, width/32] F8_E8M0 (one scale per 32 x 32 block) with p in w1, w3 (rows = intermediate,
  width = hidden) and w2 (rows = hidden, width = intermediate); archive members uint8.

Every loader checks the model identity (a ModelProfile: the reference's pinned checkpoint by default), the
layer range, each tensor's name / dtype / shape / bytes, every archive member's NPY header before NumPy
allocates, and each tensor's SHA-256, in that order; writers record the same fields, so fixtures for the
synthetic stores this build benchmarks are made the way the reference's fetchers make theirs.
"""

from __future__ import annotations

import hashlib
import json
import re
from pathlib import Path

import numpy as np

from .store import REFERENCE_PROFILE, ModelProfile, read_bounded_npz, read_manifest

GATE_KIND, ROUTER_KIND, SHARED_KIND = "gate_projection_fixture", "router_bias_fixture", "shared_expert_fp8"
BIAS_NAMES = ("bias", "bias_vl")


def _sha(array) -> str:
    return hashlib.sha256(memoryview(np.ascontiguousarray(array)).cast("B")).hexdigest()


def _layer(manifest: dict, profile: ModelProfile) -> int:
    layer = manifest.get("layer")
    if type(layer) is not int or not 0 <= layer < profile.layers:
        raise ValueError("Fixture layer is outside the pinned backbone")
    return layer


def _identity(manifest: dict, kind: str, profile: ModelProfile, message: str):
    if (manifest.get("kind"), manifest.get("model"), manifest.get("revision")) != (kind, profile.model,
                                                                                   profile.revision):
        raise ValueError(message)


def _write(directory: Path, archive: str, arrays: dict, manifest: dict) -> Path:
    directory = Path(directory)
    directory.mkdir(parents=True, exist_ok=True)
    np.savez(directory / archive, **arrays)
    (directory / "manifest.json").write_text(json.dumps(manifest, indent=2) + "\n", encoding="utf-8")
    return directory / archive


# ---- gate -------------------------------------------------------------------------------------------------

def gate_shape(profile: ModelProfile = REFERENCE_PROFILE) -> tuple:
    return (profile.experts, profile.hidden)


def validate_gate_weight(weight, profile: ModelProfile = REFERENCE_PROFILE):
    """The gate matrix as finite BF16 bits of the model's shape (gate.py:62-64)."""
    if (not isinstance(weight, np.ndarray) or weight.dtype != np.uint16 or weight.shape != gate_shape(profile)
            or np.any((weight & 0x7F80) == 0x7F80)):
        raise ValueError("Gate weight must contain the original finite BF16 matrix")


def write_gate_fixture(directory: Path, layer: int, weight, profile: ModelProfile = REFERENCE_PROFILE) -> Path:
    validate_gate_weight(weight, profile)
    _layer({"layer": layer}, profile)
    manifest = {"kind": GATE_KIND, "model": profile.model, "revision": profile.revision, "layer": layer,
                "tensor": {"name": f"layers.{layer}.ffn.gate.weight", "dtype": "BF16", "shape": list(weight.shape),
                           "bytes": weight.nbytes, "sha256": _sha(weight)}, "source": "synthetic"}
    return _write(directory, "native-gate.npz", {"weight": weight}, manifest)


def load_gate_fixture(path: Path, profile: ModelProfile = REFERENCE_PROFILE):
    """(BF16 weight bits [experts, hidden], manifest) -- the checks of gate.py:67-99."""
    path = Path(path)
    shape = gate_shape(profile)
    nbytes = shape[0] * shape[1] * 2
    if path.stat().st_size > nbytes + 64 * 1024:
        raise ValueError("Gate archive exceeds its bounded fixture size")
    manifest = read_manifest(path)
    _identity(manifest, GATE_KIND, profile, "Gate fixture differs from the pinned source")
    layer = _layer(manifest, profile)
    tensor = manifest.get("tensor", {})
    if (tensor.get("name"), tensor.get("dtype"), tensor.get("shape"), tensor.get("bytes")) != (
            f"layers.{layer}.ffn.gate.weight", "BF16", list(shape), nbytes):
        raise ValueError("Gate tensor identity/layout differs from the fixture")
    weight = read_bounded_npz(path, {"weight": (shape, np.uint16)}, "Gate")["weight"]
    validate_gate_weight(weight, profile)
    if _sha(weight) != tensor.get("sha256"):
        raise ValueError("Gate weight differs from its original source hash")
    return weight, manifest


# ---- router biases ----------------------------------------------------------------------------------------

def validate_router_arrays(arrays: dict, profile: ModelProfile = REFERENCE_PROFILE):
    if set(arrays) != set(BIAS_NAMES):
        raise ValueError("Router fixture requires the text and image-span biases")
    for array in arrays.values():
        if (not isinstance(array, np.ndarray) or array.dtype != np.float32 or array.shape != (profile.experts,)
                or not np.isfinite(array).all()):
            raise ValueError(f"Router bias must contain {profile.experts} finite FP32 values")


def write_router_fixture(directory: Path, layer: int, arrays: dict,
                         profile: ModelProfile = REFERENCE_PROFILE) -> Path:
    validate_router_arrays(arrays, profile)
    _layer({"layer": layer}, profile)
    tensors = [{"name": n, "tensor": f"layers.{layer}.ffn.gate.{n}", "dtype": "F32", "shape": [profile.experts],
                "bytes": 4 * profile.experts, "sha256": _sha(arrays[n])} for n in BIAS_NAMES]
    manifest = {"kind": ROUTER_KIND, "model": profile.model, "revision": profile.revision, "layer": layer,
                "config": profile.router_config(), "inference_config_sha256": profile.inference_config_sha256,
                "tensors": tensors, "source": "synthetic"}
    return _write(directory, "native-router.npz", {n: arrays[n] for n in BIAS_NAMES}, manifest)


def load_router_fixture(path: Path, profile: ModelProfile = REFERENCE_PROFILE):
    """({bias, bias_vl}, manifest) -- the checks of router.py:129-171."""
    path = Path(path)
    e = profile.experts
    if path.stat().st_size > 2 * 4 * e + 8192:
        raise ValueError("Router archive exceeds its bounded fixture size")
    manifest = read_manifest(path)
    if ((manifest.get("kind"), manifest.get("model"), manifest.get("revision"), manifest.get("config"),
         manifest.get("inference_config_sha256"))
            != (ROUTER_KIND, profile.model, profile.revision, profile.router_config(),
                profile.inference_config_sha256)):
        raise ValueError("Router fixture differs from the pinned source/configuration")
    layer = _layer(manifest, profile)
    entries = manifest.get("tensors", [])
    if len(entries) != 2 or {t.get("name") for t in entries} != set(BIAS_NAMES):
        raise ValueError("Incomplete router provenance")
    arrays = read_bounded_npz(path, {n: ((e,), np.float32) for n in BIAS_NAMES}, "Router")
    validate_router_arrays(arrays, profile)
    for entry in entries:
        name = entry["name"]
        if (entry.get("tensor"), entry.get("dtype"), entry.get("shape"), entry.get("bytes")) != (
                f"layers.{layer}.ffn.gate.{name}", "F32", [e], 4 * e):
            raise ValueError("Router tensor identity/layout differs from its manifest")
        if _sha(arrays[name]) != entry.get("sha256"):
            raise ValueError("Router bias differs from its original source hash")
    return arrays, manifest


# ---- shared expert ----------------------------------------------------------------------------------------

def shared_layout(profile: ModelProfile = REFERENCE_PROFILE) -> dict:
    """{name: shape} of the FP8 block-32 shared expert (shared.py:20-24)."""
    h, i = profile.hidden, profile.intermediate
    shapes = {"w1": (i, h), "w3": (i, h), "w2": (h, i)}
    return {f"{p}_{s}": (rows, width) if s == "weight" else (rows // 32, width // 32)
            for p, (rows, width) in shapes.items() for s in ("weight", "scale")}


def validate_shared_arrays(arrays: dict, profile: ModelProfile = REFERENCE_PROFILE):
    layout = shared_layout(profile)
    if set(arrays) != set(layout):
        raise ValueError("A shared expert requires exactly six native tensors")
    for name, shape in layout.items():
        a = arrays[name]
        if not isinstance(a, np.ndarray) or a.dtype != np.uint8 or a.shape != shape:
            raise ValueError("Shared tensor differs from the pinned FP8/block-32 layout")


def _shared_entry(layer: int, name: str, shape) -> tuple:
    projection, suffix = name.split("_")
    return (f"layers.{layer}.ffn.shared_experts.{projection}.{suffix}",
            "F8_E4M3" if suffix == "weight" else "F8_E8M0", list(shape), int(np.prod(shape)))


def validate_shared_provenance(manifest: dict, profile: ModelProfile = REFERENCE_PROFILE):
    """The checks of shared.py:35-53."""
    if (manifest.get("model"), manifest.get("revision"), manifest.get("kind"), manifest.get("swiglu_limit")) != (
            profile.model, profile.revision, SHARED_KIND, profile.swiglu_limit):
        raise ValueError("Shared provenance differs from the pinned checkpoint")
    layer = _layer(manifest, profile)
    layout = shared_layout(profile)
    entries = manifest.get("tensors", [])
    if len(entries) != 6 or {e.get("name") for e in entries} != set(layout):
        raise ValueError("Incomplete shared fixture provenance")
    for entry in entries:
        name = entry["name"]
        if ((entry.get("tensor"), entry.get("dtype"), entry.get("shape"), entry.get("bytes"))
                != _shared_entry(layer, name, layout[name])
                or not re.fullmatch(r"[0-9a-f]{64}", entry.get("sha256", ""))):
            raise ValueError("Shared tensor provenance differs from its pinned identity/layout")


def write_shared_fixture(directory: Path, layer: int, arrays: dict,
                         profile: ModelProfile = REFERENCE_PROFILE) -> Path:
    validate_shared_arrays(arrays, profile)
    _layer({"layer": layer}, profile)
    tensors = []
    for name in shared_layout(profile):
        tensor, dtype, shape, nbytes = _shared_entry(layer, name, arrays[name].shape)
        tensors.append({"name": name, "tensor": tensor, "dtype": dtype, "shape": shape, "bytes": nbytes,
                        "sha256": _sha(arrays[name])})
    manifest = {"kind": SHARED_KIND, "model": profile.model, "revision": profile.revision, "layer": layer,
                "swiglu_limit": profile.swiglu_limit, "tensors": tensors, "source": "synthetic"}
    return _write(directory, "native-shared.npz", {n: arrays[n] for n in shared_layout(profile)}, manifest)


def load_shared_fixture(path: Path, profile: ModelProfile = REFERENCE_PROFILE):
    """(six uint8 arrays, manifest) -- the checks of shared.py:108-138."""
    path = Path(path)
    manifest = read_manifest(path)
    validate_shared_provenance(manifest, profile)
    layout = shared_layout(profile)
    if path.stat().st_size > sum(int(np.prod(s)) for s in layout.values()) + 64 * 1024:
        raise ValueError("Shared archive exceeds its bounded fixture size")
    arrays = read_bounded_npz(path, {n: (s, np.uint8) for n, s in layout.items()}, "Shared")
    validate_shared_arrays(arrays, profile)
    for entry in manifest["tensors"]:
        if _sha(arrays[entry["name"]]) != entry["sha256"]:
            raise ValueError("Shared fixture bytes differ from their source hash")
    return arrays, manifest
