"""The layer fixtures (vesper_amd.fixtures) and the connected call's host-side checks, no GPU.

Gate, router-bias and shared-expert fixtures written here reload bit for bit; every refusal of the reference's
loaders (src/vesper/gate.py:67-99, src/vesper/router.py:129-171, src/vesper/shared.py:35-138) is exercised on
a fixture damaged after writing; the reference's own pinned routing configuration and layer registration
(src/vesper/router.py:16-18, src/vesper/prefix_profile.py:4-9) are checked as constants.
"""

import json

import numpy as np
import pytest

from oracle.formats import bf16_bits
from oracle.inputs import fp8_block32_expert_normal, router_weight
from vesper_amd.connected import ConnectedConfig, ConnectedMoE, bf16_activation, validate_layer
from vesper_amd.fixtures import (load_gate_fixture, load_router_fixture, load_shared_fixture, shared_layout,
                                 write_gate_fixture, write_router_fixture, write_shared_fixture)
from vesper_amd.resources import MiB
from vesper_amd.store import REFERENCE_PROFILE, ModelProfile
from vesper_amd.tiered import CacheConfig

TINY = ModelProfile("test/tiny-moe", "r1", 512, 256, 16, 3, 10.0, 48, 4, "sqrtsoftplus", 1.5, "0" * 64)


def gate(rng, profile=TINY):
    return bf16_bits(router_weight(rng, profile.experts, profile.hidden))


def biases(rng, profile=TINY):
    return {n: rng.standard_normal(profile.experts).astype(np.float32) for n in ("bias", "bias_vl")}


def damage(path, edit):
    manifest = path.parent / "manifest.json"
    original = manifest.read_text()
    m = json.loads(original)
    edit(m)
    manifest.write_text(json.dumps(m))
    return original


def test_reference_constants():
    assert REFERENCE_PROFILE.router_config() == {"experts": 384, "topk": 6, "score_func": "sqrtsoftplus",
                                                 "gate_temp": 1.0, "norm_topk_prob": True, "route_scale": 1.5,
                                                 "normalization_epsilon": 1e-20}
    layout = shared_layout(REFERENCE_PROFILE)
    assert sum(int(np.prod(s)) for s in layout.values()) == 35_424_000       # the reference's SHARED_BYTES
    assert layout["w2_scale"] == (160, 72)
    for layer in (0, 2, 3, 20, 25):
        assert validate_layer(layer, REFERENCE_PROFILE) == layer
    for layer, profile in ((1, "qualified"), (4, "qualified"), (26, "token_prefix"), (40, "backbone_probe"),
                           (0, "other"), (True, "qualified")):
        with pytest.raises(ValueError, match="Unregistered"):
            validate_layer(layer, REFERENCE_PROFILE, profile)
    assert validate_layer(1, REFERENCE_PROFILE, "token_prefix") == 1
    assert validate_layer(39, REFERENCE_PROFILE, "backbone_probe") == 39
    assert validate_layer(2, TINY) == 2
    with pytest.raises(ValueError):
        validate_layer(3, TINY)


def test_gate_fixture_round_trip_and_refusals(tmp_path):
    rng = np.random.default_rng(1)
    weight = gate(rng)
    path = write_gate_fixture(tmp_path / "gate", 2, weight, TINY)
    got, manifest = load_gate_fixture(path, TINY)
    np.testing.assert_array_equal(got, weight)
    assert manifest["tensor"]["name"] == "layers.2.ffn.gate.weight" and manifest["layer"] == 2
    with pytest.raises(ValueError, match="pinned source"):
        load_gate_fixture(path)                                     # a TINY fixture is not the reference model
    for edit, message in ((lambda m: m.update(layer=3), "pinned backbone"),
                          (lambda m: m["tensor"].update(dtype="F32"), "identity/layout"),
                          (lambda m: m["tensor"].update(sha256="0" * 64), "source hash"),
                          (lambda m: m.update(kind="router_bias_fixture"), "pinned source")):
        original = damage(path, edit)
        with pytest.raises(ValueError, match=message):
            load_gate_fixture(path, TINY)
        (path.parent / "manifest.json").write_text(original)
    bad = weight.copy()
    bad[3, 7] = 0x7F80                                              # +inf
    with pytest.raises(ValueError, match="finite BF16"):
        write_gate_fixture(tmp_path / "bad", 0, bad, TINY)
    np.savez(path, weight=weight.astype(np.float32).view(np.uint32).astype(np.uint16))
    with pytest.raises(ValueError, match="source hash"):
        load_gate_fixture(path, TINY)
    np.savez(path, weight=weight, extra=weight[:1])
    with pytest.raises(ValueError, match="exactly"):
        load_gate_fixture(path, TINY)
    np.savez(path, weight=weight.astype(np.int16))
    with pytest.raises(ValueError, match="header"):
        load_gate_fixture(path, TINY)


def test_router_fixture_round_trip_and_refusals(tmp_path):
    rng = np.random.default_rng(2)
    arrays = biases(rng)
    path = write_router_fixture(tmp_path / "router", 1, arrays, TINY)
    got, manifest = load_router_fixture(path, TINY)
    for n in arrays:
        np.testing.assert_array_equal(got[n], arrays[n])
    assert manifest["config"] == TINY.router_config()
    for edit, message in ((lambda m: m["config"].update(topk=5), "configuration"),
                          (lambda m: m.update(inference_config_sha256="1" * 64), "configuration"),
                          (lambda m: m["tensors"].pop(), "Incomplete"),
                          (lambda m: m["tensors"][0].update(shape=[15]), "identity/layout"),
                          (lambda m: m["tensors"][1].update(sha256="f" * 64), "source hash")):
        original = damage(path, edit)
        with pytest.raises(ValueError, match=message):
            load_router_fixture(path, TINY)
        (path.parent / "manifest.json").write_text(original)
    with pytest.raises(ValueError, match="finite FP32"):
        write_router_fixture(tmp_path / "bad", 0, {"bias": arrays["bias"], "bias_vl": arrays["bias"] * np.inf}, TINY)
    np.savez(path, bias=arrays["bias"], bias_vl=arrays["bias_vl"].astype(np.float64))
    with pytest.raises(ValueError, match="header|exceeds"):
        load_router_fixture(path, TINY)


def test_shared_fixture_round_trip_and_refusals(tmp_path):
    rng = np.random.default_rng(3)
    arrays = fp8_block32_expert_normal(rng, TINY.hidden, TINY.intermediate)
    path = write_shared_fixture(tmp_path / "shared", 0, arrays, TINY)
    got, manifest = load_shared_fixture(path, TINY)
    for n in arrays:
        np.testing.assert_array_equal(got[n], arrays[n])
    assert {t["dtype"] for t in manifest["tensors"]} == {"F8_E4M3", "F8_E8M0"}
    for edit, message in ((lambda m: m.update(swiglu_limit=0.0), "pinned checkpoint"),
                          (lambda m: m["tensors"][2].update(tensor="layers.0.ffn.experts.0.w3.weight"),
                           "identity/layout"),
                          (lambda m: m["tensors"][5].update(sha256="abc"), "identity/layout"),
                          (lambda m: m["tensors"][4].update(sha256="0" * 64), "source hash"),
                          (lambda m: m.update(layer=-1), "pinned backbone")):
        original = damage(path, edit)
        with pytest.raises(ValueError, match=message):
            load_shared_fixture(path, TINY)
        (path.parent / "manifest.json").write_text(original)
    short = dict(arrays)
    short["w2_scale"] = short["w2_scale"][:-1]
    with pytest.raises(ValueError, match="FP8/block-32"):
        write_shared_fixture(tmp_path / "bad", 0, short, TINY)


def test_connected_host_checks():
    with pytest.raises(ValueError, match="component reservation"):
        ConnectedConfig(cache=CacheConfig(host_cap_bytes=256 * MiB, helper_device=None, helper_slots=0))
    config = ConnectedConfig()
    assert config.cache.helper_slots == 0 and config.cache.integrity_mode == "gpu-sha256"
    values, bits = bf16_activation(np.array([1.0, -2.5, 3.0e38, 0.0], np.float32).repeat(128), 512)
    assert bits.dtype == np.uint16 and values.shape == (512,) and bits[0] == 0x3F80
    with pytest.raises(ValueError, match="finite BF16"):
        bf16_activation(np.full(512, 0x7F80, np.uint16), 512)
    with pytest.raises(ValueError, match="per token"):
        bf16_activation(np.zeros(511, np.float32), 512)
    with pytest.raises(ValueError, match="per token"):
        bf16_activation(np.zeros(512, np.float64), 512)
    # the provider contract a block or backbone relies on, before anything is opened
    moe = ConnectedMoE("store", "gate.npz", "router.npz", "shared.npz", layer=2)
    assert moe.layer == 2 and moe.stack is None and moe.config.cache.primary_device == 0
    with pytest.raises(RuntimeError, match="context manager"):
        moe.forward(np.zeros(5120, np.float32))
    with pytest.raises(ValueError, match="BLAS"):
        ConnectedMoE("store", "gate.npz", "router.npz", "shared.npz", cublas_library="libcublas.so")
    with pytest.raises(ValueError, match="source factory"):
        ConnectedMoE("store", "gate.npz", "router.npz", "shared.npz", source_factory=3)
