"""GPU parity of the store-backed boundary: TieredExpertRuntime(store, CacheConfig) and
ConnectedMoE(store, gate_fixture, router_fixture, shared_fixture, config) (src/vesper/tiered.py:130-216,
src/vesper/connected.py:56-213).

* TieredExpertRuntime at the reference model's shapes, in both integrity modes: every call's stage dict is
  bit-identical to ResidentExpert on the same expert, whichever tier (store, RAM, GPU slot) served it; the
  tier sequence, read counts and audit byte counters are the exclusive-tier policy's; a byte flipped in the
  store file is refused.
* ConnectedMoE over a 16-expert store and fixtures written here: logits, routing and the routed sum before
  the shared expert are bit-identical to the resident decode layer (MoELayer without a shared expert) on
  the same weights, for one token and for five; the output is that sum plus the FP8 shared expert's BF16
  rows, rounded once; a second call served from other tiers returns the same bits; the image-span bias
  selects differently and matches the layer built on that bias; experts missing from the store are refused
  before any store read, and the next call succeeds; a store read failing in the middle of a call fails
  that call only.
"""

import numpy as np
import pytest

from oracle.formats import bf16_bits, bf16_values
from oracle.inputs import activations, mxfp4_expert
from tests.helpers import write_layer
from vesper_amd.config import MoEConfig
from vesper_amd.connected import ConnectedConfig, ConnectedMoE
from vesper_amd.expert import ResidentExpert
from vesper_amd.layer import ExpertBank, MoELayer
from vesper_amd.resources import GiB, MiB
from vesper_amd.store import REFERENCE_PROFILE, ModelProfile, NativeStore, build_store
from vesper_amd.tiered import CacheConfig, TieredExpertRuntime

pytestmark = pytest.mark.gpu

SMALL = ModelProfile("test/small-moe", "r1", 512, 256, 16, 3, 10.0, 48, 4, "sqrtsoftplus", 1.5, "0" * 64)
LAYER = 1


def cache_config(mode, slots, ram_experts, profile, max_store):
    return CacheConfig(host_cap_bytes=512 * MiB, ram_cache_bytes=ram_experts * profile.expert_bytes,
                       available_floor=GiB, primary_slots=slots, helper_device=None, helper_slots=0,
                       integrity_mode=mode, max_store_experts=max_store, device_cap_bytes=256 * MiB)


@pytest.mark.parametrize("mode", ["readback", "gpu-sha256"])
def test_tiered_runtime_over_store_matches_resident_expert(direct_io_dir, mode):
    rng = np.random.default_rng(31)
    experts = {e: mxfp4_expert(rng, REFERENCE_PROFILE.hidden, REFERENCE_PROFILE.intermediate) for e in (3, 7, 9)}
    store = direct_io_dir / "store"
    build_store([(0, e, a) for e, a in experts.items()], store, max_experts=4)
    x = activations(rng, 1, REFERENCE_PROFILE.hidden)[0]
    weight = np.float32(0.37)
    expected = {}
    for e, arrays in experts.items():
        with ResidentExpert(arrays) as resident:
            expected[e] = resident.forward(x, weight)
    order = [3, 7, 3, 9, 7]
    size = REFERENCE_PROFILE.expert_bytes
    with TieredExpertRuntime(store, cache_config(mode, 1, 1, REFERENCE_PROFILE, 4)) as runtime:
        tiers = []
        for e in order:
            print(f"tiered {mode} expert 0:{e}", flush=True)
            got = runtime.forward(f"0:{e}", x, weight)
            tiers.append(runtime.last_event["source_tier"])
            for name, ref in expected[e].items():
                np.testing.assert_array_equal(got[name], ref[0], err_msg=f"{e} {name}")
        assert tiers == ["store", "store", "ram", "store", "store"]
        snap = runtime.snapshot()
        assert snap["primary_keys"] == ["0:7"] and snap["ram_keys"] == ["0:9"]
        assert (snap["store_direct_read_calls"], snap["store_direct_read_bytes"]) == (4, 4 * size)
        c = snap["counters"]
        assert (c["ram_hits"], c["primary_evictions"], c["ram_capacity_evictions"]) == (1, 4, 2)
        if mode == "gpu-sha256":
            assert c["primary_gpu_audit_payload_bytes"] == 5 * size and c["primary_audit_readback_bytes"] == 0
        else:
            assert c["primary_audit_readback_bytes"] == 5 * size and c["cpu_checks_deferred"] == 0
        with pytest.raises(KeyError):
            runtime.forward("0:4", x, weight)
    assert runtime.cleanup["host_buffer_reservations_bytes"] == 0
    # one flipped byte inside expert 9 (the third entry): that read is refused, the others still serve
    data = store / "experts.bin"
    raw = bytearray(data.read_bytes())
    raw[2 * size + 12345] ^= 0x10
    data.write_bytes(bytes(raw))
    with TieredExpertRuntime(store, cache_config(mode, 1, 0, REFERENCE_PROFILE, 4)) as runtime:
        np.testing.assert_array_equal(runtime.forward("0:3", x, weight)["w2"], expected[3]["w2"][0])
        with pytest.raises(ValueError, match="hash"):
            runtime.forward("0:9", x, weight)
        assert runtime.snapshot()["counters"]["integrity_failures"] == 1


@pytest.mark.parametrize("mode", ["readback", "gpu-sha256"])
def test_tiered_runtime_batch_prefetch_matches_resident_expert(direct_io_dir, mode):
    """TieredExpertRuntime.prefetch promotes a batch through the store's read-ahead pipeline (reads and host
    checks of later experts beside the uploads and audits of earlier ones): every expert lands in its own
    slot, and the calls that follow are GPU hits whose stage dicts equal ResidentExpert's bit for bit."""
    rng = np.random.default_rng(37)
    ids = (2, 5, 6, 11)
    experts = {e: mxfp4_expert(rng, REFERENCE_PROFILE.hidden, REFERENCE_PROFILE.intermediate) for e in ids}
    store = direct_io_dir / "store"
    build_store([(0, e, a) for e, a in experts.items()], store, max_experts=4)
    x = activations(rng, 1, REFERENCE_PROFILE.hidden)[0]
    weight = np.float32(0.61)
    with TieredExpertRuntime(store, cache_config(mode, 4, 0, REFERENCE_PROFILE, 4)) as runtime:
        print(f"tiered {mode} batch prefetch", flush=True)
        assert runtime.prefetch([f"0:{e}" for e in ids]) == ["store"] * 4
        for e in ids:
            got = runtime.forward(f"0:{e}", x, weight)
            assert runtime.last_event["source_tier"] == "primary_gpu"
            with ResidentExpert(experts[e]) as resident:
                ref = resident.forward(x, weight)
            for name, value in ref.items():
                np.testing.assert_array_equal(got[name], value[0], err_msg=f"{e} {name}")
        c = runtime.snapshot()["counters"]
        assert c["store_reads_completed"] == 4 and c["primary_hits"] == 4 and c["integrity_failures"] == 0
    assert runtime.cleanup["host_buffer_reservations_bytes"] == 0


class Resident:
    """The decode layer on the same weights, no shared expert: its output is the routed sum rounded once."""

    def __init__(self, ctx, experts, gate, bias):
        cfg = MoEConfig(hidden=SMALL.hidden, intermediate=SMALL.intermediate, experts=SMALL.experts,
                        top_k=SMALL.top_k, score_func=SMALL.score_func, route_scale=SMALL.route_scale,
                        swiglu_limit=SMALL.swiglu_limit, shared=None)
        self.bank = ExpertBank(ctx, cfg, cfg.experts)
        for n, arrays in experts.items():
            self.bank.upload(n, arrays)
        self.layer = MoELayer(ctx, cfg, bf16_values(gate), self.bank, bias=bias)

    def decode(self, bits):
        out = self.layer.decode(bits.reshape(-1, SMALL.hidden), diagnostics=True)
        t, e, k = out.shape[0], SMALL.experts, SMALL.top_k
        return out, {"logits": self.layer.read("logits", (t, e), np.float32),
                     "indices": self.layer.read("indices", (t, k), np.int32),
                     "weights": self.layer.read("weights", (t, k), np.float32)}

    def close(self):
        self.layer.close()
        self.bank.free()


def check_call(out, resident, bits):
    ref_out, ref = resident.decode(bits)
    t = ref_out.shape[0]
    np.testing.assert_array_equal(np.asarray(out["logits"]).reshape(t, -1).view(np.uint32),
                                  ref["logits"].view(np.uint32))
    np.testing.assert_array_equal(np.asarray(out["routing"]["indices"]).reshape(t, -1), ref["indices"])
    np.testing.assert_array_equal(np.asarray(out["routing"]["weights"]).reshape(t, -1).view(np.uint32),
                                  ref["weights"].view(np.uint32))
    agg = out["aggregation"]
    before = np.asarray(agg["before_shared_fp32"]).reshape(t, -1)
    np.testing.assert_array_equal(bf16_bits(before), ref_out)
    shared = np.asarray(out["shared"]["w2"]).reshape(t, -1)
    np.testing.assert_array_equal(np.asarray(out["output_bf16"]).reshape(t, -1),
                                  bf16_bits(before + bf16_values(shared)))
    return ref["indices"]


@pytest.mark.parametrize("mode", ["readback", "gpu-sha256"])
def test_connected_moe_over_store_matches_decode_layer(gpu_ctx, direct_io_dir, mode):
    rng = np.random.default_rng(41)
    layer = write_layer(direct_io_dir, rng, SMALL, LAYER)
    paths, experts, gate, biases = layer["paths"], layer["experts"], layer["gate"], layer["biases"]
    config = ConnectedConfig(cache=cache_config(mode, 2, 2, SMALL, 16), host_cap_bytes=1024 * MiB,
                             device_free_floor=GiB)
    one = bf16_bits(activations(rng, 1, SMALL.hidden)[0])
    five = bf16_bits(activations(rng, 5, SMALL.hidden))
    text = Resident(gpu_ctx, experts, gate, biases["bias"])
    image = Resident(gpu_ctx, experts, gate, biases["bias_vl"])
    try:
        with ConnectedMoE(*paths, config, layer=LAYER, model=SMALL) as moe:
            print(f"connected {mode}: one token", flush=True)
            first = moe.forward(one)
            assert first["output_bf16"].shape == (SMALL.hidden,) and first["routing"]["indices"].shape == (4,)
            indices = check_call(first, text, one)
            assert [ev["source_tier"] for ev in first["expert_events"]] == ["store"] * 4
            assert sorted(first["experts"]) == sorted(indices[0].tolist())
            print(f"connected {mode}: same token again", flush=True)
            again = moe.forward(one)
            # two GPU slots and a two-expert RAM tier: the first call left its first two experts in RAM and
            # its last two in the slots; each expert of the repeat is promoted from RAM, demoting the oldest
            assert [ev["source_tier"] for ev in again["expert_events"]] == ["ram"] * 4
            np.testing.assert_array_equal(again["output_bf16"], first["output_bf16"])
            print(f"connected {mode}: five tokens", flush=True)
            check_call(moe.forward(five), text, five)
            print(f"connected {mode}: image span", flush=True)
            vl = moe.forward(one, image_span=True)
            check_call(vl, image, one)
            snap = moe.snapshot()
            assert snap["calls"] == {"calls_started": 4, "calls_completed": 4, "calls_failed": 0}
            assert snap["cache"]["integrity_mode"] == mode
            assert moe.last_attempt["status"] == "pass" and moe.last_attempt["image_span"] is True
        assert moe.cleanup["parent_reservation_bytes"] == 0 and moe.cleanup["cache_reservation_bytes"] == 0
    finally:
        text.close()
        image.close()


def test_connected_moe_refuses_missing_experts_before_reading(gpu_ctx, direct_io_dir):
    rng = np.random.default_rng(43)
    # text routing never selects experts 8-15 (bias -100), image-span routing always prefers them (+100)
    high = (np.arange(SMALL.experts) >= 8).astype(np.float32) * 100
    layer = write_layer(direct_io_dir, rng, SMALL, LAYER, range(8), {"bias": -high, "bias_vl": high})
    paths, experts, gate, biases = layer["paths"], layer["experts"], layer["gate"], layer["biases"]
    config = ConnectedConfig(cache=cache_config("gpu-sha256", 2, 2, SMALL, 16), host_cap_bytes=1024 * MiB,
                             device_free_floor=GiB)
    x = bf16_bits(activations(rng, 1, SMALL.hidden)[0])
    text = Resident(gpu_ctx, experts, gate, biases["bias"])
    try:
        with ConnectedMoE(*paths, config, layer=LAYER, model=SMALL) as moe:
            with pytest.raises(KeyError, match="absent"):
                moe.forward(x, image_span=True)
            attempt = moe.last_attempt
            assert attempt["status"] == "failed" and attempt["completed_expert_ids"] == []
            assert attempt["store_direct_read_calls"] == 0
            check_call(moe.forward(x), text, x)                      # a fresh accumulator after the refusal
            with pytest.raises(ValueError, match="boolean"):
                moe.forward(x, image_span=1)
            assert moe.snapshot()["calls"] == {"calls_started": 2, "calls_completed": 1, "calls_failed": 1}
        with pytest.raises(ValueError, match="Unregistered"):
            ConnectedMoE(*paths, config, layer=3, model=SMALL)
        with pytest.raises(ValueError, match="selected layer"):
            with ConnectedMoE(*paths, config, layer=0, model=SMALL):
                pass
    finally:
        text.close()


class FailingStore(NativeStore):
    """A store whose n-th expert read fails once with OSError (an injected device-read fault)."""

    def __init__(self, *args, fail_at=3, **kwargs):
        super().__init__(*args, **kwargs)
        self.fail_at, self.reads = fail_at, 0

    def read_into(self, key, target):
        self.reads += 1
        if self.reads == self.fail_at:
            raise OSError("injected read failure")
        return super().read_into(key, target)


def test_connected_moe_injected_read_failure_then_fresh_call(gpu_ctx, direct_io_dir):
    """The reference's injected-expert-failure case (tests/test_connected.py:35-70 of the reference): a read
    failing in the middle of a call fails that call with the experts completed so far recorded and publishes
    nothing; the next call starts from a zeroed accumulator and matches the resident layer."""
    rng = np.random.default_rng(47)
    layer = write_layer(direct_io_dir, rng, SMALL, LAYER)
    paths, experts, gate, biases = layer["paths"], layer["experts"], layer["gate"], layer["biases"]
    config = ConnectedConfig(cache=cache_config("gpu-sha256", 2, 2, SMALL, 16), host_cap_bytes=1024 * MiB,
                             device_free_floor=GiB)
    x = bf16_bits(activations(rng, 1, SMALL.hidden)[0])
    text = Resident(gpu_ctx, experts, gate, biases["bias"])

    def factory(path, budget):
        return FailingStore(path, budget, max_experts=16, profile=SMALL, fail_at=3)
    try:
        with ConnectedMoE(*paths, config, layer=LAYER, model=SMALL, source_factory=factory) as moe:
            with pytest.raises(OSError, match="injected"):
                moe.forward(x)
            attempt = moe.last_attempt
            assert attempt["status"] == "failed" and len(attempt["completed_expert_ids"]) == 2
            check_call(moe.forward(x), text, x)
            assert moe.snapshot()["calls"] == {"calls_started": 2, "calls_completed": 1, "calls_failed": 1}
        assert moe.cleanup["parent_reservation_bytes"] == 0 and moe.cleanup["cache_reservation_bytes"] == 0
    finally:
        text.close()
