"""The connected MoE as a transformer's per-layer provider (the call shapes of src/vesper/backbone.py:63 and
src/vesper/block.py:43-92,140-147), on the GPU.

A fake backbone walks two layers, each a ConnectedMoE over its own store and fixtures: the MoE input of a
layer is the previous layer's residual stream (x + MoE(x), one BF16 rounding), passed as the flat BF16
vector the backbone passes, with image_span False. Every layer's routing equals the oracle's on the
kernel's logits (indices and weight bits) and its output is within the north-star tolerance of the oracle's
full layer (FP8 shared expert). A fake block opens around one provider the way the reference's block does --
device ledgers, the combined device cap and free floor, its own allocator wrapped around each ledger --
calls forward(x.reshape(H), image_span) for a text and an image-span token, and reshapes the output to
(1, 1, H).
"""

from contextlib import ExitStack

import numpy as np
import pytest

from oracle.formats import bf16_bits, bf16_values
from oracle.inputs import activations
from oracle.moe import moe_layer
from tests.helpers import assert_close, write_layer
from vesper_amd.connected import ConnectedConfig, ConnectedMoE
from vesper_amd.resources import GiB, MiB
from vesper_amd.store import ModelProfile
from vesper_amd.tiered import CacheConfig

pytestmark = pytest.mark.gpu

SMALL = ModelProfile("test/small-moe", "r1", 512, 256, 16, 3, 10.0, 48, 4, "sqrtsoftplus", 1.5, "0" * 64)


def config():
    cache = CacheConfig(host_cap_bytes=512 * MiB, ram_cache_bytes=2 * SMALL.expert_bytes, available_floor=GiB,
                        primary_slots=2, helper_device=None, helper_slots=0, integrity_mode="gpu-sha256",
                        max_store_experts=16, device_cap_bytes=256 * MiB)
    return ConnectedConfig(cache=cache, host_cap_bytes=1024 * MiB, device_free_floor=GiB)


def oracle_layer(art, hidden_bits, logits, image_span=False):
    bias = art["biases"]["bias_vl" if image_span else "bias"]
    return moe_layer(bf16_values(hidden_bits).reshape(1, -1), bf16_values(art["gate"]), art["experts"], art["shared"],
                     top_k=SMALL.top_k, route_scale=SMALL.route_scale, score_func=SMALL.score_func, bias=bias,
                     swiglu_limit=SMALL.swiglu_limit, shared_format="fp8", logits=np.asarray(logits).reshape(1, -1))


def check_layer(out, ref):
    np.testing.assert_array_equal(out["routing"]["indices"], ref["routing"]["indices"][0])
    np.testing.assert_array_equal(out["routing"]["weights"].view(np.uint32),
                                  ref["routing"]["weights"][0].view(np.uint32))
    assert_close(out["output_bf16"], ref["output_bf16"][0], "layer output")


def test_fake_backbone_walks_two_layers(direct_io_dir):
    rng = np.random.default_rng(51)
    arts = {layer: write_layer(direct_io_dir / f"layer{layer}", rng, SMALL, layer) for layer in (0, 1)}
    hidden = bf16_bits(activations(rng, 1, SMALL.hidden)[0])
    with ExitStack() as stack:
        moe = {layer: stack.enter_context(ConnectedMoE(*art["paths"], config(), layer=layer, model=SMALL))
               for layer, art in arts.items()}
        for layer in (0, 1):
            print(f"backbone layer {layer}", flush=True)
            values = hidden.reshape(SMALL.hidden)
            out = moe[layer].forward(values, False)
            assert moe[layer].layer == layer and out["output_bf16"].shape == (SMALL.hidden,)
            check_layer(out, oracle_layer(arts[layer], values, out["logits"]))
            hidden = bf16_bits(bf16_values(values) + bf16_values(out["output_bf16"]))
        assert all(m.snapshot()["calls"]["calls_completed"] == 1 for m in moe.values())


class FakeBlock:
    """A transformer block's view of its MoE provider: the open checks and device accounting around the MoE
    call of a block step, with a 512 MiB combined device cap."""

    CAP = 512 * MiB

    def __init__(self, moe, layer, ordinal=0):
        self.moe, self.layer, self.ordinal = moe, layer, ordinal
        self.peak = 0

    def __enter__(self):
        if self.moe.stack is None:
            raise ValueError("Block operators must be open on the same device")
        if self.moe.config.cache.primary_device != self.ordinal or self.moe.layer != self.layer:
            raise ValueError("MoE device or layer differs from the block's")
        self.devices = list(self.moe.devices.values())
        self.restore = []
        for device in self.devices:
            original = device.allocate

            def allocate(size, original=original):
                if self.owned() + size > self.CAP:
                    raise MemoryError("Block allocation exceeds the combined owned GPU cap")
                return original(size)
            device.allocate = allocate
            self.restore.append((device, original))
        self.headroom()
        return self

    def owned(self):
        return sum(sum(d.allocations.values()) for d in self.devices)

    def headroom(self):
        owned = self.owned()
        self.peak = max(self.peak, owned)
        if owned > self.CAP or any(d.memory()["free"] < d.free_floor for d in self.devices):
            raise MemoryError("Block refuses work below its device reserves")

    def ffn(self, x_bits, image_span):
        self.headroom()
        result = self.moe.forward(x_bits.reshape(-1), image_span)
        self.headroom()
        return result, result["output_bf16"].reshape(1, 1, -1)

    def __exit__(self, *_):
        for device, original in self.restore:
            device.allocate = original


def test_fake_block_step_calls(direct_io_dir):
    rng = np.random.default_rng(53)
    art = write_layer(direct_io_dir, rng, SMALL, 2)
    with ConnectedMoE(*art["paths"], config(), layer=2, model=SMALL) as moe:
        with pytest.raises(ValueError, match="differs"):
            with FakeBlock(moe, layer=1):
                pass
        with FakeBlock(moe, layer=2) as block:
            for image_span in (False, True):
                x = bf16_bits(activations(rng, 1, SMALL.hidden)).reshape(1, 1, SMALL.hidden)
                print(f"block step image_span={image_span}", flush=True)
                result, output = block.ffn(x, image_span)
                assert output.shape == (1, 1, SMALL.hidden)
                check_layer(result, oracle_layer(art, x.reshape(-1), result["logits"], image_span))
            assert 0 < block.peak <= FakeBlock.CAP
            pointer = moe.devices["shared"].allocate(4096)           # the block's wrapper sits in front
            moe.devices["shared"].free(pointer)
    with pytest.raises(ValueError, match="open"):
        with FakeBlock(moe, layer=2):
            pass
