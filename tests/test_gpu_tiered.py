"""GPU tests of host-pinned expert streaming (ExpertCache / PooledExpertRuntime / OffloadDecode).

The cache moves bytes and never touches the arithmetic, so every result through it must equal the resident
path bit for bit: the tiered single-expert call against ResidentExpert, and a chain of MoE layers whose
experts stream through a cache too small to hold them (evictions on every step) against the same layers
with every expert resident.
"""

import ctypes as C

import numpy as np
import pytest

from oracle.formats import bf16_bits
from oracle.inputs import activations, mxfp4_expert
from vesper_amd import _lib
from vesper_amd.config import MoEConfig
from vesper_amd.expert import ResidentExpert
from vesper_amd.layer import ExpertBank, MoELayer
from vesper_amd.tiered import (ExpertCache, HostExpertPool, OffloadDecode, PooledExpertRuntime, decode_routed,
                               expert_key)

pytestmark = pytest.mark.gpu


def test_cache_lru_order_and_slot_bytes(gpu_ctx):
    size = 4096
    host = gpu_ctx.host_alloc_pinned(size * 5)
    view = np.ctypeslib.as_array((C.c_uint8 * (size * 5)).from_address(host))
    for i in range(5):
        view[i * size:(i + 1) * size] = np.random.default_rng(i).integers(0, 256, size, dtype=np.uint8)
    cache = ExpertCache(gpu_ctx, size, 3)
    try:
        for i in range(4):
            cache.register(i, host + i * size)
        a, b, c, d = 0, 1, 2, 3

        def ensure(keys):
            ptrs, hits = cache.ensure(keys)
            cache.wait_ready(None)
            gpu_ctx.sync()
            for k, p in zip(keys, ptrs):
                np.testing.assert_array_equal(gpu_ctx.download(p, (size,), np.uint8), view[k * size:(k + 1) * size])
            return list(hits)

        assert ensure([a, b]) == [0, 0]
        assert ensure([c]) == [0]
        assert ensure([d]) == [0]            # evicts a (least recent)
        assert ensure([b]) == [1]
        assert ensure([a]) == [0]            # evicts c; b and d stay
        assert ensure([d, b]) == [1, 1]
        st = cache.stats()
        assert (st["hits"], st["misses"], st["resident"]) == (3, 5, 3)
        with pytest.raises(ValueError):
            cache.ensure([a, a])
        with pytest.raises(ValueError):
            cache.ensure([a, b, c, d])       # more keys than slots
        with pytest.raises(ValueError):
            cache.ensure([9])                # unregistered
        with pytest.raises(ValueError):
            cache.register(7, np.zeros(size, np.uint8).ctypes.data)   # pageable memory is refused
    finally:
        cache.close()
        gpu_ctx.host_free_pinned(host)


def test_pooled_runtime_matches_resident_expert(gpu_ctx):
    cfg = MoEConfig(hidden=512, intermediate=256, experts=4, top_k=1, swiglu_limit=10.0, shared=None)
    rng = np.random.default_rng(12)
    arrays = [mxfp4_expert(rng, cfg.hidden, cfg.intermediate) for _ in range(4)]
    pool = HostExpertPool(gpu_ctx, cfg, 4)
    staging = ExpertBank(gpu_ctx, cfg, 1)
    try:
        for i, arr in enumerate(arrays):
            pool.upload_arrays(i, arr, staging)
        rt = PooledExpertRuntime(gpu_ctx, cfg, pool, {f"0:{i}": i for i in range(4)}, slots=2)
        x = activations(rng, 3, cfg.hidden)
        tiers = []
        try:
            for key in ("0:1", "0:1", "0:2", "0:3", "0:1"):
                got = rt.forward(key, x, 0.75)
                tiers.append(rt.last_event["source_tier"])
                idx = int(key.split(":")[1])
                with ResidentExpert(arrays[idx], swiglu_limit=10.0, hidden=cfg.hidden,
                                    intermediate=cfg.intermediate) as ref:
                    want = ref.forward(x, 0.75)
                for name in want:
                    np.testing.assert_array_equal(np.asarray(got[name]).view(np.uint8),
                                                  np.asarray(want[name]).view(np.uint8), err_msg=f"{key} {name}")
            with pytest.raises(KeyError):
                rt.forward("1:0", x)
        finally:
            rt.close()
        assert tiers == ["host_pinned", "primary_gpu", "host_pinned", "host_pinned", "host_pinned"]
    finally:
        staging.free()
        pool.close()


def test_gpu_sha256_admission_audit(gpu_ctx):
    """audit=True (the gpu-sha256 mode): every admitted slot is hashed on the device against its source's digest
    table before the expert runs. A source byte flipped after its table was taken makes the next admission
    fail (ValueError) and the slot is dropped, never served; with the byte restored the key is admitted
    afresh and computes what the resident expert computes."""
    cfg = MoEConfig(hidden=512, intermediate=256, experts=3, top_k=1, swiglu_limit=10.0, shared=None)
    rng = np.random.default_rng(21)
    arrays = [mxfp4_expert(rng, cfg.hidden, cfg.intermediate) for _ in range(3)]
    pool = HostExpertPool(gpu_ctx, cfg, 3)
    staging = ExpertBank(gpu_ctx, cfg, 1)
    try:
        for i, arr in enumerate(arrays):
            pool.upload_arrays(i, arr, staging)
        gpu_ctx.sync()
        rt = PooledExpertRuntime(gpu_ctx, cfg, pool, {f"0:{i}": i for i in range(3)}, slots=2, audit=True)
        x = activations(rng, 2, cfg.hidden)
        try:
            for key in ("0:1", "0:0", "0:2"):                   # 0:1 admitted, then evicted
                rt.forward(key, x, 0.5)
            snap = rt.snapshot()
            assert snap["integrity_failures"] == 0 and snap["gpu_audit_payload_bytes"] == 3 * pool.expert_bytes
            src = np.ctypeslib.as_array((C.c_uint8 * pool.expert_bytes).from_address(pool.ptr(1)))
            offset = pool.expert_bytes // 3
            src[offset] ^= 0x10
            with pytest.raises(ValueError, match="differ"):
                rt.forward("0:1", x, 0.5)
            assert rt.snapshot()["integrity_failures"] == 1
            src[offset] ^= 0x10
            got = rt.forward("0:1", x, 0.5)
            assert rt.last_event["source_tier"] == "host_pinned"   # the failed slot was not kept
            with ResidentExpert(arrays[1], swiglu_limit=10.0, hidden=cfg.hidden, intermediate=cfg.intermediate) as ref:
                want = ref.forward(x, 0.5)
            np.testing.assert_array_equal(np.asarray(got["w2"]), np.asarray(want["w2"]))
            rt.forward("0:1", x, 0.5)
            assert rt.last_event["source_tier"] == "primary_gpu"   # hits are not re-audited
            assert rt.snapshot()["gpu_audit_payload_bytes"] == 4 * pool.expert_bytes
        finally:
            rt.close()
    finally:
        staging.free()
        pool.close()


@pytest.mark.parametrize("audit", [False, True])
def test_offload_decode_equals_resident_layers(gpu_ctx, audit):
    """With audit=True every admitted slot is also verified on the copy stream (mx_sha256_verify) against
    digest tables taken on the device from the pinned sources: a clean run passes check_audit, and a source
    byte flipped before a forced admission is reported, dropped from the cache, and passes once restored."""
    cfg = MoEConfig(hidden=512, intermediate=256, experts=16, top_k=4, swiglu_limit=10.0, shared="mxfp4",
                    max_tokens=4)
    L, T, steps = 3, 4, 3
    rng = np.random.default_rng(2026)
    arrays = [[mxfp4_expert(rng, cfg.hidden, cfg.intermediate) for _ in range(cfg.experts + 1)] for _ in range(L)]
    banks, layers = [], []
    pool = HostExpertPool(gpu_ctx, cfg, L * cfg.experts)
    cache = ExpertCache(gpu_ctx, pool.expert_bytes, 20)   # 48 routed keys through 20 slots
    try:
        for l in range(L):
            bank = ExpertBank(gpu_ctx, cfg, cfg.experts + 1)
            for e in range(cfg.experts + 1):
                bank.upload(e, arrays[l][e])
            for e in range(cfg.experts):
                pool.fill_from_bank(bank, e, l * cfg.experts + e)
            banks.append(bank)
            layers.append(MoELayer(gpu_ctx, cfg, np.zeros((cfg.experts, cfg.hidden), np.float32), bank))
        off = OffloadDecode(gpu_ctx, cfg, L, lambda l, e: (pool, l * cfg.experts + e),
                            [banks[l].tiled_ptr(cfg.experts) for l in range(L)], cache, banks[0].tiled_ptr(0),
                            audit=audit)
        x = gpu_ctx.upload(bf16_bits(activations(rng, T, cfg.hidden)))
        ys = [gpu_ctx.empty((T, cfg.hidden), np.uint16) for _ in range(L)]
        ref_ys = [gpu_ctx.empty((T, cfg.hidden), np.uint16) for _ in range(L)]
        try:
            for step in range(steps):
                routing = []
                for l in range(L):
                    ids = np.stack([rng.choice(cfg.experts, cfg.top_k, replace=False) for _ in range(T)]).astype(np.int32)
                    w = rng.uniform(0.1, 1.0, (T, cfg.top_k)).astype(np.float32)
                    routing.append((ids, w))
                off.load_routing(routing)
                off.step_device(x.ptr, T, [y.ptr for y in ys], [r[0] for r in routing])
                gpu_ctx.sync(off.stream)
                for l in range(L):
                    src = x.ptr if l == 0 else ref_ys[l - 1].ptr
                    decode_routed(layers[l], src, T, off.ids[l].ptr, off.wts[l].ptr, ref_ys[l].ptr)
                gpu_ctx.sync()
                for l in range(L):
                    np.testing.assert_array_equal(ys[l].download(), ref_ys[l].download(), err_msg=f"step {step} layer {l}")
            st = cache.stats()
            assert st["misses"] > 20 and st["hits"] > 0
            if audit:
                off.check_audit()
                assert off.audited_slots == st["misses"]
                ids = np.tile(np.array([3, 5, 7, 9], np.int32), (T, 1))
                routing = [(ids, np.full((T, cfg.top_k), 0.25, np.float32))] * L
                off.load_routing(routing)
                src = np.ctypeslib.as_array((C.c_uint8 * pool.expert_bytes).from_address(pool.ptr(5)))   # layer 0, expert 5
                src[777] ^= 0x01
                cache.forget(expert_key(0, 5))
                off.step_device(x.ptr, T, [y.ptr for y in ys], [r[0] for r in routing])
                gpu_ctx.sync()
                assert np.all(ys[0].download() == 0x7FC0), "the audit gate did not poison layer 0"
                for l in range(1, L):   # later layers inherit the NaN through their inputs
                    v = ys[l].download()
                    assert np.all(((v & 0x7F80) == 0x7F80) & ((v & 0x7F) != 0)), f"layer {l} output is not NaN"
                with pytest.raises(ValueError, match="0:5"):
                    off.check_audit()
                src[777] ^= 0x01
                off.step_device(x.ptr, T, [y.ptr for y in ys], [r[0] for r in routing])
                off.check_audit()
                assert not np.any((ys[-1].download() & 0x7F80) == 0x7F80)
            off.check_routes()
            with pytest.raises(ValueError, match="outside the pinned model"):
                off.load_routing([(np.full((T, cfg.top_k), cfg.experts, np.int32), np.ones((T, cfg.top_k), np.float32))] * L)
            with pytest.raises(ValueError, match="differs from the routing loaded"):
                off.step_device(x.ptr, T, [y.ptr for y in ys], [r[0] + 1 for r in routing])
        finally:
            off.close()
            for d in [x] + ys + ref_ys:
                d.free()
    finally:
        for layer in layers:
            layer.close()
        for bank in banks:
            bank.free()
        cache.close()
        pool.close()


def test_decode_routed_repairs_invalid_routing(gpu_ctx):
    """Out-of-range and repeated ids are replaced (weight 0) so the call stays in bounds and counted in the
    layer's routing error word: the result equals the call with the repaired routing, the word reads 2 after
    the bad call and 0 after the good one, and prefill counts the same replacements."""
    cfg = MoEConfig(hidden=512, intermediate=256, experts=8, top_k=2, shared=None, max_tokens=4)
    rng = np.random.default_rng(4)
    bank = ExpertBank(gpu_ctx, cfg, cfg.experts)
    for e in range(cfg.experts):
        bank.upload(e, mxfp4_expert(rng, cfg.hidden, cfg.intermediate))
    layer = MoELayer(gpu_ctx, cfg, np.zeros((cfg.experts, cfg.hidden), np.float32), bank)
    try:
        x = gpu_ctx.upload(bf16_bits(activations(rng, 2, cfg.hidden)))
        bad = gpu_ctx.upload(np.array([[3, 3], [99, 5]], np.int32))
        w = gpu_ctx.upload(np.array([[0.5, 0.7], [0.2, 0.9]], np.float32))
        good = gpu_ctx.upload(np.array([[3, 0], [0, 5]], np.int32))
        w_good = gpu_ctx.upload(np.array([[0.5, 0.0], [0.0, 0.9]], np.float32))
        y1, y2 = gpu_ctx.empty((2, cfg.hidden), np.uint16), gpu_ctx.empty((2, cfg.hidden), np.uint16)
        assert layer.route_errors() == 0
        decode_routed(layer, x.ptr, 2, bad.ptr, w.ptr, y1.ptr)
        assert layer.route_errors() == 2
        decode_routed(layer, x.ptr, 2, good.ptr, w_good.ptr, y2.ptr)
        assert layer.route_errors() == 0
        gpu_ctx.sync()
        np.testing.assert_array_equal(y1.download(), y2.download())
        nbytes = layer.workspace_bytes(2)
        ws = gpu_ctx.malloc(nbytes)
        try:
            layer.prefill_device(x.ptr, 2, y1.ptr, ws, nbytes, bad.ptr, w.ptr)
            assert layer.route_errors() == 2
            layer.prefill_device(x.ptr, 2, y2.ptr, ws, nbytes, good.ptr, w_good.ptr)
            assert layer.route_errors(clear=False) == 0
            gpu_ctx.sync()
            np.testing.assert_array_equal(y1.download(), y2.download())
        finally:
            gpu_ctx.free(ws)
        for d in (x, bad, w, good, w_good, y1, y2):
            d.free()
    finally:
        layer.close()
        bank.free()
