"""The allocation-free tiled expert call (mx_expert_forward_tiled_noalloc) against the allocating entry point
(mx_expert_forward_tiled), through the C ABI: output and every stage buffer bit-identical, on two calls in a
row -- 16 tokens of the BASELINE expert, then 3 tokens of a smaller expert, so the second call runs on what
the first left in the fixed array -- and sizes beyond the array refused before any device work."""

import ctypes as C

import numpy as np
import pytest

from oracle.formats import bf16_bits
from oracle.inputs import activations, mxfp4_expert
from vesper_amd import _lib
from vesper_amd.config import MoEConfig
from vesper_amd.layer import ExpertBank

pytestmark = pytest.mark.gpu
STAGES = ("q", "s", "w1", "w3", "down_input", "trace", "down_q", "down_s")


def stage_buffers(ctx, t, h, i):
    shapes = {"q": ((t, h), np.uint8), "s": ((t, h // 32), np.uint8), "w1": ((t, i), np.uint16),
              "w3": ((t, i), np.uint16), "down_input": ((t, i), np.uint16), "trace": ((t, i, 5), np.float32),
              "down_q": ((t, i), np.uint8), "down_s": ((t, i // 32), np.uint8)}
    return {n: ctx.empty(*shapes[n]) for n in STAGES}


def run(ctx, entry, tiled, h, i, x, t, route, limit, with_stages):
    y = ctx.empty((t, h), np.uint16)
    bufs = stage_buffers(ctx, t, h, i) if with_stages else None
    stages = C.byref(_lib.MxExpertStages(*[bufs[n].ptr for n in STAGES])) if bufs else None
    getattr(ctx.lib, entry)(ctx._h(), C.c_void_p(tiled), h, i, C.c_void_p(x.ptr), t, C.c_float(limit),
                            C.c_void_p(route.ptr), C.c_void_p(y.ptr), stages, None)
    ctx.sync()
    out = {"y": y.download()}
    if bufs:
        out.update({n: b.download() for n, b in bufs.items()})
    for d in [y] + (list(bufs.values()) if bufs else []):
        d.free()
    return out


@pytest.mark.parametrize("with_stages", [False, True])
def test_noalloc_call_equals_the_allocating_call(gpu_ctx, with_stages):
    rng = np.random.default_rng(777)
    for h, i, t, limit in ((7168, 2048, 16, 0.0), (1024, 512, 3, 10.0)):
        cfg = MoEConfig(hidden=h, intermediate=i, experts=1, top_k=1, shared=None)
        bank = ExpertBank(gpu_ctx, cfg, 1)
        bank.upload(0, mxfp4_expert(rng, h, i))
        x = gpu_ctx.upload(bf16_bits(activations(rng, t, h)))
        route = gpu_ctx.upload(rng.uniform(0.1, 2.5, t).astype(np.float32))
        try:
            ref = run(gpu_ctx, "expert_forward_tiled", bank.tiled_ptr(0), h, i, x, t, route, limit, with_stages)
            got = run(gpu_ctx, "expert_forward_tiled_noalloc", bank.tiled_ptr(0), h, i, x, t, route, limit,
                      with_stages)
            assert set(got) == set(ref)
            for name in ref:
                np.testing.assert_array_equal(got[name], ref[name], err_msg=f"{h}x{i} T={t} {name}")
            assert not np.all(got["y"] == 0)
        finally:
            x.free()
            route.free()
            bank.free()


def test_noalloc_call_refuses_sizes_beyond_its_array(gpu_ctx):
    """16 tokens of a 32768 x 32768 expert need more than the fixed 1 MiB: refused (ValueError) before any
    launch -- the tiled pointer is never read, so any aligned address serves."""
    x = gpu_ctx.empty((16, 256), np.uint16)
    y = gpu_ctx.empty((16, 256), np.uint16)
    try:
        with pytest.raises(ValueError, match="fixed"):
            gpu_ctx.lib.expert_forward_tiled_noalloc(gpu_ctx._h(), C.c_void_p(x.ptr), 32768, 32768,
                                                     C.c_void_p(x.ptr), 16, C.c_float(0.0), None, C.c_void_p(y.ptr),
                                                     None, None)
    finally:
        x.free()
        y.free()
