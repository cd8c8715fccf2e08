"""The device-native tiled expert layout (mx_tile_expert / mx_untile_expert).

The conversion is checked three ways: against an independent NumPy construction of the
layout from its definition (gather by index arrays, not the kernel's loop), by the exact
round trip tiled -> reference, and through the decode layer, whose expert outputs are
compared with the oracle run on the reference-layout arrays (test_gpu_moe)."""

import ctypes as C

import numpy as np
import pytest

from oracle.inputs import mxfp4_expert
from vesper_amd import _lib
from vesper_amd.config import MoEConfig
from vesper_amd.layer import TENSORS, ExpertBank

pytestmark = pytest.mark.gpu


def tile_numpy(arrays, hidden, intermediate):
    """The tiled blob built from the layout's definition with fancy indexing."""
    H, I = hidden, intermediate
    blocks = {n: arrays[n].reshape(arrays[n].shape[0], -1, 16) for n in ("w1_weight", "w3_weight", "w2_weight")}
    g, c, t, l = np.meshgrid(np.arange(I // 32), np.arange(H // 128), np.arange(4), np.arange(64), indexing="ij")
    m, q = l % 16, l // 16
    row, blk = 32 * g + 8 * t + (m & 7), 4 * c + q
    gu = np.where((m < 8)[..., None], blocks["w1_weight"][row, blk], blocks["w3_weight"][row, blk])
    su = np.where(m < 8, arrays["w1_scale"][row, blk], arrays["w3_scale"][row, blk]).astype(np.uint32)
    gu_s = (su << (8 * t)).sum(axis=2, dtype=np.uint64).astype(np.uint32)       # [g, c, l], byte t = tile t
    b, c, t, l = np.meshgrid(np.arange(H // 64), np.arange(I // 128), np.arange(4), np.arange(64), indexing="ij")
    m, q = l % 16, l // 16
    row, blk = 64 * b + 16 * t + m, 4 * c + q
    dn = blocks["w2_weight"][row, blk]
    dn_s = (arrays["w2_scale"][row, blk].astype(np.uint32) << (8 * t)).sum(axis=2, dtype=np.uint64).astype(np.uint32)
    return np.concatenate([gu.reshape(-1), gu_s.reshape(-1).view(np.uint8), dn.reshape(-1),
                           dn_s.reshape(-1).view(np.uint8)])


@pytest.mark.parametrize("hidden,intermediate", [(256, 128), (512, 384), (5120, 2304)])
def test_tiled_layout_matches_definition_and_round_trips(gpu_ctx, hidden, intermediate):
    rng = np.random.default_rng(hidden + intermediate)
    arrays = mxfp4_expert(rng, hidden, intermediate)
    cfg = MoEConfig(hidden=hidden, intermediate=intermediate, experts=2, top_k=1, shared=None)
    bank = ExpertBank(gpu_ctx, cfg, 2)
    try:
        bank.upload(1, arrays)
        tiled = gpu_ctx.download(bank.tiled_ptr(1), (bank.expert_bytes,), np.uint8)
        np.testing.assert_array_equal(tiled, tile_numpy(arrays, hidden, intermediate))
        back = bank.download(1)
        for name in TENSORS:
            np.testing.assert_array_equal(back[name], arrays[name], err_msg=name)
    finally:
        bank.free()


def test_tile_refuses_bad_shapes_and_alignment(gpu_ctx):
    lib = gpu_ctx.lib
    assert lib.cdll.mx_tiled_expert_bytes(7168, 2048) == 23_396_352
    cfg = MoEConfig(hidden=256, intermediate=128, experts=1, top_k=1, shared=None)
    bank = ExpertBank(gpu_ctx, cfg, 1)
    try:
        ptrs = bank._staging_ptrs()
        with pytest.raises(ValueError):
            lib.tile_expert(gpu_ctx._h(), C.byref(ptrs), 256, 100, C.c_void_p(bank.tiled_ptr(0)), None)
        with pytest.raises(ValueError):
            lib.tile_expert(gpu_ctx._h(), C.byref(ptrs), 256, 128, C.c_void_p(bank.tiled_ptr(0) + 16), None)
    finally:
        bank.free()
