"""GPU parity of the format hooks and the block GEMV (bit-exact against the oracle)."""

import numpy as np
import pytest

from oracle.formats import (bf16_bits, bf16_values, e4m3_values, encode_e4m3, mxfp4_gemv_spec, quantize_activation,
                            unpack_fp4)
from tests.helpers import assert_gemv_close, exact_activation
from tests.test_oracle_formats import conversion_space
from vesper_amd import _lib, conformance

pytestmark = pytest.mark.gpu


def test_dequant_all_codes_all_scales(gpu_ctx):
    packed = np.tile(np.array([0x10, 0x32, 0x54, 0x76, 0x98, 0xBA, 0xDC, 0xFE], np.uint8), (256, 2))
    scales = np.arange(256, dtype=np.uint8).reshape(256, 1)
    got = conformance.decode_fp4(gpu_ctx, packed, scales)
    assert conformance.compare(unpack_fp4(packed, scales), got, "dequant")["status"] == "pass"


def test_dequant_random_expert_matrix(gpu_ctx):
    rng = np.random.default_rng(1)
    packed = rng.integers(0, 256, (256, 1024), dtype=np.uint8)
    scales = rng.integers(118, 127, (256, 64), dtype=np.uint8)
    got = conformance.decode_fp4(gpu_ctx, packed, scales)
    np.testing.assert_array_equal(got.view(np.uint32), unpack_fp4(packed, scales).view(np.uint32))


def test_encode_e4m3_conformance_space(gpu_ctx):
    space = conversion_space()
    got = conformance.encode_fp8(gpu_ctx, space)
    assert conformance.compare(encode_e4m3(space), got, "e4m3")["status"] == "pass"


def test_activation_quantizer_reference_cases(gpu_ctx):
    rng = np.random.default_rng(20261018)
    x = rng.standard_normal((64, 512)).astype(np.float32)
    x *= np.ldexp(np.ones((64, 1), np.float32), rng.integers(-20, 16, (64, 1)))
    x[0] = 0
    x[1, 0::2], x[1, 1::2] = 0.0, -0.0
    x[2] = np.float32(1e-30)
    x = bf16_values(bf16_bits(x))
    q, s = conformance.activation32(gpu_ctx, x)
    q_ref, s_ref = quantize_activation(x)
    np.testing.assert_array_equal(s, s_ref)
    np.testing.assert_array_equal(q, q_ref)
    # the BF16-input entry point agrees with the FP32 one
    xd = gpu_ctx.upload(bf16_bits(x))
    qd, sd = gpu_ctx.empty(q.shape, np.uint8), gpu_ctx.empty(s.shape, np.uint8)
    gpu_ctx.lib.act_quant32(gpu_ctx._h(), _lib.vp(xd), _lib.vp(qd), _lib.vp(sd), 64, 512, None)
    np.testing.assert_array_equal(qd.download(), q_ref)
    np.testing.assert_array_equal(sd.download(), s_ref)
    for d in (xd, qd, sd):
        d.free()


def run_gemv(ctx, q, sa, w, sw):
    t, k = q.shape
    n = w.shape[0]
    dev = [ctx.upload(np.ascontiguousarray(a)) for a in (q, sa, w, sw)]
    y = ctx.empty((t, n), np.uint16)
    try:
        ctx.lib.gemv_mxfp4(ctx._h(), *[_lib.vp(d) for d in dev], _lib.vp(y), t, n, k, None)
        return y.download()
    finally:
        for d in dev + [y]:
            d.free()


@pytest.mark.parametrize("tokens,n,k", [(1, 64, 128), (3, 128, 256), (16, 192, 512), (5, 7168, 2048)])
def test_block_gemv_is_exact_on_exactly_representable_inputs(gpu_ctx, tokens, n, k):
    """Every partial sum is a multiple of 2^-2 below 2^22, so any summation order is exact: this
    pins the MFMA operand layouts (K split, nibble order, token columns, output rows) and which
    E8M0 scale multiplies which 32-element block, bit for bit."""
    rng = np.random.default_rng(n * 31 + k + tokens)
    x = exact_activation(rng, tokens, k)
    q, sa = quantize_activation(x)
    np.testing.assert_array_equal((e4m3_values(q) * np.repeat(2.0 ** (sa.astype(np.float64) - 127), 32, 1)), x)
    w = rng.integers(0, 256, (n, k // 2), dtype=np.uint8)
    sw = rng.integers(126, 129, (n, k // 32), dtype=np.uint8)
    got = run_gemv(gpu_ctx, q, sa, w, sw)
    np.testing.assert_array_equal(got, mxfp4_gemv_spec(q, sa, w, sw))


def test_block_gemv_random_inputs_close_to_in_order_sum(gpu_ctx):
    rng = np.random.default_rng(42)
    x = bf16_values(bf16_bits(rng.standard_normal((4, 2048)).astype(np.float32)))
    q, sa = quantize_activation(x)
    w = rng.integers(0, 256, (1024, 1024), dtype=np.uint8)
    sw = rng.integers(118, 127, (1024, 64), dtype=np.uint8)
    got = run_gemv(gpu_ctx, q, sa, w, sw)
    ref = mxfp4_gemv_spec(q, sa, w, sw)
    assert_gemv_close(got, ref, "random GEMV")


def test_hardware_e4m3_packing_matches_the_encoder_on_every_float(gpu_ctx):
    """The prefill epilogue packs E4M3 codes with the gfx950 conversion instruction; on every one of the
    2^32 FP32 inputs (clamped to +-448 as the quantizers clamp) it must give the software encoder's code,
    which test_encode_e4m3_conformance_space pins to the oracle."""
    import ctypes as C
    mismatches = C.c_uint64(1)
    gpu_ctx.lib.check_e4m3_pack(gpu_ctx._h(), C.byref(mismatches))
    assert mismatches.value == 0
