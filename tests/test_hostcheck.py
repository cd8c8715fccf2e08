"""The device numerics header (mx_numerics.h), compiled for the CPU, matches the oracle exhaustively.

The same header is compiled by hipcc into the gfx950 kernels, so these checks
pin the kernels' scalar arithmetic without a GPU.
"""

import ctypes as C
from pathlib import Path

import numpy as np
import pytest

from oracle.formats import (bf16_bits, bf16_values, e4m3_values, e8m0_values, encode_e4m3, fp4_values,
                            quantize_activation)
from tests.test_oracle_formats import conversion_space

LIB = Path(__file__).resolve().parents[1] / "vesper_amd" / "libmxmoe_hostcheck.so"


@pytest.fixture(scope="module")
def host():
    assert LIB.exists(), "build first: python -m vesper_amd.build"
    lib = C.CDLL(str(LIB))
    P, I64 = C.c_void_p, C.c_int64
    for name in ("mxh_e4m3_encode", "mxh_e4m3_decode", "mxh_fp4_decode", "mxh_e8m0_decode", "mxh_bf16_bits"):
        getattr(lib, name).argtypes = [P, P, I64]
    lib.mxh_act_quant32.argtypes = [P, P, P, I64, I64]
    return lib


def call(fn, values, out_dtype):
    values = np.ascontiguousarray(values)
    out = np.empty(values.shape, out_dtype)
    fn(values.ctypes.data, out.ctypes.data, values.size)
    return out


def test_e4m3_encode_matches_oracle_on_conformance_space_and_specials(host):
    space = np.concatenate([conversion_space(),
                            np.array([np.inf, -np.inf, np.nan, 1e-45, -1e-45, 3e38, 447.99, 464.0, 480.0],
                                     np.float32)])
    np.testing.assert_array_equal(call(host.mxh_e4m3_encode, space, np.uint8), encode_e4m3(space))


def test_e4m3_encode_matches_oracle_on_random_fp32_bits(host):
    rng = np.random.default_rng(11)
    bits = rng.integers(0, 2 ** 32, 2_000_000, dtype=np.uint64).astype(np.uint32)
    values = bits.view(np.float32)
    np.testing.assert_array_equal(call(host.mxh_e4m3_encode, values, np.uint8), encode_e4m3(values))


def test_decoders_match_oracle_on_every_code(host):
    codes = np.arange(256, dtype=np.uint8)
    got = call(host.mxh_e4m3_decode, codes, np.float32)
    want = e4m3_values(codes)
    finite = ~np.isnan(want)
    np.testing.assert_array_equal(got[finite].view(np.uint32), want[finite].view(np.uint32))
    assert np.isnan(got[~finite]).all()
    got = call(host.mxh_fp4_decode, codes[:16], np.float32)
    np.testing.assert_array_equal(got.view(np.uint32), fp4_values(codes[:16]).view(np.uint32))
    got = call(host.mxh_e8m0_decode, codes, np.float32)
    want = e8m0_values(codes)
    np.testing.assert_array_equal(got[:255].view(np.uint32), want[:255].view(np.uint32))
    assert np.isnan(got[255])


def test_bf16_rounding_matches_oracle(host):
    rng = np.random.default_rng(12)
    bits = np.concatenate([rng.integers(0, 2 ** 32, 1_000_000, dtype=np.uint64).astype(np.uint32),
                           np.array([0x3F808000, 0x3F818000, 0x80000000, 0x7F7FFFFF, 0x7FC00001, 0xFF800001],
                                    np.uint32)])
    values = bits.view(np.float32)
    np.testing.assert_array_equal(call(host.mxh_bf16_bits, values, np.uint16), bf16_bits(values))


def test_activation_quantizer_matches_oracle(host):
    rng = np.random.default_rng(20261018)
    x = rng.standard_normal((64, 512)).astype(np.float32)
    x *= np.ldexp(np.ones((64, 1), np.float32), rng.integers(-20, 16, (64, 1)))
    x[0] = 0
    x[1, 0::2], x[1, 1::2] = 0.0, -0.0
    x[2] = np.float32(1e-30)
    x[3] = bf16_values(np.arange(0x0001, 0x0201, dtype=np.uint16))    # BF16 subnormals
    x[4, :32] = 448.0 * 2 ** 20
    q, s = np.empty(x.shape, np.uint8), np.empty((64, 16), np.uint8)
    host.mxh_act_quant32(x.ctypes.data, q.ctypes.data, s.ctypes.data, 64, 512)
    q_ref, s_ref = quantize_activation(x)
    np.testing.assert_array_equal(s, s_ref)
    np.testing.assert_array_equal(q, q_ref)


def test_act128_quotient_equals_the_division_over_the_quantizer_domain(host):
    """The block-128 quantizers divide by the block scale with mx::act128_quotient (one reciprocal per
    block, then x * inv corrected by one fused multiply-add). Exhaustively, over every BF16 x of either
    sign (and NaN) and every scale act128_scale(amax) with |x| <= amax, amax up to infinity: the quotient
    equals the IEEE division bit for bit wherever |x / s| >= 2^-90, and every E4M3 code equals the
    division's -- so the quantizers' codes are those of act_quant_value(x, s), which the oracle follows."""
    fn = host.mxh_act128_quotient_check
    fn.restype = C.c_int64
    fn.argtypes = [C.POINTER(C.c_int64), C.POINTER(C.c_float), C.POINTER(C.c_int64)]
    codes, qmax, pairs = C.c_int64(), C.c_float(), C.c_int64()
    differing = fn(C.byref(codes), C.byref(qmax), C.byref(pairs))
    assert pairs.value > 850_000_000
    assert codes.value == 0
    assert differing == 0 or qmax.value < 2.0 ** -90
