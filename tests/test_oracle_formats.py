"""Pins the oracle's format codecs and block GEMV (CPU only).

Goldens restate tests/test_formats.py:11-60 of the reference; the exhaustive
checks compare the oracle's bit-arithmetic encoders with independent methods
(nearest-value search, torch casts, exact rational arithmetic).
"""

from fractions import Fraction

import numpy as np
import pytest

from oracle.formats import (bf16_bits, bf16_values, e4m3_values, e8m0_values, encode_e4m3, fp4_values,
                            mxfp4_gemv_fp32, mxfp4_gemv_spec, quantize_activation, split_nibbles, unpack_fp4,
                            fp8_block32_gemv_fp32)


def conversion_space():
    """All finite BF16 values plus FP32 values at and +-1 ulp around every E4M3 midpoint
    (the set of src/vesper/conformance.py:53-62)."""
    space = bf16_values(np.arange(65536, dtype=np.uint16))
    space = space[np.isfinite(space)]
    levels = e4m3_values(np.arange(127, dtype=np.uint8))
    mid = ((levels[:-1] + levels[1:]) / np.float32(2)).astype(np.float32)
    return np.concatenate([space, mid, -mid, np.nextafter(mid, np.float32(np.inf)),
                           np.nextafter(mid, np.float32(-np.inf))]).astype(np.float32)


def nearest_search_e4m3(values):
    """Independent encoder: nearest of the 127 non-negative levels, ties to the even code."""
    levels = e4m3_values(np.arange(127, dtype=np.uint8)).astype(np.float64)
    out = np.empty(values.shape, np.uint8)
    for start in range(0, values.size, 4096):
        v = values[start:start + 4096].astype(np.float64)
        mag = np.minimum(np.abs(v), 448.0)
        dist = np.abs(mag[:, None] - levels[None, :])
        best = dist.min(axis=1, keepdims=True)
        candidates = dist == best
        even = candidates & ((np.arange(127) % 2) == 0)[None, :]
        pick = np.where(even.any(axis=1), even.argmax(axis=1), candidates.argmax(axis=1))
        out[start:start + 4096] = pick.astype(np.uint8) | np.where(np.signbit(v), 0x80, 0).astype(np.uint8)
    return out


def test_fp4_known_values_and_signed_zero():
    expected = np.array([0, .5, 1, 1.5, 2, 3, 4, 6, -0., -.5, -1, -1.5, -2, -3, -4, -6], np.float32)
    np.testing.assert_array_equal(fp4_values(np.arange(16, dtype=np.uint8)).view(np.uint32),
                                  expected.view(np.uint32))
    with pytest.raises(ValueError):
        fp4_values(np.array([16], np.uint8))


def test_e8m0_special_and_normal_scales():
    values = e8m0_values(np.array([0, 1, 126, 127, 128, 254, 255], np.uint8))
    np.testing.assert_array_equal(values[:6], np.array([2.**-127, 2.**-126, .5, 1, 2, 2.**127], np.float32))
    assert values[0].view(np.uint32) == 0x00400000
    assert np.isnan(values[-1])
    all_codes = e8m0_values(np.arange(255, dtype=np.uint8)).astype(np.float64)
    np.testing.assert_array_equal(all_codes, 2.0 ** (np.arange(255) - 127.0))


def test_fp4_nibble_order_and_scale():
    actual = unpack_fp4(np.full((1, 16), 0x98, np.uint8), np.array([[128]], np.uint8))
    assert np.signbit(actual[0, 0]) and actual[0, 0] == 0      # low nibble 8 = -0, even index
    assert actual[0, 1] == -1                                   # high nibble 9 = -0.5, x2
    packed = np.array([[0x10, 0x32, 0x54, 0x76, 0x98, 0xBA, 0xDC, 0xFE] * 2], np.uint8)
    np.testing.assert_array_equal(split_nibbles(packed)[0, :16], np.arange(16))


def test_dequant_all_codes_all_scales_is_exact_product():
    packed = np.tile(np.array([0x10, 0x32, 0x54, 0x76, 0x98, 0xBA, 0xDC, 0xFE], np.uint8), (256, 2))
    scales = np.arange(256, dtype=np.uint8).reshape(256, 1)
    out = unpack_fp4(packed, scales)
    codes = np.tile(np.arange(16), 2)
    for c in range(255):
        exact = fp4_values(codes.astype(np.uint8)).astype(np.float64) * 2.0 ** (c - 127)
        with np.errstate(over="ignore"):
            np.testing.assert_array_equal(out[c].view(np.uint32), exact.astype(np.float32).view(np.uint32))
    assert np.isnan(out[255]).all()


def test_e4m3_known_ties_and_saturation():
    inputs = np.array([0., -0., 1., 1.0625, 1.1875, 448., 1000., 2.**-10], np.float32)
    np.testing.assert_array_equal(encode_e4m3(inputs), [0, 128, 56, 56, 58, 126, 126, 0])
    assert encode_e4m3(np.array([np.nan], np.float32))[0] == 127


def test_all_finite_e4m3_codes_round_trip():
    codes = np.arange(256, dtype=np.uint8)
    codes = codes[(codes & 127) != 127]
    np.testing.assert_array_equal(encode_e4m3(e4m3_values(codes)), codes)


def test_e4m3_encoder_matches_nearest_search_on_conformance_space():
    space = conversion_space()
    np.testing.assert_array_equal(encode_e4m3(space), nearest_search_e4m3(space))


def test_e4m3_codec_matches_torch_float8():
    torch = pytest.importorskip("torch")
    space = conversion_space()
    space = space[np.abs(space) <= 448]
    ours = encode_e4m3(space)
    theirs = torch.from_numpy(space).to(torch.float8_e4m3fn).view(torch.uint8).numpy()
    np.testing.assert_array_equal(ours, theirs)
    codes = torch.arange(256, dtype=torch.int32).to(torch.uint8)
    decoded = codes.view(torch.float8_e4m3fn).to(torch.float32).numpy()
    mine = e4m3_values(np.arange(256, dtype=np.uint8))
    finite = np.isfinite(decoded)
    np.testing.assert_array_equal(mine[finite].view(np.uint32), decoded[finite].view(np.uint32))
    np.testing.assert_array_equal(np.isnan(mine), np.isnan(decoded))


def test_bf16_ties_round_to_even_and_match_torch():
    values = np.array([0x3F808000, 0x3F818000, 0x80000000], np.uint32).view(np.float32)
    np.testing.assert_array_equal(bf16_bits(values), [0x3F80, 0x3F82, 0x8000])
    torch = pytest.importorskip("torch")
    rng = np.random.default_rng(0)
    bits = np.concatenate([rng.integers(0, 2 ** 32, 200000, dtype=np.uint64).astype(np.uint32),
                           np.array([0x7F7FFFFF, 0x7F7F8000, 0x00008000, 0x80018000, 0x7F800000], np.uint32)])
    values = bits.view(np.float32)
    values = values[~np.isnan(values)]
    theirs = torch.from_numpy(values).to(torch.bfloat16).view(torch.int16).numpy().view(np.uint16)
    np.testing.assert_array_equal(bf16_bits(values), theirs)


def test_zero_activation_uses_reference_amax_floor():
    values = np.zeros((2, 32), np.float32)
    values[1] = -0.
    quantized, scales = quantize_activation(values)
    np.testing.assert_array_equal(scales, [[105], [105]])
    assert (quantized[0] == 0).all() and (quantized[1] == 128).all()


def test_activation_rejects_nonfinite_and_partial_blocks():
    with pytest.raises(ValueError):
        quantize_activation(np.ones(31, np.float32))
    with pytest.raises(ValueError):
        quantize_activation(np.full(32, np.inf, np.float32))


def test_activation_scale_is_ceil_log2_and_codes_round_to_nearest():
    rng = np.random.default_rng(20261018)
    x = rng.standard_normal((64, 512)).astype(np.float32)
    x *= np.ldexp(np.ones((64, 1), np.float32), rng.integers(-20, 16, (64, 1)))
    x = bf16_values(bf16_bits(x))
    q, s = quantize_activation(x)
    amax = np.maximum(np.abs(x.reshape(64, 16, 32)).max(-1), np.float32(1e-4))
    scaled = (amax * np.float32(1 / 448)).astype(np.float32).astype(np.float64)
    np.testing.assert_array_equal(s.astype(np.int64) - 127, np.ceil(np.log2(scaled)).astype(np.int64))
    decoded = e4m3_values(q).reshape(64, 16, 32).astype(np.float64) * 2.0 ** (s.astype(np.float64) - 127)[..., None]
    target = x.reshape(64, 16, 32).astype(np.float64)
    # every code is a nearest E4M3 level of x / 2^e
    levels = np.sort(np.concatenate([e4m3_values(np.arange(127, dtype=np.uint8)),
                                     -e4m3_values(np.arange(1, 127, dtype=np.uint8))]).astype(np.float64))
    normalized = target / 2.0 ** (s.astype(np.float64) - 127)[..., None]
    err = np.abs(decoded / 2.0 ** (s.astype(np.float64) - 127)[..., None] - normalized)
    best = np.abs(normalized[..., None] - levels).min(-1)
    np.testing.assert_array_equal(err, best)


def _exact_gemv(q, s, packed, ws):
    """Rational arithmetic: exact block dots, rounded to FP32 once, then the FP32 in-order sum."""
    a = e4m3_values(q)
    w = unpack_fp4(packed, np.full(ws.shape, 127, np.uint8))
    n, k = w.shape
    out = np.zeros(n, np.float32)
    for row in range(n):
        total = np.float32(0)
        for g in range(k // 32):
            dot = sum(Fraction(float(a[g * 32 + j])) * Fraction(float(w[row, g * 32 + j])) for j in range(32))
            dot32 = np.float32(float(dot))
            assert Fraction(float(np.float64(float(dot)))) == dot   # float64 holds the block dot exactly
            total = np.float32(total + np.float32(np.float32(dot32 * e8m0_values(s[g])) * e8m0_values(ws[row, g])))
        out[row] = total
    return out


def test_block_gemv_matches_exact_rational_arithmetic():
    rng = np.random.default_rng(7)
    x = bf16_values(bf16_bits(rng.standard_normal(256).astype(np.float32)))
    q, s = quantize_activation(x)
    packed = rng.integers(0, 256, (12, 128), dtype=np.uint8)
    ws = rng.integers(115, 129, (12, 8), dtype=np.uint8)
    np.testing.assert_array_equal(mxfp4_gemv_fp32(q, s, packed, ws)[0].view(np.uint32),
                                  _exact_gemv(q, s, packed, ws).view(np.uint32))


def test_block_gemv_sums_groups_in_order_in_fp32():
    # Scaled group values (2^24, 1, -2^24): in-order FP32 addition rounds 2^24 + 1 to 2^24
    # (tie to even), so the spec gives 0 where the exact sum is 1; with 2 in the middle it is 2.
    q = np.zeros((1, 96), np.uint8)
    packed = np.zeros((1, 48), np.uint8)
    q[0, 0], q[0, 32], q[0, 64] = 0x38, 0x38, 0x38                   # 1.0 at the first K of each group
    packed[0, 0], packed[0, 16], packed[0, 32] = 0x02, 0x02, 0x0A    # +1, +1, -1 in the low nibbles
    s = np.array([[127, 127, 127]], np.uint8)
    ws = np.array([[127 + 24, 127, 127 + 24]], np.uint8)
    assert mxfp4_gemv_fp32(q, s, packed, ws)[0, 0] == 0.0
    ws[0, 1] = 128
    assert mxfp4_gemv_fp32(q, s, packed, ws)[0, 0] == 2.0
    np.testing.assert_array_equal(mxfp4_gemv_spec(q, s, packed, ws), [[0x4000]])


def test_block_gemv_nibble_order():
    q = np.zeros((1, 32), np.uint8)
    packed = np.zeros((1, 16), np.uint8)
    s, ws = np.array([[127]], np.uint8), np.array([[127]], np.uint8)
    packed[0, 0] = 0x20             # K=0 -> code 0, K=1 -> code 2 (1.0)
    q[0, 0] = 0x38                  # activation 1.0 at K=0 only
    assert mxfp4_gemv_fp32(q, s, packed, ws)[0, 0] == 0.0
    q[0, 1] = 0x40                  # activation 2.0 at K=1
    assert mxfp4_gemv_fp32(q, s, packed, ws)[0, 0] == 2.0


def test_fp8_block32_scale_index_is_row_block():
    rng = np.random.default_rng(3)
    q, s = quantize_activation(bf16_values(bf16_bits(rng.standard_normal((2, 64)).astype(np.float32))))
    w = rng.integers(0, 126, (64, 64), dtype=np.uint8)
    ws = np.array([[127, 128], [126, 127]], np.uint8)
    out = fp8_block32_gemv_fp32(q, s, w, ws)
    a = e4m3_values(q).astype(np.float64) * np.repeat(2.0 ** (s.astype(np.float64) - 127), 32, axis=1)
    wv = e4m3_values(w).astype(np.float64) * np.repeat(np.repeat(2.0 ** (ws.astype(np.float64) - 127), 32, 0), 32, 1)
    np.testing.assert_allclose(out, a @ wv.T, rtol=2e-5, atol=1e-3)
