"""The FP8 projection oracle (oracle/projections.py), pinned independently of its own formulas."""

from fractions import Fraction

import numpy as np
import pytest

from oracle.formats import e4m3_values, encode_e4m3, fma_f32, fp8_block32_gemv_fp32
from oracle.projections import (CONFIG3_LAYOUT, fp8_block128_gemm_fp32, fp8_projection, fp8_reference_fp32,
                                fp8_weights, quantize_activation_128)


def round_f32(value: Fraction) -> np.float32:
    """The FP32 nearest to an exact rational (ties to the even significand), by exact comparison of the
    neighbours of a first guess -- independent of any floating-point rounding chain."""
    guess = np.float32(float(value))
    candidates = [np.nextafter(guess, np.float32(-np.inf)), guess, np.nextafter(guess, np.float32(np.inf))]
    def key(c):
        return (abs(Fraction(float(c)) - value), int(np.array(c).view(np.uint32)) & 1)
    return min(candidates, key=key)


def test_fma_f32_is_the_correctly_rounded_fused_result():
    """fma_f32 against exact rational arithmetic: random operands over many magnitudes, and two designed
    cases where the float64 sum lands exactly halfway between two FP32 values while the exact value does
    not (the naive double rounding would round the tie to even, the wrong way)."""
    rng = np.random.default_rng(77)
    a = (rng.standard_normal(4000) * np.exp2(rng.integers(-20, 20, 4000))).astype(np.float32)
    b = (rng.standard_normal(4000) * np.exp2(rng.integers(-20, 20, 4000))).astype(np.float32)
    c = (rng.standard_normal(4000) * np.exp2(rng.integers(-40, 40, 4000))).astype(np.float32)
    lo, hi = np.float32(1 - 2.0 ** -20), np.float32(1 + 2.0 ** -20)       # lo * hi = 1 - 2^-40 exactly
    big = np.float32(2.0 ** 24 + 2)
    a = np.concatenate([a, [lo, lo]]).astype(np.float32)
    b = np.concatenate([b, [-hi, hi]]).astype(np.float32)
    c = np.concatenate([c, [big, big]]).astype(np.float32)
    got = fma_f32(a, b, c)
    for i in range(len(a)):
        want = round_f32(Fraction(float(a[i])) * Fraction(float(b[i])) + Fraction(float(c[i])))
        assert got[i] == want, (i, a[i], b[i], c[i], got[i], want)
    assert got[-2] == np.float32(2.0 ** 24 + 2) and got[-1] == np.float32(2.0 ** 24 + 2)
    naive = (a[-2:].astype(np.float64) * b[-2:] + c[-2:]).astype(np.float32)
    assert list(naive) == [np.float32(2.0 ** 24), np.float32(2.0 ** 24 + 4)]   # what the fix corrects


def small_int_codes(rng, shape, lo=-8, hi=8):
    """E4M3 codes of small integers (exactly representable)."""
    return encode_e4m3(rng.integers(lo, hi + 1, shape).astype(np.float32))


def test_quantizer_closed_form_cases():
    x = np.zeros((3, 256), np.float32)
    x[1, :128] = np.linspace(-448, 448, 128, dtype=np.float32)       # amax 448 -> scale exactly 1
    x[2, 128:] = 1e-6                                                # below the floor
    q, s = quantize_activation_128(x)
    assert s.dtype == np.float32 and s.shape == (3, 2)
    floor_scale = np.float32(np.float32(1e-4) / np.float32(448))
    assert s[0, 0] == floor_scale and np.all(q[0] == 0)
    assert s[1, 0] == np.float32(1.0)
    np.testing.assert_array_equal(q[1, :128], encode_e4m3(x[1, :128]))
    assert s[2, 1] == floor_scale
    # every code times its scale is within half an E4M3 step of the input (relative 2^-4)
    rng = np.random.default_rng(1)
    x = rng.standard_normal((4, 512)).astype(np.float32) * 3
    q, s = quantize_activation_128(x)
    back = e4m3_values(q).reshape(4, 4, 128) * s[..., None]
    err = np.abs(back.reshape(4, 512) - x)
    assert np.all(err <= np.maximum(np.abs(x) * 2.0 ** -4, np.repeat(s, 128, 1) * 2.0 ** -10))


def test_block128_gemm_equals_integer_matmul_on_unit_scales():
    rng = np.random.default_rng(2)
    q = small_int_codes(rng, (5, 384))
    w = small_int_codes(rng, (200, 384))
    got = fp8_block128_gemm_fp32(q, np.ones((5, 3), np.float32), w, np.ones((2, 3), np.float32))
    ints = e4m3_values(q).astype(np.int64) @ e4m3_values(w).astype(np.int64).T
    np.testing.assert_array_equal(got, ints.astype(np.float32))


def test_block128_scaling_is_per_block_and_in_order():
    """Each weight row has one or two nonzero K blocks: the result is, per block in K order, the exact
    rational d * f32(sa * sw) added to the running FP32 sum with one rounding -- computed here with
    Fractions and an exact nearest-FP32 search."""
    rng = np.random.default_rng(3)
    t, n, k = 2, 130, 256
    q = encode_e4m3(rng.standard_normal((t, k)).astype(np.float32))
    w = np.zeros((n, k), np.uint8)
    used = rng.integers(1, 4, n)                          # bit g set: block g is nonzero
    for r in range(n):
        for g in range(2):
            if used[r] >> g & 1:
                w[r, 128 * g:128 * g + 128] = encode_e4m3(rng.standard_normal(128).astype(np.float32))
    sa = np.exp2(rng.integers(-6, 6, (t, 2))).astype(np.float32) * np.float32(1.5)
    sw = np.exp2(rng.uniform(-8, -2, (2, 2))).astype(np.float32)
    got = fp8_block128_gemm_fp32(q, sa, w, sw)
    for i in range(t):
        for r in range(n):
            acc = np.float32(0.0)
            for g in range(2):
                d = sum(Fraction(float(a)) * Fraction(float(b)) for a, b in
                        zip(e4m3_values(q[i, 128 * g:128 * g + 128]), e4m3_values(w[r, 128 * g:128 * g + 128])))
                d32 = round_f32(d)
                scale = round_f32(Fraction(float(sa[i, g])) * Fraction(float(sw[r // 128, g])))
                acc = round_f32(Fraction(float(d32)) * Fraction(float(scale)) + Fraction(float(acc)))
            assert got[i, r] == acc


def test_profiles_agree_on_unit_scales_and_exact_inputs():
    """Block 32 (E8M0 127 = 1.0) and block 128 (FP32 1.0) give identical sums on integer inputs."""
    rng = np.random.default_rng(4)
    q = small_int_codes(rng, (3, 512))
    w = small_int_codes(rng, (128, 512))
    b32 = fp8_block32_gemv_fp32(q, np.full((3, 16), 127, np.uint8), w, np.full((4, 16), 127, np.uint8))
    b128 = fp8_block128_gemm_fp32(q, np.ones((3, 4), np.float32), w, np.ones((1, 4), np.float32))
    np.testing.assert_array_equal(b32, b128)


def test_linearity_in_power_of_two_weight_scales():
    rng = np.random.default_rng(5)
    w, sw = fp8_weights(rng, 256, 256, 128)
    x = rng.standard_normal((2, 256)).astype(np.float32)
    a = fp8_projection(x, w, sw, 128)["output_fp32"]
    b = fp8_projection(x, w, sw * np.float32(4), 128)["output_fp32"]
    np.testing.assert_array_equal(b, a * np.float32(4))


@pytest.mark.parametrize("block", [32, 128])
def test_projection_tracks_the_unquantized_product(block):
    rng = np.random.default_rng(6 + block)
    w, sw = fp8_weights(rng, 256, 1024, block)
    x = rng.standard_normal((4, 1024)).astype(np.float32)
    got = fp8_projection(x, w, sw, block)["output_fp32"].astype(np.float64)
    ref = fp8_reference_fp32(x, w, sw, block).astype(np.float64)
    cos = float((got * ref).sum() / np.sqrt((got * got).sum() * (ref * ref).sum()))
    assert cos > 0.999


def test_config3_layout_and_weights():
    assert CONFIG3_LAYOUT == {"q_a": (1536, 7168), "q_b": (24576, 1536), "kv_a": (576, 7168), "o": (7168, 16384)}
    total = sum(r * c for r, c in CONFIG3_LAYOUT.values())
    assert total == 170_328_064
    w, s = fp8_weights(np.random.default_rng(0), 576, 256, 128)
    assert s.shape == (5, 2) and np.all((w & 0x7F) != 0x7F)
    assert np.all((s >= 2.0 ** -8) & (s <= 2.0 ** -2))


def test_kv_round32_round_trips_representable_blocks():
    """A block built as E4M3 values x 2^k with its largest code 448 x 2^k present is recovered exactly:
    codes, the scale 127 + k and the rounded values equal the input; an all-zero block keeps zeros with
    the floor's scale (105)."""
    from oracle.formats import bf16_bits, e4m3_values, encode_e4m3
    from oracle.projections import kv_round32
    rng = np.random.default_rng(32)
    codes = rng.integers(0, 126, (4, 32)).astype(np.uint8) | (rng.integers(0, 2, (4, 32)).astype(np.uint8) << 7)
    codes[:, 5] = 0x7E                                           # 448
    k = np.array([-6, 0, 3, -20])
    x = (e4m3_values(codes).astype(np.float64) * np.exp2(k)[:, None]).astype(np.float32)
    x = np.concatenate([x, np.zeros((1, 32), np.float32)])
    rounded, q, s = kv_round32(bf16_bits(x))
    np.testing.assert_array_equal(q[:4], codes)
    np.testing.assert_array_equal(s[:4, 0], 127 + k)
    np.testing.assert_array_equal(rounded, bf16_bits(x))
    assert s[4, 0] == 105 and not q[4].any()
    assert (encode_e4m3(np.float32(448.0)) == 0x7E).all()


def test_wo_a_grouped_indexes_groups_and_rows():
    """One-hot weights: row r of group g reads element (r + 3 g) mod K of activation group g, so every
    output is a known rounded input value times the weight's block scale."""
    from oracle.formats import bf16_bits, bf16_values
    from oracle.projections import kv_round32, wo_a_grouped
    groups, rows, width, t = 4, 64, 128, 3
    rng = np.random.default_rng(8)
    codes = np.zeros((groups * rows, width), np.uint8)
    r = np.arange(groups * rows)
    col = (r % rows + 3 * (r // rows)) % width
    codes[r, col] = 0x38                                         # E4M3 1.0
    scales = rng.integers(124, 130, (groups * rows // 32, width // 32), dtype=np.uint8)
    x = bf16_bits(rng.standard_normal((t, groups, width)).astype(np.float32))
    out = wo_a_grouped(x, codes, scales, groups=groups)
    rounded = bf16_values(kv_round32(x)[0]).reshape(t, groups, width)
    ws = np.exp2(scales.astype(np.float64) - 127)[r // 32, col // 32]
    want = rounded[:, r // rows, col] * ws[None, :]
    np.testing.assert_array_equal(out["output_bf16"].reshape(t, -1), bf16_bits(want.astype(np.float32)))
