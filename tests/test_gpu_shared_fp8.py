"""GPU parity of the FP8 block-32 shared expert (ResidentSharedExpert, src/vesper/shared.py:141-170).

Stage by stage against the oracle (expert_forward with fmt="fp8"): the quantizers and the SwiGLU epilogue
bit-exact on the kernel's own intermediate values, W1/W3 exact on designed exactly-representable
inputs, the GEMVs within the GEMV bar on random inputs, the output within the north-star tolerance.
"""

import numpy as np
import pytest

from oracle.expert import expert_forward, swiglu
from oracle.formats import encode_e4m3, fp8_block32_gemv_fp32, quantize_activation
from oracle.inputs import activations, fp8_block32_expert, fp8_block32_expert_normal
from tests.helpers import assert_close, assert_gemv_close, exact_activation
from vesper_amd.shared import ResidentSharedExpert

pytestmark = pytest.mark.gpu


def check_fp8_stages(got, x, arrays, limit):
    ref = expert_forward(x, arrays, None, limit, fmt="fp8")
    np.testing.assert_array_equal(got["q"], ref["q"])
    np.testing.assert_array_equal(got["s"], ref["s"])
    for name in ("w1", "w3"):
        assert_gemv_close(got[name], ref[name], name, min_equal=0.90)
    down_input, trace = swiglu(got["w1"], got["w3"], limit, None)
    np.testing.assert_array_equal(got["down_input"].view(np.uint32), down_input.view(np.uint32))
    np.testing.assert_array_equal(got["trace"].view(np.uint32), trace.view(np.uint32))
    dq, ds = quantize_activation(got["down_input"])
    np.testing.assert_array_equal(got["down_q"], dq)
    np.testing.assert_array_equal(got["down_s"], ds)
    own = fp8_block32_gemv_fp32(got["down_q"], got["down_s"], arrays["w2_weight"], arrays["w2_scale"])
    from oracle.formats import bf16_bits
    assert_gemv_close(got["w2"], bf16_bits(own), "w2 on the kernel's own down input", min_equal=0.90)
    assert_close(got["w2"], ref["w2"], "shared expert output")


@pytest.mark.parametrize("hidden,intermediate,tokens,limit", [(256, 128, 1, 10.0), (512, 256, 3, 0.0),
                                                               (1024, 512, 16, 10.0)])
def test_fp8_shared_expert_stages(hidden, intermediate, tokens, limit):
    """Checkpoint-like weights (N(0, 0.02) quantized per 32 x 32 block). Codes drawn uniformly make the
    weights heavy-tailed (magnitudes spread over 2^-9 .. 448), so one activation code flipped by a
    reordered sum, times a 448 weight, dominates an output; that distribution stays in the exact and
    GEMV checks."""
    rng = np.random.default_rng(hidden * 7 + tokens)
    arrays = fp8_block32_expert_normal(rng, hidden, intermediate)
    x = activations(rng, tokens, hidden)
    with ResidentSharedExpert(arrays, swiglu_limit=limit, hidden=hidden, intermediate=intermediate) as shared:
        assert shared.fmt == "fp8"
        got = shared.forward(x)
    check_fp8_stages(got, x, arrays, limit)


def test_fp8_shared_gate_up_exact_on_representable_inputs():
    rng = np.random.default_rng(9)
    hidden, intermediate = 512, 256
    arrays = fp8_block32_expert(rng, hidden, intermediate, scale_lo=126, scale_hi=128)
    for name in ("w1_weight", "w3_weight"):
        arrays[name] = encode_e4m3(rng.integers(-8, 9, arrays[name].shape).astype(np.float32))
    x = exact_activation(rng, 4, hidden)
    with ResidentSharedExpert(arrays, swiglu_limit=0.0, hidden=hidden, intermediate=intermediate) as shared:
        got = shared.forward(x)
    q, s = quantize_activation(x)
    from oracle.formats import bf16_bits
    for name in ("w1", "w3"):
        want = bf16_bits(fp8_block32_gemv_fp32(q, s, arrays[f"{name}_weight"], arrays[f"{name}_scale"]))
        np.testing.assert_array_equal(got[name], want)


def test_reference_shared_expert_shapes_one_token():
    """The reference's shared expert: E4M3 W1/W3 [2304, 5120], W2 [5120, 2304], 32 x 32 E8M0, clamp 10."""
    rng = np.random.default_rng(20261018)
    arrays = fp8_block32_expert_normal(rng, 5120, 2304)
    x = activations(rng, 1, 5120)
    with ResidentSharedExpert(arrays, hidden=5120, intermediate=2304) as shared:
        got = shared.forward(x[0])
        with pytest.raises(ValueError):
            shared.forward(x, 0.5)
    assert got["w2"].shape == (1, 5120) and got["down_s"].shape == (1, 72)
    check_fp8_stages(got, x, arrays, 10.0)


def test_fp8_gemv_bar_on_uniform_codes():
    rng = np.random.default_rng(21)
    arrays = fp8_block32_expert(rng, 512, 256)
    x = activations(rng, 5, 512)
    with ResidentSharedExpert(arrays, swiglu_limit=10.0, hidden=512, intermediate=256) as shared:
        got = shared.forward(x)
    ref = expert_forward(x, arrays, None, 10.0, fmt="fp8")
    for name in ("w1", "w3"):
        assert_gemv_close(got[name], ref[name], name, min_equal=0.90)


def test_fp8_shared_layout_refused_before_device():
    rng = np.random.default_rng(1)
    arrays = fp8_block32_expert(rng, 256, 128)
    arrays["w2_scale"] = arrays["w2_scale"][:, :2]
    with pytest.raises(ValueError):
        ResidentSharedExpert(arrays, hidden=256, intermediate=128)
