"""GPU parity of one expert, stage by stage (ExpertExecutor.execute, src/vesper/expert.py:51-79).

Bit-exact: the activation quantization, the W1/W3 GEMVs (fp4_gemv_spec's arithmetic: each
32-block dot rounded once to FP32, scaled, and added in ascending block order), the SwiGLU
epilogue and the down-input quantization. W2 (a different FP32 summation order) matches the
in-order sum in >= 97% of BF16 results with every difference within 2^-7 of the row's largest
magnitude, and the expert output meets the tolerance (max rel err 1e-2, cosine 0.9999).
"""

import numpy as np
import pytest

from oracle.expert import expert_forward, expert_reference_stages, swiglu
from oracle.formats import bf16_bits, mxfp4_gemv_spec, quantize_activation
from oracle.inputs import SEEDS, activations, mxfp4_expert
from tests.helpers import assert_close, assert_gemv_close, exact_activation
from vesper_amd.expert import BF16ActivationExpert, ExpertExecutor, ResidentExpert
from vesper_amd.shared import ResidentSharedExpert

pytestmark = pytest.mark.gpu


def check_stages(got, x, arrays, route, limit):
    ref = expert_forward(x, arrays, route, limit)
    np.testing.assert_array_equal(got["q"], ref["q"])
    np.testing.assert_array_equal(got["s"], ref["s"])
    for name in ("w1", "w3"):   # fp4_gemv_spec's per-block rounding and order: bit for bit
        np.testing.assert_array_equal(got[name], ref[name], err_msg=name)
    # epilogue on the kernel's own W1/W3: bit-exact
    down_input, trace = swiglu(got["w1"], got["w3"], limit, route)
    np.testing.assert_array_equal(got["down_input"].view(np.uint32), down_input.view(np.uint32))
    np.testing.assert_array_equal(got["trace"].view(np.uint32), trace.view(np.uint32))
    dq, ds = quantize_activation(got["down_input"])
    np.testing.assert_array_equal(got["down_q"], dq)
    np.testing.assert_array_equal(got["down_s"], ds)
    w2_own = mxfp4_gemv_spec(got["down_q"], got["down_s"], arrays["w2_weight"], arrays["w2_scale"])
    assert_gemv_close(got["w2"], w2_own, "w2 on the kernel's own down input")
    assert_close(got["w2"], ref["w2"], "expert output")
    return ref


@pytest.mark.parametrize("hidden,intermediate,tokens,limit", [(256, 128, 1, 10.0), (512, 256, 3, 0.0),
                                                               (1024, 512, 16, 10.0)])
def test_expert_stages_random(hidden, intermediate, tokens, limit):
    rng = np.random.default_rng(hidden + tokens)
    arrays = mxfp4_expert(rng, hidden, intermediate)
    x = activations(rng, tokens, hidden)
    route = rng.uniform(0.05, 1.5, tokens).astype(np.float32)
    with ResidentExpert(arrays, swiglu_limit=limit, hidden=hidden, intermediate=intermediate) as expert:
        got = expert.forward(x, route)
    check_stages(got, x, arrays, route, limit)


def test_expert_gate_up_exact_on_representable_inputs():
    rng = np.random.default_rng(77)
    hidden, intermediate = 1024, 256
    arrays = mxfp4_expert(rng, hidden, intermediate, scale_lo=126, scale_hi=128)
    x = exact_activation(rng, 5, hidden)
    with ResidentExpert(arrays, swiglu_limit=0.0, hidden=hidden, intermediate=intermediate) as expert:
        got = expert.forward(x, np.ones(5, np.float32))
    q, s = quantize_activation(x)
    np.testing.assert_array_equal(got["w1"], mxfp4_gemv_spec(q, s, arrays["w1_weight"], arrays["w1_scale"]))
    np.testing.assert_array_equal(got["w3"], mxfp4_gemv_spec(q, s, arrays["w3_weight"], arrays["w3_scale"]))


@pytest.mark.parametrize("tokens", [1, 16])
def test_gate_up_bit_exact_at_benchmark_shapes(tokens):
    """W1/W3 of a 7168 x 2048 expert on random inputs (uniform nibbles, E8M0 codes in [118, 126], x ~ N(0, 1))
    equal mxfp4_gemv_spec (formats.py:97-118) bit for bit."""
    rng = np.random.default_rng(20261018 + tokens)
    arrays = mxfp4_expert(rng, 7168, 2048)
    x = activations(rng, tokens, 7168)
    with ResidentExpert(arrays, swiglu_limit=10.0, hidden=7168, intermediate=2048) as expert:
        got = expert.forward(x, np.ones(tokens, np.float32))
    q, s = quantize_activation(x)
    for name in ("w1", "w3"):
        ref = mxfp4_gemv_spec(q, s, arrays[name + "_weight"], arrays[name + "_scale"])
        np.testing.assert_array_equal(got[name], ref, err_msg=name)


def test_reference_model_shapes_and_clamp():
    """The reference's own expert shapes (5120 x 2304, clamp 10) on one token."""
    rng = np.random.default_rng(20261018)
    arrays = mxfp4_expert(rng, 5120, 2304)
    x = activations(rng, 1, 5120)
    with ResidentExpert(arrays, swiglu_limit=10.0, hidden=5120, intermediate=2304) as expert:
        got = expert.forward(x[0], 0.75)
    assert got["q"].shape == (1, 5120) and got["down_s"].shape == (1, 72)
    check_stages(got, x, arrays, np.array([0.75], np.float32), 10.0)


def test_shared_expert_is_unweighted_and_executor_validates_before_device():
    rng = np.random.default_rng(3)
    arrays = mxfp4_expert(rng, 256, 128)
    x = activations(rng, 2, 256)
    with ResidentSharedExpert(arrays, swiglu_limit=0.0, hidden=256, intermediate=128) as shared:
        got = shared.forward(x)
        with pytest.raises(ValueError):
            shared.forward(x, 0.5)
        with pytest.raises(ValueError):
            shared.forward(np.full((2, 256), np.inf, np.float32))
        with pytest.raises(ValueError):
            shared.forward(np.zeros((17, 256), np.float32))
    check_stages(got, x, arrays, None, 0.0)
    with ExpertExecutor(hidden=256, intermediate=128) as ex:
        with pytest.raises(ValueError):
            ex.execute(x, {"w1_weight": 0})


@pytest.mark.parametrize("seed", SEEDS)
def test_canonical_seeds(seed):
    """The reference's canonical seed set (src/vesper/expert_reference.py:110): the W4A8 expert stage by stage
    and the BF16-activation expert (configuration 0's formula) on the same weights, two tokens each."""
    rng = np.random.default_rng(seed)
    hidden, intermediate = 1024, 512
    arrays = mxfp4_expert(rng, hidden, intermediate)
    x = activations(rng, 2, hidden)
    route = np.array([1.0, 0.5], np.float32)
    with ResidentExpert(arrays, swiglu_limit=10.0, hidden=hidden, intermediate=intermediate) as expert:
        got = expert.forward(x, route)
    check_stages(got, x, arrays, route, 10.0)
    with BF16ActivationExpert(arrays, hidden=hidden, intermediate=intermediate) as expert:
        out = expert.forward(x, route)
    assert_close(out["y"], expert_reference_stages(x, arrays, route)["y"], f"configuration 0, seed {seed}")
