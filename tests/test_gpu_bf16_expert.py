"""GPU parity of the configuration-0 expert (BF16 activations, FP32 accumulation; mx_expert_forward_bf16).

* BASELINE configuration 0 itself (7168 x 2048, E8M0 codes in [118, 126], one token): y within the
  north-star tolerance of the float64 formula (max relative error 1e-2, cosine 0.9999); the FP32
  intermediates g = W1 x, u = W3 x and h within 1e-5 (normwise) of it.
* Exact inputs (small integer activations, E8M0 codes in [124, 127]): every partial sum is exactly
  representable, so g and u equal the float64 values bit for bit -- a wrong nibble order, scale byte or tile
  row fails this.
* The reference model's shapes with a route weight; several token counts (one, two and four token groups);
  each token's result is identical whether it runs alone or in a batch.
"""

import numpy as np
import pytest

from oracle.expert import expert_reference_stages
from oracle.formats import bf16_bits
from oracle.inputs import activations, mxfp4_expert
from tests.helpers import assert_close
from vesper_amd.expert import BF16ActivationExpert

pytestmark = pytest.mark.gpu


def normwise(got, ref):
    ref = np.asarray(ref, np.float64)
    return float(np.linalg.norm(np.asarray(got, np.float64) - ref) / max(np.linalg.norm(ref), 1e-300))


def check(out, ref, what):
    i = ref["g"].shape[1]
    assert normwise(out["gu"][:, :i], ref["g"]) < 1e-5, what
    assert normwise(out["gu"][:, i:], ref["u"]) < 1e-5, what
    assert normwise(out["h"], ref["h"]) < 1e-5, what
    assert_close(out["y"], ref["y"], what)


def test_configuration_0_one_token():
    rng = np.random.default_rng(20261018)
    arrays = mxfp4_expert(rng, 7168, 2048)
    x = activations(rng, 1, 7168)
    with BF16ActivationExpert(arrays, hidden=7168, intermediate=2048) as expert:
        out = expert.forward(x[0])
    check(out, expert_reference_stages(x, arrays), "configuration 0")


def test_exact_inputs_give_exact_gate_and_up():
    rng = np.random.default_rng(5)
    h, i = 1024, 512
    arrays = mxfp4_expert(rng, h, i, scale_lo=124, scale_hi=127)
    x = rng.integers(-3, 4, (3, h)).astype(np.float32)
    with BF16ActivationExpert(arrays, hidden=h, intermediate=i) as expert:
        out = expert.forward(bf16_bits(x))
    ref = expert_reference_stages(x, arrays)
    np.testing.assert_array_equal(out["gu"][:, :i], ref["g"].astype(np.float32))
    np.testing.assert_array_equal(out["gu"][:, i:], ref["u"].astype(np.float32))


def test_reference_shapes_with_route_weight():
    rng = np.random.default_rng(7)
    arrays = mxfp4_expert(rng, 5120, 2304)
    x = activations(rng, 2, 5120)
    w = np.array([0.37, 1.25], np.float32)
    with BF16ActivationExpert(arrays) as expert:
        out = expert.forward(x, w)
    check(out, expert_reference_stages(x, arrays, w), "reference shapes")


@pytest.mark.parametrize("tokens", [5, 16])
def test_token_groups_and_batch_invariance(tokens):
    rng = np.random.default_rng(tokens)
    h, i = 1024, 512
    arrays = mxfp4_expert(rng, h, i)
    x = activations(rng, tokens, h)
    with BF16ActivationExpert(arrays, hidden=h, intermediate=i) as expert:
        out = expert.forward(x)
        check(out, expert_reference_stages(x, arrays), f"T={tokens}")
        for row in (0, tokens - 1):
            alone = expert.forward(x[row])
            for name in ("gu", "h", "y"):
                np.testing.assert_array_equal(alone[name][0], out[name][row], err_msg=f"{name} row {row}")


def test_refusals_before_device_work():
    rng = np.random.default_rng(1)
    with pytest.raises(ValueError, match="hidden <= 8192"):
        BF16ActivationExpert(mxfp4_expert(rng, 8320, 128), hidden=8320, intermediate=128)
    arrays = mxfp4_expert(rng, 256, 128)
    with BF16ActivationExpert(arrays, hidden=256, intermediate=128) as expert:
        with pytest.raises(ValueError, match="1 to 16"):
            expert.forward(np.zeros((17, 256), np.float32))
        with pytest.raises(ValueError, match="finite"):
            expert.forward(np.zeros(256, np.float32), np.float32(np.nan))
