"""Shared test utilities: tolerance metrics and designed inputs."""

import numpy as np

from oracle.formats import bf16_values

# The north-star tolerance for FFN/MoE outputs against the FP32 oracle (BF16 out):
# normwise max relative error <= 1e-2 and cosine similarity >= 0.9999.
MAX_REL_ERR = 1e-2
MIN_COSINE = 0.9999


def as_f64(bits_or_values):
    a = np.asarray(bits_or_values)
    return (bf16_values(a) if a.dtype == np.uint16 else a).astype(np.float64)


def max_rel_err(got, ref) -> float:
    g, r = as_f64(got), as_f64(ref)
    return float(np.max(np.abs(g - r)) / max(np.max(np.abs(r)), 1e-30))


def cosine(got, ref) -> float:
    g, r = as_f64(got).ravel(), as_f64(ref).ravel()
    return float(g @ r / max(np.linalg.norm(g) * np.linalg.norm(r), 1e-300))


def assert_close(got, ref, what=""):
    err, cos = max_rel_err(got, ref), cosine(got, ref)
    assert err <= MAX_REL_ERR and cos >= MIN_COSINE, f"{what}: max_rel_err={err:.3e} cosine={cos:.8f}"


def bf16_ulp_diff(a, b) -> np.ndarray:
    """Distance in BF16 units in the last place between two BF16 bit arrays (same-sign ordering)."""
    def key(x):
        x = np.asarray(x, np.uint16).astype(np.int32)
        return np.where(x & 0x8000, -(x & 0x7FFF), x)
    return np.abs(key(a) - key(b))


def assert_gemv_close(got, ref, what="", min_equal=0.97):
    """GEMV outputs from a different FP32 summation order than the in-order oracle: almost all BF16
    results identical, and every difference within 2^-7 of the row's largest magnitude (an ulp bound
    is meaningless where a sum cancels to near zero). The equal fraction guards against systematic
    errors (a wrong scale, operand or layout changes nearly every output): `min_equal` is 0.97 for
    E2M1 x E4M3 products (5 significant bits); FP8 x FP8 products carry 8 and the MFMA rounds its four
    scaled 32-blocks once instead of four times, so a reordered sum lands on the other side of a BF16
    rounding boundary more often, and small samples (a few hundred outputs) vary; those callers pass 0.90."""
    ulps = bf16_ulp_diff(got, ref)
    equal = float(np.mean(ulps == 0))
    g, r = as_f64(got), as_f64(ref)
    scale = np.max(np.abs(r), axis=-1, keepdims=True)
    worst = float(np.max(np.abs(g - r) / np.maximum(scale, 1e-30)))
    assert equal >= min_equal and worst <= 2 ** -7, \
        f"{what}: equal fraction {equal:.4f}, worst normwise diff {worst:.3e}"


def exact_activation(rng, tokens, hidden):
    """Inputs whose per-32 quantization is exact: integers in [-16, 16] with one element per block
    set to +-448 (scale 2^0) or +-224 (scale 2^-1), so every E4M3 code times its scale is the input."""
    x = rng.integers(-16, 17, (tokens, hidden)).astype(np.float32)
    blocks = hidden // 32
    pick = rng.integers(0, 32, (tokens, blocks))
    big = rng.choice(np.array([448.0, -448.0, 224.0, -224.0], np.float32), (tokens, blocks))
    for t in range(tokens):
        x[t, np.arange(blocks) * 32 + pick[t]] = big[t]
    return x


def write_layer(root, rng, profile, layer, stored=None, bias_shift=None):
    """One MoE layer of `profile` as the reference's on-disk artifacts under `root`: an expert store (the
    experts in `stored`, all by default), gate, router-bias and FP8 shared-expert fixtures. Returns
    {"paths": (store, gate, router, shared), "experts", "gate" (BF16 bits), "biases", "shared"}."""
    from oracle.formats import bf16_bits
    from oracle.inputs import fp8_block32_expert_normal, mxfp4_expert, router_weight
    from vesper_amd.fixtures import write_gate_fixture, write_router_fixture, write_shared_fixture
    from vesper_amd.store import build_store

    h, i, e = profile.hidden, profile.intermediate, profile.experts
    stored = range(e) if stored is None else stored
    experts = {n: mxfp4_expert(rng, h, i) for n in range(e)}
    build_store([(layer, n, experts[n]) for n in stored], root / "store", max_experts=len(stored), profile=profile)
    gate = bf16_bits(router_weight(rng, e, h))
    biases = {n: (rng.standard_normal(e) * 0.05).astype(np.float32) for n in ("bias", "bias_vl")}
    for name, shift in (bias_shift or {}).items():
        biases[name] = biases[name] + np.asarray(shift, np.float32)
    shared = fp8_block32_expert_normal(rng, h, i)
    paths = (root / "store", write_gate_fixture(root / "gate", layer, gate, profile),
             write_router_fixture(root / "router", layer, biases, profile),
             write_shared_fixture(root / "shared", layer, shared, profile))
    return {"paths": paths, "experts": experts, "gate": gate, "biases": biases, "shared": shared}
