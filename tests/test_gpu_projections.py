"""GPU parity of the FP8 block-scaled projections (NativeProjections.fp8, projections.py:135-154).

* The per-128 activation quantizer: bit-exact against the oracle (codes and FP32 scales).
* The tiled weight layout: against an independent NumPy construction from its definition.
* The product: exact on designed inputs whose every partial sum is representable (both profiles), so
  the operand layouts and scale placement are pinned bit for bit; random inputs within the GEMV bar;
  configuration-3 shapes at T = 1, 16, 300 and 2048 (the GEMM and split-K branches the benchmark times,
  sampled tokens; at 2048 also on exact inputs, bit for bit) and the reference shapes within the
  north-star tolerance.
"""

import ctypes as C

import numpy as np
import pytest

from oracle.formats import bf16_bits, bf16_values, encode_e4m3, quantize_activation
from oracle.projections import (CONFIG3_LAYOUT, fp8_block128_gemm_fp32, fp8_projection, fp8_weights,
                                quantize_activation_128)
from tests.helpers import assert_close, assert_gemv_close
from vesper_amd import _lib
from vesper_amd.projections import FP8_LAYOUT, NativeProjections

pytestmark = pytest.mark.gpu


def tile_numpy(w, sw, block):
    n, k = w.shape
    g, c, t, h, l = np.meshgrid(np.arange(n // 64), np.arange(k // 128), np.arange(4), np.arange(2), np.arange(64),
                                indexing="ij")
    rows = 64 * g + 16 * t + (l % 16)
    k0 = 128 * c + 64 * h + 16 * (l // 16)
    pieces = w[rows[..., None], k0[..., None] + np.arange(16)]
    out = [pieces.reshape(-1)]
    if block == 32:
        g, c, l = np.meshgrid(np.arange(n // 64), np.arange(k // 128), np.arange(64), indexing="ij")
        word = np.zeros(g.shape, np.uint32)
        for t in range(4):
            word |= sw[(64 * g + 16 * t) // 32, 4 * c + l // 16].astype(np.uint32) << (8 * t)
        out.append(word.reshape(-1).view(np.uint8))
    else:
        out.append(np.ascontiguousarray(sw, np.float32).reshape(-1).view(np.uint8))
    return np.concatenate(out)                               # the blob's tail padding is not defined


def arrays_for(layout, block, rng, layer=0):
    arrays = {}
    for name, (rows, width) in layout.items():
        w, s = fp8_weights(rng, rows, width, block)
        arrays[f"layers.{layer}.attn.{name}.weight"] = w
        arrays[f"layers.{layer}.attn.{name}.scale"] = s
    return arrays


@pytest.mark.parametrize("offset", [0, 2])
def test_act_quant128_bit_exact(gpu_ctx, offset):
    """offset 0: 16-byte aligned buffers (8 values per lane); offset 2 values: the 4-byte aligned path."""
    rng = np.random.default_rng(7)
    x = rng.standard_normal((9, 1024)).astype(np.float32)
    x *= np.ldexp(np.ones((9, 1), np.float32), rng.integers(-30, 10, (9, 1)))
    x[0] = 0
    x[1, :128] = 448.0
    x[2, 256:384] = -1e-7
    bits = bf16_bits(x)
    padded = np.concatenate([np.zeros(offset, np.uint16), bits.ravel()])
    xd = gpu_ctx.upload(padded)
    q = gpu_ctx.empty((9 * 1024 + 2 * offset,), np.uint8)
    s = gpu_ctx.empty((9, 8), np.float32)
    gpu_ctx.lib.act_quant128(gpu_ctx._h(), _lib.vp(xd.ptr + 2 * offset), _lib.vp(q.ptr + 2 * offset), _lib.vp(s), 9,
                             1024, None)
    q_ref, s_ref = quantize_activation_128(bf16_values(bits))
    np.testing.assert_array_equal(s.download().view(np.uint32), s_ref.view(np.uint32))
    np.testing.assert_array_equal(q.download()[2 * offset:].reshape(9, 1024), q_ref)
    for d in (xd, q, s):
        d.free()


@pytest.mark.parametrize("block", [32, 128])
def test_tiled_layout_matches_definition(gpu_ctx, block):
    rng = np.random.default_rng(block)
    w, sw = fp8_weights(rng, 192, 384, block)
    wd, sd = gpu_ctx.upload(w), gpu_ctx.upload(sw)
    n = int(gpu_ctx.lib.cdll.mx_fp8_tiled_bytes(192, 384, block))
    blob = gpu_ctx.malloc(n)
    try:
        gpu_ctx.lib.fp8_tile(gpu_ctx._h(), _lib.vp(wd), _lib.vp(sd), 192, 384, block, C.c_void_p(blob), None)
        got = gpu_ctx.download(blob, (n,), np.uint8)
        want = tile_numpy(w, sw, block)
        assert n == (len(want) + 255) // 256 * 256
        np.testing.assert_array_equal(got[:len(want)], want)
    finally:
        gpu_ctx.free(blob)
        wd.free()
        sd.free()


def run_projection(block, w, sw, x_bits):
    rows, width = w.shape
    layout = {"p": (rows, width)}
    arrays = {"layers.0.attn.p.weight": w, "layers.0.attn.p.scale": sw}
    with NativeProjections(arrays, block=block, layout=layout) as proj:
        return proj.fp8("p", x_bits)


def exact_case(block, tokens, rows, width, wmax, xmax, seed):
    """Small-integer codes, power-of-two scales: every partial sum is exact, so any order gives the
    same FP32 result and the trace must equal the oracle bit for bit."""
    rng = np.random.default_rng(seed)
    codes = encode_e4m3(np.arange(-wmax, wmax + 1, dtype=np.float32))      # the integers' E4M3 codes
    w = codes[rng.integers(-wmax, wmax + 1, (rows, width)) + wmax]
    if block == 32:
        sw = rng.integers(125, 130, (rows // 32, width // 32), dtype=np.uint8)
        x = rng.integers(-xmax, xmax + 1, (tokens, width)).astype(np.float32)
        x[:, ::32] = 448.0                                   # per-32 scale 2^0: codes are the integers
    else:
        sw = np.exp2(rng.integers(-8, -2, ((rows + 127) // 128, width // 128))).astype(np.float32)
        x = rng.integers(-xmax, xmax + 1, (tokens, width)).astype(np.float32)
        x[:, ::128] = 448.0                                  # per-128 scale exactly 1
    return w, sw, x


@pytest.mark.parametrize("block", [32, 128])
@pytest.mark.parametrize("tokens", [1, 5, 16, 21, 40, 200])
def test_exact_on_representable_inputs(block, tokens):
    rows, width = (128, 512) if tokens <= 32 else (320, 640)       # 320 rows: a partial 256-row GEMM tile
    w, sw, x = exact_case(block, tokens, rows, width, 8, 16, block * 100 + tokens)
    check_exact(block, w, sw, x)


@pytest.mark.parametrize("block", [32, 128])
def test_exact_through_the_split_k_gemm(block):
    """200 tokens x 320 rows over K = 2048: the GEMM splits K in two and adds the FP32 partial sums in
    split order; magnitudes stay small enough (|sum| < 2^16 units of the smallest scale) to be exact."""
    w, sw, x = exact_case(block, 200, 320, 2048, 1, 2, 7 + block)
    check_exact(block, w, sw, x)


@pytest.mark.parametrize("block", [32, 128])
@pytest.mark.parametrize("tokens,rows,width", [(33, 64, 128), (129, 64, 256), (33, 192, 384), (257, 128, 128)])
def test_exact_gemm_edges(block, tokens, rows, width):
    """The GEMM's 3-stage LDS ring at its edges: one K chunk (nothing copied ahead), a single 64-row group
    in a 256-row workgroup, token counts just past the GEMV's limit and a partial last tile."""
    w, sw, x = exact_case(block, tokens, rows, width, 8, 16, 1000 * block + tokens + rows + width)
    check_exact(block, w, sw, x)


@pytest.mark.parametrize("block", [32, 128])
@pytest.mark.parametrize("tokens,rows,width,wmax,xmax", [(512, 320, 640, 8, 16), (600, 64, 128, 8, 16),
                                                         (777, 192, 2048, 1, 2)])
def test_exact_long_batches(block, tokens, rows, width, wmax, xmax):
    """Several 128-token tiles: a partial last row tile, one K chunk with a single 64-row group and a
    partial last token tile, and K = 2048 split in two."""
    w, sw, x = exact_case(block, tokens, rows, width, wmax, xmax, 3000 * block + tokens + rows + width)
    check_exact(block, w, sw, x)


@pytest.mark.parametrize("block", [32, 128])
@pytest.mark.parametrize("tokens", [1, 21])
def test_exact_through_the_split_k_gemv(block, tokens):
    """K = 2048 splits the GEMV's K four ways; the last workgroup of each tile adds the partial sums in
    split order. Three calls in a row on one weight set, each with new activations, each exact: a tile
    counter left behind by one call would leave the next call's outputs unwritten."""
    w, sw, _ = exact_case(block, tokens, 192, 2048, 4, 8, 31 + block + tokens)
    rows, width = w.shape
    arrays = {"layers.0.attn.p.weight": w, "layers.0.attn.p.scale": sw}
    with NativeProjections(arrays, block=block, layout={"p": (rows, width)}) as proj:
        for call in range(3):
            _, _, x = exact_case(block, tokens, rows, width, 4, 8, 100 * call + block + tokens)
            bits = bf16_bits(x)
            got = proj.fp8("p", bits)
            ref = fp8_projection(bf16_values(bits), w, sw, block)
            np.testing.assert_array_equal(got["output_fp32"].view(np.uint32), ref["output_fp32"].view(np.uint32),
                                          err_msg=f"call {call}")
            np.testing.assert_array_equal(got["output_bf16"], ref["output_bf16"], err_msg=f"call {call}")


def project_both_ways(proj, ctx, name, bits, rows, width):
    """One projection of BF16 `bits` with the activation codes and scales requested (the quantizer kernel
    runs first) and without them (block 128 at <= 4 tokens: the GEMV quantizes in LDS). Returns
    (trace, y) of each."""
    tokens = bits.shape[0]
    x = ctx.upload(bits)
    q = ctx.empty((tokens, width), np.uint8)
    s = ctx.empty((tokens, width // 128), np.float32)
    outs = []
    try:
        for with_codes in (True, False):
            trace = ctx.empty((tokens, rows), np.float32)
            y = ctx.empty((tokens, rows), np.uint16)
            proj.project_device(name, x.ptr, tokens, y.ptr, trace_ptr=trace, q_ptr=q if with_codes else None,
                                s_ptr=s if with_codes else None)
            outs.append((trace.download(), y.download()))
            trace.free()
            y.free()
    finally:
        for d in (x, q, s):
            d.free()
    return outs


@pytest.mark.parametrize("tokens", [1, 3, 4])
@pytest.mark.parametrize("rows,width", [(256, 1024), (128, 2048), (576, 7168)])
def test_gemv_quantizing_in_lds_equals_the_quantizer_path(gpu_ctx, tokens, rows, width):
    """Block 128 at <= 4 tokens without requested codes: the GEMV quantizes its own K range with the
    quantizer kernel's arithmetic, so FP32 sums and BF16 outputs equal the two-launch path bit for bit
    (random inputs), and the oracle's exactly on representable inputs."""
    rng = np.random.default_rng(tokens * 1000 + rows + width)
    w, sw = fp8_weights(rng, rows, width, 128)
    arrays = {"layers.0.attn.p.weight": w, "layers.0.attn.p.scale": sw}
    with NativeProjections(arrays, block=128, layout={"p": (rows, width)}) as proj:
        bits = bf16_bits(rng.standard_normal((tokens, width)).astype(np.float32))
        (t_q, y_q), (t_f, y_f) = project_both_ways(proj, gpu_ctx, "p", bits, rows, width)
        np.testing.assert_array_equal(t_f.view(np.uint32), t_q.view(np.uint32))
        np.testing.assert_array_equal(y_f, y_q)
    w, sw, x = exact_case(128, tokens, rows, width, 2, 4, 7 * tokens + rows)   # sums below 2^24 units of 2^-8
    arrays = {"layers.0.attn.p.weight": w, "layers.0.attn.p.scale": sw}
    with NativeProjections(arrays, block=128, layout={"p": (rows, width)}) as proj:
        bits = bf16_bits(x)
        ref = fp8_projection(bf16_values(bits), w, sw, 128)
        (_, _), (t_f, y_f) = project_both_ways(proj, gpu_ctx, "p", bits, rows, width)
        np.testing.assert_array_equal(t_f.view(np.uint32), ref["output_fp32"].view(np.uint32))
        np.testing.assert_array_equal(y_f, ref["output_bf16"])


@pytest.mark.parametrize("rows,width,tokens", [(4096, 2048, 1), (4096, 2048, 3), (16384, 1024, 1), (16384, 1024, 4),
                                               (4096, 16384, 1), (4096, 16384, 2)])
def test_tile_gemv_shapes_equal_the_quantizer_path_and_the_oracle(gpu_ctx, rows, width, tokens):
    """The block-128 tile GEMV's other workgroup shapes (the test above runs 1 tile x 8 K parts): 2 tiles x 8
    parts (256-1023 tiles) and 2 tiles x 4 parts (1024 tiles and more), with 1, 2 and 4 in-kernel
    quantization passes, and the unfused tile kernel where a wave's blocks exceed its LDS rows (16384 wide
    at 2 tokens). Random inputs: the same bits with or without codes requested; exact inputs: the oracle's
    bits."""
    rng = np.random.default_rng(tokens * 7 + rows + width)
    w, sw = fp8_weights(rng, rows, width, 128)
    arrays = {"layers.0.attn.p.weight": w, "layers.0.attn.p.scale": sw}
    with NativeProjections(arrays, block=128, layout={"p": (rows, width)}) as proj:
        bits = bf16_bits(rng.standard_normal((tokens, width)).astype(np.float32))
        (t_q, y_q), (t_f, y_f) = project_both_ways(proj, gpu_ctx, "p", bits, rows, width)
        np.testing.assert_array_equal(t_f.view(np.uint32), t_q.view(np.uint32))
        np.testing.assert_array_equal(y_f, y_q)
    w, sw, x = exact_case(128, tokens, rows, width, 2, 4, 11 * tokens + rows + width)
    arrays = {"layers.0.attn.p.weight": w, "layers.0.attn.p.scale": sw}
    with NativeProjections(arrays, block=128, layout={"p": (rows, width)}) as proj:
        bits = bf16_bits(x)
        ref = fp8_projection(bf16_values(bits), w, sw, 128)
        (_, _), (t_f, y_f) = project_both_ways(proj, gpu_ctx, "p", bits, rows, width)
        np.testing.assert_array_equal(t_f.view(np.uint32), ref["output_fp32"].view(np.uint32))
        np.testing.assert_array_equal(y_f, ref["output_bf16"])


def check_exact(block, w, sw, x):
    bits = bf16_bits(x)
    got = run_projection(block, w, sw, bits)
    ref = fp8_projection(bf16_values(bits), w, sw, block)
    np.testing.assert_array_equal(got["input_fp8"], ref["input_fp8"])
    scale_key = "scale_e8m0" if block == 32 else "scale_f32"
    np.testing.assert_array_equal(got[scale_key].view(np.uint8), np.asarray(ref["scale"]).view(np.uint8))
    np.testing.assert_array_equal(got["output_fp32"].view(np.uint32), ref["output_fp32"].view(np.uint32))
    np.testing.assert_array_equal(got["output_bf16"], ref["output_bf16"])


@pytest.mark.parametrize("block", [32, 128])
def test_random_inputs_close_to_ordered_sum(block):
    rng = np.random.default_rng(11 + block)
    w, sw = fp8_weights(rng, 320, 2048, block)
    bits = bf16_bits(rng.standard_normal((7, 2048)).astype(np.float32))
    got = run_projection(block, w, sw, bits)
    ref = fp8_projection(bf16_values(bits), w, sw, block)
    np.testing.assert_array_equal(got["input_fp8"], ref["input_fp8"])
    assert_gemv_close(got["output_bf16"], ref["output_bf16"], f"block {block}", min_equal=0.90)
    assert_close(got["output_bf16"], ref["output_bf16"], f"block {block}")


@pytest.mark.parametrize("tokens", [1, 16, 300])
def test_config3_projections_within_tolerance(tokens):
    rng = np.random.default_rng(20261018 + tokens)
    arrays = arrays_for(CONFIG3_LAYOUT, 128, rng)
    x = {name: bf16_bits(rng.standard_normal((tokens, width)).astype(np.float32))
         for name, (_, width) in CONFIG3_LAYOUT.items()}
    with NativeProjections(arrays, block=128) as proj:
        for name, (rows, width) in CONFIG3_LAYOUT.items():
            got = proj.fp8(name, x[name])
            ref = fp8_projection(bf16_values(x[name]), arrays[f"layers.0.attn.{name}.weight"],
                                 arrays[f"layers.0.attn.{name}.scale"], 128)
            assert got["output_bf16"].shape == (tokens, rows)
            np.testing.assert_array_equal(got["input_fp8"], ref["input_fp8"])
            assert_close(got["output_bf16"], ref["output_bf16"], name)


@pytest.mark.parametrize("tokens", [1, 16, 2048])
def test_config3_stacked_q_a_kv_a(tokens):
    """q_a and kv_a as one projection of their stacked rows (the benchmark's timed form, 2112 rows: the last
    128-row scale block half full): sampled tokens within the bar of the oracle, for both row ranges."""
    rng = np.random.default_rng(30 + tokens)
    layout = {"q_kv_a": (1536 + 576, 7168)}
    arrays = arrays_for(layout, 128, rng)
    x = bf16_bits(rng.standard_normal((tokens, 7168)).astype(np.float32))
    sample = np.unique(np.concatenate([[0, tokens - 1], rng.choice(tokens, min(tokens, 32), replace=False)]))
    with NativeProjections(arrays, block=128, layout=layout) as proj:
        got = proj.fp8("q_kv_a", x)
    ref = fp8_projection(bf16_values(x[sample]), arrays["layers.0.attn.q_kv_a.weight"],
                         arrays["layers.0.attn.q_kv_a.scale"], 128)
    for rows, name in ((slice(0, 1536), "q_a rows"), (slice(1536, 2112), "kv_a rows")):
        assert_close(got["output_bf16"][sample][:, rows], ref["output_bf16"][:, rows], f"{name} T={tokens}")


def test_config3_T2048_sampled_tokens_within_tolerance():
    """All four configuration-3 projections at the benchmark's 2048 tokens: the whole batch runs through the
    GEMM (q_a and kv_a with K split too), and 64 sampled tokens (first and last included, spread over every
    128-token tile) are compared with the oracle: codes bit-exact, outputs within the north-star bar."""
    tokens = 2048
    rng = np.random.default_rng(20262048)
    arrays = arrays_for(CONFIG3_LAYOUT, 128, rng)
    sample = np.unique(np.concatenate([[0, tokens - 1], rng.choice(tokens, 62, replace=False)]))
    with NativeProjections(arrays, block=128) as proj:
        for name, (rows, width) in CONFIG3_LAYOUT.items():
            x = bf16_bits(rng.standard_normal((tokens, width)).astype(np.float32))
            got = proj.fp8(name, x)
            ref = fp8_projection(bf16_values(x[sample]), arrays[f"layers.0.attn.{name}.weight"],
                                 arrays[f"layers.0.attn.{name}.scale"], 128)
            assert got["output_bf16"].shape == (tokens, rows)
            np.testing.assert_array_equal(got["input_fp8"][sample], ref["input_fp8"])
            np.testing.assert_array_equal(got["scale_f32"][sample].view(np.uint32), ref["scale"].view(np.uint32))
            assert_close(got["output_bf16"][sample], ref["output_bf16"], f"{name} T={tokens}")
            assert_gemv_close(got["output_bf16"][sample], ref["output_bf16"], f"{name} T={tokens}", min_equal=0.90)


def test_config3_T2048_exact_sampled_tokens():
    """The four configuration-3 shapes at 2048 tokens on exact inputs (small integer codes, power-of-two
    scales, |sums| below 2^16 units of the smallest scale, so every partial sum is representable): the GEMM's
    tiling, copy pipeline and K splits at the benchmark's shapes are pinned bit for bit on 64 sampled tokens,
    tile edges included."""
    tokens = 2048
    rng = np.random.default_rng(20262049)
    sample = np.unique(np.concatenate([[0, 127, 128, tokens - 1], rng.choice(tokens, 60, replace=False)]))
    for i, (name, (rows, width)) in enumerate(CONFIG3_LAYOUT.items()):
        w, sw, x = exact_case(128, tokens, rows, width, 1, 2, 777 + i)
        bits = bf16_bits(x)
        got = run_projection(128, w, sw, bits)
        ref = fp8_projection(bf16_values(bits[sample]), w, sw, 128)
        np.testing.assert_array_equal(got["output_fp32"][sample].view(np.uint32), ref["output_fp32"].view(np.uint32),
                                      err_msg=name)
        np.testing.assert_array_equal(got["output_bf16"][sample], ref["output_bf16"], err_msg=name)


def test_reference_shapes_block32_and_refusals():
    rng = np.random.default_rng(5)
    arrays = arrays_for(FP8_LAYOUT, 32, rng)
    proj = NativeProjections(arrays, block=32)
    with proj:
        open_stats = proj.stats()
        assert open_stats["owned_context_active"] and open_stats["host_reserved_bytes"] == 512 * 2 ** 20
        assert open_stats["device_owned_bytes"] >= proj.resident_bytes
        x = bf16_bits(rng.standard_normal((2, 4, 5120)).astype(np.float32))
        got = proj.fp8("wq_a", x)
        assert got["output_bf16"].shape == (2, 4, 1280) and got["scale_e8m0"].shape == (2, 4, 160)
        ref = fp8_projection(bf16_values(x.reshape(8, 5120)), arrays["layers.0.attn.wq_a.weight"],
                             arrays["layers.0.attn.wq_a.scale"], 32)
        assert_close(got["output_bf16"].reshape(8, 1280), ref["output_bf16"], "wq_a")
        with pytest.raises(ValueError):
            proj.fp8("wq_a", x.astype(np.float32))
        with pytest.raises(ValueError):
            proj.fp8("wq_a", np.full((1, 5120), 0x7F80, np.uint16))
        with pytest.raises(ValueError):
            proj.fp8("wo_a", x)
    # the reference's stats() keys (projections.py:189-195); the ledger is released and the peak kept on close
    closed = proj.stats()
    assert set(closed) == {"host_allowance_bytes", "host_reserved_bytes", "device_peak_owned_bytes",
                           "device_owned_bytes", "owned_context_active", "reservation_is_RSS_limit",
                           "driver_module_memory_excluded"}
    assert not closed["owned_context_active"] and closed["host_reserved_bytes"] == 0 == closed["device_owned_bytes"]
    assert closed["host_allowance_bytes"] == 512 * 2 ** 20
    assert closed["device_peak_owned_bytes"] >= proj.resident_bytes
    bad = dict(arrays)
    bad["layers.0.attn.wkv.scale"] = np.full((16, 160), 255, np.uint8)
    with pytest.raises(ValueError):
        NativeProjections(bad, block=32)


def wo_a_arrays(w, sw):
    """The grouped projection's weights beside one tiny block-32 projection (the runtime tiles both)."""
    rng = np.random.default_rng(0)
    arrays = arrays_for({"p": (64, 128)}, 32, rng)
    arrays["layers.0.attn.wo_a.weight"] = w
    arrays["layers.0.attn.wo_a.scale"] = sw
    return arrays


def test_kv_round32_and_window_rounding_bit_exact():
    from oracle.projections import kv_round32
    rng = np.random.default_rng(512)
    v = rng.standard_normal((2, 7, 512)).astype(np.float32) * np.exp2(rng.integers(-12, 8, (2, 7, 1)))
    v[0, 3] = 0.0                                                # zero blocks: the floor scale
    v[1, 2, :32] = np.float32(1e-30)                              # below the floor
    bits = bf16_bits(v)
    w, sw = fp8_weights(rng, 8192, 4096, 32)
    with NativeProjections(wo_a_arrays(w, sw), block=32, layout={"p": (64, 128)}) as proj:
        got = proj.round_window(bits)
        with pytest.raises(ValueError, match="window"):
            proj.round_window(np.concatenate([bits, bits[:1]]))      # a batch of 3
    rounded, q, s = kv_round32(bits)
    np.testing.assert_array_equal(got["rounded_bf16"], rounded)
    np.testing.assert_array_equal(got["codes_fp8"], q)
    np.testing.assert_array_equal(got["scales_e8m0"], s)


def test_grouped_projection_exact_on_representable_inputs():
    """Small-integer weight codes with power-of-two block scales, and activations whose per-32 scale is
    2^0 (each block holds 448): every partial sum is exact in FP32, so the BF16 outputs equal the oracle's
    bit for bit -- and each group reads its own activations (distinct per group)."""
    from oracle.projections import wo_a_grouped
    rng = np.random.default_rng(4096)
    w = encode_e4m3(rng.integers(-8, 9, (8192, 4096)).astype(np.float32))
    sw = rng.integers(125, 130, (256, 128), dtype=np.uint8)
    for tokens in (1, 5):
        x = rng.integers(-16, 17, (tokens, 8, 4096)).astype(np.float32)
        x[..., ::32] = 448.0
        bits = bf16_bits(x)
        with NativeProjections(wo_a_arrays(w, sw), block=32, layout={"p": (64, 128)}) as proj:
            got = proj.grouped(bits)
        ref = wo_a_grouped(bits, w, sw)
        np.testing.assert_array_equal(got["input_fp8"], ref["input_fp8"])
        np.testing.assert_array_equal(got["scale_e8m0"], ref["scale_e8m0"])
        np.testing.assert_array_equal(got["rounded_bf16"], ref["rounded_bf16"])
        np.testing.assert_array_equal(got["output_bf16"], ref["output_bf16"].reshape(tokens, 8, 1024))


@pytest.mark.parametrize("lead", [(1,), (8,), (2, 3)])
def test_grouped_projection_random_within_tolerance(lead):
    from oracle.projections import wo_a_grouped
    rng = np.random.default_rng(sum(lead) + 17)
    w, sw = fp8_weights(rng, 8192, 4096, 32)
    bits = bf16_bits(rng.standard_normal((*lead, 8, 4096)).astype(np.float32))
    with NativeProjections(wo_a_arrays(w, sw), block=32, layout={"p": (64, 128)}) as proj:
        got = proj.grouped(bits)
        with pytest.raises(ValueError):
            proj.grouped(bits[..., :2048].copy())
        with pytest.raises(ValueError):
            proj.grouped(np.zeros((33, 8, 4096), np.uint16))
    ref = wo_a_grouped(bits, w, sw)
    assert got["output_bf16"].shape == (*lead, 8, 1024)
    np.testing.assert_array_equal(got["rounded_bf16"], ref["rounded_bf16"])
    assert_close(got["output_bf16"].reshape(-1, 8192), ref["output_bf16"].reshape(-1, 8192), "wo_a grouped")
