"""Device format hooks and the exact-bit comparator (mirrors src/vesper/conformance.py:15-122).

decode_fp4 / encode_fp8 / activation32 run the bit-exact format kernels
(mx_dequant_mxfp4, mx_encode_e4m3, mx_act_quant32_f32) on NumPy inputs and
return NumPy results; compare() reports mismatches with the reference's
semantics (exact FP32 bits, NaN by classification, signed zero preserved).
"""

from __future__ import annotations

import numpy as np

from . import _lib


def compare(expected: np.ndarray, actual: np.ndarray, label: str) -> dict:
    """Exact-bit comparison report with the reference's result keys (src/vesper/conformance.py:15-28).

    Floating arrays are compared as their storage words, so signed zeros differ; two NaNs of any payload
    count as equal. Other dtypes compare storage values directly."""
    if (expected.shape, expected.dtype) != (actual.shape, actual.dtype):
        return {"check": label, "status": "fail", "reason": "shape_or_dtype_mismatch"}
    floating = expected.dtype.kind == "f"
    if floating:
        word = np.dtype(f"u{expected.dtype.itemsize}")
        differs = np.not_equal(expected.view(word), actual.view(word))
        np.logical_and(differs, ~np.logical_and(np.isnan(expected), np.isnan(actual)), out=differs)
    else:
        differs = np.not_equal(expected, actual)
    where = np.flatnonzero(differs)
    semantics = (f"exact_float{8 * expected.dtype.itemsize}_bits_with_NaN_classification; signed_zero_preserved"
                 if floating else "exact_storage_bits")
    return {"check": label, "status": "fail" if where.size else "pass", "elements": int(expected.size),
            "mismatches": int(where.size), "comparison": semantics, "first_mismatch_indices": where[:8].tolist()}


def decode_fp4(ctx: _lib.Context, packed: np.ndarray, scales: np.ndarray) -> np.ndarray:
    packed = np.ascontiguousarray(packed, np.uint8)
    rows, k = packed.shape[0], packed.shape[1] * 2
    scales = np.ascontiguousarray(scales, np.uint8)
    if scales.shape != (rows, k // 32):
        raise ValueError("Scale shape does not match packed FP4 weights")
    pd, sd, od = ctx.upload(packed), ctx.upload(scales), ctx.empty((rows, k), np.float32)
    try:
        ctx.lib.dequant_mxfp4(ctx._h(), _lib.vp(pd), _lib.vp(sd), _lib.vp(od), rows, k, None)
        return od.download()
    finally:
        for d in (pd, sd, od):
            d.free()


def encode_fp8(ctx: _lib.Context, values: np.ndarray) -> np.ndarray:
    values = np.ascontiguousarray(values, np.float32)
    vd, od = ctx.upload(values), ctx.empty(values.shape, np.uint8)
    try:
        ctx.lib.encode_e4m3(ctx._h(), _lib.vp(vd), _lib.vp(od), values.size, None)
        return od.download()
    finally:
        vd.free()
        od.free()


def activation32(ctx: _lib.Context, values: np.ndarray):
    values = np.ascontiguousarray(values, np.float32)
    if values.ndim == 1:
        values = values.reshape(1, -1)
    rows, width = values.shape
    if width % 32 or not np.isfinite(values).all():
        raise ValueError("Activation must be finite with a width divisible by 32")
    vd, qd, sd = ctx.upload(values), ctx.empty((rows, width), np.uint8), ctx.empty((rows, width // 32), np.uint8)
    try:
        ctx.lib.act_quant32_f32(ctx._h(), _lib.vp(vd), _lib.vp(qd), _lib.vp(sd), rows, width, None)
        return qd.download(), sd.download()
    finally:
        for d in (vd, qd, sd):
            d.free()
