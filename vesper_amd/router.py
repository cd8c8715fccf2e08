"""Gate projection and routing postprocessing on the device (mirrors src/vesper/router.py:195-274
and src/vesper/gate.py:102-164).

RouterProbe(arrays{bias, bias_vl}) is a context manager with inspect(logits,
image_span, synthetic_zero_bias), inspect_selection(scores, selection) and
decision(logits), returning the reference's dict keys (scores, selection, raw,
denominator, weights, indices, tied). It is generalised from E=384/k=6/
sqrtsoftplus/x1.5 to any (E <= 1024, k <= 32, sigmoid | sqrtsoftplus, scale).
Logits may be [E] (the reference's single row) or [T, E].
"""

from __future__ import annotations

import ctypes as C
import math

import numpy as np

from . import _lib
from .layer import bf16_input

ROUTER_CONFIG = {"experts": 384, "topk": 6, "score_func": "sqrtsoftplus", "route_scale": 1.5,
                 "normalization_epsilon": 1e-20}


class RouterProbe:
    def __init__(self, arrays=None, ordinal=0, *, experts=384, top_k=6, score_func="sqrtsoftplus", route_scale=1.5):
        if score_func not in _lib.MX_SCORE:
            raise ValueError("Unknown score function")
        if not 1 <= experts <= 1024 or not 1 <= top_k <= min(32, experts) or not math.isfinite(route_scale):
            raise ValueError("Router configuration outside the supported range")
        arrays = arrays or {}
        if set(arrays) - {"bias", "bias_vl"}:
            raise ValueError("Routing accepts only text and image-span biases")
        for array in arrays.values():
            if (np.asarray(array).dtype != np.float32 or np.asarray(array).shape != (experts,)
                    or not np.isfinite(array).all()):
                raise ValueError(f"Router bias must contain {experts} finite FP32 values")
        self.arrays, self.ordinal = arrays, ordinal
        self.experts, self.top_k, self.score_func, self.route_scale = experts, top_k, score_func, route_scale
        self.ctx = None
        self.inspections = 0

    def __enter__(self):
        if self.ctx is not None:
            raise RuntimeError("Router probe is already open")
        self.ctx = _lib.Context(self.ordinal)
        try:
            self.biases = {n: self.ctx.upload(np.ascontiguousarray(a, np.float32)) for n, a in self.arrays.items()}
            return self
        except BaseException:
            self.close()
            raise

    def _rows(self, values, name):
        values = np.ascontiguousarray(values, dtype=np.float32)
        if values.ndim == 1:
            values = values.reshape(1, -1)
        if values.ndim != 2 or values.shape[1] != self.experts or not np.isfinite(values).all():
            raise ValueError(f"Router probe accepts finite FP32 {name} of width {self.experts}")
        return values

    def _outputs(self, t):
        e, k = self.experts, self.top_k
        bufs = {"scores": ((t, e), np.float32), "selection": ((t, e), np.float32), "raw": ((t, k), np.float32),
                "denominator": ((t,), np.float32), "weights": ((t, k), np.float32), "indices": ((t, k), np.int32),
                "tied": ((t,), np.int32)}
        dev = {n: self.ctx.empty(shape, dtype) for n, (shape, dtype) in bufs.items()}
        out = _lib.MxRouterOut(None, dev["scores"].ptr, dev["selection"].ptr, dev["indices"].ptr,
                               dev["weights"].ptr, dev["raw"].ptr, dev["denominator"].ptr, dev["tied"].ptr)
        return dev, out

    def _collect(self, dev, single):
        result = {n: d.download() for n, d in dev.items()}
        for d in dev.values():
            d.free()
        if single:
            result = {n: v.reshape(-1) if v.ndim > 1 else v for n, v in result.items()}
            result["tied"] = result["tied"].reshape(1)
            result["denominator"] = result["denominator"].reshape(1)
        self.inspections += 1
        return result

    def inspect(self, logits, image_span=False, synthetic_zero_bias=False) -> dict:
        if self.ctx is None:
            raise RuntimeError("Use the router probe as a context manager")
        if type(image_span) is not bool or type(synthetic_zero_bias) is not bool:
            raise ValueError("Router probe mask flags must be boolean")
        single = np.asarray(logits).ndim == 1
        rows = self._rows(logits, "logits")
        t = rows.shape[0]
        bias = None
        if not synthetic_zero_bias:
            name = "bias_vl" if image_span else "bias"
            bias = self.biases.get(name)
        ld = self.ctx.upload(rows)
        dev, out = self._outputs(t)
        try:
            self.ctx.lib.router_postprocess(self.ctx._h(), _lib.vp(ld), _lib.vp(bias), t, self.experts, self.top_k,
                                            _lib.MX_SCORE[self.score_func], self.route_scale, C.byref(out), None)
            return self._collect(dev, single)
        finally:
            ld.free()

    def inspect_selection(self, scores, selection) -> dict:
        """Synthetic selection-only diagnostics (router.py:243-258)."""
        if self.ctx is None:
            raise RuntimeError("Use the router probe as a context manager")
        single = np.asarray(scores).ndim == 1
        s, sel = self._rows(scores, "scores"), self._rows(selection, "selection")
        if s.shape != sel.shape or np.any(s < 0) or np.max(s) > np.finfo(np.float32).max / 8:
            raise ValueError("Synthetic selection requires finite bounded raw scores and finite selection scores")
        t = s.shape[0]
        sd, seld = self.ctx.upload(s), self.ctx.upload(sel)
        dev, out = self._outputs(t)
        try:
            self.ctx.copy_d2d(dev["scores"].ptr, sd.ptr, s.nbytes)
            self.ctx.copy_d2d(dev["selection"].ptr, seld.ptr, sel.nbytes)
            self.ctx.lib.router_select(self.ctx._h(), _lib.vp(sd), _lib.vp(seld), t, self.experts, self.top_k,
                                       self.route_scale, C.byref(out), None)
            return self._collect(dev, single)
        finally:
            sd.free()
            seld.free()

    def decision(self, logits, image_span=False):
        result = self.inspect(logits, image_span=image_span)
        return result["weights"], result["indices"]

    def close(self):
        if self.ctx is not None:
            ctx, self.ctx = self.ctx, None
            ctx.close()

    def __exit__(self, *_):
        self.close()


class GateProjection:
    """FP32 logits = W_r (BF16 bits promoted, or FP32) . x (gate.py:102-164); any T rows."""

    def __init__(self, weight, ordinal=0):
        weight = np.asarray(weight)
        if weight.ndim != 2 or weight.dtype not in (np.dtype(np.uint16), np.dtype(np.float32)):
            raise ValueError("Gate weight must be a 2-D BF16 (uint16 bits) or FP32 matrix")
        if weight.dtype == np.uint16:
            if np.any((weight & 0x7F80) == 0x7F80):
                raise ValueError("Gate weight must contain finite BF16 values")
            weight = (weight.astype(np.uint32) << 16).view(np.float32)
        if not np.isfinite(weight).all() or weight.shape[1] % 4:
            raise ValueError("Gate weight must be finite with a width divisible by 4")
        self.weight, self.ordinal = np.ascontiguousarray(weight, np.float32), ordinal
        self.experts, self.hidden = weight.shape
        self.ctx = None
        self.calls = 0

    def __enter__(self):
        if self.ctx is not None:
            raise RuntimeError("Gate projection is already open")
        self.ctx = _lib.Context(self.ordinal)
        try:
            self.w = self.ctx.upload(self.weight)
            return self
        except BaseException:
            self.__exit__()
            raise

    def project(self, activation) -> np.ndarray:
        if self.ctx is None:
            raise RuntimeError("Use the gate projection as a context manager")
        single = np.asarray(activation).ndim == 1
        bits = bf16_input(np.asarray(activation), self.hidden)
        t = bits.shape[0]
        xd = self.ctx.upload(bits)
        out = self.ctx.empty((t, self.experts), np.float32)
        try:
            self.ctx.lib.gate_project(self.ctx._h(), _lib.vp(self.w), _lib.vp(xd), t, self.hidden, self.experts,
                                      _lib.vp(out), None)
            logits = out.download()
        finally:
            xd.free()
            out.free()
        if not np.isfinite(logits).all():
            raise ValueError("Projection output leaves the finite probe scope")
        self.calls += 1
        return logits.reshape(-1) if single else logits

    def __exit__(self, *_):
        if self.ctx is not None:
            ctx, self.ctx = self.ctx, None
            ctx.close()
