"""One expert over a few tokens with every stage returned (mirrors src/vesper/expert.py:17-114).

ExpertExecutor(ordinal, swiglu_limit, device_cap) is a context manager whose
execute(x, weights, routing_weight) takes device pointers to the six expert
tensors and returns the reference's stage dict: q, s, w1, w3, down_input,
trace, down_q, down_s, w2. Inputs are validated before any device work. The
arithmetic runs in mx_expert_forward (gfx950 scaled-MFMA kernels); T may be
1..16 tokens per call, with one routing weight per token.
"""

from __future__ import annotations

import ctypes as C
import math

import numpy as np

from . import _lib
from .layer import TENSORS, bf16_input
from .timing import Timings

MiB = 1 << 20


def _layout(hidden: int, intermediate: int) -> dict:
    return {"w1_weight": (intermediate, hidden // 2), "w1_scale": (intermediate, hidden // 32),
            "w3_weight": (intermediate, hidden // 2), "w3_scale": (intermediate, hidden // 32),
            "w2_weight": (hidden, intermediate // 2), "w2_scale": (hidden, intermediate // 32)}


def validate_expert_arrays(arrays: dict, hidden: int, intermediate: int):
    layout = _layout(hidden, intermediate)
    if set(arrays) != set(layout):
        raise ValueError("A complete expert requires exactly six native tensors")
    for name, shape in layout.items():
        a = arrays[name]
        if getattr(a, "dtype", None) != np.uint8 or tuple(a.shape) != shape:
            raise ValueError("Expert tensor layout differs from the pinned shape")


class ExpertExecutor:
    """Native expert arithmetic and reusable workspace, independent of residency."""

    def __init__(self, ordinal=0, swiglu_limit=10.0, device_cap=64 * MiB, *, hidden=5120, intermediate=2304):
        if not math.isfinite(swiglu_limit) or swiglu_limit < 0:
            raise ValueError("Invalid SwiGLU limit")
        if hidden <= 0 or hidden % 128 or intermediate <= 0 or intermediate % 128:
            raise ValueError("Expert shapes must be positive multiples of 128")
        self.ordinal, self.limit, self.device_cap = ordinal, float(swiglu_limit), device_cap
        self.hidden, self.intermediate = hidden, intermediate
        self.ctx = None
        self.timings = Timings()

    def __enter__(self):
        if self.ctx is not None:
            raise RuntimeError("Expert executor is already open")
        self.ctx = _lib.Context(self.ordinal, 0)
        try:
            t, h, i = 16, self.hidden, self.intermediate
            self.work = {"x": self.ctx.empty((t, h), np.uint16), "route": self.ctx.empty((t,), np.float32),
                         "q": self.ctx.empty((t, h), np.uint8), "s": self.ctx.empty((t, h // 32), np.uint8),
                         "w1": self.ctx.empty((t, i), np.uint16), "w3": self.ctx.empty((t, i), np.uint16),
                         "down_input": self.ctx.empty((t, i), np.uint16),
                         "trace": self.ctx.empty((t, i, 5), np.float32),
                         "down_q": self.ctx.empty((t, i), np.uint8), "down_s": self.ctx.empty((t, i // 32), np.uint8),
                         "w2": self.ctx.empty((t, h), np.uint16)}
            return self
        except BaseException:
            self.close()
            raise

    def execute(self, x, weights: dict, routing_weight=None) -> dict:
        if self.ctx is None:
            raise RuntimeError("Use the expert executor as a context manager")
        bits = bf16_input(np.asarray(x, dtype=np.float32) if np.asarray(x).dtype != np.uint16 else x, self.hidden)
        t = bits.shape[0]
        if not 1 <= t <= 16:
            raise ValueError("One expert call accepts 1 to 16 tokens")
        self._check_weights(weights)
        route = None
        if routing_weight is not None:
            route = np.broadcast_to(np.asarray(routing_weight, dtype=np.float32).reshape(-1), (t,)).copy()
            if not np.isfinite(route).all():
                raise ValueError("Routing weight must be finite")
        w = self.work
        with self.timings.section("transfer.input_h2d"):
            self.ctx.copy_h2d(w["x"].ptr, bits)
            if route is not None:
                self.ctx.copy_h2d(w["route"].ptr, route)
        stages = _lib.MxExpertStages(*[w[n].ptr for n in ("q", "s", "w1", "w3", "down_input", "trace",
                                                          "down_q", "down_s")])
        with self.timings.section("compute.kernels"):
            self._compute(weights, t, None if route is None else C.c_void_p(w["route"].ptr), stages)
            self.ctx.sync()
        h, i = self.hidden, self.intermediate
        layout = {"q": ((t, h), np.uint8), "s": ((t, h // 32), np.uint8), "w1": ((t, i), np.uint16),
                  "w3": ((t, i), np.uint16), "down_input": ((t, i), np.uint16), "trace": ((t, i, 5), np.float32),
                  "down_q": ((t, i), np.uint8), "down_s": ((t, i // 32), np.uint8), "w2": ((t, h), np.uint16)}
        with self.timings.section("transfer.diagnostics_d2h"):
            out = {name: self.ctx.download(w[name].ptr, shape, dtype) for name, (shape, dtype) in layout.items()}
        # the reference reports down_input as FP32 values of the BF16 boundary
        out["down_input"] = (out["down_input"].astype(np.uint32) << 16).view(np.float32)
        return out

    def _check_weights(self, weights):
        if set(weights) != set(TENSORS):
            raise ValueError("A complete expert requires exactly six native tensors")

    def _compute(self, weights, t, route_ptr, stages):
        """The MXFP4 expert on the reference-layout tensors at `weights` (device pointers)."""
        w = self.work
        ptrs = _lib.MxExpertPtrs(*[int(weights[n]) for n in TENSORS])
        self.ctx.lib.expert_forward(self.ctx._h(), C.byref(ptrs), _lib.MX_FMT_MXFP4, self.hidden, self.intermediate,
                                    C.c_void_p(w["x"].ptr), t, self.limit, route_ptr, C.c_void_p(w["w2"].ptr),
                                    C.byref(stages), None)

    def close(self):
        if self.ctx is not None:
            ctx, self.ctx = self.ctx, None
            ctx.close()

    def __exit__(self, *_):
        self.close()


class ResidentExpert(ExpertExecutor):
    """Uploads one expert on enter; forward(x, routing_weight) (expert.py:95-114)."""

    def __init__(self, arrays: dict, ordinal=0, swiglu_limit=10.0, *, hidden=5120, intermediate=2304):
        validate_expert_arrays(arrays, hidden, intermediate)
        super().__init__(ordinal, swiglu_limit, hidden=hidden, intermediate=intermediate)
        self.arrays = arrays
        self.weights = {}

    def __enter__(self):
        super().__enter__()
        try:
            self.device_arrays = {n: self.ctx.upload(np.ascontiguousarray(a)) for n, a in self.arrays.items()}
            self.weights = {n: a.ptr for n, a in self.device_arrays.items()}
            return self
        except BaseException:
            self.close()
            raise

    def forward(self, x, routing_weight=None) -> dict:
        return self.execute(x, self.weights, routing_weight)


class BF16ActivationExpert:
    """The benchmark's configuration-0 expert on the same MXFP4 weights: BF16 activations, FP32 accumulation,
    no activation quantization and no clamp -- y = W2 (silu(W1 x) * (W3 x)) -- where the reference's expert
    quantizes both activations to E4M3 (a separately named profile, not a replacement for ResidentExpert).

    Uploads the six tensors on enter and tiles them into the device layout the decode kernels read;
    forward(x, routing_weight=None) takes BF16 bits or FP32 values [H] or [T, H] (T <= 16) and returns
    {"gu": FP32 [T, 2I] (W1 x then W3 x), "h": FP32 [T, I], "y": BF16 bits [T, H]} (mx_expert_forward_bf16)."""

    def __init__(self, arrays: dict, ordinal=0, *, hidden=5120, intermediate=2304):
        validate_expert_arrays(arrays, hidden, intermediate)
        if hidden > 8192 or intermediate > 4096:
            raise ValueError("The BF16-activation expert supports hidden <= 8192 and intermediate <= 4096")
        self.arrays, self.ordinal = arrays, ordinal
        self.hidden, self.intermediate = hidden, intermediate
        self.ctx = None

    def __enter__(self):
        if self.ctx is not None:
            raise RuntimeError("Expert is already open")
        self.ctx = _lib.Context(self.ordinal)
        try:
            h, i, lib = self.hidden, self.intermediate, self.ctx.lib
            raw = {n: self.ctx.upload(np.ascontiguousarray(self.arrays[n])) for n in TENSORS}
            self.tiled = self.ctx.malloc(int(lib.cdll.mx_tiled_expert_bytes(h, i)))
            ptrs = _lib.MxExpertPtrs(*[raw[n].ptr for n in TENSORS])
            lib.tile_expert(self.ctx._h(), C.byref(ptrs), h, i, C.c_void_p(self.tiled), None)
            self.ctx.sync()
            for d in raw.values():
                d.free()
            t = 16
            self.work = {"x": self.ctx.empty((t, h), np.uint16), "route": self.ctx.empty((t,), np.float32),
                         "gu": self.ctx.empty((t, 2 * i), np.float32), "h": self.ctx.empty((t, i), np.float32),
                         "y": self.ctx.empty((t, h), np.uint16)}
            return self
        except BaseException:
            self.__exit__()
            raise

    def forward(self, x, routing_weight=None) -> dict:
        if self.ctx is None:
            raise RuntimeError("Use the expert as a context manager")
        bits = bf16_input(np.asarray(x) if np.asarray(x).dtype == np.uint16 else np.asarray(x, np.float32),
                          self.hidden)
        t = bits.shape[0]
        if not 1 <= t <= 16:
            raise ValueError("One expert call accepts 1 to 16 tokens")
        w = self.work
        route = None
        if routing_weight is not None:
            route = np.broadcast_to(np.asarray(routing_weight, np.float32).reshape(-1), (t,)).copy()
            if not np.isfinite(route).all():
                raise ValueError("Routing weight must be finite")
            self.ctx.copy_h2d(w["route"].ptr, route)
        self.ctx.copy_h2d(w["x"].ptr, bits)
        self.ctx.lib.expert_forward_bf16(self.ctx._h(), C.c_void_p(self.tiled), self.hidden, self.intermediate,
                                         C.c_void_p(w["x"].ptr), t,
                                         None if route is None else C.c_void_p(w["route"].ptr),
                                         C.c_void_p(w["h"].ptr), C.c_void_p(w["gu"].ptr), C.c_void_p(w["y"].ptr),
                                         None)
        self.ctx.sync()
        h, i = self.hidden, self.intermediate
        return {"gu": self.ctx.download(w["gu"].ptr, (t, 2 * i), np.float32),
                "h": self.ctx.download(w["h"].ptr, (t, i), np.float32),
                "y": self.ctx.download(w["y"].ptr, (t, h), np.uint16)}

    def __exit__(self, *_):
        if self.ctx is not None:
            ctx, self.ctx = self.ctx, None
            ctx.close()
