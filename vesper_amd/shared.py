"""Always-active shared expert (mirrors ResidentSharedExpert, src/vesper/shared.py:141-170).

Two storage formats, detected from the arrays:
* FP8 block 32 (the reference's shared expert, shared.py:20-24): w1/w3 [I, H], w2 [H, I] E4M3 with E8M0
  scales per 32 x 32 block. The weights are tiled once on enter (mx_fp8_tile) and each call runs
  mx_fp8_expert_forward: the MXFP4 expert's stage sequence with the FP8 block-32 product
  (gemv_fp8_shared, shared_probe.cu:4-49).
* MXFP4 (how the decode layer stores it, next to the routed experts): the ResidentExpert path.

forward(x) is never routing-weighted; the stage dict is the reference's (q, s, w1, w3, down_input, trace,
down_q, down_s, w2).
"""

from __future__ import annotations

import ctypes as C

import numpy as np

from . import _lib
from .expert import ExpertExecutor, validate_expert_arrays

FP8_TENSORS = ("w1_weight", "w1_scale", "w3_weight", "w3_scale", "w2_weight", "w2_scale")


def shared_fp8_layout(hidden: int, intermediate: int) -> dict:
    """Tensor shapes of the FP8 block-32 shared expert (shared.py:20-24)."""
    shapes = {"w1": (intermediate, hidden), "w3": (intermediate, hidden), "w2": (hidden, intermediate)}
    return {f"{p}_{suffix}": (rows, width) if suffix == "weight" else (rows // 32, width // 32)
            for p, (rows, width) in shapes.items() for suffix in ("weight", "scale")}


def validate_shared_arrays(arrays, hidden: int, intermediate: int):
    layout = shared_fp8_layout(hidden, intermediate)
    if set(arrays) != set(layout):
        raise ValueError("A shared expert requires exactly six native tensors")
    for name, shape in layout.items():
        a = arrays[name]
        if getattr(a, "dtype", None) != np.uint8 or tuple(a.shape) != shape:
            raise ValueError("Shared tensor differs from the pinned FP8/block-32 layout")


class ResidentSharedExpert(ExpertExecutor):
    """forward(x) = expert(x) with no routing weight (shared.py:169-170)."""

    def __init__(self, arrays: dict, ordinal=0, swiglu_limit=10.0, *, hidden=5120, intermediate=2304):
        w1 = arrays.get("w1_weight")
        self.fmt = "fp8" if getattr(w1, "shape", None) == (intermediate, hidden) else "mxfp4"
        if self.fmt == "fp8":
            validate_shared_arrays(arrays, hidden, intermediate)
        else:
            validate_expert_arrays(arrays, hidden, intermediate)
        super().__init__(ordinal, swiglu_limit, hidden=hidden, intermediate=intermediate)
        self.arrays = arrays
        self.weights = {}

    def __enter__(self):
        super().__enter__()
        try:
            self.device_arrays = {n: self.ctx.upload(np.ascontiguousarray(a)) for n, a in self.arrays.items()}
            self.weights = {n: a.ptr for n, a in self.device_arrays.items()}
            if self.fmt == "fp8":
                lib = self.ctx.lib
                self.tiled = {}
                for p in ("w1", "w3", "w2"):
                    rows, width = self.arrays[f"{p}_weight"].shape
                    blob = self.ctx.malloc(int(lib.cdll.mx_fp8_tiled_bytes(rows, width, 32)))
                    self.tiled[p] = blob
                    lib.fp8_tile(self.ctx._h(), C.c_void_p(self.weights[f"{p}_weight"]),
                                 C.c_void_p(self.weights[f"{p}_scale"]), rows, width, 32, C.c_void_p(blob), None)
                self.ctx.sync()
                # the FP8 product reads only the tiled copies: the uploaded checkpoint layout is released
                for array in self.device_arrays.values():
                    array.free()
                self.device_arrays = {}
                self.weights = dict.fromkeys(self.arrays)
            return self
        except BaseException:
            self.close()
            raise

    def _compute(self, weights, t, route_ptr, stages):
        if self.fmt != "fp8":
            return super()._compute(weights, t, route_ptr, stages)
        w = self.work
        self.ctx.lib.fp8_expert_forward(self.ctx._h(), *[C.c_void_p(self.tiled[p]) for p in ("w1", "w3", "w2")],
                                        self.hidden, self.intermediate, C.c_void_p(w["x"].ptr), t, self.limit,
                                        route_ptr, C.c_void_p(w["w2"].ptr), C.byref(stages), None)

    def forward(self, x, routing_weight=None) -> dict:
        if routing_weight is not None:
            raise ValueError("The shared expert is never routing-weighted")
        return self.execute(x, self.weights, None)
