"""FP8 E4M3 block-scaled attention projections (mirrors NativeProjections, src/vesper/projections.py:67-154).

NativeProjections(arrays, ordinal, *, layer, block) uploads each projection's E4M3 weight and scales once,
tiled for the gfx950 MFMA (mx_fp8_tile), and `fp8(name, values)` returns the reference's stage dict:
input_fp8, scale_e8m0 (block 32) or scale_f32 (block 128), output_fp32, output_bf16.

block 32 is the reference's own projection arithmetic (E8M0 scales per 32 x 32 weight block, per-32
activation quantization, `layers.{layer}.attn.{name}.{weight,scale}` arrays of FP8_LAYOUT shapes).
block 128 is BASELINE configuration 3 (FP32 scales per 128 x 128 block, per-token per-128 FP32
activation scales, CONFIG3_LAYOUT shapes). Inputs are validated before any device work. The
reference bounds a call to 8 rows; here any number of rows runs in one launch (16 tokens per MFMA
column group), and `project_device` is the pointer-level fast path.
"""

from __future__ import annotations

import ctypes as C
import math
import threading

import numpy as np

from . import _lib
from .resources import MiB, MemoryBudget

FP8_LAYOUT = {"wq_a": (1280, 5120), "wq_b": (32768, 1280), "wkv": (512, 5120), "wo_b": (5120, 8192)}
WO_A = (8192, 4096)          # the grouped output projection: 8 groups of 1024 rows over 4096 (projections.py:34)
WO_A_GROUPS = 8
GROUPED_MAX_TOKENS = 32      # grouped calls run on the decode GEMV
CONFIG3_LAYOUT = {"q_a": (1536, 7168), "q_b": (24576, 1536), "kv_a": (576, 7168), "o": (7168, 16384)}
MAX_ROWS = 1 << 16
HOST_ALLOWANCE = 512 * MiB   # host bytes an open runtime reserves for its calls' uploads and results


def validate_values(values, width):
    """Finite contiguous BF16 rows of the projection's width (projections.py:20-26, without the 8-row cap)."""
    if (not isinstance(values, np.ndarray) or values.dtype != np.uint16 or values.ndim not in (1, 2, 3)
            or values.shape[-1] != width or not values.flags.c_contiguous
            or not 1 <= math.prod(values.shape[:-1]) <= MAX_ROWS
            or np.any((values & 0x7F80) == 0x7F80)):
        raise ValueError("Expected bounded contiguous finite BF16 projection input")
    return math.prod(values.shape[:-1])


def scale_shape(rows, width, block):
    return (rows // 32, width // 32) if block == 32 else ((rows + 127) // 128, width // 128)


def validate_projection_weights(arrays, layer, layout, block):
    for name, (rows, width) in layout.items():
        for suffix, dtype, shape in (("weight", np.uint8, (rows, width)),
                                     ("scale", np.uint8 if block == 32 else np.float32, scale_shape(rows, width, block))):
            a = arrays.get(f"layers.{layer}.attn.{name}.{suffix}")
            if (not isinstance(a, np.ndarray) or a.dtype != dtype or a.shape != shape or not a.flags.c_contiguous):
                raise ValueError("Expected block-scaled FP8 Attention weights/scales")
            bad = np.any((a & 127) == 127) if suffix == "weight" else (
                np.any(a == 255) if block == 32 else not (np.isfinite(a).all() and np.all(a > 0)))
            if bad:
                raise ValueError("FP8 Attention weights/scales must be finite")


class NativeProjections:
    """Resident tiled FP8 matrices, serialized calls."""

    def __init__(self, arrays, ordinal=0, *, layer=0, block=32, layout=None):
        if block not in (32, 128):
            raise ValueError("block must be 32 or 128")
        self.layout = dict(layout or (FP8_LAYOUT if block == 32 else CONFIG3_LAYOUT))
        for rows, width in self.layout.values():
            if rows % 64 or width % 128:
                raise ValueError("projection rows must be a multiple of 64 and width of 128")
        validate_projection_weights(arrays, layer, self.layout, block)
        # wo_a (block 32 only) is optional: present, it enables grouped()
        self.has_wo_a = block == 32 and f"layers.{layer}.attn.wo_a.weight" in arrays
        if self.has_wo_a:
            validate_projection_weights(arrays, layer, {"wo_a": WO_A}, 32)
        self.arrays, self.ordinal, self.layer, self.block = arrays, ordinal, layer, block
        self.lock, self.opened, self.ctx = threading.Lock(), False, None
        self.tiled = {}
        self.budget = MemoryBudget(cap=HOST_ALLOWANCE, owner="projections")
        self._device_peak = 0   # the context's peak owned bytes, kept past close for stats()

    def __enter__(self):
        with self.lock:
            if self.opened:
                raise RuntimeError("Projection runtime is already open")
            self.budget.acquire(HOST_ALLOWANCE)
            try:
                self.ctx = _lib.Context(self.ordinal, 0)
            except BaseException:
                self.budget.release(HOST_ALLOWANCE)
                raise
            try:
                lib = self.ctx.lib
                tiled_layout = dict(self.layout, **({"wo_a": WO_A} if self.has_wo_a else {}))
                for name, (rows, width) in tiled_layout.items():
                    w = self.ctx.upload(self.arrays[f"layers.{self.layer}.attn.{name}.weight"])
                    s = self.ctx.upload(self.arrays[f"layers.{self.layer}.attn.{name}.scale"])
                    nbytes = int(lib.cdll.mx_fp8_tiled_bytes(rows, width, self.block))
                    blob = self.ctx.malloc(nbytes)
                    self.tiled[name] = blob
                    lib.fp8_tile(self.ctx._h(), _lib.vp(w), _lib.vp(s), rows, width, self.block, C.c_void_p(blob), None)
                    self.ctx.sync()
                    w.free()
                    s.free()
                self.resident_bytes = sum(int(lib.cdll.mx_fp8_tiled_bytes(r, c, self.block))
                                          for r, c in tiled_layout.values())
                self.opened = True
                return self
            except BaseException:
                self._close_context()
                raise

    def _close_context(self):
        self._device_peak = max(self._device_peak, self.ctx.owned_bytes()[1])
        self.ctx.close()
        self.ctx = None
        self.budget.release(HOST_ALLOWANCE)

    def _ready(self):
        if not self.opened:
            raise RuntimeError("Projection runtime is not open")
        self.budget.acquire(0)   # MemoryError once the machine is below its memory reserve

    def stats(self) -> dict:
        """The runtime's host reservation and device footprint (projections.py:189-195): the host allowance
        (its peak reservation) and what is reserved now, the device context's peak and live owned bytes, and
        whether the context is open. The reservation is a ledger, not a limit on the process's resident set,
        and module (code object) memory is not in the device figures."""
        live, peak = self.ctx.owned_bytes() if self.ctx is not None else (0, 0)
        return {"host_allowance_bytes": self.budget.peak, "host_reserved_bytes": self.budget.reserved,
                "device_peak_owned_bytes": max(peak, self._device_peak), "device_owned_bytes": live,
                "owned_context_active": self.ctx is not None, "reservation_is_RSS_limit": False,
                "driver_module_memory_excluded": True}

    def project_device(self, name, x_ptr, tokens, y_ptr, stream=None, trace_ptr=None, q_ptr=None, s_ptr=None):
        """y[T][rows] BF16 = projection of device BF16 x[T][width]; no host synchronisation."""
        self._ready()
        rows, width = self.layout[name]
        self.ctx.lib.fp8_projection(self.ctx._h(), C.c_void_p(self.tiled[name]), rows, width, self.block,
                                    C.c_void_p(int(x_ptr)), int(tokens), C.c_void_p(int(y_ptr)),
                                    _lib.vp(trace_ptr), _lib.vp(q_ptr), _lib.vp(s_ptr), _lib._stream(stream))

    def fp8(self, name, values):
        with self.lock:
            self._ready()
            if name not in self.layout:
                raise ValueError("Unknown FP8 Attention projection")
            rows, width = self.layout[name]
            tokens = validate_values(values, width)
            lead = values.shape[:-1]
            sdt, sw = (np.uint8, width // 32) if self.block == 32 else (np.float32, width // 128)
            x = self.ctx.upload(np.ascontiguousarray(values).reshape(tokens, width))
            q = self.ctx.empty((tokens, width), np.uint8)
            s = self.ctx.empty((tokens, sw), sdt)
            trace = self.ctx.empty((tokens, rows), np.float32)
            out = self.ctx.empty((tokens, rows), np.uint16)
            try:
                self.project_device(name, x.ptr, tokens, out.ptr, trace_ptr=trace, q_ptr=q, s_ptr=s)
                scale_key = "scale_e8m0" if self.block == 32 else "scale_f32"
                return {"input_fp8": q.download().reshape(*lead, width),
                        scale_key: s.download().reshape(*lead, sw),
                        "output_fp32": trace.download().reshape(*lead, rows),
                        "output_bf16": out.download().reshape(*lead, rows)}
            finally:
                for d in (x, q, s, trace, out):
                    d.free()

    def grouped(self, values):
        """The grouped output projection (projections.py:156-171): values [..., 8, 4096] BF16 ->
        rounded_bf16, input_fp8, scale_e8m0 [..., 8, 128] and output_bf16 [..., 8, 1024]. kv_round32's
        codes and scales feed the scaled MFMA directly (the E4M3 weights are never widened to BF16)."""
        with self.lock:
            self._ready()
            if not self.has_wo_a:
                raise ValueError("grouped() needs the block-32 wo_a weights")
            if (not isinstance(values, np.ndarray) or values.ndim not in (3, 4) or values.shape[-2:] != (8, 4096)
                    or not values.flags.c_contiguous):
                raise ValueError("Expected original eight-group BF16 output-projection input")
            tokens = validate_values(values.reshape(*values.shape[:-2], 32768), 32768)
            if tokens > GROUPED_MAX_TOKENS:
                raise ValueError(f"grouped() takes at most {GROUPED_MAX_TOKENS} tokens per call")
            rows, width = WO_A
            x = self.ctx.upload(values)
            rounded = self.ctx.empty(values.shape, np.uint16)
            q = self.ctx.empty(values.shape, np.uint8)
            s = self.ctx.empty((*values.shape[:-1], width // 32), np.uint8)
            out = self.ctx.empty((tokens, rows), np.uint16)
            lib, h = self.ctx.lib, self.ctx._h()
            try:
                lib.kv_round32(h, _lib.vp(x), values.size, _lib.vp(rounded), _lib.vp(q), _lib.vp(s), None)
                lib.fp8_grouped_projection(h, C.c_void_p(self.tiled["wo_a"]), WO_A_GROUPS, rows // WO_A_GROUPS, width,
                                           _lib.vp(q), _lib.vp(s), tokens, _lib.vp(out), None, None)
                return {"rounded_bf16": rounded.download(), "input_fp8": q.download(), "scale_e8m0": s.download(),
                        "output_bf16": out.download().reshape(*values.shape[:-2], WO_A_GROUPS, rows // WO_A_GROUPS)}
            finally:
                for d in (x, rounded, q, s, out):
                    d.free()

    def round_window(self, values):
        """Per-32 post-RoPE FP8 rounding of window KV rows [1 or 2, S, 512] (kv_round32, projections.py:
        173-188): rounded_bf16, codes_fp8 and scales_e8m0 [B, S, 16]."""
        with self.lock:
            self._ready()
            validate_values(values, 512)
            if values.ndim != 3 or values.shape[0] not in (1, 2):
                raise ValueError("Expected bounded window KV rows")
            x = self.ctx.upload(values)
            rounded = self.ctx.empty(values.shape, np.uint16)
            q = self.ctx.empty(values.shape, np.uint8)
            s = self.ctx.empty((*values.shape[:2], 16), np.uint8)
            try:
                self.ctx.lib.kv_round32(self.ctx._h(), _lib.vp(x), values.size, _lib.vp(rounded), _lib.vp(q),
                                        _lib.vp(s), None)
                return {"rounded_bf16": rounded.download(), "codes_fp8": q.download(), "scales_e8m0": s.download()}
            finally:
                for d in (x, rounded, q, s):
                    d.free()

    def __exit__(self, *_):
        with self.lock:
            self.opened = False
            if self.ctx is not None:
                self._close_context()
            self.tiled.clear()
