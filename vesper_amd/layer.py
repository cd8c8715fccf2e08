"""Resident expert bank and the batched MoE decode layer (the fast path).

ExpertBank keeps every expert of a layer in one HBM allocation in the
device-native tiled layout (mx_tile_expert): the expert kernels then read each
wave's operands as 1 KB of contiguous memory with one coalesced scale word per
chunk. Experts enter and leave the bank in the reference's per-expert layout
(w1_weight, w1_scale, w3_weight, w3_scale, w2_weight, w2_scale;
src/vesper/storage.py:33-41) through a one-expert staging area and the
bit-exact tile/untile conversion. MoELayer drives mx_moe_decode: router,
top-k + plan, fused expert GEMVs and ordered combine in five kernel launches on
one stream, with inputs resident in HBM.
"""

from __future__ import annotations

import ctypes as C

import numpy as np

from . import _lib
from .config import MoEConfig

TENSORS = ("w1_weight", "w1_scale", "w3_weight", "w3_scale", "w2_weight", "w2_scale")

# Plan struct layout (mx_moe.hip `Plan`): 8 header ints, then per-slot arrays.
_MAX_TOKENS, _MAX_TOPK = 16, 32
_MAX_SLOTS = _MAX_TOKENS * _MAX_TOPK + 1


def _plan_views(raw: np.ndarray) -> dict:
    words = raw.view(np.int32)
    o = 8
    out = {"n_slots": int(words[0]), "n_routed": int(words[1]), "total_rows": int(words[2]),
           "tokens": int(words[3]), "top_k": int(words[4])}
    for name in ("slot_expert", "slot_ntok", "slot_row0", "slot_weighted"):
        out[name] = words[o:o + _MAX_SLOTS]
        o += _MAX_SLOTS
    out["slot_tok"] = words[o:o + _MAX_SLOTS * _MAX_TOKENS].reshape(_MAX_SLOTS, _MAX_TOKENS)
    o += _MAX_SLOTS * _MAX_TOKENS
    out["slot_w"] = words[o:o + _MAX_SLOTS * _MAX_TOKENS].view(np.float32).reshape(_MAX_SLOTS, _MAX_TOKENS)
    o += _MAX_SLOTS * _MAX_TOKENS
    out["tok_rows"] = words[o:o + _MAX_TOKENS * (_MAX_TOPK + 1)].reshape(_MAX_TOKENS, _MAX_TOPK + 1)
    return out


class ExpertBank:
    """`count` experts of one layer resident in a single device allocation (tiled layout)."""

    def __init__(self, ctx: _lib.Context, config: MoEConfig, count: int):
        self.ctx, self.config, self.count = ctx, config, int(count)
        layout = config.expert_layout()
        self.offsets, offset = {}, 0
        for name in TENSORS:
            rows, cols = layout[name]
            self.offsets[name] = (offset, (rows, cols))
            offset += rows * cols
        self.expert_bytes = int(ctx.lib.cdll.mx_tiled_expert_bytes(config.hidden, config.intermediate))
        if self.expert_bytes != offset or offset % 256:
            raise ValueError("expert shapes must be multiples of 128 (tiled and reference sizes agree)")
        self.base = ctx.malloc(self.expert_bytes * self.count)
        self._staging = 0

    def tiled_ptr(self, expert: int) -> int:
        if not 0 <= expert < self.count:
            raise ValueError("expert index outside the bank")
        return self.base + expert * self.expert_bytes

    def _stage(self) -> int:
        if not self._staging:
            self._staging = self.ctx.malloc(self.expert_bytes)
        return self._staging

    def _staging_ptrs(self) -> _lib.MxExpertPtrs:
        base = self._stage()
        return _lib.MxExpertPtrs(*[base + self.offsets[n][0] for n in TENSORS])

    def upload(self, expert: int, arrays: dict, stream=None):
        """Reference-layout arrays -> staging -> tiled slot `expert`."""
        validate_expert_arrays(arrays, self.config)
        dst = self.tiled_ptr(expert)
        ptrs = self._staging_ptrs()
        for name in TENSORS:
            self.ctx.copy_h2d(getattr(ptrs, name), np.ascontiguousarray(arrays[name], np.uint8), stream)
        self.ctx.lib.tile_expert(self.ctx._h(), C.byref(ptrs), self.config.hidden, self.config.intermediate,
                                 C.c_void_p(dst), _lib._stream(stream))

    def download(self, expert: int) -> dict:
        """Tiled slot `expert` -> reference-layout arrays (bit-exact inverse of upload)."""
        src = self.tiled_ptr(expert)
        ptrs = self._staging_ptrs()
        self.ctx.lib.untile_expert(self.ctx._h(), C.c_void_p(src), self.config.hidden, self.config.intermediate,
                                   C.byref(ptrs), None)
        return {name: self.ctx.download(getattr(ptrs, name), shape, np.uint8)
                for name, (_, shape) in self.offsets.items()}

    def fill_synthetic(self, seed: int, scale_lo: int = 118, scale_hi: int = 126, stream=None):
        """BASELINE inputs generated in HBM: uniform packed bytes, E8M0 codes uniform in [lo, hi], drawn in
        the reference layout (one seed per expert tensor) and tiled into place."""
        ptrs = self._staging_ptrs()
        for e in range(self.count):
            for t, name in enumerate(TENSORS):
                _, (rows, cols) = self.offsets[name]
                lo, hi = (0, 255) if name.endswith("weight") else (scale_lo, scale_hi)
                self.ctx.fill_uniform_u8(getattr(ptrs, name), rows * cols, (seed * 1_000_003 + e * 8 + t), lo, hi,
                                         stream)
            self.ctx.lib.tile_expert(self.ctx._h(), C.byref(ptrs), self.config.hidden, self.config.intermediate,
                                     C.c_void_p(self.tiled_ptr(e)), _lib._stream(stream))

    def free(self):
        for attr in ("base", "_staging"):
            ptr = getattr(self, attr)
            if ptr:
                self.ctx.free(ptr)
                setattr(self, attr, 0)


def validate_expert_arrays(arrays: dict, config: MoEConfig):
    """Layout check before any device work (checkpoint.py:143-149, test_expert_boundaries.py)."""
    layout = config.expert_layout()
    if set(arrays) != set(layout):
        raise ValueError("A complete expert requires exactly six native tensors")
    for name, shape in layout.items():
        a = arrays[name]
        if not isinstance(a, np.ndarray) or a.dtype != np.uint8 or a.shape != shape:
            raise ValueError("Expert tensor layout differs from the pinned shape")


class MoELayer:
    """One routed MoE layer resident on the device; `decode` runs T <= 16 tokens."""

    def __init__(self, ctx: _lib.Context, config: MoEConfig, router_weight, bank: ExpertBank, bias=None):
        if bank.count != config.experts + (1 if config.shared else 0):
            raise ValueError("expert bank size must be experts (+1 for the shared expert)")
        self.ctx, self.config, self.bank = ctx, config, bank
        self.lib = ctx.lib
        self._owned = []
        self.router_weight = self._device_f32(router_weight, (config.experts, config.hidden))
        self.bias = None if bias is None else self._device_f32(bias, (config.experts,))
        cfg = _lib.MxMoeConfig(config.hidden, config.intermediate, config.experts, config.top_k,
                               _lib.MX_SCORE[config.score_func], config.route_scale, config.swiglu_limit,
                               _lib.MX_FMT_MXFP4 if config.shared else -1, config.max_tokens)
        table = (C.c_void_p * config.experts)(*[bank.tiled_ptr(e) for e in range(config.experts)])
        shared = C.c_void_p(bank.tiled_ptr(config.experts)) if config.shared else None
        handle = C.c_void_p()
        self.lib.layer_create(ctx._h(), C.byref(cfg), _lib.vp(self.router_weight), _lib.vp(self.bias),
                              table, shared, C.byref(handle))
        self.handle = handle

    def _device_f32(self, value, shape):
        if isinstance(value, _lib.DeviceArray):
            if value.dtype != np.float32 or value.shape != shape:
                raise ValueError(f"expected an FP32 device array of shape {shape}")
            return value
        array = np.ascontiguousarray(value, dtype=np.float32)
        if array.shape != shape or not np.isfinite(array).all():
            raise ValueError(f"expected finite FP32 values of shape {shape}")
        dev = self.ctx.upload(array)
        self._owned.append(dev)
        return dev

    def close(self):
        if self.handle:
            handle, self.handle = self.handle, C.c_void_p()
            self.lib.layer_destroy(handle)
        for dev in self._owned:
            dev.free()
        self._owned.clear()

    def __enter__(self):
        return self

    def __exit__(self, *_):
        self.close()

    # -- fast path --------------------------------------------------------------------------
    def decode_device(self, x_ptr: int, tokens: int, y_ptr: int, stream=None, diagnostics: bool = False):
        """y = MoE(x) with x, y device BF16 [tokens, hidden]; no host synchronisation."""
        self.lib.moe_decode(self.handle, C.c_void_p(int(x_ptr)), int(tokens), C.c_void_p(int(y_ptr)),
                            int(bool(diagnostics)), _lib._stream(stream))

    def decode(self, x, diagnostics: bool = False) -> np.ndarray:
        """Host convenience: BF16 bits or FP32 [T, H] in, BF16 bits [T, H] out."""
        bits = bf16_input(x, self.config.hidden)
        t = bits.shape[0]
        xd = self.ctx.upload(bits)
        yd = self.ctx.empty((t, self.config.hidden), np.uint16)
        try:
            self.decode_device(xd.ptr, t, yd.ptr, diagnostics=diagnostics)
            return yd.download()
        finally:
            xd.free()
            yd.free()

    # -- prefill ----------------------------------------------------------------------------
    def workspace_bytes(self, tokens: int) -> int:
        return int(self.lib.cdll.mx_prefill_workspace_bytes(self.handle, int(tokens)))

    def prefill_device(self, x_ptr: int, tokens: int, y_ptr: int, workspace: int, workspace_bytes: int,
                       ids_ptr=None, weights_ptr=None, stream=None):
        """y = MoE(x) for `tokens` rows as grouped GEMMs (mx_moe_prefill); routing given by device ids/weights
        [T, k] or, when both are None, by the layer's router. No host synchronisation."""
        self.lib.moe_prefill(self.handle, C.c_void_p(int(x_ptr)), int(tokens), _lib.vp(ids_ptr), _lib.vp(weights_ptr),
                             C.c_void_p(int(y_ptr)), C.c_void_p(int(workspace)), int(workspace_bytes),
                             _lib._stream(stream))

    def prefill(self, x, ids=None, weights=None, stages: bool = False):
        """Host convenience: BF16 bits or FP32 [T, H] in (and optional int32 ids / FP32 weights [T, k]),
        BF16 bits [T, H] out. With stages=True also the call's intermediate stages (mx_prefill_stage_offsets):
        (y, {"down_q" [rows, I], "down_s" [rows, I/32], "pair_row" [T, k], "row0" [E + 1],
        "expert_out" [T, k + 1, H] (token t's experts in ascending ID, the shared expert last)})."""
        bits = bf16_input(x, self.config.hidden)
        t = bits.shape[0]
        k = self.config.top_k
        if (ids is None) != (weights is None):
            raise ValueError("routing ids and weights are given together or not at all")
        if ids is not None:
            ids = np.ascontiguousarray(ids, dtype=np.int32)
            weights = np.ascontiguousarray(weights, dtype=np.float32)
            if ids.shape != (t, k) or weights.shape != (t, k):
                raise ValueError(f"routing must be [{t}, {k}]")
            if ids.min() < 0 or ids.max() >= self.config.experts or np.any(np.diff(np.sort(ids, 1), axis=1) == 0):
                raise ValueError("routing ids must be distinct experts of the layer")
            if not np.isfinite(weights).all():
                raise ValueError("route weights must be finite")
        nbytes = self.workspace_bytes(t)
        xd = self.ctx.upload(bits)
        yd = self.ctx.empty((t, self.config.hidden), np.uint16)
        ws = self.ctx.malloc(nbytes)
        dev = [self.ctx.upload(ids), self.ctx.upload(weights)] if ids is not None else [None, None]
        try:
            self.prefill_device(xd.ptr, t, yd.ptr, ws, nbytes, dev[0], dev[1])
            y = yd.download()
            if not stages:
                return y
            cfg = self.config
            at = (C.c_uint64 * 5)()
            self.lib.prefill_stage_offsets(self.handle, t, at)
            rows = t * cfg.top_k + (t if cfg.shared else 0)
            i = cfg.intermediate
            return y, {"down_q": self.ctx.download(ws + at[0], (rows, i), np.uint8),
                       "down_s": self.ctx.download(ws + at[1], (rows, i // 32), np.uint8),
                       "pair_row": self.ctx.download(ws + at[2], (t, cfg.top_k), np.int32),
                       "row0": self.ctx.download(ws + at[3], (cfg.experts + 1,), np.int32),
                       "expert_out": self.ctx.download(ws + at[4], (t, cfg.top_k + 1, cfg.hidden), np.uint16)}
        finally:
            for d in [xd, yd] + [d for d in dev if d is not None]:
                d.free()
            self.ctx.free(ws)

    def route_errors(self, clear: bool = True, stream=None) -> int:
        """Routing ids that routed decode / prefill replaced since the last clear (synchronises `stream`)."""
        count = C.c_uint32()
        self.lib.layer_route_errors(self.handle, C.byref(count), int(bool(clear)), _lib._stream(stream))
        return int(count.value)

    # -- diagnostics ------------------------------------------------------------------------
    def buffer(self, name: str):
        p, n = C.c_void_p(), C.c_uint64()
        self.lib.layer_buffer(self.handle, _lib.BUFFERS[name], C.byref(p), C.byref(n))
        return int(p.value), int(n.value)

    def read(self, name: str, shape, dtype) -> np.ndarray:
        p, n = self.buffer(name)
        want = int(np.prod(shape)) * np.dtype(dtype).itemsize
        if want > n:
            raise ValueError(f"buffer {name} holds {n} bytes, {want} requested")
        return self.ctx.download(p, shape, dtype)

    def plan(self) -> dict:
        p, n = self.buffer("plan")
        return _plan_views(self.ctx.download(p, (n,), np.uint8))

    STAGES = {"router": 0, "route_plan": 1, "gateup": 2, "down": 3, "combine": 4}

    def time_stage(self, stage: str, iters: int = 20, stream=None) -> float:
        """Average us per launch of one stage of the most recent decode call, re-launched `iters` times
        back to back with HIP events around the loop (mx_layer_time_stage)."""
        us = C.c_float()
        self.lib.layer_time_stage(self.handle, self.STAGES[stage], int(iters), C.byref(us), _lib._stream(stream))
        return float(us.value)

    def profile(self, enable: bool):
        ms = (C.c_float * 4)()
        calls = C.c_int32()
        self.lib.layer_profile(self.handle, int(bool(enable)), ms, C.byref(calls))
        return {"router": ms[0], "gateup": ms[1], "down": ms[2], "combine": ms[3], "calls": calls.value}


def bf16_input(x, hidden: int) -> np.ndarray:
    """[T, H] BF16 storage bits from BF16 bits or FP32 values (connected.py:45-53, batched)."""
    x = np.asarray(x)
    if x.ndim == 1:
        x = x.reshape(1, -1)
    if x.ndim != 2 or x.shape[1] != hidden or x.dtype not in (np.dtype(np.uint16), np.dtype(np.float32)):
        raise ValueError(f"MoE input must be BF16 storage bits or FP32 values of shape (T, {hidden})")
    if x.dtype == np.uint16:
        bits = np.ascontiguousarray(x)
    else:
        b = np.ascontiguousarray(x, dtype=np.float32).view(np.uint32).astype(np.uint64)
        nan = ((b & 0x7F800000) == 0x7F800000) & ((b & 0x7FFFFF) != 0)
        bits = np.where(nan, (b >> 16) | 0x40, (b + 0x7FFF + ((b >> 16) & 1)) >> 16).astype(np.uint16)
    if np.any((bits & 0x7F80) == 0x7F80):
        raise ValueError("MoE activation leaves the finite BF16 scope")
    return bits
