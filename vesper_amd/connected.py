"""A routed MoE layer call with every stage returned (mirrors ConnectedMoE, src/vesper/connected.py:56-213).

ConnectedMoE(layer).forward(activation, image_span) -> {input_bf16, logits, routing,
experts{id -> stage dict}, shared, aggregation{after_expert_<id>_fp32 ...,
before_shared_fp32, after_shared_fp32, output_bf16}, output_bf16}.

The arithmetic is one mx_moe_decode call with diagnostics on (router, top-k
plan, fused expert kernels, fused ordered combine). The aggregation snapshots
are then replayed from the kernels' own BF16 expert outputs with the
MoEAccumulator kernels (zero, per-expert row adds in ascending ID, shared
last), exactly the reference's stepwise order; its final BF16 output must
equal the fused combine's, which the call checks. Nested calls are refused,
as in the reference (connected.py:131-133).
"""

from __future__ import annotations

import threading
import time

import numpy as np

from . import _lib
from .layer import MoELayer, bf16_input


class ConnectedMoE:
    def __init__(self, layer: MoELayer):
        self.layer = layer
        self.config = layer.config
        self.lock = threading.RLock()
        self.active = False
        self.stats = {"calls_started": 0, "calls_completed": 0, "calls_failed": 0}
        self.last_attempt = None

    def __enter__(self):
        return self

    def __exit__(self, *_):
        with self.lock:
            if self.active:
                raise RuntimeError("Cannot close connected MoE during a live call")

    def forward(self, activation, image_span=False) -> dict:
        if type(image_span) is not bool:
            raise ValueError("Connected image-span flag must be boolean")
        cfg = self.config
        bits = bf16_input(activation, cfg.hidden)
        t = bits.shape[0]
        if not 1 <= t <= cfg.max_tokens:
            raise ValueError(f"Connected MoE accepts 1 to {cfg.max_tokens} tokens per call")
        with self.lock:
            if self.active:
                raise RuntimeError("Nested MoE calls would overwrite live workspaces")
            self.active = True
            self.stats["calls_started"] += 1
            attempt = {"status": "running", "stage": "decode", "tokens": t}
            self.last_attempt = attempt
            started = time.perf_counter()
            try:
                result = self._forward(bits, t)
                attempt.update(status="pass", stage="complete",
                               indices=result["routing"]["indices"].tolist())
                self.stats["calls_completed"] += 1
                return result
            except BaseException as error:
                self.stats["calls_failed"] += 1
                attempt.update(status="failed", error_type=type(error).__name__)
                raise
            finally:
                attempt["wall_ms"] = (time.perf_counter() - started) * 1000
                self.active = False

    def _forward(self, bits, t):
        cfg, layer, ctx = self.config, self.layer, self.layer.ctx
        e, k, h, i = cfg.experts, cfg.top_k, cfg.hidden, cfg.intermediate
        xd, yd = ctx.upload(bits), ctx.empty((t, h), np.uint16)
        try:
            layer.decode_device(xd.ptr, t, yd.ptr, diagnostics=True)
            ctx.sync()
            output = yd.download()
        finally:
            xd.free()
            yd.free()
        routing = {"logits": layer.read("logits", (t, e), np.float32),
                   "scores": layer.read("scores", (t, e), np.float32),
                   "selection": layer.read("selection", (t, e), np.float32),
                   "raw": layer.read("raw", (t, k), np.float32),
                   "denominator": layer.read("denominator", (t,), np.float32),
                   "weights": layer.read("weights", (t, k), np.float32),
                   "indices": layer.read("indices", (t, k), np.int32),
                   "tied": layer.read("tied", (t,), np.int32)}
        plan = layer.plan()
        rows = plan["total_rows"]
        xq = layer.read("xq", (t, h), np.uint8)
        xs = layer.read("xs", (t, h // 32), np.uint8)
        w1 = layer.read("w1", (rows, i), np.uint16)
        w3 = layer.read("w3", (rows, i), np.uint16)
        din = layer.read("down_input", (rows, i), np.uint16)
        trace = layer.read("trace", (rows, i, 5), np.float32)
        dq = layer.read("down_q", (rows, i), np.uint8)
        ds = layer.read("down_s", (rows, i // 32), np.uint8)
        eout = layer.read("expert_out", (rows, h), np.uint16)

        def stages(slot):
            r0, n = int(plan["slot_row0"][slot]), int(plan["slot_ntok"][slot])
            toks = plan["slot_tok"][slot, :n]
            sl = slice(r0, r0 + n)
            return {"tokens": toks.copy(), "q": xq[toks], "s": xs[toks], "w1": w1[sl], "w3": w3[sl],
                    "down_input": (din[sl].astype(np.uint32) << 16).view(np.float32), "trace": trace[sl],
                    "down_q": dq[sl], "down_s": ds[sl], "w2": eout[sl]}

        experts = {int(plan["slot_expert"][s]): stages(s) for s in range(plan["n_routed"])}
        shared = stages(plan["n_routed"]) if cfg.shared else None
        aggregation = self._aggregate(plan, t)
        if not np.array_equal(aggregation["output_bf16"], output):
            raise RuntimeError("Fused combine differs from the stepwise ordered accumulation")
        return {"input_bf16": bits, "logits": routing["logits"], "routing": routing, "experts": experts,
                "shared": shared, "aggregation": aggregation, "output_bf16": output}

    def _aggregate(self, plan, t):
        """Stepwise ordered accumulation over the kernels' BF16 expert rows (moe.py:96-135)."""
        ctx, layer, h = self.layer.ctx, self.layer, self.config.hidden
        lib, hc = ctx.lib, ctx._h()
        eout_ptr, _ = layer.buffer("expert_out")
        total = ctx.empty((t, h), np.float32)
        rows_dev = ctx.empty((16,), np.int32)
        out = ctx.empty((t, h), np.uint16)
        stages = {}
        try:
            lib.acc_zero(hc, _lib.vp(total), t * h, None)
            for s in range(plan["n_routed"]):
                r0, n = int(plan["slot_row0"][s]), int(plan["slot_ntok"][s])
                ctx.copy_h2d(rows_dev.ptr, plan["slot_tok"][s, :n].astype(np.int32))
                lib.acc_add_rows(hc, _lib.vp(total), _lib.vp(eout_ptr + r0 * h * 2), _lib.vp(rows_dev), n, h, None)
                stages[f"after_expert_{int(plan['slot_expert'][s])}_fp32"] = total.download()
            stages["before_shared_fp32"] = total.download()
            if self.config.shared:
                r0 = int(plan["slot_row0"][plan["n_routed"]])
                lib.acc_add(hc, _lib.vp(total), _lib.vp(eout_ptr + r0 * h * 2), t * h, None)
            stages["after_shared_fp32"] = total.download()
            lib.acc_finish(hc, _lib.vp(total), _lib.vp(out), t * h, None)
            stages["output_bf16"] = out.download()
            return stages
        finally:
            total.free()
            rows_dev.free()
            out.free()
