"""One MoE layer call with every stage returned (the reference's ConnectedMoE, src/vesper/connected.py:24-213).

Two forms:

* ConnectedMoE(store, gate_fixture, router_fixture, shared_fixture, config, *, layer, profile, source_factory):
  the reference's constructor and call. The layer's resident weights come from the three fixture pairs
  (vesper_amd.fixtures), its routed experts from the on-disk store through the exclusive tiers
  (TieredExpertRuntime). forward(activation, image_span) runs the gate projection (the router kernel's FP32
  dot products), the routing postprocess with the text or image-span bias, the participation plan, each
  selected expert in ascending ID from whichever tier holds it, the FP8 shared expert, and the ordered FP32
  accumulation with one BF16 rounding -- each stage a HIP kernel call -- and returns the reference's dict
  {input_bf16, logits, routing, experts, expert_events, shared, aggregation, output_bf16}. Selected experts
  missing from the store are refused before any expert I/O; a failed call returns nothing and the next one
  starts from a zeroed accumulator; nested calls are refused. Activations are one token [hidden] as in the
  reference, or up to 16 tokens [T, hidden].
* ConnectedLayer(layer): the same dict for a resident MoELayer, from one mx_moe_decode call with
  diagnostics on. The aggregation snapshots are replayed from the kernels' own BF16 expert rows with the
  accumulator kernels (zero, per-expert row adds in ascending ID, shared last); the replay's BF16 output
  must equal the fused combine's, which the call checks.

The helper-GPU tier of the reference's default configuration needs a second device; ConnectedConfig's
default cache here has none (one GPU), and is otherwise the reference's (two primary slots, a two-expert RAM
tier, GPU SHA-256 audits, 48-expert stores).
"""

from __future__ import annotations

import hashlib
import threading
import time
from contextlib import ExitStack
from dataclasses import asdict, dataclass, field
from pathlib import Path

import numpy as np

from . import _lib
from .fixtures import load_gate_fixture, load_router_fixture, load_shared_fixture
from .layer import MoELayer, bf16_input
from .moe import MoEAccumulator, participation
from .resources import GiB, MiB, MemoryBudget, physical_memory
from .router import GateProjection, RouterProbe
from .shared import ResidentSharedExpert
from .store import REFERENCE_PROFILE, ModelProfile, expert_key
from .tiered import CacheConfig, TieredExpertRuntime

REGISTERED_LAYERS = (0, 2, 3, 20, 21, 22, 23, 24, 25)
LAYER_PROFILES = ("qualified", "token_prefix", "backbone_probe")
MAX_CALL_TOKENS = 16


def validate_layer(layer, model: ModelProfile, profile: str = "qualified") -> int:
    """The layers a connected call may use (src/vesper/prefix_profile.py:4-9): for the reference's pinned
    model the registered layers (plus layer 1 for "token_prefix", any layer for "backbone_probe"); for any
    other model every layer of it."""
    if type(layer) is not int or profile not in LAYER_PROFILES:
        raise ValueError("Unregistered original layer/profile")
    if model != REFERENCE_PROFILE or profile == "backbone_probe":
        allowed = 0 <= layer < model.layers
    else:
        allowed = layer in REGISTERED_LAYERS or (profile == "token_prefix" and layer == 1)
    if not allowed:
        raise ValueError("Unregistered original layer/profile")
    return layer


def _cache_config() -> CacheConfig:
    return CacheConfig(host_cap_bytes=128 * MiB, ram_cache_bytes=2 * REFERENCE_PROFILE.expert_bytes, primary_slots=2,
                       helper_device=None, helper_slots=0, integrity_mode="gpu-sha256", max_store_experts=48)


@dataclass(frozen=True)
class ConnectedConfig:
    """The call's caps (src/vesper/connected.py:30-43): the cache's own configuration, the host bytes the
    whole call may reserve (the cache's cap plus 132 MiB for fixtures, upload staging and the accumulator),
    the explicit device bytes of every component together, and the device's free-memory floor."""
    cache: CacheConfig = field(default_factory=_cache_config)
    host_cap_bytes: int = 320 * MiB
    primary_explicit_cap_bytes: int = 128 * MiB
    device_free_floor: int = GiB

    def __post_init__(self):
        if self.host_cap_bytes < self.cache.host_cap_bytes + 132 * MiB:
            raise ValueError("Connected host cap must cover all component reservation allowances")
        if self.primary_explicit_cap_bytes <= 0 or self.device_free_floor < 0:
            raise ValueError("Invalid connected GPU allocation cap")


class DeviceLedger:
    """A component's device context in the shape of the reference's Device ledger (src/vesper/cuda.py:93-191)
    as a transformer block reads it around a MoE call (src/vesper/block.py:43-92): `allocations` (the
    context's live explicit bytes, as one entry), `peak`, `memory()`, `free_floor` and `allocate` / `free`."""

    def __init__(self, ctx: _lib.Context, free_floor: int):
        self.ctx, self.free_floor, self.ordinal = ctx, free_floor, ctx.ordinal

    @property
    def allocations(self) -> dict:
        return {"explicit": self.ctx.owned_bytes()[0]}

    @property
    def peak(self) -> int:
        return self.ctx.owned_bytes()[1]

    def memory(self) -> dict:
        return self.ctx.memory()

    def allocate(self, size: int) -> int:
        return self.ctx.malloc(size)

    def free(self, pointer: int):
        self.ctx.free(pointer)


def bf16_activation(activation, hidden: int):
    """(FP32 values, BF16 bits) of an activation given as BF16 bits or FP32 values, refused unless every value
    is a finite BF16 (src/vesper/connected.py:46-53)."""
    x = np.asarray(activation)
    if x.ndim not in (1, 2) or x.shape[-1] != hidden or x.dtype not in (np.dtype(np.uint16), np.dtype(np.float32)):
        raise ValueError(f"Connected MoE accepts {hidden:,} BF16 storage bits or FP32 activation values per token")
    bits = bf16_input(x, hidden).reshape(x.shape)
    values = (bits.astype(np.uint32) << 16).view(np.float32)
    if not np.isfinite(values).all():
        raise ValueError("Connected activation leaves the finite BF16 scope")
    return np.ascontiguousarray(values), bits


class ConnectedMoE:
    """Serial calls of one registered layer over the store (src/vesper/connected.py:56-213)."""

    def __init__(self, store: Path, gate_fixture: Path, router_fixture: Path, shared_fixture: Path,
                 config: ConnectedConfig | None = None, *, cublas_library=None, layer=0, profile="qualified",
                 source_factory=None, model: ModelProfile = REFERENCE_PROFILE):
        if cublas_library is not None:
            raise ValueError("The gate projection runs as a HIP kernel; no BLAS library is loaded")
        self.layer = validate_layer(layer, model, profile)
        self.model = model
        self.store_path, self.gate_fixture = Path(store), Path(gate_fixture)
        self.router_fixture, self.shared_fixture = Path(router_fixture), Path(shared_fixture)
        self.config = config or ConnectedConfig()
        if source_factory is not None and not callable(source_factory):
            raise ValueError("Expected an explicit expert source factory")
        self.source_factory = source_factory
        self.stack, self.active = None, False
        self.lock = threading.RLock()
        self.stats = {"calls_started": 0, "calls_completed": 0, "calls_failed": 0}
        self.last_attempt = None

    def __enter__(self):
        if self.stack is not None:
            raise RuntimeError("Connected MoE is already open")
        self.stack = ExitStack()
        c, m = self.config, self.model
        self.budget = MemoryBudget(c.host_cap_bytes, c.cache.available_floor, owner="connected")
        try:
            allowance = c.cache.host_cap_bytes + 100 * MiB       # the cache's cap + fixtures and staging
            self.budget.acquire(allowance)
            self.stack.callback(self.budget.release, allowance)
            weight, self.gate_manifest = load_gate_fixture(self.gate_fixture, m)
            biases, self.router_manifest = load_router_fixture(self.router_fixture, m)
            shared, self.shared_manifest = load_shared_fixture(self.shared_fixture, m)
            if any(man["layer"] != self.layer for man in (self.gate_manifest, self.router_manifest,
                                                           self.shared_manifest)):
                raise ValueError("Connected gate, router and shared artifacts must match the selected layer")
            ordinal = c.cache.primary_device
            self.gate = self.stack.enter_context(GateProjection(weight, ordinal))
            self.router = self.stack.enter_context(RouterProbe(biases, ordinal, experts=m.experts, top_k=m.top_k,
                                                               score_func=m.score_func, route_scale=m.route_scale))
            self.shared = self.stack.enter_context(ResidentSharedExpert(shared, ordinal, m.swiglu_limit,
                                                                        hidden=m.hidden, intermediate=m.intermediate))
            self.accumulator = self.stack.enter_context(MoEAccumulator(ordinal, MAX_CALL_TOKENS, hidden=m.hidden,
                                                                       experts=m.experts, top_k=m.top_k))
            self.experts = self.stack.enter_context(TieredExpertRuntime(self.store_path, c.cache,
                                                                        source_factory=self.source_factory, model=m,
                                                                        max_tokens=MAX_CALL_TOKENS))
            if any(entry["provenance"]["layer"] != self.layer for entry in self.experts.store.entries.values()):
                raise ValueError("Connected store contains artifacts from another layer")
            self.contexts = {"gate": self.gate.ctx, "router": self.router.ctx, "shared": self.shared.ctx,
                             "accumulator": self.accumulator.ctx, "cache_primary": self.experts.ctx}
            self.devices = {n: DeviceLedger(ctx, c.device_free_floor) for n, ctx in self.contexts.items()}
            self.helper_device = None
            self.minimum_available = physical_memory()["available"]
            self._headroom()
            return self
        except BaseException:
            self.stack.close()
            self.stack = None
            raise

    def _headroom(self):
        """Host reserve, the combined explicit device cap and the device's free floor, checked around a call."""
        available = physical_memory()["available"]
        self.minimum_available = min(self.minimum_available, available)
        self.budget.acquire(0, available)
        total = sum(sum(device.allocations.values()) for device in self.devices.values())
        if total > self.config.primary_explicit_cap_bytes:
            raise MemoryError("Combined native GPU buffers exceed the connected explicit cap")
        if self.devices["cache_primary"].memory()["free"] < self.config.device_free_floor:
            raise MemoryError("Connected runtime refuses work below the GPU reserve")

    def forward(self, activation, image_span=False) -> dict:
        if self.stack is None:
            raise RuntimeError("Use connected MoE as a context manager")
        if type(image_span) is not bool:
            raise ValueError("Connected image-span flag must be boolean")
        m = self.model
        x, bits = bf16_activation(activation, m.hidden)
        single = x.ndim == 1
        rows = bits.reshape(-1, m.hidden)
        t = rows.shape[0]
        if not 1 <= t <= MAX_CALL_TOKENS:
            raise ValueError(f"Connected MoE accepts 1 to {MAX_CALL_TOKENS} tokens per call")
        with self.lock:
            if self.active:
                raise RuntimeError("Nested MoE calls would overwrite live workspaces")
            before = self.experts.snapshot()
            self.active = True
            self.stats["calls_started"] += 1
            attempt = {"status": "running", "input_bf16_sha256": hashlib.sha256(bits.tobytes()).hexdigest(),
                       "image_span": image_span, "completed_expert_ids": [], "stage": "headroom"}
            self.last_attempt = attempt
            started = time.perf_counter()
            try:
                self.experts.cache.enforce_pressure()
                self._headroom()
                attempt["stage"] = "gate"
                logits = self.gate.project(rows)
                routing = self.router.inspect(logits, image_span)
                weights, indices = routing["weights"], routing["indices"]
                selected = participation(indices, t, experts=m.experts, top_k=m.top_k)
                attempt.update(indices=indices.tolist(), weight_bits=weights.view(np.uint32).tolist())
                missing = [e for e in selected if expert_key(self.layer, e, m) not in self.experts.store.entries]
                if missing:
                    raise KeyError(f"Selected original experts absent from this bounded store: {missing}")
                self.accumulator.begin(indices)
                outputs, stages, events = {}, {}, []
                for expert, token_rows in selected.items():
                    attempt["stage"] = f"expert:{expert}"
                    rank = np.argmax(indices[token_rows] == expert, axis=1)
                    route = weights[token_rows, rank]
                    result = self.experts.forward(expert_key(self.layer, expert, m), rows[token_rows], route)
                    outputs[expert] = result
                    events.append(dict(self.experts.last_event))
                    stages[f"after_expert_{expert}_fp32"] = self.accumulator.add(expert, result["w2"])
                    attempt["completed_expert_ids"].append(expert)
                attempt["stage"] = "shared"
                shared = self.shared.forward(rows)
                attempt["stage"] = "final_accumulation"
                stages.update(self.accumulator.finish(shared["w2"]))
                self.experts.cache.enforce_pressure()
                self._headroom()
                attempt.update(status="pass", stage="complete")
                self.stats["calls_completed"] += 1
                if single:
                    routing = {n: v.reshape(-1) for n, v in routing.items()}
                    logits = logits.reshape(-1)
                    shared = {n: v[0] for n, v in shared.items()}
                    stages = {n: v.reshape(-1) for n, v in stages.items()}
                    outputs = {e: {n: v[0] for n, v in r.items()} for e, r in outputs.items()}
                return {"input_bf16": bits, "logits": logits, "routing": routing, "experts": outputs,
                        "expert_events": events, "shared": shared, "aggregation": stages,
                        "output_bf16": stages["output_bf16"]}
            except BaseException as error:
                self.stats["calls_failed"] += 1
                attempt.update(status="failed", error_type=type(error).__name__)
                raise
            finally:
                try:
                    after = self.experts.snapshot()
                    attempt.update(wall_ms=(time.perf_counter() - started) * 1000,
                                   store_direct_read_calls=after["store_direct_read_calls"]
                                   - before["store_direct_read_calls"],
                                   store_direct_read_bytes=after["store_direct_read_bytes"]
                                   - before["store_direct_read_bytes"],
                                   cache_counter_delta={n: after["counters"][n] - v
                                                        for n, v in before["counters"].items()})
                finally:
                    self.active = False

    def snapshot(self) -> dict:
        if self.stack is None:
            raise RuntimeError("Connected MoE is closed")
        return {"calls": dict(self.stats), "cache": self.experts.snapshot(),
                "combined_host_reservation_peak_bytes": self.budget.peak,
                "combined_host_cap_bytes": self.budget.cap,
                "minimum_observed_host_available_bytes": self.minimum_available,
                "host_available_floor_bytes": self.budget.available_floor,
                "component_peak_explicit_device_bytes": {n: d.peak for n, d in self.devices.items()},
                "primary_explicit_cap_bytes": self.config.primary_explicit_cap_bytes,
                "cache_config": asdict(self.config.cache), "device": self.gate.ctx.device_name()[1]}

    def __exit__(self, *_):
        with self.lock:
            if self.active:
                raise RuntimeError("Cannot close connected MoE during a live call")
            live = {n: ctx.owned_bytes()[0] for n, ctx in self.contexts.items()} if self.stack is not None else {}
            if self.stack is not None:
                self.stack.close()
                self.stack = None
            self.cleanup = {"parent_reservation_bytes": self.budget.reserved,
                            "cache_reservation_bytes": self.experts.budget.reserved,
                            "explicit_live_bytes_before_close": live}


class ConnectedLayer:
    """ConnectedMoE's call over a resident MoELayer (one fused decode with diagnostics, replayed stepwise)."""

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
