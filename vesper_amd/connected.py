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
from contextlib import ExitStack, contextmanager
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
    """Serial calls of one registered layer over the store, behind the reference's constructor, call and
    records (src/vesper/connected.py:56-213: forward, snapshot, last_attempt, cleanup, stats).

    Opening loads the three fixtures, opens the five components on one exit stack -- gate projection, router
    probe, shared expert, accumulator, and the tiered expert runtime over the store -- and checks that the
    fixtures and every stored expert belong to the selected layer. A call is the pipeline
    route -> run the selected experts -> combine, with the host and device reserves checked before and after
    it; the call's record (last_attempt) is kept by one context manager that takes the lock, refuses nesting,
    counts the call, marks it passed or failed, and, either way, adds its wall time and the store and cache
    counters it moved. A failed call returns nothing and the next one starts from a zeroed accumulator."""

    CALL_COUNTERS = ("calls_started", "calls_completed", "calls_failed")

    def __init__(self, store: Path, gate_fixture: Path, router_fixture: Path, shared_fixture: Path,
                 config: ConnectedConfig | None = None, *, cublas_library=None, layer=0, profile="qualified",
                 source_factory=None, model: ModelProfile = REFERENCE_PROFILE):
        if cublas_library is not None:
            raise ValueError("The gate projection runs as a HIP kernel; no BLAS library is loaded")
        if source_factory is not None and not callable(source_factory):
            raise ValueError("Expected an explicit expert source factory")
        self.layer, self.model = validate_layer(layer, model, profile), model
        self.store_path = Path(store)
        self.gate_fixture, self.router_fixture, self.shared_fixture = map(Path, (gate_fixture, router_fixture,
                                                                                 shared_fixture))
        self.config, self.source_factory = config or ConnectedConfig(), source_factory
        self.stats = dict.fromkeys(self.CALL_COUNTERS, 0)
        self.lock = threading.RLock()
        self.stack, self.active, self.last_attempt = None, False, None

    # -- opening ---------------------------------------------------------------------------------------------
    def _fixtures(self):
        """(gate weight, router biases, shared expert) of the selected layer."""
        m = self.model
        (weight, self.gate_manifest), (biases, self.router_manifest), (shared, self.shared_manifest) = (
            load(path, m) for load, path in ((load_gate_fixture, self.gate_fixture),
                                            (load_router_fixture, self.router_fixture),
                                            (load_shared_fixture, self.shared_fixture)))
        layers = {man["layer"] for man in (self.gate_manifest, self.router_manifest, self.shared_manifest)}
        if layers != {self.layer}:
            raise ValueError("Connected gate, router and shared artifacts must match the selected layer")
        return weight, biases, shared

    def _components(self, stack: ExitStack, weight, biases, shared):
        c, m = self.config, self.model
        gpu = c.cache.primary_device
        self.gate = stack.enter_context(GateProjection(weight, gpu))
        self.router = stack.enter_context(RouterProbe(biases, gpu, experts=m.experts, top_k=m.top_k,
                                                      score_func=m.score_func, route_scale=m.route_scale))
        self.shared = stack.enter_context(ResidentSharedExpert(shared, gpu, m.swiglu_limit, hidden=m.hidden,
                                                               intermediate=m.intermediate))
        self.accumulator = stack.enter_context(MoEAccumulator(gpu, MAX_CALL_TOKENS, hidden=m.hidden,
                                                              experts=m.experts, top_k=m.top_k))
        self.experts = stack.enter_context(TieredExpertRuntime(self.store_path, c.cache, model=m,
                                                               source_factory=self.source_factory,
                                                               max_tokens=MAX_CALL_TOKENS))
        if any(entry["provenance"]["layer"] != self.layer for entry in self.experts.store.entries.values()):
            raise ValueError("Connected store contains artifacts from another layer")
        self.contexts = {"gate": self.gate.ctx, "router": self.router.ctx, "shared": self.shared.ctx,
                         "accumulator": self.accumulator.ctx, "cache_primary": self.experts.ctx}
        self.devices = {name: DeviceLedger(ctx, c.device_free_floor) for name, ctx in self.contexts.items()}
        self.helper_device = None

    def __enter__(self):
        if self.stack is not None:
            raise RuntimeError("Connected MoE is already open")
        c = self.config
        self.budget = MemoryBudget(c.host_cap_bytes, c.cache.available_floor, owner="connected")
        with ExitStack() as stack:   # unwinds only when opening fails: pop_all() takes the resources over
            allowance = c.cache.host_cap_bytes + 100 * MiB   # the cache's own cap + fixtures and upload staging
            self.budget.acquire(allowance)
            stack.callback(self.budget.release, allowance)
            self._components(stack, *self._fixtures())
            self.minimum_available = physical_memory()["available"]
            self._headroom()
            self.stack = stack.pop_all()
        return self

    # -- reserves --------------------------------------------------------------------------------------------
    def _headroom(self):
        """The host reserve (tracking the lowest available memory seen), the components' combined explicit
        device bytes against the cap, and the compute device's free-memory floor."""
        host_free = physical_memory()["available"]
        self.minimum_available = min(host_free, self.minimum_available)
        self.budget.acquire(0, host_free)   # MemoryError below the reserve
        if sum(ledger.allocations["explicit"] for ledger in self.devices.values()) > \
                self.config.primary_explicit_cap_bytes:
            raise MemoryError("Combined native GPU buffers exceed the connected explicit cap")
        if self.devices["cache_primary"].memory()["free"] < self.config.device_free_floor:
            raise MemoryError("Connected runtime refuses work below the GPU reserve")

    def _reserves(self):
        self.experts.cache.enforce_pressure()
        self._headroom()

    # -- one call --------------------------------------------------------------------------------------------
    @contextmanager
    def _attempt(self, bits: np.ndarray, image_span: bool):
        with self.lock:
            if self.active:
                raise RuntimeError("Nested MoE calls would overwrite live workspaces")
            record = {"status": "running", "input_bf16_sha256": hashlib.sha256(bits.tobytes()).hexdigest(),
                      "image_span": image_span, "completed_expert_ids": [], "stage": "headroom"}
            baseline, clock = self.experts.snapshot(), time.perf_counter()
            self.active, self.last_attempt = True, record
            self.stats["calls_started"] += 1
            try:
                yield record
            except BaseException as error:
                self.stats["calls_failed"] += 1
                record.update(status="failed", error_type=type(error).__name__)
                raise
            else:
                record.update(status="pass", stage="complete")
                self.stats["calls_completed"] += 1
            finally:
                try:
                    now = self.experts.snapshot()
                    moved = {n: now[n] - baseline[n] for n in ("store_direct_read_calls", "store_direct_read_bytes")}
                    record.update(wall_ms=(time.perf_counter() - clock) * 1000, **moved,
                                  cache_counter_delta={n: now["counters"][n] - v
                                                       for n, v in baseline["counters"].items()})
                finally:
                    self.active = False

    def _route(self, rows: np.ndarray, image_span: bool, record: dict):
        """Gate logits, the routing postprocess, and per selected expert (ascending ID) its token rows and
        their route weights; selected experts missing from the store are refused before any expert I/O."""
        m = self.model
        record["stage"] = "gate"
        logits = self.gate.project(rows)
        routing = self.router.inspect(logits, image_span)
        indices, weights = routing["indices"], routing["weights"]
        record.update(indices=indices.tolist(), weight_bits=weights.view(np.uint32).tolist())
        plan = participation(indices, rows.shape[0], experts=m.experts, top_k=m.top_k)
        absent = [e for e in plan if expert_key(self.layer, e, m) not in self.experts.store.entries]
        if absent:
            raise KeyError(f"Selected original experts absent from this bounded store: {absent}")
        routes = {}
        for expert, token_rows in plan.items():
            rank = (indices[token_rows] == expert).argmax(axis=1)   # the expert's position in each token's list
            routes[expert] = (token_rows, weights[token_rows, rank])
        return logits, routing, routes

    def _run_experts(self, rows: np.ndarray, routes: dict, record: dict):
        """Each routed expert from whichever tier holds it, its rows added to the accumulator in order."""
        results, events, snapshots = {}, [], {}
        for expert, (token_rows, route) in routes.items():
            record["stage"] = f"expert:{expert}"
            out = self.experts.forward(expert_key(self.layer, expert, self.model), rows[token_rows], route)
            events.append(dict(self.experts.last_event))
            snapshots[f"after_expert_{expert}_fp32"] = self.accumulator.add(expert, out["w2"])
            results[expert] = out
            record["completed_expert_ids"].append(expert)
        return results, events, snapshots

    def forward(self, activation, image_span=False) -> dict:
        if self.stack is None:
            raise RuntimeError("Use connected MoE as a context manager")
        if type(image_span) is not bool:
            raise ValueError("Connected image-span flag must be boolean")
        _, bits = bf16_activation(activation, self.model.hidden)
        rows = bits.reshape(-1, self.model.hidden)
        if not 1 <= rows.shape[0] <= MAX_CALL_TOKENS:
            raise ValueError(f"Connected MoE accepts 1 to {MAX_CALL_TOKENS} tokens per call")
        with self._attempt(bits, image_span) as record:
            self._reserves()
            logits, routing, routes = self._route(rows, image_span, record)
            self.accumulator.begin(routing["indices"])
            experts, events, aggregation = self._run_experts(rows, routes, record)
            record["stage"] = "shared"
            shared = self.shared.forward(rows)
            record["stage"] = "final_accumulation"
            aggregation.update(self.accumulator.finish(shared["w2"]))
            self._reserves()
        if bits.ndim == 1:   # one token given as [hidden]: drop the token axis, as the reference's call returns
            first = lambda v: v[0]
            flat = lambda v: v.reshape(-1)
            logits, routing, aggregation = flat(logits), _map(flat, routing), _map(flat, aggregation)
            shared = _map(first, shared)
            experts = {e: _map(first, r) for e, r in experts.items()}
        return {"input_bf16": bits, "logits": logits, "routing": routing, "experts": experts,
                "expert_events": events, "shared": shared, "aggregation": aggregation,
                "output_bf16": aggregation["output_bf16"]}

    # -- records ---------------------------------------------------------------------------------------------
    def snapshot(self) -> dict:
        if self.stack is None:
            raise RuntimeError("Connected MoE is closed")
        b, c = self.budget, self.config
        return {"calls": dict(self.stats), "cache": self.experts.snapshot(),
                "combined_host_reservation_peak_bytes": b.peak, "combined_host_cap_bytes": b.cap,
                "minimum_observed_host_available_bytes": self.minimum_available,
                "host_available_floor_bytes": b.available_floor,
                "component_peak_explicit_device_bytes": {n: ledger.peak for n, ledger in self.devices.items()},
                "primary_explicit_cap_bytes": c.primary_explicit_cap_bytes, "cache_config": asdict(c.cache),
                "device": self.gate.ctx.device_name()[1]}

    def __exit__(self, *_):
        with self.lock:
            if self.active:
                raise RuntimeError("Cannot close connected MoE during a live call")
            live = {}
            if self.stack is not None:
                live = {n: ctx.owned_bytes()[0] for n, ctx in self.contexts.items()}
                stack, self.stack = self.stack, None
                stack.close()
            self.cleanup = {"parent_reservation_bytes": self.budget.reserved,
                            "cache_reservation_bytes": self.experts.budget.reserved,
                            "explicit_live_bytes_before_close": live}


def _map(fn, mapping: dict) -> dict:
    return {name: fn(value) for name, value in mapping.items()}


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
