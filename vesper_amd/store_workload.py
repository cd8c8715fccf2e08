"""Store -> HBM promotion of single experts through the exclusive tiers, used by bench.py.

  python -m vesper_amd.store_workload --experts 8

Writes a store of `experts` + 1 synthetic experts at the reference model's shapes (18.8 MB each, random
bytes: promotion does not look at the values) to a directory whose filesystem accepts O_DIRECT, flushes it
to the device, and then requests every expert once through TieredExpertRuntime's tiers with one GPU slot
and no RAM tier, so every request is a store read promoted into HBM. The first request warms up and is not
counted. Both integrity modes run on fresh runtimes.

Per mode, the median per expert of each stage (the runtime's own timing sections): the O_DIRECT read, the
copy into pinned staging, the host SHA-256 checks (whole expert and each tensor against the manifest), the
H2D copy + tiling into the slot, and the upload audit (readback: D2H + host SHA-256; gpu-sha256: the 4 KiB
digest table on the host and the hash on the GPU). Reported rates: expert bytes / the whole promotion
("store_to_hbm"), / the direct read alone ("direct_read") and / the H2D + tiling alone. Then the same
experts as one pipelined batch per mode ("batch": TieredExpertRuntime.prefetch into as many GPU slots), whose
rate is the batch's bytes over its wall time.
"""

from __future__ import annotations

import argparse
import json
import os
import shutil
import sys
import tempfile
import time
from pathlib import Path

import numpy as np

ROOT = Path(__file__).resolve().parents[1]


def _direct_io_ok(directory: Path) -> bool:
    probe = directory / ".direct_probe"
    try:
        probe.write_bytes(b"\0" * 4096)
        os.close(os.open(probe, os.O_RDONLY | os.O_DIRECT))
        return True
    except OSError:
        return False
    finally:
        probe.unlink(missing_ok=True)


def scratch_directory() -> Path:
    """A new empty directory on a filesystem that accepts O_DIRECT: the system temp directory, else one beside
    the package."""
    for parent in (None, ROOT):
        directory = Path(tempfile.mkdtemp(prefix=".direct_io_store_", dir=parent))
        if _direct_io_ok(directory):
            return directory
        shutil.rmtree(directory, ignore_errors=True)
    raise RuntimeError("no filesystem here accepts O_DIRECT reads")


def write_store(directory: Path, count: int, seed: int, profile) -> list:
    from .store import build_store, tensor_layout
    rng = np.random.default_rng(seed)
    layout = tensor_layout(profile)
    items = []
    for expert in range(count):
        blob = rng.integers(0, 256, profile.expert_bytes, dtype=np.uint8)
        arrays = {n: blob[r["offset"]:r["offset"] + r["bytes"]].reshape(r["shape"]) for n, r in layout.items()}
        items.append((0, expert, arrays))
    build_store(items, directory, max_experts=count, profile=profile)
    fd = os.open(directory / "experts.bin", os.O_RDONLY)
    try:
        os.fsync(fd)
    finally:
        os.close(fd)
    return [f"0:{expert}" for expert in range(count)]


STAGES = {"direct_read": ("storage.direct_read",), "staging_copy": ("host.store_staging_copy",),
          "host_sha256": ("integrity.cpu_sha256", "integrity.prepare_cpu_chunks"),
          "h2d_and_tile": ("transfer.primary_h2d",), "audit_d2h": ("transfer.primary_d2h",),
          "audit_gpu": ("integrity.gpu_sha256", "integrity.gpu_digest_d2h")}


def promote(store: Path, keys: list, mode: str, profile) -> dict:
    from .resources import GiB, MiB
    from .tiered import CacheConfig, TieredExpertRuntime
    config = CacheConfig(host_cap_bytes=1024 * MiB, ram_cache_bytes=0, available_floor=GiB, primary_slots=1,
                         helper_device=None, helper_slots=0, integrity_mode=mode, max_store_experts=len(keys),
                         device_cap_bytes=512 * MiB, profile=True)
    size = profile.expert_bytes
    walls, stages = [], {name: [] for name in STAGES}
    with TieredExpertRuntime(store, config, model=profile) as runtime:
        timings = runtime.timings
        for i, key in enumerate(keys):
            before = timings.snapshot()
            start = time.perf_counter()
            with runtime.cache.acquire(key) as (_, origin):
                pass
            wall = (time.perf_counter() - start) * 1e3
            if origin != "store":
                raise RuntimeError(f"expected a store read for {key}, got {origin}")
            if i == 0:
                continue                       # warm-up: first kernel launches and allocations
            delta = timings.since(before)
            walls.append(wall)
            for name, sections in STAGES.items():
                stages[name].append(sum(delta.get(s, {"total_ms": 0.0})["total_ms"] for s in sections))
        counters = runtime.snapshot()["counters"]
    med = {name: float(np.median(v)) for name, v in stages.items()}
    wall = float(np.median(walls))

    def rate(ms):
        return round(size / (ms * 1e-3) / 1e9, 2) if ms > 0 else None

    return {"experts_timed": len(walls), "expert_bytes": size, "ms_per_expert": round(wall, 3),
            "store_to_hbm_GB_per_s": rate(wall), "direct_read_GB_per_s": rate(med["direct_read"]),
            "h2d_and_tile_GB_per_s": rate(med["h2d_and_tile"]),
            "stage_ms": {name: round(v, 3) for name, v in med.items()},
            "integrity_failures": counters["integrity_failures"]}


def promote_batch(store: Path, keys: list, mode: str, profile, depth: int = 6, readers: int = 3) -> dict:
    """keys[0] promoted alone (warm-up), then keys[1:] as one pipelined batch (TieredExpertRuntime.prefetch:
    store reads and host checks of later experts overlap the uploads and audits of earlier ones) into as
    many GPU slots; wall time of the batch."""
    from .resources import GiB, MiB
    from .tiered import CacheConfig, TieredExpertRuntime
    batch = keys[1:]
    config = CacheConfig(host_cap_bytes=2048 * MiB, ram_cache_bytes=0, available_floor=GiB,
                         primary_slots=len(batch), helper_device=None, helper_slots=0, integrity_mode=mode,
                         max_store_experts=len(keys), device_cap_bytes=2048 * MiB, profile=False)
    size = profile.expert_bytes
    with TieredExpertRuntime(store, config, model=profile) as runtime:
        runtime.prefetch(keys[:1])
        start = time.perf_counter()
        origins = runtime.prefetch(batch, depth=depth, readers=readers)
        wall = time.perf_counter() - start
        if origins != ["store"] * len(batch):
            raise RuntimeError(f"expected store reads for the batch, got {origins}")
        counters = runtime.snapshot()["counters"]
    return {"experts": len(batch), "expert_bytes": size, "ms": round(wall * 1e3, 2),
            "ms_per_expert": round(wall * 1e3 / len(batch), 3),
            "store_to_hbm_GB_per_s": round(len(batch) * size / wall / 1e9, 2), "pipeline_depth": depth,
            "reader_threads": readers, "integrity_failures": counters["integrity_failures"]}


def run(experts: int = 8, seed: int = 20261018) -> dict:
    from .store import REFERENCE_PROFILE
    directory = scratch_directory()
    try:
        keys = write_store(directory / "store", experts + 1, seed, REFERENCE_PROFILE)
        out = {mode: promote(directory / "store", keys, mode, REFERENCE_PROFILE)
               for mode in ("readback", "gpu-sha256")}
        out["batch"] = {mode: promote_batch(directory / "store", keys, mode, REFERENCE_PROFILE)
                        for mode in ("readback", "gpu-sha256")}
        if os.environ.get("VESPER_STORE_SWEEP"):
            out["batch_sweep"] = {f"{d}x{r}": promote_batch(directory / "store", keys, "gpu-sha256",
                                                            REFERENCE_PROFILE, d, r)
                                  for d, r in ((3, 2), (6, 3), (8, 4))}
        out["note"] = ("readback / gpu-sha256: one expert per request, store read -> pinned staging -> HBM slot "
                       "(tiled), with the mode's checks; medians over the timed experts. batch: the same experts "
                       "as one pipelined promotion (reads, host SHA-256 and uploads of different experts overlap)")
        return out
    finally:
        shutil.rmtree(directory, ignore_errors=True)


def main():
    p = argparse.ArgumentParser(description=__doc__)
    p.add_argument("--experts", type=int, default=8)
    args = p.parse_args()
    print(json.dumps(run(args.experts)), flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
