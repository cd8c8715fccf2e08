"""The on-disk expert store (the reference's format, src/vesper/storage.py:20-186), read and written here.

Format (kept identical so a store written by either side opens in the other):

* `experts.bin`: whole experts back to back, each the six tensors in checkpoint order -- w1_weight [I, H/2],
  w1_scale [I, H/32], w3_*, w2_weight [H, I/2], w2_scale [H, I/32], row-major bytes -- entry n at byte
  n x expert_bytes (a multiple of 4096, so every expert is an aligned direct read).
* `manifest.json`: schema_version 1, kind "vesper_native_expert_store", the model and revision the experts
  came from, expert_bytes, file name and size, the tensor layout ({name: offset, bytes, shape}), and per
  entry its key "layer:expert", offset, bytes, the SHA-256 of the whole expert and its provenance (the
  expert-fixture manifest: identity, and name / checkpoint tensor / dtype / shape / bytes / SHA-256 of each
  tensor).

The model identity the store is checked against is a ModelProfile: REFERENCE_PROFILE is the reference's
pinned checkpoint (hidden 5120, intermediate 2304, 384 experts, 40 layers, swiglu_limit 10, at most 48
experts per store); BASELINE_PROFILE describes seeded synthetic stores at the DeepSeek-V3 shapes this build
benchmarks (7168 x 2048, 256 experts). Validation happens before any expert byte is trusted; reads go
through DirectReader (O_DIRECT); a read is refused unless its SHA-256 (and, on request, every tensor's)
matches the manifest.
"""

from __future__ import annotations

import hashlib
import json
import threading
from concurrent.futures import ThreadPoolExecutor
import os
import re
import zipfile
from dataclasses import dataclass
from pathlib import Path

import numpy as np

from .disk import PAGE, DirectReader
from .integrity import HASHERS, digest_shape, hash_chunks_native
from .resources import MemoryBudget, MiB
from .timing import Timings

STORE_KIND = "vesper_native_expert_store"
EXPERT_KIND = "complete_expert"
PROJECTIONS = ("w1", "w3", "w2")


@dataclass(frozen=True)
class ModelProfile:
    model: str
    revision: str
    hidden: int
    intermediate: int
    experts: int
    layers: int
    swiglu_limit: float
    max_store_experts: int
    top_k: int = 6
    score_func: str = "sqrtsoftplus"
    route_scale: float = 1.5
    inference_config_sha256: str = ""   # the released routing configuration a router fixture is pinned to

    def router_config(self) -> dict:
        """The routing configuration a router fixture records (src/vesper/router.py:16-17 for the reference)."""
        return {"experts": self.experts, "topk": self.top_k, "score_func": self.score_func, "gate_temp": 1.0,
                "norm_topk_prob": True, "route_scale": self.route_scale, "normalization_epsilon": 1e-20}

    def expert_layout(self) -> dict:
        """{tensor name: (rows, bytes per row)} in checkpoint order (src/vesper/checkpoint.py:139-141)."""
        h, i = self.hidden, self.intermediate
        shapes = {"w1": (i, h), "w3": (i, h), "w2": (h, i)}
        return {f"{p}_{s}": (shapes[p][0], shapes[p][1] // d) for p in PROJECTIONS for s, d in (("weight", 2),
                                                                                                   ("scale", 32))}

    @property
    def expert_bytes(self) -> int:
        return sum(r * c for r, c in self.expert_layout().values())


REFERENCE_PROFILE = ModelProfile("deepseek-ai/DeepSeek-V4.1-Flash-1017", "1bae0e1088993b9b82de08f59de5be5a34e42170",
                                 5120, 2304, 384, 40, 10.0, 48, 6, "sqrtsoftplus", 1.5,
                                 "2e84f45cf1dac8c7fcbb200e96667d4b913275690668ed496f24c7747207a809")
BASELINE_PROFILE = ModelProfile("synthetic/deepseek-v3-style-moe", "seeded-20261018", 7168, 2048, 256, 61, 0.0,
                                61 * 256, 8, "sigmoid", 2.5)


def validate_store_limit(limit, profile: ModelProfile = REFERENCE_PROFILE):
    if type(limit) is not int or not 1 <= limit <= profile.max_store_experts:
        raise ValueError(f"Explicit native-store limit must be one to {profile.max_store_experts} experts")


def validate_expert_identity(layer, expert, profile: ModelProfile = REFERENCE_PROFILE):
    if type(layer) is not int or type(expert) is not int or not (0 <= layer < profile.layers
                                                                 and 0 <= expert < profile.experts):
        raise ValueError("Expert identity is outside the pinned model")


def expert_key(layer: int, expert: int, profile: ModelProfile = REFERENCE_PROFILE) -> str:
    validate_expert_identity(layer, expert, profile)
    return f"{layer}:{expert}"


def tensor_layout(profile: ModelProfile = REFERENCE_PROFILE) -> dict:
    """{name: {offset, bytes, shape}} of one expert's bytes."""
    layout, at = {}, 0
    for name, (rows, cols) in profile.expert_layout().items():
        layout[name] = {"offset": at, "bytes": rows * cols, "shape": [rows, cols]}
        at += rows * cols
    return layout


def _hex(data) -> str:
    return hashlib.sha256(memoryview(np.ascontiguousarray(data)).cast("B")).hexdigest()


def _hex_parallel(views) -> list:
    """The SHA-256 of each view, on the host hashing threads: the whole-expert digest and the per-tensor
    digests of one read run on separate cores, and the whole-expert chain bounds the wall time."""
    return [f.result() for f in [HASHERS.submit(_hex, v) for v in views]]


def expert_provenance(layer: int, expert: int, arrays: dict, profile: ModelProfile = REFERENCE_PROFILE,
                      source: str = "synthetic") -> dict:
    """The expert-fixture manifest of six arrays (the shape src/vesper/checkpoint.py:215-222 records)."""
    validate_expert_identity(layer, expert, profile)
    tensors = []
    for name, (rows, cols) in profile.expert_layout().items():
        projection, suffix = name.split("_")
        tensors.append({"name": name, "tensor": f"layers.{layer}.ffn.experts.{expert}.{projection}.{suffix}",
                        "dtype": "I8" if suffix == "weight" else "F8_E8M0", "shape": [rows, cols],
                        "bytes": rows * cols, "sha256": _hex(arrays[name])})
    return {"kind": EXPERT_KIND, "model": profile.model, "revision": profile.revision, "layer": layer,
            "expert": expert, "swiglu_limit": profile.swiglu_limit, "source": source, "tensors": tensors}


def validate_expert_provenance(manifest: dict, profile: ModelProfile = REFERENCE_PROFILE):
    """The checks of src/vesper/checkpoint.py:157-174 against `profile`."""
    identity = (manifest.get("model"), manifest.get("revision"), manifest.get("kind"), manifest.get("swiglu_limit"))
    if identity != (profile.model, profile.revision, EXPERT_KIND, profile.swiglu_limit):
        raise ValueError("Expert provenance differs from the pinned checkpoint and probe scope")
    layer, expert = manifest.get("layer"), manifest.get("expert")
    validate_expert_identity(layer, expert, profile)
    layout = profile.expert_layout()
    entries = manifest.get("tensors", [])
    if len(entries) != len(layout) or {e.get("name") for e in entries} != set(layout):
        raise ValueError("Incomplete expert fixture provenance")
    for entry in entries:
        name = entry["name"]
        projection, suffix = name.split("_")
        expected = (f"layers.{layer}.ffn.experts.{expert}.{projection}.{suffix}",
                    "I8" if suffix == "weight" else "F8_E8M0", list(layout[name]), layout[name][0] * layout[name][1])
        if ((entry.get("tensor"), entry.get("dtype"), entry.get("shape"), entry.get("bytes")) != expected
                or not re.fullmatch(r"[0-9a-f]{64}", entry.get("sha256", ""))):
            raise ValueError("Expert tensor provenance differs from its pinned identity and layout")


def validate_expert_arrays(arrays: dict, profile: ModelProfile = REFERENCE_PROFILE):
    layout = profile.expert_layout()
    if set(arrays) != set(layout):
        raise ValueError("A complete expert requires exactly six native tensors")
    for name, shape in layout.items():
        a = arrays[name]
        if not isinstance(a, np.ndarray) or a.dtype != np.uint8 or a.shape != shape:
            raise ValueError("Expert tensor layout differs from the pinned shape")


# ---- expert fixtures (native-expert.npz + manifest.json, src/vesper/checkpoint.py:177-260) ------------------

def write_expert_fixture(directory: Path, layer: int, expert: int, arrays: dict,
                         profile: ModelProfile = REFERENCE_PROFILE) -> Path:
    """One expert as the reference's fixture pair; returns the archive path."""
    validate_expert_arrays(arrays, profile)
    directory = Path(directory)
    directory.mkdir(parents=True, exist_ok=True)
    manifest = expert_provenance(layer, expert, arrays, profile)
    np.savez(directory / "native-expert.npz", **{name: arrays[name] for name in profile.expert_layout()})
    (directory / "manifest.json").write_text(json.dumps(manifest, indent=2) + "\n", encoding="utf-8")
    return directory / "native-expert.npz"


def read_manifest(path: Path, limit: int = 65536) -> dict:
    """The manifest.json beside an archive, refused above `limit` bytes before it is parsed."""
    with (Path(path).parent / "manifest.json").open("rb") as stream:
        raw = stream.read(limit + 1)
    if len(raw) > limit:
        raise ValueError("Excessive fixture metadata")
    return json.loads(raw)


def read_bounded_npz(path: Path, members: dict, what: str) -> dict:
    """{name: array} of an .npz archive holding exactly the members {name: (shape, dtype)}: the member list,
    each member's stored size and its NPY header (version, shape, C order, dtype) are checked before NumPy
    allocates anything, and nothing is unpickled."""
    with zipfile.ZipFile(path) as archive:
        if sorted(archive.namelist()) != sorted(f"{name}.npy" for name in members):
            raise ValueError(f"{what} archive does not hold exactly its {len(members)} tensors")
        for name, (shape, dtype) in members.items():
            info = archive.getinfo(f"{name}.npy")
            if info.file_size > int(np.prod(shape)) * np.dtype(dtype).itemsize + 1024:
                raise ValueError(f"{what} archive member exceeds its bounded size")
            with archive.open(info) as stream:
                version = np.lib.format.read_magic(stream)
                if version not in ((1, 0), (2, 0)):
                    raise ValueError(f"Unsupported {what.lower()} array header")
                read_header = (np.lib.format.read_array_header_1_0 if version == (1, 0)
                               else np.lib.format.read_array_header_2_0)
                stored, fortran, stored_dtype = read_header(stream, max_header_size=1024)
                if stored != tuple(shape) or fortran or stored_dtype != np.dtype(dtype):
                    raise ValueError(f"{what} archive header differs from the bounded native layout")
    with np.load(path, allow_pickle=False) as archive:
        return {name: archive[name].copy() for name in members}


def load_expert_fixture(path: Path, profile: ModelProfile = REFERENCE_PROFILE):
    """(arrays, manifest) of a fixture; every member's header is bounded before NumPy allocates."""
    path = Path(path)
    manifest = read_manifest(path)
    validate_expert_provenance(manifest, profile)
    layout = profile.expert_layout()
    arrays = read_bounded_npz(path, {name: (shape, np.uint8) for name, shape in layout.items()}, "Expert")
    validate_expert_arrays(arrays, profile)
    for entry in manifest["tensors"]:
        if _hex(arrays[entry["name"]]) != entry["sha256"]:
            raise ValueError("Expert fixture bytes differ from their source hash")
    return arrays, manifest


# ---- the store ----------------------------------------------------------------------------------------------

def build_store(experts, directory: Path, *, max_experts=4, profile: ModelProfile = REFERENCE_PROFILE) -> dict:
    """Write a new store from `experts`: fixture archive paths (as the reference's build_store takes) or
    (layer, expert, arrays) triples. Refuses an existing directory; on failure removes only what it wrote."""
    validate_store_limit(max_experts, profile)
    items = list(experts)
    if not 1 <= len(items) <= max_experts:
        raise ValueError("Expert fixture count exceeds the explicit native-store limit")
    directory = Path(directory).resolve()
    if directory.exists():
        raise FileExistsError("Refusing to replace an existing native store")
    size = profile.expert_bytes
    if size % PAGE:
        raise ValueError("Expert bytes must be a multiple of 4096 for direct reads")
    directory.mkdir(parents=True)
    entries, seen = [], set()
    try:
        with (directory / "experts.bin").open("xb", buffering=0) as out:
            for item in items:
                if isinstance(item, (str, Path)):
                    arrays, provenance = load_expert_fixture(Path(item), profile)
                else:
                    layer, expert, arrays = item
                    validate_expert_arrays(arrays, profile)
                    provenance = expert_provenance(layer, expert, arrays, profile)
                key = expert_key(provenance["layer"], provenance["expert"], profile)
                if key in seen:
                    raise ValueError("Store entries must identify different original experts")
                seen.add(key)
                digest, offset = hashlib.sha256(), out.tell()
                for name in profile.expert_layout():
                    raw = memoryview(np.ascontiguousarray(arrays[name])).cast("B")
                    digest.update(raw)
                    if out.write(raw) != len(raw):
                        raise OSError("Short native-store write")
                entries.append({"key": key, "offset": offset, "bytes": size, "sha256": digest.hexdigest(),
                                "provenance": provenance})
            os.fsync(out.fileno())
        manifest = {"schema_version": 1, "kind": STORE_KIND, "model": profile.model, "revision": profile.revision,
                    "expert_bytes": size, "file": "experts.bin", "file_bytes": len(entries) * size,
                    "layout": tensor_layout(profile), "entries": entries}
        (directory / "manifest.json").write_text(json.dumps(manifest, indent=2) + "\n", encoding="utf-8")
    except BaseException:
        for name in ("manifest.json", "experts.bin"):
            (directory / name).unlink(missing_ok=True)
        directory.rmdir()
        raise
    return {"probe": "build_native_store", "status": "pass", "experts": len(entries),
            "file_bytes": len(entries) * size, "model": profile.model, "revision": profile.revision}


class NativeStore:
    """A validated store opened read-only: metadata checked on construction, one direct-I/O buffer while open
    (src/vesper/storage.py:95-186)."""

    def __init__(self, directory: Path, budget: MemoryBudget, *, max_experts=4,
                 profile: ModelProfile = REFERENCE_PROFILE):
        validate_store_limit(max_experts, profile)
        self.profile = profile
        self.directory = Path(directory).resolve(strict=True)
        self.budget, self.reader = budget, None
        self.timings = Timings()
        self.gpu_integrity, self.expected_chunks = False, {}
        self.read_calls, self.bytes_read = 0, 0
        self._count_lock = threading.Lock()
        with (self.directory / "manifest.json").open("rb") as stream:
            raw = stream.read(MiB + 1)
        if len(raw) > MiB:
            raise ValueError("Native-store metadata exceeds the probe's bounded scope")
        self.manifest = m = json.loads(raw)
        self.size = profile.expert_bytes
        header = (m.get("schema_version"), m.get("kind"), m.get("model"), m.get("revision"), m.get("expert_bytes"),
                  m.get("file"))
        if header != (1, STORE_KIND, profile.model, profile.revision, self.size, "experts.bin"):
            raise ValueError("Native store does not match the pinned format")
        if m.get("layout") != tensor_layout(profile) or not 1 <= len(m.get("entries", [])) <= max_experts:
            raise ValueError("Unexpected native-store layout or probe size")
        self.entries = {}
        for ordinal, entry in enumerate(m["entries"]):
            provenance = entry.get("provenance", {})
            validate_expert_provenance(provenance, profile)
            key = expert_key(provenance["layer"], provenance["expert"], profile)
            if (entry.get("key") != key or key in self.entries or entry.get("offset") != ordinal * self.size
                    or entry.get("bytes") != self.size or not re.fullmatch(r"[0-9a-f]{64}", entry.get("sha256", ""))):
                raise ValueError("Invalid or overlapping native-store entry")
            self.entries[key] = entry
        self.path = self.directory / "experts.bin"
        if m.get("file_bytes") != len(self.entries) * self.size or self.path.stat().st_size != m["file_bytes"]:
            raise ValueError("Native store file size differs from its complete entries")

    def __enter__(self):
        if self.reader is not None:
            raise RuntimeError("Native store is already open")
        self.reader = DirectReader(self.path, self.size, self.budget)
        return self

    def __exit__(self, *_):
        for key in list(self.expected_chunks):
            table = self.expected_chunks.pop(key)
            self.budget.release(table.nbytes, category="integrity")
        if self.reader is not None:
            self.reader.close()
            self.reader = None

    def validate(self, key: str, data: np.ndarray, *, tensors: bool = False):
        """Refuse (ValueError) bytes whose SHA-256 differs from the manifest's -- the whole expert, and each
        tensor against its provenance when `tensors`."""
        with self.timings.section("integrity.cpu_sha256"):
            entry = self.entries[key]
            if data.dtype != np.uint8 or data.shape != (self.size,) or not data.flags.c_contiguous:
                raise ValueError("Native-store payload layout differs from one expert")
            layout = self.manifest["layout"]
            named = entry["provenance"]["tensors"] if tensors else []
            regions = [layout[t["name"]] for t in named]
            views = [data] + [data[r["offset"]:r["offset"] + r["bytes"]] for r in regions]
            digests = _hex_parallel(views) if named else [_hex(data)]
            if digests[0] != entry["sha256"]:
                raise ValueError("Native expert bytes differ from the store hash")
            for tensor, digest in zip(named, digests[1:]):
                if digest != tensor["sha256"]:
                    raise ValueError("Native expert tensor differs from its original source hash")

    def check_bytes(self, key: str, data: np.ndarray):
        """validate(key, data, tensors=True) from any thread (no timing section), counted as one store read."""
        entry = self.entries[key]
        if data.dtype != np.uint8 or data.shape != (self.size,) or not data.flags.c_contiguous:
            raise ValueError("Native-store payload layout differs from one expert")
        layout = self.manifest["layout"]
        named = entry["provenance"]["tensors"]
        digests = _hex_parallel([data] + [data[layout[t["name"]]["offset"]:layout[t["name"]]["offset"]
                                                 + layout[t["name"]]["bytes"]] for t in named])
        with self._count_lock:
            self.read_calls += 1
            self.bytes_read += self.size
        if digests[0] != entry["sha256"]:
            raise ValueError("Native expert bytes differ from the store hash")
        for tensor, digest in zip(named, digests[1:]):
            if digest != tensor["sha256"]:
                raise ValueError("Native expert tensor differs from its original source hash")

    def adopt_table(self, key: str, table: np.ndarray):
        """Keep a verified read's 4 KiB digest table for the GPU audit (charged to the budget)."""
        if key in self.expected_chunks:
            return
        self.budget.acquire(table.nbytes, category="integrity")
        self.expected_chunks[key] = table

    def _after_read(self, key: str, target: np.ndarray):
        """Check the bytes just read against the manifest; with gpu_integrity, also build their 4 KiB digest
        table for the GPU audit -- on a hashing thread while the manifest digests run (the table's Python loop
        and the large GIL-free digests overlap), kept only if the bytes pass."""
        self.read_calls += 1
        self.bytes_read += self.size
        if not (self.gpu_integrity and key not in self.expected_chunks):
            self.validate(key, target, tensors=True)
            return
        shape = digest_shape(self.size)
        self.budget.acquire(shape[0] * shape[1], category="integrity")
        try:
            table = np.empty(shape, np.uint8)
            pending = HASHERS.submit(hash_chunks_native, target, table)
            try:
                self.validate(key, target, tensors=True)
            finally:
                with self.timings.section("integrity.prepare_cpu_chunks"):
                    pending.result()
            table.setflags(write=False)
            self.expected_chunks[key] = table
        except BaseException:
            self.budget.release(shape[0] * shape[1], category="integrity")
            raise

    def prefetch(self, keys, *, depth: int = 6, readers: int = 3, chunk_parts: int = 4) -> "StorePipeline":
        """A pipeline that reads and verifies `keys` (store entries, in order) ahead of their use; see
        StorePipeline."""
        if self.reader is None:
            raise RuntimeError("Native store is closed")
        return StorePipeline(self, keys, depth=depth, readers=readers, chunk_parts=chunk_parts)

    def read_into(self, key: str, target: np.ndarray):
        """Direct read of `key` into the reader's buffer, copied into `target` (one expert of bytes), then
        checked; with gpu_integrity set, the verified bytes' 4 KiB digest table is kept for the GPU audit."""
        if self.reader is None:
            raise RuntimeError("Native store is closed")
        entry = self.entries[key]
        with self.timings.section("storage.direct_read"):
            self.reader.read(entry["offset"], self.size)
        with self.timings.section("host.store_staging_copy"):
            np.copyto(target, self.reader.array())
        self._after_read(key, target)


def _page_aligned(size: int) -> np.ndarray:
    """`size` bytes starting on a page boundary (what an O_DIRECT read may target)."""
    raw = np.empty(size + PAGE, np.uint8)
    skip = (-raw.ctypes.data) % PAGE
    return raw[skip:skip + size]


class StorePipeline:
    """Reads and verifies a sequence of store entries ahead of their upload (a batch promotion).

    `readers` threads each take the next entry in order, read it with O_DIRECT straight into one of `depth`
    page-aligned host buffers (reserved in the store's budget), and check it as read_into does: the whole
    expert's and each tensor's SHA-256 against the manifest and, in GPU-integrity mode, the 4 KiB digest
    table for the upload audit -- the digests on the shared hashing threads, so several entries hash at
    once. get(key) returns the verified buffer of the next entry in order (waiting for it) or raises its
    read or check error; the caller copies it out and calls release(). Reads of later entries, their
    hashing and the caller's uploads of earlier ones therefore overlap. Budget: depth x one expert."""

    def __init__(self, store: NativeStore, keys, *, depth: int = 6, readers: int = 3, chunk_parts: int = 4):
        keys = list(keys)
        self.chunk_parts = chunk_parts
        if depth < 1 or readers < 1 or readers > depth:
            raise ValueError("A store pipeline needs 1 <= readers <= depth")
        for key in keys:
            if key not in store.entries:
                raise KeyError("Requested expert is absent from the pinned native store")
        self.store, self.keys, self.size = store, keys, store.size
        self.depth = depth
        store.budget.acquire(depth * self.size, category="scratch")
        self._buffers = [_page_aligned(self.size) for _ in range(depth)]
        self._free = list(range(depth))
        self._cond = threading.Condition()
        self._closed = False
        self._handle = os.open(store.path, os.O_RDONLY | os.O_DIRECT)
        self._pool = ThreadPoolExecutor(max_workers=readers, thread_name_prefix="vesper-store-read")
        self._futures = [self._pool.submit(self._fetch, key) for key in keys]
        self._next = 0

    def _take_buffer(self) -> int:
        with self._cond:
            while not self._free and not self._closed:
                self._cond.wait()
            if self._closed:
                raise RuntimeError("Store pipeline is closed")
            return self._free.pop(0)

    def release(self, index: int):
        with self._cond:
            self._free.append(index)
            self._cond.notify()

    def _fetch(self, key):
        index = self._take_buffer()
        try:
            data = self._buffers[index]
            if os.preadv(self._handle, [memoryview(data)], self.store.entries[key]["offset"]) != self.size:
                raise OSError("Short direct read")
            self.store.check_bytes(key, data)
            table = None
            if self.store.gpu_integrity and key not in self.store.expected_chunks:
                table = np.empty(digest_shape(self.size), np.uint8)
                hash_chunks_native(data, table, self.chunk_parts)
                table.setflags(write=False)
            return index, data, table
        except BaseException:
            self.release(index)
            raise

    def next_key(self):
        """The entry get() returns next (None when all are consumed)."""
        return self.keys[self._next] if self._next < len(self.keys) else None

    def get(self, key):
        """(buffer index, verified bytes, digest table or None) of the next entry, which must be `key`."""
        if self._next >= len(self.keys) or self.keys[self._next] != key:
            raise RuntimeError("Store pipeline entries are consumed in order")
        future = self._futures[self._next]
        self._next += 1
        return future.result()

    def close(self):
        with self._cond:
            self._closed = True
            self._cond.notify_all()
        for future in self._futures:
            future.cancel()
        self._pool.shutdown(wait=True)
        os.close(self._handle)
        self._buffers, self._futures = [], []
        self.store.budget.release(self.depth * self.size, category="scratch")

    def __enter__(self):
        return self

    def __exit__(self, *_):
        self.close()
