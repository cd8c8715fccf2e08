"""ctypes binding of libmxmoe.so (the C ABI declared in include/mxmoe.h).

Replaces the reference's ctypes binding of libcuda/NVRTC (src/vesper/cuda.py:28-315):
the library is built ahead of time for gfx950 and loaded from this package
directory. There is no fallback: if the library is missing, every entry point
raises.
"""

from __future__ import annotations

import ctypes as C
import threading
from pathlib import Path

import numpy as np

PKG = Path(__file__).resolve().parent
LIB_PATH = PKG / "libmxmoe.so"

MX_OK, MX_ERR_INVALID, MX_ERR_MEMORY, MX_ERR_STATE, MX_ERR_HIP = 0, -1, -2, -3, -4
MX_FMT_MXFP4, MX_FMT_FP8_BLOCK32 = 0, 1
MX_SCORE = {"sigmoid": 0, "sqrtsoftplus": 1}
BUFFERS = {"logits": 0, "scores": 1, "selection": 2, "indices": 3, "weights": 4, "xq": 5, "xs": 6, "plan": 7,
           "w1": 8, "w3": 9, "down_input": 10, "down_q": 11, "down_s": 12, "expert_out": 13, "trace": 14,
           "raw": 15, "denominator": 16, "tied": 17}


class HipError(RuntimeError):
    """A HIP runtime failure (the reference's CudaError, src/vesper/cuda.py:18-19)."""


CudaError = HipError


class MxExpertPtrs(C.Structure):
    _fields_ = [(name, C.c_void_p) for name in
                ("w1_weight", "w1_scale", "w3_weight", "w3_scale", "w2_weight", "w2_scale")]


class MxExpertStages(C.Structure):
    _fields_ = [(name, C.c_void_p) for name in
                ("q", "s", "w1", "w3", "down_input", "trace", "down_q", "down_s")]


class MxRouterOut(C.Structure):
    _fields_ = [(name, C.c_void_p) for name in
                ("logits", "scores", "selection", "indices", "weights", "raw", "denominator", "tied")]


class MxMoeConfig(C.Structure):
    _fields_ = [("hidden", C.c_int32), ("intermediate", C.c_int32), ("experts", C.c_int32),
                ("top_k", C.c_int32), ("score_func", C.c_int32), ("route_scale", C.c_float),
                ("swiglu_limit", C.c_float), ("shared_format", C.c_int32), ("max_tokens", C.c_int32)]


_P, _I32, _I64, _U64, _F = C.c_void_p, C.c_int32, C.c_int64, C.c_uint64, C.c_float
SIGNATURES = {
    "mx_last_error": ([], C.c_char_p),
    "mx_device_count": ([], C.c_int),
    "mx_create": ([C.c_int, _U64, C.POINTER(_P)], C.c_int),
    "mx_destroy": ([_P], C.c_int),
    "mx_device_name": ([_P, C.c_char_p, C.c_size_t, C.c_char_p, C.c_size_t], C.c_int),
    "mx_device_memory": ([_P, C.POINTER(_U64), C.POINTER(_U64)], C.c_int),
    "mx_malloc": ([_P, _U64, C.POINTER(_P)], C.c_int),
    "mx_free": ([_P, _P], C.c_int),
    "mx_owned_bytes": ([_P, C.POINTER(_U64), C.POINTER(_U64)], C.c_int),
    "mx_host_alloc_pinned": ([_P, _U64, C.POINTER(_P)], C.c_int),
    "mx_host_free_pinned": ([_P, _P], C.c_int),
    "mx_memcpy_h2d": ([_P, _P, _P, _U64, _P], C.c_int),
    "mx_memcpy_d2h": ([_P, _P, _P, _U64, _P], C.c_int),
    "mx_memcpy_d2d": ([_P, _P, _P, _U64, _P], C.c_int),
    "mx_stream_create": ([_P, C.POINTER(_P)], C.c_int),
    "mx_stream_destroy": ([_P, _P], C.c_int),
    "mx_stream_sync": ([_P, _P], C.c_int),
    "mx_device_sync": ([_P], C.c_int),
    "mx_event_create": ([_P, C.POINTER(_P)], C.c_int),
    "mx_event_destroy": ([_P, _P], C.c_int),
    "mx_event_record": ([_P, _P, _P], C.c_int),
    "mx_event_sync": ([_P, _P], C.c_int),
    "mx_event_elapsed_ms": ([_P, _P, _P, C.POINTER(_F)], C.c_int),
    "mx_stream_wait_event": ([_P, _P, _P], C.c_int),
    "mx_fill_uniform_u8": ([_P, _P, _U64, _U64, C.c_uint32, C.c_uint32, _P], C.c_int),
    "mx_dequant_mxfp4": ([_P, _P, _P, _P, _I64, _I64, _P], C.c_int),
    "mx_encode_e4m3": ([_P, _P, _P, _I64, _P], C.c_int),
    "mx_act_quant32": ([_P, _P, _P, _P, _I64, _I64, _P], C.c_int),
    "mx_act_quant32_f32": ([_P, _P, _P, _P, _I64, _I64, _P], C.c_int),
    "mx_gemv_mxfp4": ([_P, _P, _P, _P, _P, _P, _I32, _I32, _I32, _P], C.c_int),
    "mx_expert_forward": ([_P, C.POINTER(MxExpertPtrs), _I32, _I32, _I32, _P, _I32, _F, _P, _P,
                           C.POINTER(MxExpertStages), _P], C.c_int),
    "mx_router": ([_P, _P, _P, _P, _I32, _I32, _I32, _I32, _I32, _F, C.POINTER(MxRouterOut), _P], C.c_int),
    "mx_router_postprocess": ([_P, _P, _P, _I32, _I32, _I32, _I32, _F, C.POINTER(MxRouterOut), _P], C.c_int),
    "mx_router_select": ([_P, _P, _P, _I32, _I32, _I32, _F, C.POINTER(MxRouterOut), _P], C.c_int),
    "mx_gate_project": ([_P, _P, _P, _I32, _I32, _I32, _P, _P], C.c_int),
    "mx_acc_zero": ([_P, _P, _I64, _P], C.c_int),
    "mx_acc_add_rows": ([_P, _P, _P, _P, _I32, _I32, _P], C.c_int),
    "mx_acc_add": ([_P, _P, _P, _I64, _P], C.c_int),
    "mx_acc_finish": ([_P, _P, _P, _I64, _P], C.c_int),
    "mx_tiled_expert_bytes": ([_I32, _I32], _U64),
    "mx_tile_expert": ([_P, C.POINTER(MxExpertPtrs), _I32, _I32, _P, _P], C.c_int),
    "mx_untile_expert": ([_P, _P, _I32, _I32, C.POINTER(MxExpertPtrs), _P], C.c_int),
    "mx_layer_create": ([_P, C.POINTER(MxMoeConfig), _P, _P, C.POINTER(_P), _P, C.POINTER(_P)], C.c_int),
    "mx_layer_destroy": ([_P], C.c_int),
    "mx_layer_set_expert": ([_P, _I32, _P, _P], C.c_int),
    "mx_moe_decode": ([_P, _P, _I32, _P, _I32, _P], C.c_int),
    "mx_layer_buffer": ([_P, _I32, C.POINTER(_P), C.POINTER(_U64)], C.c_int),
    "mx_layer_profile": ([_P, _I32, C.POINTER(_F), C.POINTER(_I32)], C.c_int),
    "mx_layer_time_stage": ([_P, _I32, _I32, C.POINTER(_F), _P], C.c_int),
    "mx_prefill_workspace_bytes": ([_P, _I32], _U64),
    "mx_prefill_stage_offsets": ([_P, _I32, _P], C.c_int),
    "mx_moe_decode_routed": ([_P, _P, _I32, _P, _P, _P, _P], C.c_int),
    "mx_expert_forward_tiled": ([_P, _P, _I32, _I32, _P, _I32, _F, _P, _P, C.POINTER(MxExpertStages), _P], C.c_int),
    "mx_expert_forward_bf16": ([_P, _P, _I32, _I32, _P, _I32, _P, _P, _P, _P, _P], C.c_int),
    "mx_expert_forward_tiled_noalloc": ([_P, _P, _I32, _I32, _P, _I32, _F, _P, _P, C.POINTER(MxExpertStages), _P],
                                        C.c_int),
    "mx_layer_set_experts": ([_P, _I32, _P, _P, _P], C.c_int),
    "mx_layer_route_errors": ([_P, C.POINTER(C.c_uint32), _I32, _P], C.c_int),
    "mx_cache_create": ([_P, _U64, _I32, C.POINTER(_P)], C.c_int),
    "mx_cache_destroy": ([_P], C.c_int),
    "mx_cache_register": ([_P, C.c_int64, _P], C.c_int),
    "mx_cache_ensure": ([_P, _P, _I32, _P, _P], C.c_int),
    "mx_cache_ready_event": ([_P, C.POINTER(_P)], C.c_int),
    "mx_cache_forget": ([_P, C.c_int64], C.c_int),
    "mx_cache_release": ([_P, _P, _I32, _P], C.c_int),
    "mx_cache_copy_stream": ([_P, C.POINTER(_P)], C.c_int),
    "mx_cache_stats": ([_P, C.POINTER(_U64), C.POINTER(_U64), C.POINTER(_U64), C.POINTER(C.c_double),
                        C.POINTER(_I32)], C.c_int),
    "mx_cache_set_timing": ([_P, _I32], C.c_int),
    "mx_moe_prefill": ([_P, _P, _I32, _P, _P, _P, _P, _U64, _P], C.c_int),
    "mx_fp8_tiled_bytes": ([_I32, _I32, _I32], _U64),
    "mx_fp8_tile": ([_P, _P, _P, _I32, _I32, _I32, _P, _P], C.c_int),
    "mx_act_quant128": ([_P, _P, _P, _P, _I64, _I64, _P], C.c_int),
    "mx_fp8_projection": ([_P, _P, _I32, _I32, _I32, _P, _I32, _P, _P, _P, _P, _P], C.c_int),
    "mx_fp8_expert_forward": ([_P, _P, _P, _P, _I32, _I32, _P, _I32, _F, _P, _P, C.POINTER(MxExpertStages), _P],
                              C.c_int),
    "mx_copy_kernel": ([_P, _P, _P, _U64, _P], C.c_int),
    "mx_read_kernel": ([_P, _P, _U64, _P, _P], C.c_int),
    "mx_fp8_grouped_projection": ([_P, _P, _I32, _I32, _I32, _P, _P, _I32, _P, _P, _P], C.c_int),
    "mx_kv_round32": ([_P, _P, _I64, _P, _P, _P, _P], C.c_int),
    "mx_sha256_chunks": ([_P, _P, _U64, _P, _P], C.c_int),
    "mx_host_sha256_chunks": ([_P, _U64, _P, _I32], C.c_int),
    "mx_sha256_verify": ([_P, C.POINTER(_P), C.POINTER(_P), _P, _I32, _U64, _P, _P], C.c_int),
    "mx_audit_gate": ([_P, _P, _I32, _P, _I32, _P, _U64, _P], C.c_int),
    "mx_owned_size": ([_P, _P, C.POINTER(_U64)], C.c_int),
    "mx_check_e4m3_pack": ([_P, C.POINTER(_U64)], C.c_int),
}

_lock = threading.Lock()
_lib = None


class Library:
    """Typed handle on libmxmoe.so; attribute access returns a status-checked callable."""

    def __init__(self, path: Path):
        self.path = path
        self.cdll = C.CDLL(str(path))
        for name, (args, res) in SIGNATURES.items():
            fn = getattr(self.cdll, name)
            fn.argtypes, fn.restype = args, res

    def last_error(self) -> str:
        return self.cdll.mx_last_error().decode(errors="replace")

    def device_count(self) -> int:
        return int(self.cdll.mx_device_count())

    def check(self, status: int, what: str = ""):
        if status == MX_OK:
            return
        message = f"{what}: {self.last_error()}" if what else self.last_error()
        if status == MX_ERR_INVALID:
            raise ValueError(message)
        if status == MX_ERR_MEMORY:
            raise MemoryError(message)
        if status == MX_ERR_STATE:
            raise RuntimeError(message)
        raise HipError(message)

    def __getattr__(self, name):
        fn = getattr(self.cdll, "mx_" + name)

        def call(*args):
            status = fn(*args)
            if fn.restype is C.c_int and name not in ("device_count",):
                self.check(status, "mx_" + name)
            return status
        return call


def load() -> Library:
    """Load the built library (raises when it is absent: there is no CPU fallback)."""
    global _lib
    with _lock:
        if _lib is None:
            if not LIB_PATH.exists():
                raise RuntimeError(f"{LIB_PATH} is not built; run `python -m vesper_amd.build` "
                                   "(the HIP path has no fallback)")
            _lib = Library(LIB_PATH)
        return _lib


def ptr(value) -> int | None:
    """Integer device address of a DeviceArray / int / None."""
    if value is None:
        return None
    if isinstance(value, DeviceArray):
        return value.ptr
    return int(value)


class DeviceArray:
    """A device allocation owned by a Context, with a NumPy shape/dtype for transfers."""

    def __init__(self, ctx: "Context", shape, dtype, ptr_value: int):
        self.ctx, self.shape, self.dtype, self.ptr = ctx, tuple(shape), np.dtype(dtype), ptr_value

    @property
    def nbytes(self) -> int:
        return int(np.prod(self.shape, dtype=np.int64)) * self.dtype.itemsize

    def download(self, stream=None) -> np.ndarray:
        return self.ctx.download(self.ptr, self.shape, self.dtype, stream)

    def upload(self, array, stream=None):
        array = np.ascontiguousarray(array, dtype=self.dtype)
        if array.nbytes != self.nbytes:
            raise ValueError("upload size differs from the device array")
        self.ctx.copy_h2d(self.ptr, array, stream)

    def free(self):
        if self.ptr:
            self.ctx.free(self.ptr)
            self.ptr = 0

    def __int__(self):
        return self.ptr


class Context:
    """One device context (the reference's Device, src/vesper/cuda.py:93-191)."""

    def __init__(self, ordinal: int = 0, cap: int = 0):
        self.lib = load()
        handle = C.c_void_p()
        self.lib.create(ordinal, cap, C.byref(handle))
        self.handle, self.ordinal = handle, ordinal

    def _h(self):
        if not self.handle:
            raise RuntimeError("device context is closed")
        return self.handle

    def close(self):
        if self.handle:
            handle, self.handle = self.handle, C.c_void_p()
            self.lib.destroy(handle)

    def __enter__(self):
        return self

    def __exit__(self, *_):
        self.close()

    def device_name(self):
        name, arch = C.create_string_buffer(256), C.create_string_buffer(64)
        self.lib.device_name(self._h(), name, 256, arch, 64)
        return name.value.decode(), arch.value.decode()

    def memory(self) -> dict:
        """{"free", "total"} bytes of the device (Device.memory, cuda.py:115-119)."""
        free, total = C.c_uint64(), C.c_uint64()
        self.lib.device_memory(self._h(), C.byref(free), C.byref(total))
        return {"free": free.value, "total": total.value}

    def malloc(self, nbytes: int) -> int:
        p = C.c_void_p()
        self.lib.malloc(self._h(), int(nbytes), C.byref(p))
        return int(p.value)

    def free(self, p: int):
        self.lib.free(self._h(), C.c_void_p(int(p)))

    def owned_size(self, p: int) -> int:
        """Bytes of the allocation this context owns at base pointer p (0 if none)."""
        size = C.c_uint64()
        self.lib.owned_size(self._h(), C.c_void_p(int(p)), C.byref(size))
        return size.value

    def owned_bytes(self):
        live, peak = C.c_uint64(), C.c_uint64()
        self.lib.owned_bytes(self._h(), C.byref(live), C.byref(peak))
        return live.value, peak.value

    def empty(self, shape, dtype) -> DeviceArray:
        shape = tuple(int(s) for s in np.atleast_1d(shape)) if not isinstance(shape, tuple) else shape
        nbytes = max(int(np.prod(shape, dtype=np.int64)) * np.dtype(dtype).itemsize, 1)
        return DeviceArray(self, shape, dtype, self.malloc(nbytes))

    def upload(self, array, stream=None) -> DeviceArray:
        array = np.ascontiguousarray(array)
        out = self.empty(array.shape, array.dtype)
        self.copy_h2d(out.ptr, array, stream)
        return out

    def copy_h2d(self, dst: int, array: np.ndarray, stream=None):
        array = np.ascontiguousarray(array)
        if array.nbytes:
            self.lib.memcpy_h2d(self._h(), C.c_void_p(int(dst)), array.ctypes.data_as(C.c_void_p), array.nbytes,
                                _stream(stream))
            # pageable source: make the copy complete before the caller may reuse the array
            self.sync(stream)

    def download(self, src: int, shape, dtype, stream=None) -> np.ndarray:
        out = np.empty(shape, dtype=dtype)
        if out.nbytes:
            self.lib.memcpy_d2h(self._h(), out.ctypes.data_as(C.c_void_p), C.c_void_p(int(src)), out.nbytes,
                                _stream(stream))
        return out

    def copy_d2d(self, dst: int, src: int, nbytes: int, stream=None):
        self.lib.memcpy_d2d(self._h(), C.c_void_p(int(dst)), C.c_void_p(int(src)), int(nbytes), _stream(stream))

    def sync(self, stream=None):
        if stream is None:
            self.lib.device_sync(self._h())
        else:
            self.lib.stream_sync(self._h(), _stream(stream))

    def host_alloc_pinned(self, nbytes: int) -> int:
        """Pinned host memory (hipHostMalloc through the context; Pinned, cuda.py:200-222)."""
        p = C.c_void_p()
        self.lib.host_alloc_pinned(self._h(), int(nbytes), C.byref(p))
        return int(p.value)

    def host_free_pinned(self, p: int):
        self.lib.host_free_pinned(self._h(), C.c_void_p(int(p)))

    def stream(self) -> int:
        s = C.c_void_p()
        self.lib.stream_create(self._h(), C.byref(s))
        return int(s.value)

    def destroy_stream(self, s: int):
        self.lib.stream_destroy(self._h(), C.c_void_p(int(s)))

    def event(self) -> int:
        e = C.c_void_p()
        self.lib.event_create(self._h(), C.byref(e))
        return int(e.value)

    def record(self, event: int, stream=None):
        self.lib.event_record(self._h(), C.c_void_p(event), _stream(stream))

    def elapsed_ms(self, start: int, stop: int) -> float:
        ms = C.c_float()
        self.lib.event_sync(self._h(), C.c_void_p(stop))
        self.lib.event_elapsed_ms(self._h(), C.c_void_p(start), C.c_void_p(stop), C.byref(ms))
        return float(ms.value)

    def destroy_event(self, e: int):
        self.lib.event_destroy(self._h(), C.c_void_p(e))

    def fill_uniform_u8(self, dst: int, nbytes: int, seed: int, lo: int, hi: int, stream=None):
        self.lib.fill_uniform_u8(self._h(), C.c_void_p(int(dst)), int(nbytes), int(seed) & (2 ** 64 - 1),
                                 int(lo), int(hi), _stream(stream))


def _stream(stream):
    return None if stream is None else C.c_void_p(int(stream))


def vp(value):
    """ctypes void* of a device address (None stays NULL)."""
    p = ptr(value)
    return None if p is None else C.c_void_p(p)
