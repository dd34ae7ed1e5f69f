"""ctypes binding of the gfx950 HIP backend (include/kansai_hip.h).

The reference binds its C++ backends with nanobind (python/bindings.cpp of
the reference); nanobind is not installed in this image, so the same C ABI
is bound with the standard library's ctypes, which releases the GIL around
every foreign call (the reference releases it with gil_scoped_release,
python/bindings.cpp:237-271).

Status codes map to the exceptions the reference raises for the same
conditions: a NaN/inf reaching a quantizer -> ValueError (round(nan) in
python/kansai/quantize.py:69); allocation failure -> MemoryError
(std::bad_alloc from core/src/Storage.cpp:30); anything else ->
RuntimeError (the std::runtime_error of the reference backends).

There is no CPU fallback: if the library is missing or no gfx950 device is
present, every entry point raises.
"""

from __future__ import annotations

import ctypes
import os
import threading

_HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(_HERE, "lib", "libkansai_hip.so")

KH_OK = 0
KH_ERR_NO_DEVICE = 1
KH_ERR_INVALID_ARG = 2
KH_ERR_OOM = 3
KH_ERR_NONFINITE = 4
KH_ERR_HIP = 5

_vp = ctypes.c_void_p
_i64 = ctypes.c_int64
_int = ctypes.c_int
_size = ctypes.c_size_t
_dbl = ctypes.c_double

# name -> argtypes (all return int status unless listed in _RESTYPES)
_SIGNATURES = {
    "kh_available": [],
    "kh_init": [_int],
    "kh_last_error": [],
    "kh_device_info": [ctypes.c_char_p, _size, ctypes.POINTER(_int), ctypes.POINTER(_int), ctypes.POINTER(_int),
                       ctypes.POINTER(_int), ctypes.POINTER(_size)],
    "kh_synchronize": [],
    "kh_get_stream": [ctypes.POINTER(_vp)],
    "kh_alloc": [_size, ctypes.POINTER(_vp)],
    "kh_free": [_vp],
    "kh_pool_trim": [],
    "kh_pool_stats": [ctypes.POINTER(_size), ctypes.POINTER(_size), ctypes.POINTER(_size)],
    "kh_pool_requests": [ctypes.POINTER(_size)],
    "kh_scratch_stats": [ctypes.POINTER(_size), ctypes.POINTER(_size), ctypes.POINTER(_size)],
    "kh_memcpy_h2d": [_vp, _vp, _size],
    "kh_memcpy_d2h": [_vp, _vp, _size],
    "kh_memcpy_d2d": [_vp, _vp, _size],
    "kh_event_create": [ctypes.POINTER(_vp)],
    "kh_event_record": [_vp],
    "kh_event_elapsed_ms": [_vp, _vp, ctypes.POINTER(ctypes.c_float)],
    "kh_event_destroy": [_vp],
    "kh_graph_capture_begin": [],
    "kh_graph_capture_end": [ctypes.POINTER(_vp)],
    "kh_graph_launch": [_vp],
    "kh_graph_destroy": [_vp],
    "kh_quantize_tensor": [_vp, _i64, _vp, _vp],
    "kh_quantize_rows": [_vp, _i64, _i64, _vp, _vp],
    "kh_quantize_cols_packed": [_vp, _i64, _i64, _vp, _vp],
    "kh_quantize_tensor_packed": [_vp, _i64, _i64, _vp, _vp],
    "kh_dequantize_tensor": [_vp, _i64, _vp, _vp],
    "kh_dequantize_rows": [_vp, _i64, _i64, _vp, _vp],
    "kh_dequantize_packed": [_vp, _i64, _i64, _vp, _i64, _vp],
    "kh_dequantize_acc": [_vp, _i64, _i64, _vp, _int, _vp, _int, _vp, _vp],
    "kh_gemm_i8": [_vp, _vp, _i64, _i64, _i64, _vp, _int, _vp, _int, _vp, _vp, _vp],
    "kh_gemm_i8_ex": [_vp, _vp, _i64, _i64, _i64, _vp, _int, _vp, _int, _vp, _int, _vp, _vp, _vp, _int,
                      ctypes.POINTER(ctypes.c_int)],
    "kh_gemm_i8_quant": [_vp, _vp, _i64, _i64, _i64, _vp, _int, _vp, _int, _vp, _int, _vp, _vp, _vp],
    "kh_gemm_i8_quant_rows": [_vp, _vp, _i64, _i64, _i64, _vp, _int, _vp, _int, _vp, _int, _vp, _vp],
    "kh_gemm_i8_qload": [_vp, _i64, _i64, _i64, _vp, _int, _vp, _vp, _int, _vp, _int, _vp, _vp, _vp, _vp, _int,
                         ctypes.POINTER(ctypes.c_int)],
    "kh_gemm_i8_qload_rows": [_vp, _i64, _i64, _i64, _vp, _int, _vp, _vp, _int, _vp, _int, _vp, _vp, _vp],
    "kh_absmax_parts": [_vp, _i64, _vp, _int, ctypes.POINTER(ctypes.c_int)],
    "kh_quantize_tensor_parts": [_vp, _i64, _vp, _int, _vp, _vp],
    "kh_layernorm_ex": [_vp, _i64, _int, _vp, _vp, ctypes.c_float, _vp, _vp, _int, ctypes.POINTER(ctypes.c_int)],
    "kh_layernorm_quant": [_vp, _i64, _int, _vp, _vp, ctypes.c_float, _vp, _vp],
    "kh_causal_attention_ex": [_vp, _int, _int, _int, _int, _vp, _vp, _int, ctypes.POINTER(ctypes.c_int)],
    "kh_layernorm_quant_rows": [_vp, _i64, _int, _vp, _vp, ctypes.c_float, _vp, _vp],
    "kh_attention_ex": [_vp, _int, _int, _int, _int, _int, _vp, _vp, _int, ctypes.POINTER(ctypes.c_int)],
    "kh_attention_rows": [_vp, _int, _int, _int, _int, _int, _vp, _vp],
    "kh_attention_masked": [_vp, _int, _int, _int, _int, _int, _vp, _i64, _i64, _i64, _i64, _vp, _vp],
    "kh_linear_i8": [_vp, _i64, _i64, _vp, _i64, _vp, _int, _vp, _vp, _vp, _vp],
    "kh_linear_i8_noalloc": [_vp, _i64, _i64, _vp, _i64, _vp, _int, _vp, _vp],
    "kh_linear_i8_tensor": [_vp, _i64, _i64, _vp, _i64, _vp, _int, _vp, _vp, _vp, _vp],
    "kh_matmul_f32": [_vp, _vp, _vp, _i64, _i64, _i64, _vp],
    "kh_probe_mfma_i8": [_vp, _i64, _i64, ctypes.POINTER(ctypes.c_double), ctypes.POINTER(ctypes.c_double)],
    "kh_probe_stream_read": [_vp, _i64],
    "kh_add": [_vp, _vp, _vp, _i64],
    "kh_add_bias": [_vp, _vp, _vp, _i64, _i64, _int],
    "kh_relu": [_vp, _vp, _i64],
    "kh_embedding": [_vp, _i64, _int, _vp, _int, _vp, _int, _vp],
    "kh_layernorm": [_vp, _i64, _int, _vp, _vp, ctypes.c_float, _vp],
    "kh_gelu": [_vp, _vp, _i64],
    "kh_causal_attention": [_vp, _int, _int, _int, _int, _vp],
}
_RESTYPES = {"kh_last_error": ctypes.c_char_p}

_lib = None
_lock = threading.Lock()


class HipUnavailable(RuntimeError):
    """The HIP library or a gfx950 device is missing."""


def exported_symbols():
    """Every entry point include/kansai_hip.h declares (checked by tests)."""
    return list(_SIGNATURES)


def load_library(path: str = LIB_PATH):
    """Loads the shared library (without touching the GPU)."""
    global _lib
    with _lock:
        if _lib is None:
            if not os.path.exists(path):
                raise HipUnavailable(f"{path} is missing: build it with `python -m kansaiml_amd.build`")
            lib = ctypes.CDLL(path)
            for name, args in _SIGNATURES.items():
                fn = getattr(lib, name)
                fn.argtypes = args
                fn.restype = _RESTYPES.get(name, _int)
            _lib = lib
    return _lib


def lib():
    return _lib if _lib is not None else load_library()


def last_error() -> str:
    msg = lib().kh_last_error()
    return msg.decode() if msg else ""


def check(rc: int, what: str = ""):
    if rc == KH_OK:
        return
    msg = last_error() or what
    if rc == KH_ERR_NONFINITE:
        raise ValueError(msg)
    if rc == KH_ERR_OOM:
        raise MemoryError(msg)
    if rc == KH_ERR_NO_DEVICE:
        raise HipUnavailable(msg)
    raise RuntimeError(msg)


def call(name: str, *args):
    """Calls an entry point and raises on a nonzero status."""
    check(getattr(lib(), name)(*args), name)


def available() -> bool:
    """kan::metal::available()'s counterpart: never raises."""
    try:
        return bool(lib().kh_available())
    except Exception:
        return False


def synchronize():
    call("kh_synchronize")


def device_info() -> dict:
    name = ctypes.create_string_buffer(64)
    cus, clk, mclk, bus = _int(), _int(), _int(), _int()
    mem = _size()
    call("kh_device_info", name, 64, ctypes.byref(cus), ctypes.byref(clk), ctypes.byref(mclk), ctypes.byref(bus),
         ctypes.byref(mem))
    return {"arch": name.value.decode(), "cus": cus.value, "clock_khz": clk.value, "mem_clock_khz": mclk.value,
            "bus_width": bus.value, "total_mem": mem.value}


def pool_stats() -> dict:
    a, b, c, r = _size(), _size(), _size(), _size()
    call("kh_pool_stats", ctypes.byref(a), ctypes.byref(b), ctypes.byref(c))
    call("kh_pool_requests", ctypes.byref(r))
    return {"in_use": a.value, "cached": b.value, "driver_allocs": c.value, "requests": r.value}


def scratch_stats() -> dict:
    a, b, c = _size(), _size(), _size()
    call("kh_scratch_stats", ctypes.byref(a), ctypes.byref(b), ctypes.byref(c))
    return {"bytes": a.value, "requests": b.value, "driver_allocs": c.value}


class Event:
    """A HIP event recorded on the library stream (kernel timing)."""

    def __init__(self):
        p = _vp()
        call("kh_event_create", ctypes.byref(p))
        self.ptr = p

    def record(self):
        call("kh_event_record", self.ptr)

    def elapsed_ms(self, end: "Event") -> float:
        ms = ctypes.c_float()
        call("kh_event_elapsed_ms", self.ptr, end.ptr, ctypes.byref(ms))
        return ms.value

    def __del__(self):
        try:
            if self.ptr:
                _lib.kh_event_destroy(self.ptr)
        except Exception:
            pass
