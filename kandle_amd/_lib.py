"""ctypes binding of libkandle_hip.so (the C ABI declared in include/kandle_hip.h).

Loading fails loudly: there is no CPU or PyTorch fallback anywhere in kandle_amd.  Every wrapper
checks the return code and raises KandleHipError with the library's error text.
"""
from __future__ import annotations

import ctypes as C
from pathlib import Path

LIB_PATH = Path(__file__).resolve().parent / "libkandle_hip.so"

KH_F32, KH_BF16, KH_I32 = 0, 1, 2


class KandleHipError(RuntimeError):
    """A HIP backend call failed (bad argument, HIP runtime error, or out of memory)."""


class AllocStats(C.Structure):
    _fields_ = [
        ("live_bytes", C.c_uint64),
        ("cached_bytes", C.c_uint64),
        ("peak_bytes", C.c_uint64),
        ("n_device_allocs", C.c_uint64),
        ("n_cache_hits", C.c_uint64),
    ]


# name -> (restype, argtypes); every entry point returns int (0 = success) unless stated.
_vp, _i, _i64, _f, _sz = C.c_void_p, C.c_int, C.c_int64, C.c_float, C.c_size_t
_i64p = C.POINTER(C.c_int64)
_vpp = C.POINTER(C.c_void_p)
SIGNATURES = {
    "kh_init": [_i],
    "kh_device_count": [C.POINTER(C.c_int)],
    "kh_set_debug": [_i],
    "kh_is_capturing": [],
    "kh_alloc": [C.POINTER(C.c_void_p), _sz],
    "kh_free": [_vp],
    "kh_empty_cache": [],
    "kh_get_alloc_stats": [C.POINTER(AllocStats)],
    "kh_memcpy_h2d": [_vp, _vp, _sz],
    "kh_memcpy_d2h": [_vp, _vp, _sz],
    "kh_memcpy_d2d": [_vp, _vp, _sz],
    "kh_synchronize": [],
    "kh_event_create": [C.POINTER(C.c_void_p)],
    "kh_event_destroy": [_vp],
    "kh_event_record": [_vp],
    "kh_event_elapsed_ms": [_vp, _vp, C.POINTER(C.c_float)],
    "kh_fill": [_vp, _i64, _f, _i],
    "kh_copy_strided": [_vp, _i64, _vp, _i, _i64p, _i64p, _i, _i],
    "kh_binary": [_i, _vp, _vp, _vp, _i64, _i],
    "kh_map_strided": [_i, _i, _i64p, _vp, _i64p, _i, _vp, _i64p, _i, _vp, _i64p, _i, C.c_double, C.c_double],
    "kh_silu": [_vp, _vp, _i64, _i],
    "kh_silu_mul": [_vp, _i64, _vp, _i64, _vp, _i64, _i64, _i64, _i],
    "kh_index_select": [_vp, _i64, _vp, _i64, _i64, _vp, _i, _i],
    "kh_index_select_dim": [_vp, _i64, _i64, _i64, _vp, _i64, _vp, _i, _i],
    "kh_argmax": [_vp, _i64, _i64, _vp, _i],
    "kh_rms_norm": [_vp, _i64, _vp, _vp, _i64, _i64, _i64, _f, _i, _i],
    "kh_qk_norm_rope": [_vp, _vp, _vp, _vp, _vp, _vp, _vp, _vp, _vp, _vp, _i64, _i64, _i, _i, _i, _i64p, _f, _i,
                        _i64],
    "kh_greedy_advance": [_vp, _vp, _vp, _vp, _i64, _i64],
    "kh_sample": [_vp, _i64, _i, C.c_double, _i, C.c_double, C.c_uint64, _vp, _vp, _vp, _i, _vp, _vp],
    "kh_philox4x32_10": [C.c_uint64, _vp, _i64, _vp],
    "kh_sample_set_path": [_i],
    "kh_decode_attention_block": [_vp, _vp, _vp, _vp, _f, _vp, _vp, _vp, _i, _i, _i64, _vp, _f, _vp, _i64, _i64,
                                  _vp, _i],
    "kh_graph_begin_capture": [],
    "kh_graph_end_capture": [_vpp],
    "kh_graph_launch": [_vp],
    "kh_graph_destroy": [_vp],
    "kh_unary": [_i, _vp, _vp, _i64, _i],
    "kh_arange": [_vp, _i64, C.c_double, C.c_double, _i],
    "kh_flash_attention": [_vp, _vp, _vp, _vp, _i, _i, _i, _i64, _i64, _i, _i64p, _f, _i, _i],
    "kh_flash_attention_split": [_vp, _vp, _vp, _vp, _i, _i, _i, _i64, _i64, _i, _i64p, _f, _i],
    "kh_flash_attention_masked": [_vp, _vp, _vp, _vp, _i, _i, _i, _i64, _i64, _i, _i64p, _f, _vp, _i64p, _i, _i],
    "kh_decode_attention": [_vp, _vp, _vp, _vp, _vp, _i, _i, _i, _i, _i64, _i64p, _f, _i],
    "kh_decode_attention_noalloc": [_vp, _vp, _vp, _vp, _vp, _i, _i, _i, _i, _i64, _i64p, _f, _i],
    "kh_gemm": [_vp, _i64, _vp, _i64, _vp, _i64, _vp, _i64, _vp, _i64, _i64, _i64, _f, _f, _i, _i, _i],
    "kh_gemm_ex": [_vp, _i64, _i, _vp, _i64, _i, _vp, _i64, _vp, _i64, _vp, _i64, _i64, _i64, _f, _f, _i, _i],
    "kh_gemv_fused": [_i, _vp, _vp, _vp, _f, _vp, _i64, _vp, _vp, _vp, _i64, _i64, _f, _f, _i, _i],
    "kh_gemv_swiglu": [_i, _vp, _vp, _f, _vp, _i64, _vp, _i64, _i64, _i],
    "kh_gemm_swiglu": [_vp, _i64, _vp, _i64, _vp, _i64, _i64, _i64, _i64, _i],
    "kh_gemm_qk_norm_rope": [_vp, _i64, _vp, _i64, _i64, _i64, _i64, _i, _i, _i, _vp, _vp, _vp, _vp, _vp, _vp, _vp,
                             _i64p, _f, _i64, _i],
    "kh_gemm_qk_norm_rope_table": [_vp, _i64, _vp, _i64, _i64, _i64, _i64, _i, _i, _i, _vp, _vp, _vp, _vp, _vp, _vp,
                                   _vp, _i64p, _f, _i64, _i, _vp],
    "kh_rope_table": [_vp, _i64, _vp, _i, _vp],
    "kh_gemm_split_count": [_i64, _i64, _i64, C.POINTER(C.c_int)],
    "kh_gemm_splitk_partials": [_vp, _i64, _vp, _i64, _vp, _i64, _i64, _i64, _i, _i],
    "kh_add_rms_norm": [_vp, _i, _i64, _vp, _vp, _vp, _i64, _i64, _f, _i],
}

_lib = None


def load() -> C.CDLL:
    """Load libkandle_hip.so once; raise if it has not been built."""
    global _lib
    if _lib is None:
        if not LIB_PATH.exists():
            raise KandleHipError(
                f"{LIB_PATH} is missing: build it with `python -m kandle_amd.build` (there is no fallback path)"
            )
        L = C.CDLL(str(LIB_PATH))
        for name, argtypes in SIGNATURES.items():
            fn = getattr(L, name)
            fn.argtypes = argtypes
            fn.restype = C.c_int
        L.kh_last_error.argtypes = []
        L.kh_last_error.restype = C.c_char_p
        _lib = L
    return _lib


def check(rc: int, what: str = "") -> None:
    if rc != 0:
        msg = load().kh_last_error().decode(errors="replace")
        raise KandleHipError(f"{what or 'kandle_hip'} failed (code {rc}): {msg}")


def call(name: str, *args) -> None:
    """Call an entry point and raise on a non-zero return code."""
    check(getattr(load(), name)(*args), name)


def is_capturing() -> bool:
    """True while a graph capture is open on the library stream (kh_is_capturing)."""
    return bool(load().kh_is_capturing())


def i64_array(values) -> C.Array:
    vals = [int(v) for v in values]
    return (C.c_int64 * max(1, len(vals)))(*vals)


def device_count() -> int:
    n = C.c_int(0)
    call("kh_device_count", C.byref(n))
    return n.value


_initialized_device = None


def init(device: int = 0) -> None:
    global _initialized_device
    if _initialized_device is None:
        call("kh_init", int(device))
        _initialized_device = int(device)
    elif _initialized_device != device:
        raise KandleHipError(f"already initialised on device {_initialized_device}")


def is_initialized() -> bool:
    return _initialized_device is not None


def alloc(nbytes: int) -> int:
    p = C.c_void_p()
    call("kh_alloc", C.byref(p), int(nbytes))
    return int(p.value or 0)


def free(ptr: int) -> None:
    call("kh_free", C.c_void_p(ptr))


def alloc_stats() -> dict:
    s = AllocStats()
    call("kh_get_alloc_stats", C.byref(s))
    return {f: int(getattr(s, f)) for f, _ in AllocStats._fields_}


def synchronize() -> None:
    call("kh_synchronize")


class Event:
    """A HIP event recorded on the library stream (for timing)."""

    def __init__(self):
        p = C.c_void_p()
        call("kh_event_create", C.byref(p))
        self.handle = p

    def record(self) -> None:
        call("kh_event_record", self.handle)

    def elapsed_ms(self, end: "Event") -> float:
        ms = C.c_float(0.0)
        call("kh_event_elapsed_ms", self.handle, end.handle, C.byref(ms))
        return float(ms.value)

    def __del__(self):
        try:
            if self.handle and _lib is not None:
                _lib.kh_event_destroy(self.handle)
        except Exception:
            pass


def init_check() -> None:
    """Raise unless the library has been initialised on a device."""
    if _initialized_device is None:
        raise KandleHipError("the HIP backend is not initialised: call HipBackend.create() first")
