"""ctypes binding of libtrellis_sparse.so (C ABI in include/tsc.h).

The library is loaded from this package directory.  If it is missing the import of any op fails
loudly: there is no CPU fallback behind this API.
"""
from __future__ import annotations

import ctypes
import re
import threading
from pathlib import Path

PKG_DIR = Path(__file__).resolve().parent
LIB_PATH = PKG_DIR / "libtrellis_sparse.so"
HEADER_PATH = PKG_DIR.parent / "include" / "tsc.h"

TSC_OK, TSC_ERR_INVALID, TSC_ERR_UNSUPPORTED, TSC_ERR_HIP, TSC_ERR_OOM = range(5)
TSC_F32, TSC_F16, TSC_BF16 = 0, 1, 2
TSC_MAP_DUPLICATE, TSC_MAP_OUT_OF_RANGE = 1, 2
TSC_MAP_AUTO, TSC_MAP_BITMAP, TSC_MAP_RADIX = 0, 1, 2
TSC_EPI_BIAS, TSC_EPI_BIAS_RESIDUAL, TSC_EPI_BIAS_LN_SILU = 0, 1, 2
TSC_ST_RAW = -1
# safetensors header dtype strings in tsc_st_dtype order, with their element sizes
ST_DTYPES = ("F32", "F16", "BF16", "F64", "I64", "I32", "I16", "I8", "U8", "BOOL", "U16", "U32",
             "U64", "F8_E4M3", "F8_E5M2")
ST_SIZES = (4, 2, 2, 8, 8, 4, 2, 1, 1, 1, 2, 4, 8, 1, 1)

MAP_METHODS = {"auto": TSC_MAP_AUTO, "bitmap": TSC_MAP_BITMAP, "radix": TSC_MAP_RADIX}


class TscError(RuntimeError):
    """A libtrellis_sparse call returned a non-zero status."""

    def __init__(self, status: int, message: str):
        super().__init__(f"[tsc status {status}] {message}")
        self.status = status


_lib = None
_lock = threading.Lock()

_P = ctypes.c_void_p
_I32 = ctypes.c_int32
_I64 = ctypes.c_int64
_F32 = ctypes.c_float
_SZ = ctypes.c_size_t

_SIGNATURES = {
    "tsc_version": (_I32, []),
    "tsc_last_error": (ctypes.c_char_p, []),
    "tsc_ctx_create": (_I32, [_I32, _P, ctypes.POINTER(_P)]),
    "tsc_ctx_destroy": (_I32, [_P]),
    "tsc_ctx_set_stream": (_I32, [_P, _P]),
    "tsc_ctx_stream": (_P, [_P]),
    "tsc_sync": (_I32, [_P]),
    "tsc_malloc": (_I32, [_P, _SZ, ctypes.POINTER(_P)]),
    "tsc_free": (_I32, [_P, _P]),
    "tsc_memcpy_h2d": (_I32, [_P, _P, _P, _SZ]),
    "tsc_memcpy_d2h": (_I32, [_P, _P, _P, _SZ]),
    "tsc_memset_zero": (_I32, [_P, _P, _SZ]),
    "tsc_map_key_bytes": (_I32, [_I32, _I32, _I32, _I32]),
    "tsc_map_build": (_I32, [_P, _P, _I64, _I32, _I32, _I32, _I32, _P, _P, _I32, _P, _P, _P, _P]),
    "tsc_map_write_floor": (_I32, [_P, _P, _I64, _P]),
    "tsc_map_conv_order": (_I32, [_P, _P, _P, _I64, _P]),
    "tsc_map_gather_plan_bytes": (_I64, [_I64]),
    "tsc_map_gather_plan": (_I32, [_P, _P, _P, _I64, _I32, _I32, _I32, _I32, _P]),
    "tsc_conv_planned": (_I32, [_P, _I32, _P, _P, _P, _P, _P, _I64, _I32, _I32, _I32, _P, _P, _P,
                                _F32, _P]),
    "tsc_conv": (_I32, [_P, _I32, _P, _P, _P, _P, _P, _I64, _I32, _I32, _P]),
    "tsc_conv_fused": (_I32, [_P, _I32, _P, _P, _P, _P, _P, _I64, _I32, _I32, _I32, _P, _P, _P,
                              _F32, _P]),
    "tsc_conv_fused_noalloc": (_I32, [_P, _I32, _P, _P, _P, _P, _P, _I64, _I32, _I32, _I32, _P, _P,
                                      _P, _F32, _P]),
    "tsc_layernorm": (_I32, [_P, _I32, _P, _I64, _I32, _P, _P, _F32, _I32, _P]),
    "tsc_silu": (_I32, [_P, _I32, _P, _I64, _P]),
    "tsc_add": (_I32, [_P, _I32, _P, _P, _I64, _P]),
    "tsc_resblock": (_I32, [_P, _I32, _P, _P, _P, _I64, _I32, _P, _P, _P, _P, _F32, _P, _P, _P]),
    "tsc_linear": (_I32, [_P, _I32, _P, _I64, _I32, _P, _P, _P, _I32, _P]),
    "tsc_subdivide_count": (_I32, [_P, _P, _I64, ctypes.POINTER(_I64)]),
    "tsc_subdivide": (_I32, [_P, _P, _I64, _I32, _P, _I32, _P, _P, _P]),
    "tsc_attention": (_I32, [_P, _I32, _P, _P, _P, _P, _P, _I32, _I64, _I64, _I32, _I32, _F32,
                             _I32, _P]),
    "tsc_st_open": (_I32, [ctypes.c_char_p, ctypes.POINTER(_P)]),
    "tsc_st_close": (_I32, [_P]),
    "tsc_st_counts": (_I32, [_P, ctypes.POINTER(_I64), ctypes.POINTER(_I64), ctypes.POINTER(_I64)]),
    "tsc_st_name": (_I32, [_P, _I64, ctypes.c_char_p, _I32]),
    "tsc_st_metadata": (_I32, [_P, _I64, ctypes.c_char_p, _I32, ctypes.c_char_p, _I32]),
    "tsc_st_info": (_I32, [_P, ctypes.c_char_p, ctypes.POINTER(_I32), ctypes.POINTER(_I32),
                           ctypes.POINTER(_I64), _I32, ctypes.POINTER(_I64)]),
    "tsc_st_load": (_I32, [_P, _P, ctypes.c_char_p, _I32, _P]),
    "tsc_profile_enable": (_I32, [_P, _I32]),
    "tsc_profile_collect": (_I32, [_P, ctypes.POINTER(_I32)]),
    "tsc_profile_entry": (_I32, [_P, _I32, ctypes.c_char_p, _I32, ctypes.POINTER(ctypes.c_double),
                                 ctypes.POINTER(_I64)]),
    "tsc_profile_reset": (_I32, [_P]),
}


def header_symbols() -> list[str]:
    """Names of every function declared in include/tsc.h."""
    text = HEADER_PATH.read_text()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(tsc_[a-z0-9_]+)\s*\(", text)))


def load_library():
    """Load libtrellis_sparse.so and declare its C signatures (no GPU call is made)."""
    global _lib
    with _lock:
        if _lib is not None:
            return _lib
        if not LIB_PATH.exists():
            raise TscError(TSC_ERR_UNSUPPORTED,
                           f"{LIB_PATH} is not built; run __graft_entry__.build() or build.py")
        lib = ctypes.CDLL(str(LIB_PATH))
        for name, (res, args) in _SIGNATURES.items():
            fn = getattr(lib, name)
            fn.restype = res
            fn.argtypes = args
        _lib = lib
        return lib


def check(status: int) -> None:
    if status != TSC_OK:
        msg = _lib.tsc_last_error().decode(errors="replace") if _lib is not None else ""
        raise TscError(status, msg)


class Context:
    """One tsc_ctx per device, following torch's current stream on that device."""

    def __init__(self, device: int):
        import torch

        self.lib = load_library()
        self.device = device
        stream = torch.cuda.current_stream(device).cuda_stream
        h = _P()
        check(self.lib.tsc_ctx_create(device, _P(stream), ctypes.byref(h)))
        self.handle = h
        self._stream = stream

    def bind(self):
        """Point the context at torch's current stream; returns the raw handle."""
        import torch

        s = torch.cuda.current_stream(self.device).cuda_stream
        if s != self._stream:
            check(self.lib.tsc_ctx_set_stream(self.handle, _P(s)))
            self._stream = s
        return self.handle

    def sync(self):
        check(self.lib.tsc_sync(self.handle))

    def profile(self, on: bool) -> None:
        """Bracket every kernel this context launches with hipEvents (per-kernel timing)."""
        check(self.lib.tsc_profile_enable(self.handle, int(on)))

    def profile_results(self) -> dict:
        """{kernel name: (total ms, launches)} over the launches since the last reset."""
        n = _I32()
        check(self.lib.tsc_profile_collect(self.handle, ctypes.byref(n)))
        out = {}
        buf = ctypes.create_string_buffer(256)
        ms, cnt = ctypes.c_double(), _I64()
        for i in range(n.value):
            check(self.lib.tsc_profile_entry(self.handle, i, buf, 256, ctypes.byref(ms), ctypes.byref(cnt)))
            out[buf.value.decode()] = (ms.value, cnt.value)
        return out

    def profile_reset(self) -> None:
        check(self.lib.tsc_profile_reset(self.handle))


_contexts: dict[int, Context] = {}


def context(device: int) -> Context:
    with _lock:
        ctx = _contexts.get(device)
    if ctx is None:
        ctx = Context(device)
        with _lock:
            _contexts[device] = ctx
    return ctx
