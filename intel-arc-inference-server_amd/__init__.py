"""MI355X-native decode loop - host-side Python binding of libmi355x_decode.so.

The product is the HIP library and its C ABI (include/mi355x_decode.h); this module
only loads it with ctypes and declares the signatures. There is no fallback: if the
library is missing, loading fails with an error naming the build step.
"""
import ctypes as C
import os
import re

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(HERE)
LIB_PATH = os.path.join(HERE, "libmi355x_decode.so")
HEADER = os.path.join(ROOT, "include", "mi355x_decode.h")

_lib = None

u8, u16, u32, u64, i32, f32, sz, vp = (C.c_uint8, C.c_uint16, C.c_uint32, C.c_uint64, C.c_int,
                                        C.c_float, C.c_size_t, C.c_void_p)

# name -> (restype, argtypes)
SIGNATURES = {
    "mi_last_error": (C.c_char_p, []),
    "mi_malloc": (i32, [C.POINTER(vp), sz]),
    "mi_free": (i32, [vp]),
    "mi_memcpy_h2d": (i32, [vp, vp, sz, vp]),
    "mi_memcpy_d2h": (i32, [vp, vp, sz, vp]),
    "mi_memcpy_d2d": (i32, [vp, vp, sz, vp]),
    "mi_stream_sync": (i32, [vp]),
    "mi_device_sync": (i32, []),
    "mi_event_create": (i32, [C.POINTER(vp)]),
    "mi_event_record": (i32, [vp, vp]),
    "mi_event_elapsed_ms": (i32, [vp, vp, C.POINTER(f32)]),
    "mi_event_destroy": (i32, [vp]),
    "mi_fill_u32": (i32, [vp, sz, u64, vp]),
    "mi_fill_f16": (i32, [vp, sz, u64, i32, f32, f32, vp]),
    "mi_fill_f32": (i32, [vp, sz, u64, i32, f32, f32, i32, vp]),
    "mi_fill_i8": (i32, [vp, sz, u64, i32, i32, vp]),
    "mi_int4_dequant": (i32, [vp, vp, vp, u32, u32, vp]),
    "mi_gemv_w4a16": (i32, [vp, vp, vp, vp, u32, u32, u32, u32, vp]),
    "mi_gemv_pick_s": (u32, [u32, u32]),
    "mi_fold_partials": (i32, [vp, vp, vp, u32, u32, u32, vp]),
    "mi_stream_read": (i32, [vp, sz, vp, vp]),
}


class MiError(RuntimeError):
    pass


def lib():
    """The loaded library (raises MiError if it has not been built)."""
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            raise MiError(f"{LIB_PATH} is missing: run `python __graft_entry__.py` (build()) first")
        L = C.CDLL(LIB_PATH)
        for name, (res, args) in SIGNATURES.items():
            fn = getattr(L, name)
            fn.restype = res
            fn.argtypes = args
        _lib = L
    return _lib


def check(rc, what=""):
    """Raise MiError on a non-zero return code, with the library's message."""
    if rc != 0:
        msg = lib().mi_last_error().decode(errors="replace")
        raise MiError(f"{what or 'call'} failed ({rc}): {msg}")
    return rc


def call(name, *args):
    return check(getattr(lib(), name)(*args), name)


def header_functions():
    """Every function the public header declares (for the export check)."""
    with open(HEADER) as f:
        text = f.read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(mi_[a-z0-9_]+)\s*\(", text)))
