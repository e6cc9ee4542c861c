"""ctypes binding of libtriton_llm_hip.so (the C ABI in include/triton_llm_hip.h).

This module only loads the library and declares argument types; it performs
no GPU call on import.  The library is looked up in-tree
(``triton_llm/_lib/libtriton_llm_hip.so``) or at ``$TRITON_LLM_HIP_LIB``.
There is no fallback implementation: if the library is missing, every entry
point raises.
"""

from __future__ import annotations

import ctypes
import os

from ._build import LIB_PATH

DTYPE_F32 = 0
DTYPE_F16 = 1
DTYPE_BF16 = 2

_c_int = ctypes.c_int
_c_i64 = ctypes.c_int64
_c_size = ctypes.c_size_t
_c_float = ctypes.c_float
_vp = ctypes.c_void_p
_i64p = ctypes.POINTER(ctypes.c_int64)

# name -> (restype, argtypes).  Kept in the order of include/triton_llm_hip.h.
SIGNATURES: dict[str, tuple[object, list[object]]] = {
    "tl_device_count": (_c_int, [ctypes.POINTER(_c_int)]),
    "tl_init": (_c_int, [_c_int]),
    "tl_default_stream": (_vp, []),
    "tl_malloc": (_c_int, [ctypes.POINTER(_vp), _c_size]),
    "tl_free": (_c_int, [_vp]),
    "tl_memcpy_htod": (_c_int, [_vp, _vp, _c_size]),
    "tl_memcpy_dtoh": (_c_int, [_vp, _vp, _c_size]),
    "tl_memcpy_dtod": (_c_int, [_vp, _vp, _c_size]),
    "tl_memset": (_c_int, [_vp, _c_int, _c_size]),
    "tl_synchronize": (_c_int, []),
    "tl_error_string": (ctypes.c_char_p, [_c_int]),
    "tl_event_create": (_c_int, [ctypes.POINTER(_vp)]),
    "tl_event_destroy": (_c_int, [_vp]),
    "tl_event_record": (_c_int, [_vp, _vp]),
    "tl_event_synchronize": (_c_int, [_vp]),
    "tl_event_elapsed_ms": (_c_int, [ctypes.POINTER(_c_float), _vp, _vp]),
    "tl_graph_capture_begin": (_c_int, [_vp]),
    "tl_graph_capture_end": (_c_int, [_vp, ctypes.POINTER(_vp)]),
    "tl_graph_launch": (_c_int, [_vp, _vp]),
    "tl_graph_destroy": (_c_int, [_vp]),
    "tl_rope_inplace": (
        _c_int,
        [_vp, _vp, _vp, _c_i64, _c_i64, _c_int, _c_int, _c_int, _c_int, _vp],
    ),
    "tl_attention_fwd_workspace_bytes": (_c_size, [_c_int, _c_int, _c_int, _c_int, _c_int]),
    "tl_attention_fwd_workspace_bytes_split": (
        _c_size, [_c_int, _c_int, _c_int, _c_int, _c_int, _c_int, _c_int, _c_int]),
    "tl_attention_fwd": (
        _c_int,
        [_vp, _vp, _vp, _vp, _vp, _c_size,
         _c_int, _c_int, _c_int, _c_int, _c_int, _c_int,
         _i64p, _i64p, _i64p, _i64p,
         _c_float, _c_int, _c_int, _vp],
    ),
    "tl_decode_split_size": (_c_int, [_c_int, _c_int, _c_int]),
    "tl_attention_decode_workspace_bytes": (_c_size, [_c_int, _c_int, _c_int, _c_int, _c_int]),
    "tl_attention_decode": (
        _c_int,
        [_vp, _vp, _vp, _vp, _c_int, _vp, _vp, _c_size,
         _c_int, _c_int, _c_int, _c_int, _c_int,
         _i64p, _i64p, _i64p, _i64p,
         _c_float, _c_int, _c_int, _vp],
    ),
    "tl_attention_decode_append": (
        _c_int,
        [_vp, _vp, _vp, _vp, _vp, _vp, _vp, _vp, _c_int, _vp, _vp, _c_size,
         _c_int, _c_int, _c_int, _c_int, _c_int,
         _i64p, _i64p, _i64p, _i64p, _i64p, _i64p,
         _c_float, _c_int, _c_int, _vp],
    ),
    "tl_attention_decode_noalloc": (
        _c_int,
        [_vp, _vp, _vp, _vp, _c_int, _vp,
         _c_int, _c_int, _c_int, _c_int, _c_int,
         _i64p, _i64p, _i64p, _i64p,
         _c_float, _c_int, _c_int, _vp],
    ),
    "tl_rope_kv_append": (
        _c_int,
        [_vp, _vp, _vp, _vp, _vp, _vp, _vp, _vp,
         _c_int, _c_int, _c_int, _c_int, _c_int, _c_int, _c_int,
         _i64p, _i64p, _i64p, _i64p, _i64p, _c_int, _vp],
    ),
    "tl_rms_norm": (_c_int, [_vp, _vp, _vp, _c_int, _c_int, _c_float, _c_int, _vp]),
    "tl_add_rms_norm": (_c_int, [_vp, _vp, _vp, _vp, _vp, _c_int, _c_int, _c_float, _c_int, _vp]),
    "tl_swiglu": (_c_int, [_vp, _vp, _vp, ctypes.c_int64, _c_int, _vp]),
    "tl_add": (_c_int, [_vp, _vp, _vp, ctypes.c_int64, _c_int, _vp]),
    "tl_gemm_workspace_bytes": (_c_size, [_c_int, _c_int, _c_int, _c_int]),
    "tl_gemm": (
        _c_int,
        [_vp, _vp, _vp, _c_int, _c_int, _c_int, ctypes.c_int64, ctypes.c_int64, ctypes.c_int64,
         _vp, _c_size, _c_int, _vp],
    ),
    "tl_gemm_grouped_workspace_bytes": (_c_size, [_c_int, _c_int, _c_int, ctypes.POINTER(_c_int), _c_int]),
    "tl_gemm_grouped": (
        _c_int,
        [_vp, _c_int, _c_int, ctypes.c_int64, _c_int, ctypes.POINTER(_vp), ctypes.POINTER(_vp),
         ctypes.POINTER(_c_int), _i64p, _i64p, _vp, _c_size, _c_int, _vp],
    ),
    "tl_sample_max_vocab": (_c_int, []),
    "tl_sample_workspace_bytes": (_c_size, [_c_int, _c_int]),
    "tl_sample": (_c_int, [_vp, _c_int, _c_int, _c_i64, _c_float, _c_int, _vp, _vp, _vp, _c_size, _c_int, _vp]),
    "tl_sample_row": (_c_int, [_vp, _c_int, _c_float, _c_int, ctypes.c_double, _vp, _vp, _c_size, _c_int, _vp]),
}

_lib: ctypes.CDLL | None = None


def library_path() -> str:
    return os.environ.get("TRITON_LLM_HIP_LIB", LIB_PATH)


def load() -> ctypes.CDLL:
    """Load the HIP library (once) and declare every exported signature."""
    global _lib
    if _lib is not None:
        return _lib
    path = library_path()
    if not os.path.exists(path):
        raise RuntimeError(
            f"triton_llm HIP library not found at {path}; build it with "
            "`python -c 'import __graft_entry__; __graft_entry__.build()'` "
            "(hipcc, gfx950). There is no CPU fallback."
        )
    lib = ctypes.CDLL(path)
    for name, (res, args) in SIGNATURES.items():
        fn = getattr(lib, name)  # AttributeError if the symbol is missing
        fn.restype = res
        fn.argtypes = args
    _lib = lib
    return lib


def noalloc_scratch_bytes() -> int:
    """Size of tl_attention_decode_noalloc's static scratch, read from the
    loaded library's data symbol (the header's
    TL_DECODE_NOALLOC_SCRATCH_BYTES)."""
    return int(ctypes.c_size_t.in_dll(load(), "tl_decode_noalloc_scratch_bytes").value)


def strides(*vals: int) -> ctypes.Array:
    """Pack element strides into the int64[] the C ABI takes."""
    arr = (ctypes.c_int64 * len(vals))(*[int(v) for v in vals])
    return arr


def error_string(status: int) -> str:
    try:
        msg = load().tl_error_string(int(status))
        return msg.decode() if msg else str(status)
    except Exception:  # pragma: no cover - library unavailable
        return str(status)
