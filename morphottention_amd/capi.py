"""ctypes view of the C ABI in ``libmorphottention_hip.so``.

The library is the drop-in boundary declared in ``include/morphottention.h``.
PyTorch must be imported first so that the HIP runtime it ships is the one the
library binds to (both carry the soname ``libamdhip64.so.7``).
"""

from __future__ import annotations

import ctypes
import os

import torch  # noqa: F401  (loads the HIP runtime before the library)

LIB_PATH = os.path.join(os.path.dirname(os.path.abspath(__file__)), "libmorphottention_hip.so")

_lib = None


def lib() -> ctypes.CDLL:
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            raise ImportError(f"{LIB_PATH} is missing; build it with `python morphottention_amd/build.py`")
        L = ctypes.CDLL(LIB_PATH)
        i64, vp, sz = ctypes.c_int64, ctypes.c_void_p, ctypes.c_size_t
        L.morpho_version.restype = ctypes.c_int
        L.morpho_status_string.restype = ctypes.c_char_p
        L.morpho_status_string.argtypes = [ctypes.c_int]
        L.morpho_last_error.restype = ctypes.c_char_p
        L.morpho_forward_workspace_size.restype = sz
        L.morpho_forward_workspace_size.argtypes = [i64] * 5
        L.morpho_backward_workspace_size.restype = sz
        L.morpho_backward_workspace_size.argtypes = [i64] * 5 + [ctypes.c_int]
        L.morpho_backward_workspace_size_for_mode.restype = sz
        L.morpho_backward_workspace_size_for_mode.argtypes = [i64] * 5 + [ctypes.c_int, ctypes.c_int]
        L.morpho_forward.restype = ctypes.c_int
        L.morpho_forward.argtypes = [vp] * 5 + [vp, vp] + [i64] * 5 + [ctypes.c_float, ctypes.c_int, vp, sz, vp]
        L.morpho_forward_noalloc.restype = ctypes.c_int
        L.morpho_forward_noalloc.argtypes = [vp] * 5 + [vp, vp] + [i64] * 5 + [ctypes.c_float, ctypes.c_int, vp]
        L.morpho_backward.restype = ctypes.c_int
        L.morpho_backward.argtypes = ([vp] * 8 + [vp] * 5 + [i64] * 5 + [ctypes.c_float, ctypes.c_int]
                                      + [vp, vp, sz, vp])
        L.morpho_soft_forward.restype = ctypes.c_int
        L.morpho_soft_forward.argtypes = ([vp] * 5 + [vp, vp, vp] + [i64] * 5
                                          + [ctypes.c_float, ctypes.c_int, ctypes.c_int, vp, sz, vp])
        L.morpho_soft_forward_workspace_size.restype = sz
        L.morpho_soft_forward_workspace_size.argtypes = [i64] * 5
        L.morpho_soft_backward_workspace_size.restype = sz
        L.morpho_soft_backward_workspace_size.argtypes = [i64] * 5 + [ctypes.c_int]
        L.morpho_soft_backward.restype = ctypes.c_int
        L.morpho_soft_backward.argtypes = ([vp] * 8 + [vp] * 6 + [i64] * 5
                                           + [ctypes.c_float, ctypes.c_int, ctypes.c_int, vp, vp, sz, vp])
        L.morpho_timing_enable.restype = ctypes.c_int
        L.morpho_timing_enable.argtypes = [ctypes.c_int]
        L.morpho_timing_only.restype = ctypes.c_int
        L.morpho_timing_only.argtypes = [ctypes.c_char_p]
        L.morpho_timing_read.restype = ctypes.c_int
        L.morpho_timing_read.argtypes = [ctypes.POINTER(ctypes.c_char_p), ctypes.POINTER(ctypes.c_float),
                                         ctypes.c_int]
        _lib = L
    return _lib


def forward_workspace_size(B: int, N: int, D: int, H: int, cube_m: int) -> int:
    return int(lib().morpho_forward_workspace_size(B, N, D, H, cube_m))


def backward_workspace_size(B: int, N: int, D: int, H: int, cube_m: int, have_forward_workspace: bool,
                            mode: int | None = None) -> int:
    """Bytes of backward workspace; ``mode`` (the bits morpho_backward gets) matters
    only with MORPHO_MODE_DETERMINISTIC, which adds the per-key-block partials."""
    if mode is None:
        return int(lib().morpho_backward_workspace_size(B, N, D, H, cube_m, int(have_forward_workspace)))
    return int(lib().morpho_backward_workspace_size_for_mode(B, N, D, H, cube_m, int(have_forward_workspace), mode))


def soft_forward_workspace_size(B: int, N: int, D: int, H: int, cube_m: int) -> int:
    return int(lib().morpho_soft_forward_workspace_size(B, N, D, H, cube_m))


def soft_backward_workspace_size(B: int, N: int, D: int, H: int, cube_m: int, have_forward_workspace: bool) -> int:
    return int(lib().morpho_soft_backward_workspace_size(B, N, D, H, cube_m, int(have_forward_workspace)))


def timing_enable(enable: bool) -> None:
    lib().morpho_timing_enable(int(enable))


def timing_only(name: str | None) -> None:
    """Time only the launches reported under ``name`` (None: all of them)."""
    lib().morpho_timing_only(name.encode() if name else None)


def timing_read(max_entries: int = 4096) -> list[tuple[str, float]]:
    names = (ctypes.c_char_p * max_entries)()
    ms = (ctypes.c_float * max_entries)()
    n = lib().morpho_timing_read(names, ms, max_entries)
    return [(names[i].decode(), float(ms[i])) for i in range(n)]
