"""ctypes bindings to ``libiqk_hip.so``, the gfx950 kernel library.

Loading never falls back to anything: a missing or stale library raises
:class:`IqkNativeError`, so no code path can silently compute on the CPU.
"""

from __future__ import annotations

import ctypes
from ctypes import c_char_p, c_int, c_int64, c_uint32, c_void_p
from pathlib import Path

from . import build
from .build import HIP_LIB, LAUNCH_EXT

ABI_VERSION = 5

OK, ERR_MEMBER, ERR_GEOMETRY, ERR_ARGUMENT, ERR_LAUNCH = 0, 1, 2, 3, 4
_CODES = {ERR_MEMBER: "unknown member", ERR_GEOMETRY: "unsized geometry",
          ERR_ARGUMENT: "bad argument", ERR_LAUNCH: "kernel launch failed"}

MEMBER_IDS = {"iq2_ks": 0, "iq2_k": 1, "iq1_s_r4": 2}

_u32p = ctypes.POINTER(ctypes.c_uint32)
_i32p = ctypes.POINTER(ctypes.c_int32)

# name -> (restype, argtypes); the declarations of include/iqk_hip.h
SIGNATURES = {
    "iqk_hip_abi_version": (c_int, []),
    "iqk_hip_last_error": (c_int, []),
    "iqk_hip_source_hash": (c_char_p, []),
    "iqk_check_gemv_geometry": (c_int, [c_int, c_int64, c_int64]),
    "iqk_check_dequant_geometry": (c_int, [c_int, c_int64, c_int64]),
    "iqk_gemv": (c_int, [c_int, c_int64, c_int64, c_int64, c_void_p, ctypes.POINTER(c_void_p), c_int,
                         c_void_p, c_uint32, c_uint32, c_void_p, c_void_p]),
    "iqk_gemv_floor": (c_int, [c_int, c_int64, c_int64, c_int64, c_void_p, ctypes.POINTER(c_void_p), c_int,
                               c_void_p, c_uint32, c_uint32, c_void_p, c_void_p]),
    "iqk_gemv_floor_grid": (c_int, [c_int, c_int64, c_int64, c_int64, c_void_p, ctypes.POINTER(c_void_p), c_int,
                                    c_void_p, c_uint32, c_uint32, c_void_p, c_void_p]),
    "iqk_stream_floor": (c_int, [c_void_p, ctypes.c_uint64, c_void_p, c_void_p]),
    "iqk_stream_floor_wide": (c_int, [c_void_p, ctypes.c_uint64, c_int, ctypes.c_uint64, c_void_p, c_void_p]),
    "iqk_gemv_sorted": (c_int, [c_int, c_int64, c_int64, c_int64, c_void_p, c_int64, ctypes.POINTER(c_void_p),
                                c_int, c_void_p, c_void_p, c_uint32, c_void_p, c_void_p]),
    "iqk_gemv_union": (c_int, [c_int, c_int64, c_int64, c_int64, c_void_p, c_int64, ctypes.POINTER(c_void_p),
                               c_int, c_void_p, c_void_p, c_uint32, c_void_p, c_void_p]),
    "iqk_dequant": (c_int, [c_int, c_int64, c_int64, c_int64, ctypes.POINTER(c_void_p), c_int,
                            c_void_p, c_int64, c_void_p, c_void_p]),
    "iqk_dequant_rows": (c_int, [c_int, c_int64, c_int64, c_int64, ctypes.POINTER(c_void_p), c_int,
                                 c_int64, c_int64, c_void_p, c_int64, c_void_p, c_void_p]),
    "iqk_dequant_floor": (c_int, [c_int, c_int64, c_int64, c_int64, ctypes.POINTER(c_void_p), c_int,
                                  c_void_p, c_int64, c_void_p, c_void_p]),
    "iqk_grouped_gemm": (c_int, [c_int64, c_int64, c_int64, c_int64, c_void_p, c_int64, c_void_p,
                                 c_void_p, c_void_p, c_void_p, c_void_p, c_void_p]),
    "iqk_route": (c_int, [c_void_p, c_int64, c_int64, c_int64, c_int64, c_int64, c_void_p, c_void_p, c_void_p,
                          c_void_p]),
    "iqk_pack": (c_int, [c_int, c_int64, c_int64, c_void_p, ctypes.POINTER(c_void_p), c_int, c_void_p]),
    "iqk_fused_gemm": (c_int, [c_int, c_int64, c_int64, c_int64, c_void_p, c_int64, ctypes.POINTER(c_void_p),
                               c_int, c_int64, c_int64, c_void_p, c_void_p, c_void_p, c_int64, c_void_p, c_void_p]),
}


class IqkNativeError(RuntimeError):
    pass


_LIB = None
_LAUNCH = None


def library_path() -> Path:
    return HIP_LIB


def load() -> ctypes.CDLL:
    """Load the kernel library (once per process); raise if it is absent."""
    global _LIB
    if _LIB is not None:
        return _LIB
    path = library_path()
    if not path.is_file():
        raise IqkNativeError(
            f"{path} is not built; run `python -m mlx_iqk_amd.build` (hipcc, gfx950)")
    lib = ctypes.CDLL(str(path))
    for name, (restype, argtypes) in SIGNATURES.items():
        fn = getattr(lib, name)
        fn.restype = restype
        fn.argtypes = argtypes
    if lib.iqk_hip_abi_version() != ABI_VERSION:
        raise IqkNativeError(
            f"{path} has ABI {lib.iqk_hip_abi_version()}, this package expects {ABI_VERSION}; rebuild it")
    built, current = lib.iqk_hip_source_hash().decode(), build.hip_source_hash()
    if built != current:
        raise IqkNativeError(
            f"{path} was built from other sources (digest {built}, sources now {current}); "
            "rebuild it with `python -m mlx_iqk_amd.build`")
    _LIB = lib
    _load_launch(built)
    return lib


def _load_launch(digest: str) -> None:
    """The CPython binding of the decode launch path (``_iqk_launch``), when it
    was built beside the library from the same sources; the launchers use
    ctypes otherwise (the same entry points, ~4 us more host time a call)."""
    global _LAUNCH
    if not LAUNCH_EXT.is_file():
        return
    import importlib.util
    spec = importlib.util.spec_from_file_location("_iqk_launch", LAUNCH_EXT)
    mod = importlib.util.module_from_spec(spec)
    spec.loader.exec_module(mod)
    if mod.source_hash() != digest:
        raise IqkNativeError(f"{LAUNCH_EXT} was built with other sources than {HIP_LIB}; rebuild both with "
                             "`python -m mlx_iqk_amd.build`")
    _LAUNCH = mod


def launcher():
    """The CPython launch binding, or None (after :func:`load`)."""
    return _LAUNCH


def check(rc: int, what: str) -> None:
    """Raise on a non-zero ABI return code."""
    if rc == OK:
        return
    detail = _CODES.get(rc, f"code {rc}")
    if rc == ERR_LAUNCH:
        detail += f" (hipError {load().iqk_hip_last_error()})"
    raise IqkNativeError(f"{what}: {detail}")


def pointer_array(ptrs) -> ctypes.Array:
    arr = (c_void_p * len(ptrs))()
    for i, p in enumerate(ptrs):
        arr[i] = p
    return arr


__all__ = ["ABI_VERSION", "MEMBER_IDS", "SIGNATURES", "IqkNativeError", "check", "library_path",
           "load", "pointer_array"]
