"""Encode shim and CPU dequantizer over the package's C++ codec.

Same surface as the reference's codec shim (src/mlx_iqk/codec.py:238-293):
``quantize(member, weights, imatrix)`` turns float rows into ik wire bytes,
``dequantize(member, wire, n)`` decodes them in float32.  The library is
``libiqk_codec.so`` (``csrc/codec/iqk_codec.cpp``), whose quantizers
reproduce ik_llama's portable search byte for byte and run rows in parallel.

``IQ1_S_R4`` wire rows come in groups of four; both calls require row counts
in multiples of four for that member.
"""

from __future__ import annotations

import ctypes
from pathlib import Path

import numpy as np

from .build import CODEC_LIB
from .format import (
    IQ1_S_R4_BLOCK_BYTES,
    IQ2_K_BLOCK_BYTES,
    IQ2_KS_BLOCK_BYTES,
    IqkFormatError,
    check_member,
    check_row_width,
    check_wire_rows,
    ik_row_bytes,
)


class IqkCodecError(RuntimeError):
    pass


_LIB = None
_F32P = ctypes.POINTER(ctypes.c_float)
_BLOCK_BYTES = {"iq2_ks": IQ2_KS_BLOCK_BYTES, "iq2_k": IQ2_K_BLOCK_BYTES,
                "iq1_s_r4": IQ1_S_R4_BLOCK_BYTES}


def library_path() -> Path:
    return CODEC_LIB


def load() -> ctypes.CDLL:
    """Load the codec library once; refuse a build whose block sizes disagree."""
    global _LIB
    if _LIB is not None:
        return _LIB
    path = library_path()
    if not path.is_file():
        raise IqkCodecError(f"{path} is not built; run `python -m mlx_iqk_amd.build`")
    lib = ctypes.CDLL(str(path))
    for m in ("iq2_k", "iq2_ks", "iq1_s_r4"):
        fn = getattr(lib, f"iqk_row_size_{m}")
        fn.restype, fn.argtypes = ctypes.c_size_t, [ctypes.c_int64]
        fn = getattr(lib, f"iqk_quantize_{m}")
        fn.restype = ctypes.c_size_t
        fn.argtypes = [_F32P, ctypes.c_void_p, ctypes.c_int64, ctypes.c_int64, _F32P]
        fn = getattr(lib, f"iqk_dequantize_{m}")
        fn.restype = ctypes.c_int
        fn.argtypes = [ctypes.c_void_p, _F32P, ctypes.c_int64, ctypes.c_int64]
        fn = getattr(lib, f"iqk_block_size_{m}")
        fn.restype, fn.argtypes = ctypes.c_size_t, []
        if fn() != _BLOCK_BYTES[m]:
            raise IqkCodecError(f"{path}: block_{m} is {fn()} bytes, the format says {_BLOCK_BYTES[m]}")
    lib.iqk_codec_set_threads.restype, lib.iqk_codec_set_threads.argtypes = None, [ctypes.c_int]
    lib.iqk_codec_threads.restype, lib.iqk_codec_threads.argtypes = ctypes.c_int, []
    _LIB = lib
    return lib


def set_threads(threads: int) -> None:
    """Worker threads the quantizers use (0 = default: IQK_CODEC_THREADS or the CPU count)."""
    load().iqk_codec_set_threads(int(threads))


def threads() -> int:
    return int(load().iqk_codec_threads())


def quantize(member: str, weights: np.ndarray, imatrix: np.ndarray | None = None) -> np.ndarray:
    """Quantize ``[rows, in_features]`` float rows to ik wire ``[rows, row_bytes]``.

    ``imatrix`` is one importance vector of ``in_features`` values reused for
    every row; ``None`` selects the member's unweighted objective.
    """
    check_member(member)
    if weights.ndim != 2:
        raise IqkFormatError(f"weights must be [rows, in_features], got {weights.shape}")
    rows, n = weights.shape
    check_row_width(n, member)
    check_wire_rows(member, rows)
    src = np.ascontiguousarray(weights, dtype=np.float32)
    row_bytes = ik_row_bytes(member, n)
    out = np.zeros((rows, row_bytes), dtype=np.uint8)
    im = None
    if imatrix is not None:
        if imatrix.shape != (n,):
            raise IqkFormatError(f"imatrix must be one vector of {n} values, got {imatrix.shape}")
        im = np.ascontiguousarray(imatrix, dtype=np.float32)
    im_ptr = im.ctypes.data_as(_F32P) if im is not None else ctypes.cast(0, _F32P)
    written = getattr(load(), f"iqk_quantize_{member}")(
        src.ctypes.data_as(_F32P), out.ctypes.data_as(ctypes.c_void_p), rows, n, im_ptr)
    if written != rows * row_bytes:
        raise IqkCodecError(f"{member} quantize wrote {written} bytes, expected {rows * row_bytes}")
    return out


def dequantize(member: str, wire: np.ndarray, in_features: int) -> np.ndarray:
    """Decode ik wire rows to float32 ``[rows, in_features]``."""
    check_member(member)
    n = check_row_width(in_features, member)
    row_bytes = ik_row_bytes(member, n)
    if wire.ndim != 2 or wire.shape[1] != row_bytes:
        raise IqkFormatError(f"{member} rows of {n} weights are {row_bytes} wire bytes, got {wire.shape}")
    buf = np.ascontiguousarray(wire, dtype=np.uint8)
    rows = check_wire_rows(member, buf.shape[0])
    out = np.zeros((rows, n), dtype=np.float32)
    rc = getattr(load(), f"iqk_dequantize_{member}")(
        buf.ctypes.data_as(ctypes.c_void_p), out.ctypes.data_as(_F32P), rows, n)
    if rc != 0:
        raise IqkCodecError(f"{member} dequantize refused geometry {n}")
    return out


__all__ = ["IqkCodecError", "dequantize", "library_path", "load", "quantize", "set_threads", "threads"]
