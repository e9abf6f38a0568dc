"""ORACLE -- test infrastructure only.

Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg may
import this module; the product never does.  It is the checker, never the
thing measured or shipped.

* :func:`dequantize` -- the plain-C restatement of the reference CPU
  dequantizers (``iqk_oracle.c``), one weight at a time from the block layouts
  (reference: vendor/ik_llama/iqk_iq2.cpp:502-562,
  vendor/ik_llama/iqk_iq1sr4.cpp:581-602).
* :func:`ref_quantize` / :func:`ref_dequantize` -- the reference's own vendored
  C++ codec, compiled from its sources into ``oracle/_ref`` by
  ``oracle/Makefile`` where ``/root/reference`` exists (absent elsewhere).
* :func:`gemv_reference`, :func:`prefill_reference` -- float64 contractions
  of oracle-dequantized weights (the reference's tests compare its kernels to
  float64, tests/test_kernels.py:161-188).

Pinning of each function is in tests/test_oracle.py.
"""

from __future__ import annotations

import ctypes
import subprocess
from pathlib import Path

import numpy as np

HERE = Path(__file__).resolve().parent
ORACLE_LIB = HERE / "liboracle.so"
REF_DIR = HERE / "_ref"
REF_LIBS = {"iq2": REF_DIR / "libiqk_ref_iq2.so", "iq1": REF_DIR / "libiqk_ref_iq1sr4.so"}
REFERENCE_SOURCES = Path("/root/reference/vendor/ik_llama")

_F32P = ctypes.POINTER(ctypes.c_float)
_ROW_BYTES = {"iq2_ks": lambda n: 2 + 70 * (n // 256), "iq2_k": lambda n: 76 * (n // 256),
              "iq1_s_r4": lambda n: 2 + 6 * (n // 32)}

_oracle = None
_ref = {}


def build(with_ref: bool | None = None) -> None:
    """Compile the oracle (and the reference codec when its sources are present)."""
    targets = ["oracle"]
    if with_ref is None:
        with_ref = REFERENCE_SOURCES.is_dir()
    if with_ref:
        targets.append("ref")
    proc = subprocess.run(["make", "-s", "-C", str(HERE)] + targets, capture_output=True, text=True)
    if proc.returncode != 0:
        raise RuntimeError(f"oracle build failed:\n{proc.stdout}\n{proc.stderr}")


def _load_oracle():
    global _oracle
    if _oracle is None:
        if not ORACLE_LIB.is_file():
            build(with_ref=False)
        lib = ctypes.CDLL(str(ORACLE_LIB))
        for m in ("iq2_ks", "iq2_k", "iq1_s_r4"):
            fn = getattr(lib, f"oracle_dequant_{m}")
            fn.restype = ctypes.c_int
            fn.argtypes = [ctypes.c_void_p, _F32P, ctypes.c_int64, ctypes.c_int64]
        _oracle = lib
    return _oracle


def row_bytes(member: str, n: int) -> int:
    return _ROW_BYTES[member](n)


def _out(rows: int, n: int, out: np.ndarray | None) -> np.ndarray:
    if out is None:
        return np.empty((rows, n), dtype=np.float32)
    assert out.dtype == np.float32 and out.shape == (rows, n) and out.flags.c_contiguous, (out.dtype, out.shape)
    return out


def dequantize(member: str, wire: np.ndarray, n: int, out: np.ndarray | None = None) -> np.ndarray:
    """Oracle float32 dequantization of ik wire rows ``[rows, row_bytes]``
    (into ``out`` when given)."""
    buf = np.ascontiguousarray(wire, dtype=np.uint8)
    assert buf.ndim == 2 and buf.shape[1] == row_bytes(member, n), (member, n, buf.shape)
    out = _out(buf.shape[0], n, out)
    rc = getattr(_load_oracle(), f"oracle_dequant_{member}")(
        buf.ctypes.data_as(ctypes.c_void_p), out.ctypes.data_as(_F32P), buf.shape[0], n)
    if rc != 0:
        raise ValueError(f"oracle refused {member} geometry rows={buf.shape[0]} n={n}")
    return out


def ref_available() -> bool:
    return all(p.is_file() for p in REF_LIBS.values())


def _load_ref(member: str):
    key = "iq1" if member == "iq1_s_r4" else "iq2"
    if key not in _ref:
        if not REF_LIBS[key].is_file():
            raise FileNotFoundError(f"{REF_LIBS[key]} not built (reference sources absent)")
        lib = ctypes.CDLL(str(REF_LIBS[key]))
        names = ("iq1_s_r4",) if key == "iq1" else ("iq2_k", "iq2_ks")
        for m in names:
            fn = getattr(lib, f"iqk_quantize_{m}")
            fn.restype = ctypes.c_size_t
            fn.argtypes = [_F32P, ctypes.c_void_p, ctypes.c_int64, ctypes.c_int64, _F32P]
            fn = getattr(lib, f"iqk_dequantize_{m}")
            fn.restype = ctypes.c_int
            fn.argtypes = [ctypes.c_void_p, _F32P, ctypes.c_int64, ctypes.c_int64]
        _ref[key] = lib
    return _ref[key]


def ref_quantize(member: str, rows: np.ndarray, imatrix: np.ndarray | None) -> np.ndarray:
    """The reference's own quantizer (compiled vendored source)."""
    src = np.ascontiguousarray(rows, dtype=np.float32)
    out = np.zeros((src.shape[0], row_bytes(member, src.shape[1])), dtype=np.uint8)
    im = None if imatrix is None else np.ascontiguousarray(imatrix, dtype=np.float32)
    im_ptr = im.ctypes.data_as(_F32P) if im is not None else ctypes.cast(0, _F32P)
    written = getattr(_load_ref(member), f"iqk_quantize_{member}")(
        src.ctypes.data_as(_F32P), out.ctypes.data_as(ctypes.c_void_p), src.shape[0], src.shape[1], im_ptr)
    if written != out.size:
        raise ValueError(f"reference quantize wrote {written} of {out.size} bytes")
    return out


def ref_dequantize(member: str, wire: np.ndarray, n: int, out: np.ndarray | None = None) -> np.ndarray:
    """The reference's own CPU dequantizer (compiled vendored source), into
    ``out`` when given."""
    buf = np.ascontiguousarray(wire, dtype=np.uint8)
    out = _out(buf.shape[0], n, out)
    rc = getattr(_load_ref(member), f"iqk_dequantize_{member}")(
        buf.ctypes.data_as(ctypes.c_void_p), out.ctypes.data_as(_F32P), buf.shape[0], n)
    if rc != 0:
        raise ValueError("reference dequantize refused the geometry")
    return out


def gemv_reference(weights: np.ndarray, sel: np.ndarray, x: np.ndarray, pairs_per_row: int) -> np.ndarray:
    """float64 ``out[m] = W[sel[m]] @ x[m // pairs_per_row]``; ``weights`` is ``[E, out, in]``."""
    w = weights.astype(np.float64)
    xs = x.astype(np.float64)
    return np.stack([w[int(e)] @ xs[m // pairs_per_row] for m, e in enumerate(sel)])


def prefill_reference(weights: np.ndarray, x: np.ndarray, indices: np.ndarray) -> np.ndarray:
    """float64 ``gather_mm(x, W^T, rhs_indices=indices)`` with fp16-rounded weights.

    The prefill route contracts fp16 weights, so the reference rounds the
    dequantized weights to fp16 first (reference: src/mlx_iqk/nn.py:234-238).
    """
    w16 = weights.astype(np.float16).astype(np.float64)
    batch = np.broadcast_shapes(x.shape[:-2], indices.shape)
    xb = np.broadcast_to(x.astype(np.float64), batch + x.shape[-2:])
    ib = np.broadcast_to(indices, batch)
    out = np.empty(batch + (x.shape[-2], w16.shape[1]), dtype=np.float64)
    for pos in np.ndindex(*batch):
        out[pos] = xb[pos] @ w16[int(ib[pos])].T
    return out


__all__ = ["build", "dequantize", "gemv_reference", "prefill_reference", "ref_available",
           "ref_dequantize", "ref_quantize", "row_bytes"]
