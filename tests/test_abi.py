"""The C ABI's host-side contract, checked without a GPU.

* every function include/iqk_hip.h and include/iqk_codec.h declare is exported
  by the built library, with the ctypes signature the package binds;
* the geometry guards refuse what the reference refuses
  (src/mlx_iqk/kernels.py:100-142) and accept the routed geometry;
* every entry point refuses a bad argument before any HIP call.
"""

from __future__ import annotations

import ctypes
import re
from pathlib import Path

import pytest

from mlx_iqk_amd import _native, build, codec

ROOT = Path(__file__).resolve().parents[1]


def _declared(header: Path) -> set[str]:
    text = re.sub(r"//[^\n]*", "", header.read_text())
    return set(re.findall(r"\b(iqk_[a-z0-9_]+)\s*\(", text))


@pytest.fixture(scope="module")
def lib():
    if not build.HIP_LIB.is_file():
        build.build_hip()
    return _native.load()


def test_every_declared_kernel_entry_point_is_exported_and_bound(lib):
    declared = _declared(ROOT / "include" / "iqk_hip.h")
    assert declared == set(_native.SIGNATURES)
    for name in declared:
        assert getattr(lib, name) is not None


def test_every_declared_codec_entry_point_is_exported():
    declared = _declared(ROOT / "include" / "iqk_codec.h")
    lib = codec.load()
    for name in declared:
        assert getattr(lib, name) is not None, name


def test_abi_version(lib):
    assert lib.iqk_hip_abi_version() == _native.ABI_VERSION


@pytest.mark.parametrize("member", (0, 1, 2))
def test_geometry_guards(lib, member):
    for n in (2048, 4096):
        assert lib.iqk_check_gemv_geometry(member, n, 2048) == 0
        assert lib.iqk_check_dequant_geometry(member, n, 4096) == 0
    for bad_n in (1024, 1536, 2560, 3072, 4352, 8192, 0, -2048):
        assert lib.iqk_check_gemv_geometry(member, bad_n, 32) == _native.ERR_GEOMETRY
        assert lib.iqk_check_dequant_geometry(member, bad_n, 32) == _native.ERR_GEOMETRY
    for bad_out in (24, 40, 100, 0, -16):
        assert lib.iqk_check_gemv_geometry(member, 2048, bad_out) == _native.ERR_GEOMETRY
    assert lib.iqk_check_dequant_geometry(member, 2048, 24) == 0  # the producer takes any row count
    assert lib.iqk_check_gemv_geometry(3, 2048, 32) == _native.ERR_MEMBER


def test_entry_points_refuse_bad_arguments_before_launching(lib):
    p = ctypes.c_void_p(16)  # never dereferenced: every call below is refused first
    streams = _native.pointer_array([16] * 5)
    # wrong stream count, null x, null output, pairs not tiling rows, bad member
    assert lib.iqk_gemv(0, 4096, 2048, 256, p, streams, 4, p, 6, 12, p, None) == _native.ERR_ARGUMENT
    assert lib.iqk_gemv(0, 4096, 2048, 256, None, streams, 5, p, 6, 12, p, None) == _native.ERR_ARGUMENT
    assert lib.iqk_gemv(0, 4096, 2048, 256, p, streams, 5, p, 6, 12, None, None) == _native.ERR_ARGUMENT
    assert lib.iqk_gemv(0, 4096, 2048, 256, p, streams, 5, p, 5, 12, p, None) == _native.ERR_ARGUMENT
    assert lib.iqk_gemv(7, 4096, 2048, 256, p, streams, 5, p, 6, 12, p, None) == _native.ERR_MEMBER
    assert lib.iqk_gemv_floor(1, 3072, 2048, 256, p, streams, 4, p, 6, 12, p, None) == _native.ERR_GEOMETRY
    assert lib.iqk_dequant(2, 2048, 32, 4, streams, 5, None, 4, p, None) == _native.ERR_ARGUMENT
    assert lib.iqk_dequant(2, 2048, 32, 4, streams, 3, None, 2, p, None) == _native.ERR_ARGUMENT
    assert lib.iqk_dequant_floor(0, 2048, 32, 0, streams, 5, None, 4, p, None) == _native.ERR_ARGUMENT
    assert lib.iqk_grouped_gemm(4080, 2048, 4, 8, p, 8, p, p, p, None, p, None) == _native.ERR_GEOMETRY
    assert lib.iqk_grouped_gemm(4096, 0, 4, 8, p, 8, p, p, p, None, p, None) == _native.ERR_GEOMETRY
    assert lib.iqk_grouped_gemm(4020, 2048, 4, 8, p, 8, p, p, p, None, p, None) == _native.ERR_GEOMETRY
    assert lib.iqk_grouped_gemm(4096, 2048, 4, 8, None, 8, p, p, p, None, p, None) == _native.ERR_ARGUMENT
    assert lib.iqk_stream_floor_wide(p, 4096, 5, 0, p, None) == _native.ERR_ARGUMENT  # 4, 8 or 16 loads
    assert lib.iqk_stream_floor_wide(p, 4100, 8, 0, p, None) == _native.ERR_ARGUMENT  # not whole 16-byte words
    assert lib.iqk_stream_floor_wide(None, 4096, 8, 0, p, None) == _native.ERR_ARGUMENT
    # empty work is a no-op success, with no launch
    assert lib.iqk_stream_floor_wide(p, 0, 8, 0, p, None) == 0
    assert lib.iqk_gemv(0, 4096, 2048, 256, p, streams, 5, p, 6, 0, p, None) == 0
    assert lib.iqk_grouped_gemm(4096, 2048, 0, 0, None, 0, None, None, None, None, None, None) == 0
    assert lib.iqk_hip_last_error() == 0


def test_library_carries_the_digest_of_its_sources(lib):
    assert lib.iqk_hip_source_hash().decode() == build.hip_source_hash()


def test_a_library_built_from_other_sources_is_refused(monkeypatch, lib):
    """A stale build (sources edited after it was compiled) never runs: the
    digest compiled into it no longer matches the sources beside it."""
    monkeypatch.setattr(_native, "_LIB", None)
    monkeypatch.setattr(build, "hip_source_hash", lambda: "0" * 16)
    with pytest.raises(_native.IqkNativeError, match="other sources"):
        _native.load()


def test_missing_library_fails_loudly(monkeypatch, tmp_path):
    monkeypatch.setattr(_native, "_LIB", None)
    monkeypatch.setattr(_native, "library_path", lambda: tmp_path / "absent.so")
    with pytest.raises(_native.IqkNativeError):
        _native.load()


def test_sorted_union_and_range_entry_points_refuse_bad_arguments(lib):
    p = ctypes.c_void_p(16)  # never dereferenced: every call below is refused first
    streams = _native.pointer_array([16] * 5)
    for fn in (lib.iqk_gemv_sorted, lib.iqk_gemv_union):
        # IQ1_S_R4 has no sorted or union form (reference: _check_iq2_member)
        assert fn(2, 4096, 2048, 256, p, 2, streams, 3, p, p, 6, p, None) == _native.ERR_MEMBER
        assert fn(2, 4096, 2048, 256, p, 2, streams, 3, p, p, 0, p, None) == _native.ERR_MEMBER
        # pairs without a token map, negative row count, unsized out
        assert fn(0, 4096, 2048, 256, p, 2, streams, 5, p, None, 6, p, None) == _native.ERR_ARGUMENT
        assert fn(0, 4096, 2048, 256, p, -1, streams, 5, p, p, 6, p, None) == _native.ERR_ARGUMENT
        assert fn(0, 4096, 2048, 256, p, 0, streams, 5, p, p, 6, p, None) == _native.ERR_ARGUMENT
        assert fn(1, 4096, 2040, 256, p, 2, streams, 4, p, p, 6, p, None) == _native.ERR_GEOMETRY
        assert fn(0, 4096, 2048, 256, p, 2, streams, 5, p, p, 0, p, None) == _native.OK  # nothing to do
    # ranges outside [0, out_features) or empty
    for start, rows in ((16, 32), (-1, 8), (0, 0), (0, 33), (31, 2)):
        assert lib.iqk_dequant_rows(0, 2048, 32, 4, streams, 5, start, rows, None, 4, p, None) == _native.ERR_GEOMETRY
    assert lib.iqk_dequant_rows(0, 2048, 32, 4, streams, 5, 0, 32, None, 3, p, None) == _native.ERR_ARGUMENT
    assert lib.iqk_dequant_rows(0, 2048, 32, 4, streams, 5, 0, 32, p, 0, p, None) == _native.OK


def test_fused_gemm_refuses_bad_arguments(lib):
    p = ctypes.c_void_p(16)  # never dereferenced: every call below is refused first
    streams = _native.pointer_array([16] * 5)
    f = lib.iqk_fused_gemm
    assert f(2, 4096, 2048, 8, p, 4, streams, 5, 0, 2048, p, p, None, 4, p, None) == _native.ERR_ARGUMENT
    assert f(7, 4096, 2048, 8, p, 4, streams, 5, 0, 2048, p, p, None, 4, p, None) == _native.ERR_MEMBER
    assert f(0, 3072, 2048, 8, p, 4, streams, 5, 0, 2048, p, p, None, 4, p, None) == _native.ERR_GEOMETRY
    for start, rows in ((0, 0), (-1, 8), (2040, 16), (0, 2049)):
        assert f(0, 4096, 2048, 8, p, 4, streams, 5, start, rows, p, p, None, 4, p, None) == _native.ERR_GEOMETRY
    assert f(0, 4096, 2048, 8, p, 4, streams, 4, 0, 2048, p, p, None, 4, p, None) == _native.ERR_ARGUMENT
    assert f(1, 4096, 2048, 8, None, 4, streams, 4, 0, 2048, p, p, None, 4, p, None) == _native.ERR_ARGUMENT
    assert f(1, 4096, 2048, 8, p, 4, streams, 4, 0, 2048, None, p, None, 4, p, None) == _native.ERR_ARGUMENT
    assert f(1, 4096, 2048, 8, p, 4, streams, 4, 0, 2048, p, p, None, 0, p, None) == _native.OK
    # 32-bit offsets: an expert plane or an x of 4 GiB or more, and an empty x, are refused
    assert f(0, 4096, 1 << 22, 8, p, 4, streams, 5, 0, 2048, p, p, None, 4, p, None) == _native.ERR_GEOMETRY
    assert f(0, 4096, 2048, 8, p, 1 << 19, streams, 5, 0, 2048, p, p, None, 4, p, None) == _native.ERR_ARGUMENT
    assert f(0, 4096, 2048, 8, p, 0, streams, 5, 0, 2048, p, p, None, 4, p, None) == _native.ERR_ARGUMENT


def test_route_refuses_bad_arguments(lib):
    p = ctypes.c_void_p(16)  # never dereferenced: every call below is refused first
    f = lib.iqk_route
    assert f(p, 8, 0, 1, 1, 8, p, p, p, None) == _native.ERR_ARGUMENT       # no experts
    assert f(p, 8, 4097, 1, 1, 8, p, p, p, None) == _native.ERR_ARGUMENT    # past the LDS counters
    assert f(p, -1, 8, 1, 1, 8, p, p, p, None) == _native.ERR_ARGUMENT
    assert f(p, 8, 8, 0, 1, 8, p, p, p, None) == _native.ERR_ARGUMENT       # rows per pair
    assert f(p, 8, 8, 1, 0, 8, p, p, p, None) == _native.ERR_ARGUMENT       # pairs per x row
    assert f(p, 8, 8, 2, 4, 3, p, p, p, None) == _native.ERR_ARGUMENT       # x holds 4 of the 2 x 2 rows named
    assert f(None, 8, 8, 1, 1, 8, p, p, p, None) == _native.ERR_ARGUMENT
    assert f(p, 8, 8, 1, 1, 8, None, p, p, None) == _native.ERR_ARGUMENT
    assert f(p, 1 << 30, 8, 2, 1, 1 << 31, p, p, p, None) == _native.ERR_ARGUMENT  # 2^31 slots
    # factors whose int64 product would overflow (2^33 x 2^31) and wrap below 2^31
    assert f(p, 1 << 33, 8, 1 << 31, 1, 8, p, p, p, None) == _native.ERR_ARGUMENT
    assert f(p, 1 << 40, 8, 1 << 24, 1, 8, p, p, p, None) == _native.ERR_ARGUMENT  # 2^64: wraps to 0
    assert f(p, 8, 8, 1, 1 << 32, 8, p, p, p, None) == _native.ERR_ARGUMENT  # pairs per x row past 32 bits


def test_pack_refuses_bad_arguments(lib):
    p = ctypes.c_void_p(16)  # never dereferenced: every call below is refused first
    streams = _native.pointer_array([16] * 5)
    f = lib.iqk_pack
    assert f(3, 2048, 8, p, streams, 5, None) == _native.ERR_MEMBER
    assert f(0, 2000, 8, p, streams, 5, None) == _native.ERR_GEOMETRY   # not a multiple of 256
    assert f(2, 2048, 6, p, streams, 3, None) == _native.ERR_GEOMETRY   # IQ1_S_R4 rows in fours
    assert f(0, 2048, 8, p, streams, 4, None) == _native.ERR_ARGUMENT   # stream count
    assert f(0, 2048, 8, None, streams, 5, None) == _native.ERR_ARGUMENT
    assert f(0, 2048, 8, ctypes.c_void_p(18), streams, 5, None) == _native.ERR_ARGUMENT  # wire alignment
    assert f(0, 2048, 8, p, _native.pointer_array([24] + [16] * 4), 5, None) == _native.ERR_ARGUMENT  # qs alignment
    assert f(0, 2048, 0, p, streams, 5, None) == _native.OK


def test_launch_binding_is_built_from_the_same_sources_and_refuses_as_the_abi(lib):
    """The CPython binding of the decode launch path calls the same entry
    points (refusals come back unchanged, before any launch)."""
    fast = _native.launcher()
    assert fast is not None, "the launch binding is built beside the library by build()"
    assert fast.source_hash() == lib.iqk_hip_source_hash().decode()
    streams = _native.pointer_array([16] * 5)
    addr = ctypes.addressof(streams)
    assert fast.gemv(0, 7, 4096, 2048, 256, 16, addr, 5, 16, 6, 12, 16, 0) == _native.ERR_MEMBER
    assert fast.gemv(0, 0, 4096, 2048, 256, 16, addr, 4, 16, 6, 12, 16, 0) == _native.ERR_ARGUMENT  # streams
    assert fast.gemv(1, 1, 3072, 2048, 256, 16, addr, 4, 16, 6, 12, 16, 0) == _native.ERR_GEOMETRY  # floor
    assert fast.gemv(2, 0, 4096, 2048, 256, 0, addr, 5, 16, 6, 12, 16, 0) == _native.ERR_ARGUMENT  # null x
    assert fast.gemv(0, 0, 4096, 2048, 256, 16, addr, 5, 16, 6, 0, 16, 0) == 0  # no pairs: no launch
    with pytest.raises(TypeError):
        fast.gemv(0, 0, 4096)
    # the narrow arguments are range-checked, not truncated into a valid call
    for bad in ((0, 1 << 31, 4096, 2048, 256, 16, addr, 5, 16, 6, 12, 16, 0),   # member past int
                (0, 0, 4096, 2048, 256, 16, addr, 1 << 32, 16, 6, 12, 16, 0),  # stream count past int
                (0, 0, 4096, 2048, 256, 16, addr, 5, 16, (1 << 32) + 6, 12, 16, 0),  # pairs a row past u32
                (0, 0, 4096, 2048, 256, 16, addr, 5, 16, 6, (1 << 32) + 12, 16, 0),  # pairs past u32
                (0, 0, 4096, 2048, 256, 16, addr, 5, 16, 6, -12, 16, 0)):
        with pytest.raises(OverflowError):
            fast.gemv(*bad)
