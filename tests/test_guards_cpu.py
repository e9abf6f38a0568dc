"""Host-side guards of the kernels and the switch module, without a GPU:
every geometry the kernels are not built for is refused at construction or
before a launch (reference: tests/test_kernels.py:81-131, the guards of
src/mlx_iqk/kernels.py:100-142 and src/mlx_iqk/nn.py)."""

from __future__ import annotations

import ctypes
import pathlib
import re

import pytest

from mlx_iqk_amd import format as fmt
from mlx_iqk_amd import kernels
from mlx_iqk_amd.kernels import IqkKernelError, SUPPORTED_IN_FEATURES
from mlx_iqk_amd.nn import IqkRuntimeError, IqkSwitchLinear

HEADER = pathlib.Path(__file__).resolve().parents[1] / "include" / "iqk_hip.h"


def test_both_routed_widths_are_the_compiled_ones():
    assert SUPPORTED_IN_FEATURES == (2048, 4096)
    assert kernels.ROWS_PER_TG == 16


@pytest.mark.parametrize("member", fmt.MEMBERS)
def test_gemv_and_producer_refuse_unsized_input_widths(member):
    for n in SUPPORTED_IN_FEATURES:
        assert kernels.check_gemv_geometry(n, 32) == (n, 32)
        assert kernels.check_dequant_geometry(n, 24) == (n, 24)
    for n in (1024, 3072, 8192):  # block multiples the kernels are not sized for
        with pytest.raises(IqkKernelError):
            kernels.check_gemv_geometry(n, 32)
        with pytest.raises(IqkKernelError):
            kernels.check_dequant_geometry(n, 32)
    for n in (4000, 0, -2048):  # not a positive multiple of the block
        with pytest.raises(fmt.IqkFormatError):
            kernels.check_gemv_geometry(n, 32)


def test_gemv_refuses_out_features_that_do_not_tile_a_wavefront():
    for out in (24, 40, 100, 0, -16):
        with pytest.raises(IqkKernelError):
            kernels.check_gemv_geometry(2048, out)
    with pytest.raises(IqkKernelError):
        kernels.check_dequant_geometry(2048, 0)


@pytest.mark.parametrize("member", fmt.MEMBERS)
def test_module_construction_refuses_unsized_widths(member):
    m = IqkSwitchLinear(member, 4, 32, 2048)
    assert tuple(m.qs.shape[:2]) == (4, 32)
    with pytest.raises(IqkKernelError):
        IqkSwitchLinear(member, 4, 32, 1024)
    with pytest.raises(IqkKernelError):
        IqkSwitchLinear(member, 4, 24, 2048)
    with pytest.raises(IqkRuntimeError):
        IqkSwitchLinear(member, 0, 32, 2048)


def test_module_construction_refuses_an_unknown_member():
    with pytest.raises(fmt.IqkFormatError):
        IqkSwitchLinear("iq3_k", 4, 32, 2048)


@pytest.mark.parametrize("member", fmt.MEMBERS)
def test_module_buffers_are_the_format_streams(member):
    m = IqkSwitchLinear(member, 3, 16, 4096)
    shapes = fmt.component_shapes(member, 3, 16, 4096)
    dtypes = kernels.stream_dtypes(member)
    assert list(m._stream_names) == list(shapes)
    for name, shape in shapes.items():
        buf = getattr(m, name)
        assert tuple(buf.shape) == shape and buf.dtype == dtypes[name]


@pytest.mark.parametrize("member", fmt.MEMBERS)
def test_kernel_input_names_follow_the_format_stream_order(member):
    streams = list(fmt.component_shapes(member, 1, 1, 2048))
    table = kernels.TABLE_INPUT_NAMES[member]
    assert kernels.gemv_input_names(member) == ["x"] + streams + [table, "sel", "dims"]
    assert kernels.dequant_input_names(member) == streams + [table]


_HEADER_NAMES = {"IQ2_KS": "iq2_ks", "IQ2_K": "iq2_k", "IQ1_S_R4": "iq1_s_r4"}
_HEADER_TYPES = {"u8": "uint8", "u16": "uint16", "u32": "uint32", "f16": "float16"}


def test_the_abi_stream_order_is_the_format_order():
    """The C header's stream table (the order `streams` arrays are read in)
    names the same streams, dtypes and counts as the format, member by member."""
    rows = re.findall(r"^//\s+(IQ\w+)\s+(.*?)\s+\((\d+) streams\)$", HEADER.read_text(), re.M)
    assert sorted(_HEADER_NAMES[r[0]] for r in rows) == sorted(fmt.MEMBERS)
    for tag, body, count in rows:
        member = _HEADER_NAMES[tag]
        pairs = [p.strip().split() for p in body.split(",")]
        names = [p[0] for p in pairs]
        types = [_HEADER_TYPES[p[1]] for p in pairs]
        want = fmt.component_dtypes(member)
        assert names == list(want) and int(count) == len(want)
        assert types == [want[k].name for k in names]


def test_a_row_of_more_pairs_than_one_launch_takes_is_refused():
    """A launch carries at most 65535 pairs; one activation row with more
    pairs than that cannot be split between launches, so it is refused before
    anything launches (the pointers below are never dereferenced)."""
    ptrs = (ctypes.c_void_p * 5)(*([16] * 5))
    for ppr in (65536, 70000, 0):
        with pytest.raises(IqkKernelError):
            kernels._gemv_launch(0, "iq2_ks", 4096, 32, 8, 16, ptrs, 5, 16, ppr, ppr, 16, 0)
