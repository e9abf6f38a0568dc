"""ik wire -> relayout on the GPU: the bytes format.pack writes, bit for bit.

format.pack (the CPU relayout, itself checked against the reference's layout
and the oracle in tests/test_format.py) is the reference here.  Odd row counts
exercise a block's 2-byte tail; full-range random wire reaches every field
value.
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

import wirepack
from mlx_iqk_amd import format as fmt
from mlx_iqk_amd import kernels
from mlx_iqk_amd.nn import IqkSwitchLinear

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("member", fmt.MEMBERS)
@pytest.mark.parametrize("n", (2048, 4096))
@pytest.mark.parametrize("rows", (4, 36, 204))
def test_gpu_pack_is_format_pack(device, member, n, rows):
    wire = wirepack.random_wire(member, rows, n, seed=rows + n, scales="sweep")
    want = fmt.pack(member, wire, n)
    got = kernels.pack(member, torch.from_numpy(np.ascontiguousarray(wire)).to(device), n)
    assert set(got) == set(want)
    for k, v in want.items():
        g = got[k].cpu().numpy()
        assert g.shape == v.shape and g.dtype == v.dtype, k
        assert np.array_equal(g.view(np.uint8), np.ascontiguousarray(v).view(np.uint8)), (member, n, rows, k)


@pytest.mark.parametrize("member", ("iq2_ks", "iq2_k"))
@pytest.mark.parametrize("rows", (1, 17, 33))
def test_gpu_pack_takes_odd_row_counts(device, member, rows):
    n = 2048
    wire = wirepack.random_wire(member, rows, n, seed=rows, scales="sweep")
    want = fmt.pack(member, wire, n)
    got = kernels.pack(member, torch.from_numpy(np.ascontiguousarray(wire)).to(device), n)
    for k, v in want.items():
        assert np.array_equal(got[k].cpu().numpy().view(np.uint8), np.ascontiguousarray(v).view(np.uint8)), k


@pytest.mark.parametrize("member", fmt.MEMBERS)
def test_load_wire_matches_load_streams(device, member):
    """A module loaded from wire on the device equals one loaded from the CPU relayout."""
    E, out, n = 4, 64, 2048
    wire = wirepack.random_wire(member, E * out, n, seed=5, scales="serving")
    shapes = fmt.component_shapes(member, E, out, n)
    a = IqkSwitchLinear(member, E, out, n, device=device)
    a.load_streams({k: np.ascontiguousarray(v).reshape(shapes[k]) for k, v in fmt.pack(member, wire, n).items()})
    b = IqkSwitchLinear(member, E, out, n, device=device)
    b.load_wire(torch.from_numpy(np.ascontiguousarray(wire)).to(device))
    for k in a.stream_names():
        assert torch.equal(getattr(a, k).view(torch.uint8), getattr(b, k).view(torch.uint8)), k
