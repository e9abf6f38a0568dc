"""The device-side route (iqk_route) against a numpy stable sort.

The route groups token-expert pairs into expert-sorted slots for the prefill
kernels.  Reference: numpy's stable argsort of the ids (an id outside
[0, E) sorted as expert 0), each pair expanded to its rows; offsets are the
cumulative slot counts.  Also the module's two prefill routes through it, at
shapes where x broadcasts over trailing dims (one launch) and where it does
not (the torch bookkeeping), against the float64 gate.
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

import wirepack
from mlx_iqk_amd import format as fmt
from mlx_iqk_amd import kernels
from mlx_iqk_amd.nn import IqkSwitchLinear
from oracle import oracle

pytestmark = pytest.mark.gpu


def _reference(ids: np.ndarray, E: int, M: int, ppx: int, n_x_rows: int):
    valid = ids.astype(np.uint32) < E
    key = np.where(valid, ids, 0).astype(np.int64)
    order = np.argsort(key, kind="stable")
    counts = np.bincount(key, minlength=E) * M
    offs = np.concatenate([[0], np.cumsum(counts)]).astype(np.int64)
    r = np.arange(M)
    x_rows = np.where(valid[order][:, None], (order // ppx)[:, None] * M + r, n_x_rows).reshape(-1)
    y_rows = (order[:, None] * M + r).reshape(-1)
    return offs, x_rows, y_rows


# past 16384 pairs a wavefront's share exceeds the ids it holds (2048), and
# its second pass reloads them round by round: 40000 (three rounds) and
# 16385 at the most experts the route serves
@pytest.mark.parametrize("P,E,M,ppx", [(12288, 256, 1, 1), (12288, 256, 1, 6), (300, 8, 3, 1), (1, 1, 1, 1),
                                       (5000, 4096, 2, 5), (1023, 33, 1, 1), (2049, 256, 1, 2),
                                       (40000, 256, 1, 8), (16385, 4096, 1, 1)])
def test_route_matches_a_stable_sort(device, P, E, M, ppx):
    print(f"route P={P} E={E} M={M} ppx={ppx}", flush=True)
    rng = np.random.default_rng(P + E)
    p = 1.0 / np.arange(1, E + 1) ** 1.1
    ids = rng.choice(E, size=P, p=p / p.sum()).astype(np.int64)
    if P > 10:  # ids past the stack: E, -1 (0xFFFFFFFF), and a large one
        ids[[3, P // 2, P - 1]] = [E, -1, E + 12345]
    n_x_rows = ((P + ppx - 1) // ppx) * M
    got = kernels.route(torch.from_numpy(ids.astype(np.int32)).to(device), E, M, ppx, n_x_rows)
    want = _reference(ids, E, M, ppx, n_x_rows)
    for g, w, name in zip(got, want, ("offsets", "x_rows", "y_rows")):
        assert np.array_equal(g.cpu().numpy().astype(np.int64), w), name
    again = kernels.route(torch.from_numpy(ids.astype(np.int32)).to(device), E, M, ppx, n_x_rows)
    assert all(torch.equal(a, b) for a, b in zip(got, again))


def test_route_of_no_pairs(device):
    offs, xr, yr = kernels.route(torch.zeros(0, dtype=torch.int32, device=device), 16)
    assert offs.cpu().numpy().tolist() == [0] * 17 and xr.numel() == 0 and yr.numel() == 0


@pytest.mark.parametrize("fused", (True, False))
@pytest.mark.parametrize("xshape,ishape", [((6, 1, 1), (6, 4)), ((1, 1), (5, 3)), ((2, 1, 1, 1), (2, 3, 4)),
                                           ((1, 4, 1), (3, 4))])
def test_prefill_route_broadcast_shapes(device, fused, xshape, ishape):
    """x batch shapes broadcast against the indices: over trailing dims only
    (the device route) and over a leading dim (x [1, 4] against [3, 4]: the
    torch bookkeeping); M = 2 rows per pair.  Both prefill routes meet the
    float64 gate."""
    n, E, out = 2048, 8, 64
    member = "iq2_k"
    wire = wirepack.random_wire(member, E * out, n, seed=wirepack.seed_for("route", xshape, ishape), scales="serving")
    shapes = fmt.component_shapes(member, E, out, n)
    module = IqkSwitchLinear(member, E, out, n, device=device)
    module.load_streams({k: np.ascontiguousarray(v).reshape(shapes[k]) for k, v in fmt.pack(member, wire, n).items()})
    ref = oracle.dequantize(member, wire, n).reshape(E, out, n)
    rng = np.random.default_rng(7)
    M = 2
    x = rng.standard_normal(xshape[:-1] + (M, n)).astype(np.float16)
    idx = rng.integers(0, E, size=ishape).astype(np.int32)
    module.fused_prefill = fused
    try:
        got = module.prefill(torch.from_numpy(x).to(device), torch.from_numpy(idx).to(device))
    finally:
        module.fused_prefill = True
    want = oracle.prefill_reference(ref, x, idx)
    g = got.float().cpu().numpy().astype(np.float64)
    assert g.shape == want.shape
    assert np.max(np.abs(g - want)) / np.max(np.abs(want)) < 3e-3
