"""The switch module on the GPU: both routes, both seams, mixed members.

Mirrors the reference's module tests (tests/test_nn.py): decode route for
small dispatches, the sorted prefill route, route agreement, the down-operand
seam with its anti-case, one layer mixing members.  References are float64
contractions of the oracle's dequantization.
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

import wirepack
from mlx_iqk_amd import format as fmt
from mlx_iqk_amd import kernels
from mlx_iqk_amd.iq1grid import grid_values
from mlx_iqk_amd.nn import (DECODE_MAT_LIMIT, IqkKernelError, IqkRuntimeError, IqkSwitchLinear, grid_table,
                             member_table, value_table)
from oracle import oracle

pytestmark = pytest.mark.gpu

EXPERTS = 8
OUT = 256


def _module(member, n, seed, device, out=OUT, experts=EXPERTS):
    wire = wirepack.random_wire(member, experts * out, n, seed=seed, scales="serving")
    streams = fmt.pack(member, wire, n)
    shapes = fmt.component_shapes(member, experts, out, n)
    module = IqkSwitchLinear(member, experts, out, n, device=device)
    module.load_streams({k: np.ascontiguousarray(v).reshape(shapes[k]) for k, v in streams.items()})
    ref = oracle.dequantize(member, wire, n).reshape(experts, out, n)
    return module, ref


def _rel(got, want):
    got = got.detach().float().cpu().numpy().astype(np.float64).reshape(want.shape)
    return np.max(np.abs(got - want)) / np.max(np.abs(want))


def test_tables_are_shared_and_exact(device):
    t = value_table(device)
    assert t.dtype == torch.float16 and value_table(device) is t
    assert np.array_equal(t.cpu().numpy().astype(np.int64), fmt.IQ2NL_VALUES.astype(np.int64))
    g = grid_table(device)
    assert g.shape == (4096,)
    assert np.array_equal(g.cpu().numpy().view(np.int8).reshape(2048, 8), grid_values())
    assert member_table("iq1_s_r4", device) is g and member_table("iq2_k", device) is t


@pytest.mark.parametrize("member", fmt.MEMBERS)
def test_load_streams_rejects_wrong_or_missing_streams(device, member):
    module, _ = _module(member, 2048, 1, device)
    streams = {k: getattr(module, k) for k in module.stream_names()}
    bad = dict(streams)
    bad["qs"] = torch.zeros((EXPERTS, OUT, 3), dtype=torch.uint32, device=device)
    with pytest.raises(IqkRuntimeError):
        module.load_streams(bad)
    missing = dict(streams)
    missing.pop(module.stream_names()[1])
    with pytest.raises(IqkRuntimeError):
        module.load_streams(missing)


@pytest.mark.parametrize("member", fmt.MEMBERS)
@pytest.mark.parametrize("n", (2048, 4096))
def test_decode_route_serves_small_dispatches(device, member, n):
    print(f"decode route {member} n={n}", flush=True)
    module, ref = _module(member, n, wirepack.seed_for(member, n), device)
    rng = np.random.default_rng(31)
    tokens, top_k = 4, 6
    assert tokens * top_k <= DECODE_MAT_LIMIT
    x = rng.standard_normal((tokens, 1, 1, n)).astype(np.float16)
    idx = rng.integers(0, EXPERTS, size=(tokens, top_k)).astype(np.int32)
    got = module(torch.from_numpy(x).to(device), torch.from_numpy(idx).to(device))
    assert tuple(got.shape) == (tokens, top_k, 1, OUT)
    want = np.stack([[ref[idx[t, k]].astype(np.float64) @ x[t, 0, 0].astype(np.float64)
                      for k in range(top_k)] for t in range(tokens)])[:, :, None, :]
    assert _rel(got, want) < 1.5e-3


@pytest.mark.parametrize("member", fmt.MEMBERS)
@pytest.mark.parametrize("n", (2048, 4096))
def test_decode_route_serves_the_down_operand_shape(device, member, n):
    module, ref = _module(member, n, wirepack.seed_for(member, n, "down"), device)
    rng = np.random.default_rng(59)
    tokens, top_k = 4, 4
    x = rng.standard_normal((tokens, top_k, 1, n)).astype(np.float16)
    idx = rng.integers(0, EXPERTS, size=(tokens, top_k)).astype(np.int32)
    got = module(torch.from_numpy(x).to(device), torch.from_numpy(idx).to(device))
    want = np.stack([[ref[idx[t, k]].astype(np.float64) @ x[t, k, 0].astype(np.float64)
                      for k in range(top_k)] for t in range(tokens)])[:, :, None, :]
    assert _rel(got, want) < 1.5e-3
    # anti-case: a module that read row 0 for every pair would differ
    shared = np.stack([[ref[idx[t, k]].astype(np.float64) @ x[t, 0, 0].astype(np.float64)
                        for k in range(top_k)] for t in range(tokens)])[:, :, None, :]
    assert np.max(np.abs(shared - want)) > 1e-2 * np.max(np.abs(want))


@pytest.mark.parametrize("member", fmt.MEMBERS)
@pytest.mark.parametrize("n", (2048, 4096))
def test_prefill_route_serves_sorted_dispatches(device, member, n):
    print(f"prefill route {member} n={n}", flush=True)
    module, ref = _module(member, n, wirepack.seed_for(member, n, "prefill"), device)
    rng = np.random.default_rng(37)
    tokens, top_k = 24, 4
    x = rng.standard_normal((tokens, 1, 1, n)).astype(np.float16)
    idx = np.sort(rng.integers(0, EXPERTS, size=(tokens, top_k)), axis=None).reshape(tokens, top_k).astype(np.int32)
    got = module(torch.from_numpy(x).to(device), torch.from_numpy(idx).to(device), sorted_indices=True)
    assert tuple(got.shape) == (tokens, top_k, 1, OUT)
    assert _rel(got, oracle.prefill_reference(ref, x, idx)) < 3e-3


@pytest.mark.parametrize("member", fmt.MEMBERS)
def test_prefill_route_serves_unsorted_and_sparse_routing(device, member):
    """Above the decode limit without sorting: pairs are grouped on the device;
    only some experts are routed, so compaction leaves slots empty."""
    n = 2048
    module, ref = _module(member, n, 43, device)
    rng = np.random.default_rng(47)
    tokens, top_k = 40, 2
    x = rng.standard_normal((tokens, 1, 1, n)).astype(np.float16)
    idx = rng.choice([1, 6, 3], size=(tokens, top_k)).astype(np.int32)
    assert idx.size > DECODE_MAT_LIMIT
    got = module(torch.from_numpy(x).to(device), torch.from_numpy(idx).to(device))
    assert _rel(got, oracle.prefill_reference(ref, x, idx)) < 3e-3


@pytest.mark.parametrize("member", fmt.MEMBERS)
def test_prefill_route_serves_the_sorted_pair_operand(device, member):
    """x [P, 1, in] with indices [P], the shape a sorting caller hands over."""
    n = 4096
    module, ref = _module(member, n, 53, device)
    rng = np.random.default_rng(61)
    P = 100
    x = rng.standard_normal((P, 1, n)).astype(np.float16)
    idx = np.sort(rng.integers(0, EXPERTS, size=P)).astype(np.int32)
    got = module(torch.from_numpy(x).to(device), torch.from_numpy(idx).to(device), sorted_indices=True)
    assert tuple(got.shape) == (P, 1, OUT)
    assert _rel(got, oracle.prefill_reference(ref, x, idx)) < 3e-3


@pytest.mark.parametrize("fused", (True, False))
@pytest.mark.parametrize("member", fmt.MEMBERS)
def test_prefill_marks_out_of_range_experts_with_nan(device, member, fused):
    """Ids outside [0, num_experts) -- the stack size, -1, and an int64 id past
    2^32 that would wrap into range as 32 bits -- reach no index op: their
    pairs come back as NaN rows, as on the decode route, and every other
    pair is unaffected.  Both prefill routes, unsorted routing."""
    n = 2048
    module, ref = _module(member, n, 211, device)
    rng = np.random.default_rng(213)
    tokens, top_k = 20, 4
    x = rng.standard_normal((tokens, 1, 1, n)).astype(np.float16)
    idx = rng.integers(0, EXPERTS, size=(tokens, top_k)).astype(np.int64)
    bad = np.zeros_like(idx, dtype=bool)
    for (t, k), e in (((3, 1), EXPERTS), ((7, 0), -1), ((11, 3), 2 ** 32 + 1), ((19, 3), EXPERTS + 100)):
        idx[t, k] = e
        bad[t, k] = True
    assert idx.size > DECODE_MAT_LIMIT
    module.fused_prefill = fused
    try:
        got = module(torch.from_numpy(x).to(device), torch.from_numpy(idx).to(device))
    finally:
        module.fused_prefill = True
    got = got.float().cpu().numpy()
    assert np.all(np.isnan(got[bad])) and not np.any(np.isnan(got[~bad]))
    want = oracle.prefill_reference(ref, x, np.where(bad, 0, idx))
    keep = got[~bad].astype(np.float64)
    assert np.max(np.abs(keep - want[~bad])) / np.max(np.abs(want[~bad])) < 3e-3
    # the decode route: the same ids, 32-bit wrap included, give NaN rows too
    dec = module(torch.from_numpy(x[:12]).to(device), torch.from_numpy(idx[:12]).to(device)).float().cpu().numpy()
    assert np.all(np.isnan(dec[bad[:12]])) and not np.any(np.isnan(dec[~bad[:12]]))


@pytest.mark.parametrize("fused", (True, False))
@pytest.mark.parametrize("member", fmt.MEMBERS)
def test_prefill_confines_non_finite_activations_to_their_rows(device, member, fused):
    """An inf in one token's activations and a NaN in another's make every
    output element of those tokens' pairs non-finite (each product with the
    inf is inf or, with a zero weight, NaN) and leave every other pair's row
    bit for bit as in the same call on clean activations: the contraction
    never mixes slots.  Both prefill routes."""
    n = 2048
    module, _ = _module(member, n, 223, device)
    rng = np.random.default_rng(227)
    tokens, top_k = 20, 4
    x = rng.standard_normal((tokens, 1, 1, n)).astype(np.float16)
    idx = rng.integers(0, EXPERTS, size=(tokens, top_k)).astype(np.int32)
    dirty = x.copy()
    dirty[5, 0, 0, n // 3] = np.inf
    dirty[13, 0, 0, 7] = np.nan
    poisoned = np.zeros((tokens, top_k), dtype=bool)
    poisoned[[5, 13]] = True
    module.fused_prefill = fused
    try:
        clean = module(torch.from_numpy(x).to(device), torch.from_numpy(idx).to(device))
        got = module(torch.from_numpy(dirty).to(device), torch.from_numpy(idx).to(device))
    finally:
        module.fused_prefill = True
    g = got.float().cpu().numpy()
    assert not np.any(np.isfinite(g[poisoned]))
    assert np.array_equal(_bits(got)[~poisoned], _bits(clean)[~poisoned])


@pytest.mark.parametrize("member", fmt.MEMBERS)
def test_the_two_routes_agree_on_the_same_dispatch(device, member):
    n = 2048
    module, _ = _module(member, n, 41, device)
    rng = np.random.default_rng(43)
    x = torch.from_numpy(rng.standard_normal((4, 1, 1, n)).astype(np.float16)).to(device)
    idx = torch.from_numpy(rng.integers(0, EXPERTS, size=(4, 4)).astype(np.int32)).to(device)
    decode = module.gemv(x, idx).double()
    prefill = module.prefill(x, idx).double()
    assert (decode - prefill).abs().max() / prefill.abs().max() < 3e-3


@pytest.mark.parametrize("member", fmt.MEMBERS)
def test_reloaded_streams_are_the_ones_used(device, member):
    """The module checks its streams once for the launchers; reloading them
    (new tensors at new addresses) makes the next call use the new weights on
    both routes."""
    n = 2048
    module, ref_a = _module(member, n, 71, device)
    wire_b = wirepack.random_wire(member, EXPERTS * OUT, n, seed=72, scales="serving")
    shapes = fmt.component_shapes(member, EXPERTS, OUT, n)
    ref_b = oracle.dequantize(member, wire_b, n).reshape(EXPERTS, OUT, n)
    rng = np.random.default_rng(9)
    x = rng.standard_normal((4, 1, 1, n)).astype(np.float16)
    idx = np.stack([rng.choice(EXPERTS, 3, replace=False) for _ in range(4)]).astype(np.int64)
    xt, it = torch.from_numpy(x).to(device), torch.from_numpy(idx).to(device)
    want = lambda ref: np.einsum("tn,tkon->tko", x[:, 0, 0].astype(np.float64), ref[idx].astype(np.float64))
    for sorted_ in (False, True):
        assert _rel(module(xt, it, sorted_indices=sorted_)[..., 0, :], want(ref_a)) < 3e-3
    module.load_streams({k: np.ascontiguousarray(v).reshape(shapes[k]) for k, v in fmt.pack(member, wire_b, n).items()})
    for sorted_ in (False, True):
        assert _rel(module(xt, it, sorted_indices=sorted_)[..., 0, :], want(ref_b)) < 3e-3


@pytest.mark.parametrize("member", fmt.MEMBERS)
def test_gemv_refuses_a_pair_count_that_does_not_tile_the_rows(device, member):
    module, _ = _module(member, 2048, 61, device)
    x = torch.zeros((3, 1, 1, 2048), dtype=torch.float16, device=device)
    idx = torch.zeros((1, 4), dtype=torch.int32, device=device)
    with pytest.raises(IqkRuntimeError):
        module.gemv(x, idx)


def test_one_layer_can_mix_members(device):
    rng = np.random.default_rng(47)
    projections = [
        ("gate", *_module("iq2_ks", 4096, 51, device), 4096),
        ("up", *_module("iq2_k", 4096, 53, device), 4096),
        ("down", *_module("iq1_s_r4", 2048, 57, device, out=512), 2048),
    ]
    tokens, top_k = 4, 4
    idx = rng.integers(0, EXPERTS, size=(tokens, top_k)).astype(np.int32)
    for name, module, ref, n in projections:
        x = rng.standard_normal((tokens, 1, 1, n)).astype(np.float16)
        got = module(torch.from_numpy(x).to(device), torch.from_numpy(idx).to(device))
        want = np.stack([[ref[idx[t, k]].astype(np.float64) @ x[t, 0, 0].astype(np.float64)
                          for k in range(top_k)] for t in range(tokens)])[:, :, None, :]
        assert _rel(got, want) < 1.5e-3, name


def test_routed_geometry_at_full_size(device):
    """256 experts at the gate/up geometry: sampled rows of a top-6 dispatch.

    Full-size parity through a size-independent property: every sampled
    output row equals its float64 reference, whichever expert it came from.
    """
    print("full-size routed geometry", flush=True)
    member, E, out, n = "iq2_ks", 256, 2048, 4096
    wire = wirepack.random_wire(member, E * out, n, seed=2024, scales="serving")
    shapes = fmt.component_shapes(member, E, out, n)
    module = IqkSwitchLinear(member, E, out, n, device=device)
    module.load_streams({k: np.ascontiguousarray(v).reshape(shapes[k])
                         for k, v in fmt.pack(member, wire, n).items()})
    rng = np.random.default_rng(6)
    sel = rng.choice(E, 6, replace=False).astype(np.int32)
    x = rng.standard_normal((1, 1, 1, n)).astype(np.float16)
    got = module(torch.from_numpy(x).to(device), torch.from_numpy(sel[None]).to(device))
    got = got.float().cpu().numpy().reshape(6, out).astype(np.float64)
    rows = rng.choice(out, 64, replace=False)
    for k, e in enumerate(sel):
        w = oracle.dequantize(member, wire[e * out + rows], n).astype(np.float64)
        want = w @ x[0, 0, 0].astype(np.float64)
        assert np.max(np.abs(got[k, rows] - want)) / np.max(np.abs(want)) < 1.5e-3, e


# -- sorted and union GEMVs (reference: tests/test_nn.py:180-295) ------------

IQ2 = ("iq2_ks", "iq2_k")


def _union_operands(idx, top_k, device):
    """Pairs sorted by expert: the sorted ids, each pair's token row, the
    order and its inverse."""
    flat = torch.from_numpy(np.ascontiguousarray(idx).reshape(-1).astype(np.int64)).to(device)
    order = torch.argsort(flat, stable=True)
    sorted_ids = flat[order].to(torch.int32)
    toks = (order // top_k).to(torch.int32)
    inv = torch.argsort(order)
    return sorted_ids, toks, order, inv


def _bits(t):
    return t.contiguous().view(torch.int16).cpu().numpy()


@pytest.mark.parametrize("member", IQ2)
@pytest.mark.parametrize("n", (2048, 4096))
@pytest.mark.parametrize("out", (OUT, 48))
def test_union_gemv_is_bit_identical_to_the_pair_gemv(device, member, n, out):
    """Duplicate-heavy selection: runs start at pair 0 and end at the last
    pair.  out=48 is not a multiple of the 32-row MFMA workgroup, so the
    VALU GEMV serves it."""
    print(f"union gemv {member} n={n} out={out}", flush=True)
    module, _ = _module(member, n, wirepack.seed_for(member, n, "union"), device, out=out)
    rng = np.random.default_rng(71)
    tokens, top_k = 6, 6
    idx = rng.integers(0, 5, size=(tokens, top_k)).astype(np.int32)
    x = torch.from_numpy(rng.standard_normal((tokens, 1, 1, n)).astype(np.float16)).to(device)
    pair = module.gemv(x, torch.from_numpy(idx).to(device))
    sorted_ids, toks, _order, inv = _union_operands(idx, top_k, device)
    got = module.gemv_union(x, sorted_ids, toks)
    assert tuple(got.shape) == (tokens * top_k, out)
    assert np.array_equal(_bits(got[inv].reshape(pair.shape)), _bits(pair))


@pytest.mark.parametrize("member", IQ2)
@pytest.mark.parametrize("n", (2048, 4096))
def test_union_gemv_serves_the_down_operand_shape(device, member, n):
    """One activation row per pair: toks is the sort order itself."""
    module, ref = _module(member, n, wirepack.seed_for(member, n, "union_down"), device)
    rng = np.random.default_rng(73)
    tokens, top_k = 6, 6
    idx = rng.integers(0, 5, size=(tokens, top_k)).astype(np.int32)
    xn = rng.standard_normal((tokens, top_k, 1, n)).astype(np.float16)
    x = torch.from_numpy(xn).to(device)
    pair = module.gemv(x, torch.from_numpy(idx).to(device))
    sorted_ids, _toks, order, inv = _union_operands(idx, top_k, device)
    got = module.gemv_union(x, sorted_ids, order.to(torch.int32))[inv].reshape(pair.shape)
    assert np.array_equal(_bits(got), _bits(pair))
    want = np.stack([[ref[idx[t, k]].astype(np.float64) @ xn[t, k, 0].astype(np.float64)
                      for k in range(top_k)] for t in range(tokens)])[:, :, None, :]
    assert _rel(got, want) < 1.5e-3


@pytest.mark.parametrize("member", IQ2)
def test_union_gemv_covers_the_run_extremes(device, member):
    """A single all-pairs run and an all-distinct selection both serve."""
    n = 2048
    module, _ = _module(member, n, 79, device)
    rng = np.random.default_rng(83)
    tokens, top_k = 4, 2
    x = torch.from_numpy(rng.standard_normal((tokens, 1, 1, n)).astype(np.float16)).to(device)
    for idx in (np.full((tokens, top_k), 3, dtype=np.int32),
                np.arange(tokens * top_k, dtype=np.int32).reshape(tokens, top_k)):
        pair = module.gemv(x, torch.from_numpy(idx).to(device))
        sorted_ids, toks, _order, inv = _union_operands(idx, top_k, device)
        for fn in (module.gemv_union, module.gemv_sorted):
            got = fn(x, sorted_ids, toks)[inv].reshape(pair.shape)
            assert np.array_equal(_bits(got), _bits(pair))


@pytest.mark.parametrize("member", IQ2)
def test_union_runs_past_the_id_batch_and_invalid_ids(device, member):
    """Runs of 1 to 10 pairs and ids beyond the stack (0xFFFFFFFF first, the
    stack size last): the union form equals the sorted form bit for bit, and
    invalid ids give NaN rows."""
    n = 2048
    module, _ = _module(member, n, 97, device)
    runs = [(0xFFFFFFFF, 1), (0, 10), (1, 1), (2, 7), (3, 8), (1, 3), (EXPERTS, 3)]
    ids = np.concatenate([np.full(k, e, dtype=np.uint32) for e, k in runs])
    rng = np.random.default_rng(101)
    rows = 9
    x = torch.from_numpy(rng.standard_normal((rows, n)).astype(np.float16)).to(device)
    toks = torch.from_numpy(rng.integers(0, rows, size=ids.size).astype(np.int32)).to(device)
    sel = torch.from_numpy(ids.view(np.int32)).to(device)
    ys, yu = (kernels.gemv_sorted(member, x, module._streams(), sel, toks, EXPERTS, OUT, union=u)
              for u in (False, True))
    assert np.array_equal(_bits(yu), _bits(ys))
    bad = ids >= EXPERTS
    y = yu.float().cpu().numpy()
    assert np.all(np.isnan(y[bad])) and not np.any(np.isnan(y[~bad]))


@pytest.mark.parametrize("member", IQ2)
@pytest.mark.parametrize("tail", (0, 1, 2))
def test_union_serves_every_run_layout_of_a_workgroup(device, member, tail):
    """A union workgroup serves pairs 3z .. 3z+2: one run of three, runs of
    two and one in either order, three runs, an id repeated after another
    (unsorted input), invalid ids inside and at the edge of a group, and a
    last group of 1 or 2 pairs.  Equal to the sorted form bit for bit, NaN
    rows exactly for the invalid ids; also for 1 and 2 pairs in all."""
    n = 2048
    module, _ = _module(member, n, 103, device)
    groups = [(5, 5, 5), (5, 5, 6), (6, 7, 7), (1, 2, 3), (2, 4, 2), (EXPERTS, 0, 0), (0, 0xFFFFFFFF, 1),
              (3, 3, EXPERTS)]
    ids = np.array([e for grp in groups for e in grp] + [4, 4][:tail], dtype=np.uint32)
    rng = np.random.default_rng(107 + tail)
    rows = 7
    x = torch.from_numpy(rng.standard_normal((rows, n)).astype(np.float16)).to(device)
    for k in (ids.size, 1, 2):
        print(f"union run layouts {member} pairs={k}", flush=True)
        sel = torch.from_numpy(ids[:k].view(np.int32)).to(device)
        toks = torch.from_numpy(rng.integers(0, rows, size=k).astype(np.int32)).to(device)
        ys, yu = (kernels.gemv_sorted(member, x, module._streams(), sel, toks, EXPERTS, OUT, union=u)
                  for u in (False, True))
        assert np.array_equal(_bits(yu), _bits(ys))
        bad = ids[:k] >= EXPERTS
        y = yu.float().cpu().numpy()
        assert np.all(np.isnan(y[bad])) and not np.any(np.isnan(y[~bad]))


@pytest.mark.parametrize("member", IQ2)
@pytest.mark.parametrize("n", (2048, 4096))
@pytest.mark.parametrize("out", (OUT, 48))
def test_sorted_gemv_is_bit_identical_to_the_pair_gemv(device, member, n, out):
    module, _ = _module(member, n, wirepack.seed_for(member, n, "adj"), device, out=out)
    rng = np.random.default_rng(91)
    tokens, top_k = 6, 6
    idx = rng.integers(0, 5, size=(tokens, top_k)).astype(np.int32)
    x = torch.from_numpy(rng.standard_normal((tokens, 1, 1, n)).astype(np.float16)).to(device)
    pair = module.gemv(x, torch.from_numpy(idx).to(device))
    sorted_ids, toks, _order, inv = _union_operands(idx, top_k, device)
    got = module.gemv_sorted(x, sorted_ids, toks)
    assert np.array_equal(_bits(got[inv].reshape(pair.shape)), _bits(pair))


@pytest.mark.parametrize("method", ("gemv_sorted", "gemv_union"))
@pytest.mark.parametrize("member", IQ2)
def test_sorted_and_union_refuse_a_toks_pair_mismatch(device, member, method):
    module, _ = _module(member, 2048, 93, device)
    x = torch.zeros((2, 1, 1, 2048), dtype=torch.float16, device=device)
    sorted_ids = torch.zeros(8, dtype=torch.int32, device=device)
    toks = torch.zeros(6, dtype=torch.int32, device=device)
    with pytest.raises(IqkRuntimeError):
        getattr(module, method)(x, sorted_ids, toks)


@pytest.mark.parametrize("method", ("gemv_sorted", "gemv_union"))
def test_sorted_and_union_refuse_iq1_s_r4(device, method):
    """The recorded sorted/union formulations cover the IQ2 members only."""
    module, _ = _module("iq1_s_r4", 2048, 95, device)
    x = torch.zeros((2, 1, 1, 2048), dtype=torch.float16, device=device)
    ids = torch.zeros(4, dtype=torch.int32, device=device)
    with pytest.raises(IqkKernelError):
        getattr(module, method)(x, ids, ids)


@pytest.mark.parametrize("method", ("gemv_sorted", "gemv_union"))
@pytest.mark.parametrize("out", (OUT, 48))
def test_sorted_and_union_mark_out_of_range_rows(device, method, out):
    """A token row beyond x, or an id beyond the stack, gives a NaN output
    row and reads nothing out of bounds; the other rows are unaffected."""
    module, _ = _module("iq2_ks", 2048, 97, device, out=out)
    rng = np.random.default_rng(99)
    x = torch.from_numpy(rng.standard_normal((3, 1, 1, 2048)).astype(np.float16)).to(device)
    ids = torch.tensor([1, 1, 1, 2, EXPERTS, 5], dtype=torch.int32, device=device)
    toks = torch.tensor([0, 3, 2, 1, 0, 2], dtype=torch.int32, device=device)
    got = getattr(module, method)(x, ids, toks)
    bad = torch.tensor([False, True, False, False, True, False])
    assert torch.isnan(got[bad.to(device)]).all()
    good_ids = torch.tensor([[1], [1], [2], [5]], dtype=torch.int32, device=device)
    good_x = x.reshape(3, -1)[torch.tensor([0, 2, 1, 2], device=device)].reshape(4, 1, 1, -1)
    want = module.gemv(good_x, good_ids).reshape(4, out)
    assert np.array_equal(_bits(got[(~bad).to(device)]), _bits(want))


@pytest.mark.parametrize("member", IQ2)
def test_union_gemv_at_the_routed_geometry(device, member):
    """256 experts, gate/up geometry, the multi-token verify shape: 8 tokens x
    top-6 over a pool of 9 experts (long runs: most workgroups serve two
    pairs) and over all experts (mostly one-pair workgroups); bit-identical
    to the pair GEMV."""
    print(f"union gemv routed geometry {member}", flush=True)
    E, out, n = 256, 2048, 4096
    wire = wirepack.random_wire(member, E * out, n, seed=2025, scales="serving")
    shapes = fmt.component_shapes(member, E, out, n)
    module = IqkSwitchLinear(member, E, out, n, device=device)
    module.load_streams({k: np.ascontiguousarray(v).reshape(shapes[k])
                         for k, v in fmt.pack(member, wire, n).items()})
    rng = np.random.default_rng(8)
    tokens, top_k = 8, 6
    for pool in (rng.choice(E, 9, replace=False), np.arange(E)):
        idx = np.stack([rng.choice(pool, top_k, replace=False) for _ in range(tokens)]).astype(np.int32)
        x = torch.from_numpy(rng.standard_normal((tokens, 1, 1, n)).astype(np.float16)).to(device)
        pair = module.gemv(x, torch.from_numpy(idx).to(device))
        sorted_ids, toks, _order, inv = _union_operands(idx, top_k, device)
        for fn in (module.gemv_union, module.gemv_sorted):
            got = fn(x, sorted_ids, toks)[inv].reshape(pair.shape)
            assert np.array_equal(_bits(got), _bits(pair))


# -- range producer and range matmul (reference: tests/test_nn.py:329-377) --


@pytest.mark.parametrize("member", fmt.MEMBERS)
@pytest.mark.parametrize("n", (2048, 4096))
def test_dequantized_range_matches_the_full_slice(device, member, n):
    """Every range is the same slice of the full reconstruction and of the
    oracle's dequantization (fp16 bits: the CPU dequantizer's float32 values
    rounded once)."""
    module, ref = _module(member, n, wirepack.seed_for(member, n, "range"), device)
    full = _bits(module.dequantized())
    want = ref.astype(np.float16).view(np.int16)
    assert np.array_equal(full, want)
    for start, rows in ((0, 8), (8, 8), (16, 16), (0, 32), (24, 8), (3, 1), (5, 2), (0, OUT), (128, 128)):
        got = _bits(module.dequantized_range(start, rows))
        assert got.shape == (EXPERTS, rows, n), (start, rows)
        assert np.array_equal(got, full[:, start:start + rows]), (start, rows)
        assert np.array_equal(got, want[:, start:start + rows]), (start, rows)


@pytest.mark.parametrize("member", fmt.MEMBERS)
def test_dequantized_range_into_compacted_slots_matches_the_oracle(device, member):
    """Ranges of the experts a routing names, compacted into slots in expert
    order (the producer route's form): each slot holds the oracle's rows of its
    expert, bit for bit; slots no expert maps to stay as they were."""
    n = 2048
    module, ref = _module(member, n, wirepack.seed_for(member, n, "range-slots"), device)
    experts = [6, 1, 4]  # slot s <- experts[s]
    slot_of = np.full(EXPERTS, -1, dtype=np.int32)
    slot_of[experts] = np.arange(len(experts))
    sot = torch.from_numpy(slot_of).to(device)
    want = ref.astype(np.float16).view(np.int16)
    for start, rows in ((0, OUT), (64, 64), (4, 4), (252, 4), (96, 32)):
        out = torch.full((len(experts) + 1, rows, n), float("nan"), dtype=torch.float16, device=device)
        got = kernels.dequant(member, module._checked(), EXPERTS, OUT, n, slot_of_expert=sot,
                              n_slots=len(experts) + 1, row_start=start, rows=rows, out=out)
        got = _bits(got)
        for s, e in enumerate(experts):
            assert np.array_equal(got[s], want[e, start:start + rows]), (start, rows, e)
        assert np.isnan(out[len(experts)].float().cpu().numpy()).all(), (start, rows)


@pytest.mark.parametrize("member", fmt.MEMBERS)
def test_dequantized_range_refuses_a_bad_range(device, member):
    module, _ = _module(member, 2048, 61, device, out=32)
    for start, rows in ((0, 0), (0, 12), (0, -8), (-8, 8), (28, 8), (0, 64)):
        with pytest.raises(IqkRuntimeError):
            module.dequantized_range(start, rows)
        with pytest.raises(IqkRuntimeError):
            module.sorted_matmul_range(torch.zeros((1, 1, 2048), dtype=torch.float16, device=device),
                                       torch.zeros(1, dtype=torch.int32, device=device), start, rows)


@pytest.mark.parametrize("member", fmt.MEMBERS)
@pytest.mark.parametrize("n", (2048, 4096))
def test_sorted_matmul_range_concat_matches_the_sorted_call(device, member, n):
    """Range outputs concatenated along features equal the unsplit call, bit
    for bit; ranges narrower than one 16-column MFMA fragment included."""
    module, _ = _module(member, n, wirepack.seed_for(member, n, "nsplit"), device)
    rng = np.random.default_rng(67)
    tokens, top_k = 24, 4
    x = torch.from_numpy(rng.standard_normal((tokens, 1, 1, n)).astype(np.float16)).to(device)
    idx = np.sort(rng.integers(0, EXPERTS, size=(tokens, top_k)), axis=None).reshape(tokens, top_k)
    idx = torch.from_numpy(idx.astype(np.int32)).to(device)
    full = module(x, idx, sorted_indices=True)
    half = OUT // 2
    parts = torch.cat([module.sorted_matmul_range(x, idx, 0, half),
                       module.sorted_matmul_range(x, idx, half, half)], dim=-1)
    assert np.array_equal(_bits(parts), _bits(full))
    narrow = torch.cat([module.sorted_matmul_range(x, idx, 64 + 8 * i, 8) for i in range(2)]
                       + [module.sorted_matmul_range(x, idx, 80, 1)], dim=-1)
    assert np.array_equal(_bits(narrow), _bits(full[..., 64:81]))


@pytest.mark.parametrize("member", fmt.MEMBERS)
@pytest.mark.parametrize("fused", (False, True))
def test_sorted_matmul_range_matches_a_float64_reference(device, member, fused):
    """Each route's ranged prefill (the producer's row range + grouped GEMM,
    and the fused contraction over the range) against float64 contractions
    of the oracle's rows of that range: the reference's prefill gate, < 3e-3
    of the output range (tests/test_nn.py:337-378)."""
    n = 2048
    module, ref = _module(member, n, wirepack.seed_for(member, n, "range-f64"), device)
    module.fused_prefill = fused
    rng = np.random.default_rng(71)
    tokens, top_k = 20, 4
    xh = rng.standard_normal((tokens, 1, 1, n)).astype(np.float16)
    idx = rng.integers(0, EXPERTS, size=(tokens, top_k)).astype(np.int32)
    x = torch.from_numpy(xh).to(device)
    it = torch.from_numpy(idx).to(device)
    try:
        for start, rows in ((0, 128), (128, 64), (200, 8), (31, 1), (0, OUT)):
            got = module.sorted_matmul_range(x, it, start, rows)
            assert tuple(got.shape) == (tokens, top_k, 1, rows), (start, rows)
            got = got.float().cpu().numpy().astype(np.float64).reshape(tokens, top_k, rows)
            want = np.stack([[ref[e, start:start + rows].astype(np.float64) @ xh[t, 0, 0].astype(np.float64)
                              for e in idx[t]] for t in range(tokens)])
            rel = np.max(np.abs(got - want)) / np.max(np.abs(want))
            assert rel < 3e-3, (start, rows, rel)
    finally:
        module.fused_prefill = True


# -- fused prefill (the weights formed inside the GEMM) ---------------------


def _both_routes(module, *args, **kw):
    module.fused_prefill = True
    fused = module(*args, **kw)
    module.fused_prefill = False
    producer = module(*args, **kw)
    module.fused_prefill = True
    return fused, producer


@pytest.mark.parametrize("member", fmt.MEMBERS)
@pytest.mark.parametrize("n", (2048, 4096))
def test_fused_prefill_matches_the_producer_route(device, member, n):
    """The producer route sums fp16 weights; the fused GEMM sums IQ2_K's same
    fp16 weights, and IQ2_KS's and IQ1_S_R4's exact products n scaled by
    the row scale d afterwards, in another order: the two routes agree to
    fp16 rounding, and each meets the float64 gate."""
    print(f"fused prefill {member} n={n}", flush=True)
    module, ref = _module(member, n, wirepack.seed_for(member, n, "fused"), device)
    rng = np.random.default_rng(101)
    tokens, top_k = 40, 4
    x = rng.standard_normal((tokens, 1, 1, n)).astype(np.float16)
    idx = np.sort(rng.integers(0, EXPERTS, size=(tokens, top_k)), axis=None).reshape(tokens, top_k).astype(np.int32)
    xt, it = torch.from_numpy(x).to(device), torch.from_numpy(idx).to(device)
    fused, producer = _both_routes(module, xt, it, sorted_indices=True)
    want = oracle.prefill_reference(ref, x, idx)
    assert _rel(fused, want) < 3e-3 and _rel(producer, want) < 3e-3
    diff = (fused.float() - producer.float()).abs().max().item()
    assert diff <= 2e-3 * producer.float().abs().max().item()


@pytest.mark.parametrize("member", fmt.MEMBERS)
def test_prefill_over_more_experts_than_one_scan_round(device, member):
    """600 experts: the GEMMs' in-block work-list scan takes 256 groups a
    round, so three rounds, with empty, one-slot and multi-tile experts in
    each (the largest, 130 slots, in the last round).  Both routes meet the
    float64 gate and agree with each other."""
    E, out, n = 600, 64, 2048
    print(f"prefill over {E} experts {member}", flush=True)
    module, ref = _module(member, n, wirepack.seed_for(member, n, "many"), device, out=out, experts=E)
    rng = np.random.default_rng(149)
    counts = rng.integers(0, 4, size=E)
    counts[[3, 255, 256, 300, 511, 512, 599]] = [70, 65, 0, 64, 1, 0, 130]
    idx = np.repeat(np.arange(E), counts).astype(np.int32).reshape(-1, 1)
    x = rng.standard_normal((idx.shape[0], 1, 1, n)).astype(np.float16)
    xt, it = torch.from_numpy(x).to(device), torch.from_numpy(idx).to(device)
    fused, producer = _both_routes(module, xt, it, sorted_indices=True)
    want = oracle.prefill_reference(ref, x, idx)
    assert _rel(fused, want) < 3e-3 and _rel(producer, want) < 3e-3
    diff = (fused.float() - producer.float()).abs().max().item()
    assert diff <= 2e-3 * producer.float().abs().max().item()


@pytest.mark.parametrize("member", fmt.MEMBERS)
@pytest.mark.parametrize("out", (48, 272))
def test_fused_prefill_serves_partial_row_blocks_and_several_rows_per_pair(device, member, out):
    """out_features not a multiple of the 256-row block; x [T, M, in] with M = 3
    rows per pair, unsorted routing over a few experts."""
    n = 2048
    module, ref = _module(member, n, 103, device, out=out)
    rng = np.random.default_rng(107)
    T, M = 30, 3
    x = rng.standard_normal((T, M, n)).astype(np.float16)
    idx = rng.choice([0, 5, 2], size=T).astype(np.int32)
    fused = module.prefill(torch.from_numpy(x).to(device), torch.from_numpy(idx).to(device))
    assert tuple(fused.shape) == (T, M, out)
    want = np.stack([x[t].astype(np.float64) @ ref[idx[t]].astype(np.float64).T for t in range(T)])
    assert _rel(fused, want) < 3e-3


@pytest.mark.parametrize("member", fmt.MEMBERS)
@pytest.mark.parametrize("n", (2048, 4096))
def test_fused_prefill_experts_of_many_tiles(device, member, n):
    """Experts that span several 64-slot M-tiles, full and partial: sizes 300
    (four full tiles and a 44-slot one), 128 (two full), 200 (three full and
    an 8-slot one), 129 (two full and a one-slot one), 64, 5, 1 and 0.  Both
    routes meet the float64 gate and agree with each other, a second fused
    call repeats the first bit for bit, and row ranges concatenate to the
    unsplit call bit for bit."""
    print(f"fused prefill many tiles {member} n={n}", flush=True)
    module, ref = _module(member, n, wirepack.seed_for(member, n, "wide"), device)
    sizes = [300, 128, 200, 1, 0, 5, 64, 129]
    assert len(sizes) == EXPERTS
    idx = np.concatenate([np.full(c, e) for e, c in enumerate(sizes)]).astype(np.int32).reshape(-1, 1)
    rng = np.random.default_rng(131)
    x = rng.standard_normal((idx.shape[0], 1, 1, n)).astype(np.float16)
    xt, it = torch.from_numpy(x).to(device), torch.from_numpy(idx).to(device)
    fused, producer = _both_routes(module, xt, it, sorted_indices=True)
    want = oracle.prefill_reference(ref, x, idx)
    assert _rel(fused, want) < 3e-3 and _rel(producer, want) < 3e-3
    diff = (fused.float() - producer.float()).abs().max().item()
    assert diff <= 2e-3 * producer.float().abs().max().item()
    assert np.array_equal(_bits(module(xt, it, sorted_indices=True)), _bits(fused))
    half = OUT // 2
    parts = torch.cat([module.sorted_matmul_range(xt, it, 0, half),
                       module.sorted_matmul_range(xt, it, half, half)], dim=-1)
    assert np.array_equal(_bits(parts), _bits(fused))


@pytest.mark.parametrize("member", fmt.MEMBERS)
@pytest.mark.parametrize("n", (2048, 4096))
@pytest.mark.parametrize("scales", ("serving", "tiny"))
def test_fused_prefill_weights_are_the_producers(device, member, n, scales):
    """A one-hot activation row e_k makes a fused output the weight column k
    itself: one product w * 1 and zeros, exact in f32 and again in fp16 (IQ2_K,
    whose operands are the fp16 weights), or the exact product n * 1 times the
    row scale d, exact in f32 and rounded once to fp16 (IQ2_KS, IQ1_S_R4).  So
    every decoded weight the fused GEMM forms in registers is checked against
    the producer's dequantized stack by value (a -0 weight comes out +0 after
    the zero products, so zeros compare by value).  `tiny` scales are all
    subnormal, so many weights are subnormal or round to zero: the fused
    arithmetic must round them as the producer's f32 chain does."""
    print(f"fused weights {member} n={n} {scales}", flush=True)
    wire = wirepack.random_wire(member, EXPERTS * OUT, n, seed=wirepack.seed_for(member, n, "onehot"), scales=scales)
    shapes = fmt.component_shapes(member, EXPERTS, OUT, n)
    module = IqkSwitchLinear(member, EXPERTS, OUT, n, device=device)
    module.load_streams({k: np.ascontiguousarray(v).reshape(shapes[k]) for k, v in fmt.pack(member, wire, n).items()})
    stack = module.dequantized().float().cpu().numpy()  # [E, OUT, n]
    rng = np.random.default_rng(149)
    per_expert = 40  # two 32-slot blocks: both MFMA row blocks carry columns
    cols = np.stack([rng.choice(n, per_expert, replace=False) for _ in range(EXPERTS)])
    idx = np.repeat(np.arange(EXPERTS), per_expert).astype(np.int32).reshape(-1, 1)
    x = np.zeros((idx.shape[0], 1, 1, n), dtype=np.float16)
    x[np.arange(idx.shape[0]), 0, 0, cols.reshape(-1)] = 1.0
    module.fused_prefill = True
    got = module(torch.from_numpy(x).to(device), torch.from_numpy(idx).to(device), sorted_indices=True)
    got = got.float().cpu().numpy().reshape(EXPERTS, per_expert, OUT)
    want = np.stack([stack[e][:, cols[e]].T for e in range(EXPERTS)])
    assert np.isfinite(want).all()
    if scales == "tiny":  # the case is what it says: many subnormal weights
        assert np.mean((want != 0) & (np.abs(want) < 2.0 ** -14)) > 0.1
    assert np.array_equal(got, want)


@pytest.mark.parametrize("member", fmt.MEMBERS)
def test_fused_prefill_at_the_routed_geometry(device, member):
    """256 experts at the gate/up geometry, a Zipf-skewed 64-token top-6
    prefill: sampled output rows against float64.  IQ2_K at this width is the
    form whose super-block scales come from global memory, not LDS."""
    print(f"fused prefill routed geometry {member}", flush=True)
    E, out, n = 256, 2048, 4096
    wire = wirepack.random_wire(member, E * out, n, seed=2026, scales="serving")
    shapes = fmt.component_shapes(member, E, out, n)
    module = IqkSwitchLinear(member, E, out, n, device=device)
    module.load_streams({k: np.ascontiguousarray(v).reshape(shapes[k])
                         for k, v in fmt.pack(member, wire, n).items()})
    rng = np.random.default_rng(9)
    T, K = 64, 6
    p = 1.0 / np.arange(1, E + 1) ** 1.1
    idx = np.stack([rng.choice(E, K, replace=False, p=p / p.sum()) for _ in range(T)]).astype(np.int32)
    x = rng.standard_normal((T, 1, 1, n)).astype(np.float16)
    got = module(torch.from_numpy(x).to(device), torch.from_numpy(idx).to(device), sorted_indices=True)
    got = got.float().cpu().numpy().reshape(T, K, out).astype(np.float64)
    # whole four-row groups: IQ1_S_R4's wire interleaves the rows of a group
    rows = (4 * rng.choice(out // 4, 12, replace=False)[:, None] + np.arange(4)).reshape(-1)
    for t in range(0, T, 7):
        for k in range(K):
            w = oracle.dequantize(member, wire[idx[t, k] * out + rows], n).astype(np.float64)
            want = w @ x[t, 0, 0].astype(np.float64)
            assert np.max(np.abs(got[t, k, rows] - want)) / np.max(np.abs(want)) < 3e-3, (t, k)
