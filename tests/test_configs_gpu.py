"""The routed workloads at their full size, on the GPU, against the oracle.

One test per workload of the hot path, at the real geometry (256 experts;
gate/up [2048 x 4096], down [4096 x 2048]), so every kernel instantiation
those workloads launch runs here against the oracle:

* single IQ2_KS expert, seed-0 rows quantized by the package codec: the full
  dequantization bit-exact, then the GEMV;
* IQ2_K routed decode, 8 tokens x top-6 unsorted (the down dispatch is the
  6144-workgroup two-row-block form);
* IQ1_S_R4 routed decode, 1 token x top-6 (and 2 and 4 tokens, the two-row-
  block form) at both geometries;
* the 2048-token Zipf(1.1) mixed-member prefill (IQ2_KS gate, IQ2_K down),
  sorted, through the fused route and the producer + grouped GEMM route, and
  its gate projection in IQ1_S_R4 and in IQ2_K;
* the decode workloads and the prefill again on codec-quantized stacks.

Stacks are serving-scale random ik wire (every code, scale index and
alphabet/shift value occurs), relaid on the GPU by ``load_wire``; the
expected values are float64 contractions of ``oracle.dequantize`` of the same
wire, on sampled output rows (a size-independent property: every sampled row
equals its reference, whichever expert and token it came from).  The gates
are the reference's (tests/test_kernels.py:161-188, tests/test_nn.py:118-149):
decode ``max|d|/max|ref| < 1.5e-3``, rel-L2 <= 1e-3, > 99% of outputs at 0
fp16 ULP; prefill ``< 3e-3``.
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

import wirepack
from mlx_iqk_amd import codec
from mlx_iqk_amd import format as fmt
from mlx_iqk_amd import synth
from mlx_iqk_amd.nn import IqkSwitchLinear
from oracle import oracle

pytestmark = pytest.mark.gpu

E, TOP_K = 256, 6
GU = (2048, 4096)  # out, in
DN = (4096, 2048)

_STACKS: dict = {}


def _stack(member, out, n, seed, device):
    """A 256-expert module of serving-scale random wire (cached per test session)."""
    key = (member, out, n, seed)
    if key not in _STACKS:
        print(f"  building {member} {E}x{out}x{n} (seed {seed})", flush=True)
        wire = wirepack.random_wire(member, E * out, n, seed=seed, scales="serving")
        module = IqkSwitchLinear(member, E, out, n, device=device)
        module.load_wire(torch.from_numpy(wire).to(device))
        torch.cuda.synchronize()
        _STACKS[key] = (module, wire)
    return _STACKS[key]


@pytest.fixture(scope="module", autouse=True)
def _free_stacks():
    yield
    _STACKS.clear()
    torch.cuda.empty_cache()


def _fp16_ulp(got, want):
    def order(a):
        i = a.astype(np.float16).view(np.int16).astype(np.int64)
        return np.where(i < 0, np.int64(-32768) - i, i)
    return np.abs(order(got) - order(want))


def _rows_sample(rng, out, count, member):
    """Sampled output rows; whole four-row groups (IQ1_S_R4 wire interleaves them)."""
    groups = rng.choice(out // 4, count // 4, replace=False)
    return np.sort((4 * groups[:, None] + np.arange(4)).reshape(-1))


def _expected(member, wire, out, n, expert, rows, x):
    w = oracle.dequantize(member, wire[expert * out + rows], n).astype(np.float64)
    return w @ x.astype(np.float64)


def _check_decode(got, want, label):
    got = got.astype(np.float64)
    rel = np.max(np.abs(got - want)) / np.max(np.abs(want))
    l2 = np.linalg.norm(got - want) / np.linalg.norm(want)
    exact = float(np.mean(_fp16_ulp(got, want.astype(np.float16)) == 0))
    assert rel < 1.5e-3, (label, rel)
    assert l2 <= 1e-3, (label, l2)
    assert exact > 0.99, (label, exact)
    return rel, l2, exact


def _quantized_stack(member, out, n, seed, device, distinct=4):
    """A 256-expert module whose rows are N(0, 0.02) rows quantized by the
    package codec under a U(0.1, 1) imatrix (the workloads' stacks).
    Quantizing 256 experts is minutes of host search, so ``distinct`` experts
    are quantized and expert e holds tile e % distinct with its rows rotated
    by e // distinct (whole four-row groups), as the benchmark's stacks are
    built; every expert still owns its bytes at its own address."""
    key = ("quantized", member, out, n, seed)
    if key not in _STACKS:
        print(f"  quantizing {member} {distinct}x{out}x{n} (seed {seed}) into a {E}-expert stack", flush=True)
        tiles = [synth.quantized_rows(member, out, n, seed + t, imatrix_seed=seed + 1000) for t in range(distinct)]
        group = 4 if member == "iq1_s_r4" else 1
        wire = np.empty((E * out, tiles[0].shape[1]), dtype=np.uint8)
        for e in range(E):
            shift = group * ((e // distinct) % (out // group))
            wire[e * out:(e + 1) * out] = np.roll(tiles[e % distinct], shift, axis=0)
        module = IqkSwitchLinear(member, E, out, n, device=device)
        module.load_wire(torch.from_numpy(wire).to(device))
        torch.cuda.synchronize()
        _STACKS[key] = (module, wire)
    return _STACKS[key]


def _decode_case(device, member, tokens, seed, quantized=False):
    """Gate and down projections of one routed decode step: every pair, 64 sampled rows each."""
    rng = np.random.default_rng(seed)
    idx = np.stack([rng.choice(E, TOP_K, replace=False) for _ in range(tokens)]).astype(np.int32)
    it = torch.from_numpy(idx).to(device)
    for name, (out, n), x_shape in (("gate", GU, (tokens, 1, 1, GU[1])), ("down", DN, (tokens, TOP_K, 1, DN[1]))):
        if quantized:
            module, wire = _quantized_stack(member, out, n, wirepack.seed_for("quantized", member, name), device)
        else:
            module, wire = _stack(member, out, n, wirepack.seed_for("config", member, name), device)
        x = rng.standard_normal(x_shape).astype(np.float16)
        print(f"  {member} {name} {tokens} token(s) x top-{TOP_K}", flush=True)
        y = module(torch.from_numpy(x).to(device), it)
        assert tuple(y.shape) == (tokens, TOP_K, 1, out)
        y = y.float().cpu().numpy().reshape(tokens, TOP_K, out)
        rows = _rows_sample(rng, out, 64, member)
        got, want = [], []
        for t in range(tokens):
            for k in range(TOP_K):
                xv = x[t, 0, 0] if name == "gate" else x[t, k, 0]
                got.append(y[t, k, rows])
                want.append(_expected(member, wire, out, n, int(idx[t, k]), rows, xv))
        _check_decode(np.concatenate(got), np.concatenate(want), (member, name, tokens))


def test_single_iq2_ks_expert_quantized_from_seed_0(device):
    """One [2048 x 4096] IQ2_KS expert: rows N(0, 0.02) from default_rng(0), a
    U(0.1, 1) imatrix from default_rng(1), quantized by the package codec and
    relaid by format.pack (1122 B a row); the producer's full dequantization is
    bit-exact against the oracle, and a GEMV with x ~ N(0, 1) (default_rng(2))
    meets the decode gates on every row."""
    out, n = GU
    w = (np.random.default_rng(0).standard_normal((out, n)) * 0.02).astype(np.float32)
    imatrix = np.random.default_rng(1).uniform(0.1, 1.0, n).astype(np.float32)
    wire = codec.quantize("iq2_ks", w, imatrix)
    assert wire.shape == (out, 2 + 70 * n // 256) == (out, 1122)
    shapes = fmt.component_shapes("iq2_ks", 1, out, n)
    module = IqkSwitchLinear("iq2_ks", 1, out, n, device=device)
    module.load_streams({k: np.ascontiguousarray(v).reshape(shapes[k]) for k, v in fmt.pack("iq2_ks", wire, n).items()})
    ref = oracle.dequantize("iq2_ks", wire, n)
    got = module.dequantized().cpu().numpy()[0]
    assert np.array_equal(got.view(np.uint16), ref.astype(np.float16).view(np.uint16))
    x = np.random.default_rng(2).standard_normal(n).astype(np.float16)
    y = module(torch.from_numpy(x.reshape(1, 1, 1, n)).to(device), torch.zeros((1, 1), dtype=torch.int32,
                                                                                  device=device))
    _check_decode(y.float().cpu().numpy().reshape(out), ref.astype(np.float64) @ x.astype(np.float64), "C1")


def test_iq2_k_routed_decode_8_tokens(device):
    """IQ2_K, 256 experts, 8 tokens x top-6 unsorted: gate [2048 x 4096] (48
    pairs x 64 row groups = 3072: three pairs of a token a workgroup) and down
    [4096 x 2048] (48 pairs, 6144 row workgroups: the two-row-block form)."""
    _decode_case(device, "iq2_k", 8, seed=303)


@pytest.mark.parametrize("tokens", (1, 2, 4))
def test_iq1_s_r4_routed_decode(device, tokens):
    """IQ1_S_R4, 256 experts, top-6, at 1 token (the workload) and at 2 and 4
    tokens, where the down (2 tokens) and both projections (4 tokens) take two
    row blocks per wavefront."""
    _decode_case(device, "iq1_s_r4", tokens, seed=404 + tokens)


def test_iq2_ks_routed_decode_1_token(device):
    """IQ2_KS, 256 experts, 1 token x top-6 at both geometries."""
    _decode_case(device, "iq2_ks", 1, seed=202)


def test_iq2_ks_routed_decode_8_tokens(device):
    """IQ2_KS, 256 experts, 8 tokens x top-6: the gate's three pairs of a token
    a workgroup and the down's two-row-block form, as for IQ2_K."""
    _decode_case(device, "iq2_ks", 8, seed=208)


@pytest.mark.parametrize("member, tokens", (("iq2_ks", 1), ("iq2_k", 8), ("iq1_s_r4", 1)))
def test_routed_decode_on_codec_quantized_stacks(device, member, tokens):
    """The routed decode workloads on stacks quantized by the package codec
    from N(0, 0.02) rows (IQ2_KS 1 token, IQ2_K 8 tokens, IQ1_S_R4 1 token;
    top-6 over 256 experts, both geometries), against float64 contractions of
    the oracle's dequantization of the same wire."""
    _decode_case(device, member, tokens, seed=707 + tokens, quantized=True)


@pytest.mark.parametrize("member", ("iq2_ks", "iq1_s_r4"))
def test_row_range_producer_at_the_gate_geometry(device, member):
    """The row-range producer at [2048 x 4096] over 256 experts: a token's six
    experts compacted into slots in expert order, ranges from a half expert
    down to one four-row group, each slot's rows the oracle's bit for bit
    (reference range form: src/mlx_iqk/nn.py:171-201)."""
    from mlx_iqk_amd import kernels
    out, n = GU
    module, wire = _stack(member, out, n, wirepack.seed_for("config", member, "gate"), device)
    rng = np.random.default_rng(606)
    experts = np.sort(rng.choice(E, TOP_K, replace=False))
    slot_of = np.full(E, -1, dtype=np.int32)
    slot_of[experts] = np.arange(TOP_K, dtype=np.int32)
    sot = torch.from_numpy(slot_of).to(device)
    for start, rows in ((0, 1024), (1024, 1024), (512, 64), (2044, 4)):
        print(f"  {member} range [{start}, +{rows}) of experts {experts.tolist()}", flush=True)
        got = kernels.dequant(member, module._checked(), E, out, n, slot_of_expert=sot, n_slots=TOP_K,
                              row_start=start, rows=rows)
        got = got.view(torch.int16).cpu().numpy()
        for s, e in enumerate(experts):
            want = oracle.dequantize(member, wire[e * out + start:e * out + start + rows], n)
            assert np.array_equal(got[s], want.astype(np.float16).view(np.int16)), (member, start, rows, int(e))


@pytest.mark.parametrize("which", ("gate", "down"))
def test_decode_is_deterministic(device, which):
    """The same dispatch twice: identical fp16 bits (no atomics, fixed order),
    for the gate (three pairs a workgroup) and the down (two row blocks)."""
    geo = GU if which == "gate" else DN
    module, _ = _stack("iq2_k", *geo, wirepack.seed_for("config", "iq2_k", which), device)
    rng = np.random.default_rng(5)
    shape = (8, 1, 1, geo[1]) if which == "gate" else (8, TOP_K, 1, geo[1])
    x = torch.from_numpy(rng.standard_normal(shape).astype(np.float16)).to(device)
    idx = torch.from_numpy(np.stack([rng.choice(E, TOP_K, replace=False) for _ in range(8)]).astype(np.int32)).to(device)
    a, b = module(x, idx), module(x, idx)
    assert torch.equal(a.view(torch.int16), b.view(torch.int16))


def _zipf_prefill(device, projections, quantized=False, seed=505):
    """2048 tokens, Zipf(1.1) top-6 over 256 experts, pairs sorted by expert
    (sorted_indices=True, 12,288 pairs), for each (name, member, (out, n)):
    both routes (fused; producer + grouped GEMM) meet the prefill gate on
    sampled pairs spanning the largest and the smallest experts, agree with
    each other over the whole output, and repeat bit for bit."""
    tokens = 2048
    idx = synth.zipf_routing(tokens, E, TOP_K, 1.1, seed=seed)
    flat = idx.reshape(-1)
    order = np.argsort(flat, kind="stable")
    ids = flat[order].astype(np.int32)  # the sorting caller's pair order
    counts = np.bincount(ids, minlength=E)
    assert counts.max() > 500 and (counts > 0).sum() > 200, counts
    rng = np.random.default_rng(seed + 1)
    xtok = rng.standard_normal((tokens, GU[1])).astype(np.float16)
    # x [P, 1, in] with indices [P]: the operands of a sorting caller
    # (mlx_lm's _gather_sort, which the reference's switch layer runs under);
    # the down projection's input is an N(0, 1) fp16 intermediate
    inputs = {GU[1]: xtok[order // TOP_K].reshape(-1, 1, GU[1]),
              DN[1]: rng.standard_normal((ids.size, 1, DN[1])).astype(np.float16)}
    # sampled pairs: both ends of the sorted order, the largest expert's run, and random ones
    big = int(np.argmax(counts))
    start = int(np.searchsorted(ids, big))
    picks = np.unique(np.concatenate([[0, 1, ids.size - 1], start + np.arange(4), rng.choice(ids.size, 24, replace=False)]))
    it = torch.from_numpy(ids).to(device)
    for name, member, (out, n) in projections:
        if quantized:
            module, wire = _quantized_stack(member, out, n, wirepack.seed_for("quantized", member, name), device)
        else:
            module, wire = _stack(member, out, n, wirepack.seed_for("config", member, name), device)
        xt = torch.from_numpy(inputs[n]).to(device)
        print(f"  prefill {name} ({member}{', quantized' if quantized else ''}) fused", flush=True)
        module.fused_prefill = True
        fused = module(xt, it, sorted_indices=True)
        again = module(xt, it, sorted_indices=True)
        assert torch.equal(fused.view(torch.int16), again.view(torch.int16)), name
        print(f"  prefill {name} ({member}) producer + grouped GEMM", flush=True)
        module.fused_prefill = False
        producer = module(xt, it, sorted_indices=True)
        module.fused_prefill = True
        assert tuple(fused.shape) == tuple(producer.shape) == (ids.size, 1, out)
        f = fused.float().reshape(ids.size, out)
        p = producer.float().reshape(ids.size, out)
        assert torch.isfinite(f).all() and torch.isfinite(p).all(), name
        assert (f - p).abs().max().item() <= 2e-3 * p.abs().max().item(), name
        f, p = f.cpu().numpy(), p.cpu().numpy()
        rows = _rows_sample(rng, out, 64, member)
        for q in picks:
            want = _expected(member, wire, out, n, int(ids[q]), rows, inputs[n][q, 0])
            for got, route in ((f, "fused"), (p, "producer")):
                rel = np.max(np.abs(got[q, rows] - want)) / np.max(np.abs(want))
                assert rel < 3e-3, (name, member, route, int(q), rel)
        del fused, again, producer
        torch.cuda.empty_cache()


def test_zipf_prefill_2048_tokens_mixed_members(device):
    """The prefill workload: gate in IQ2_KS [2048 x 4096], down in IQ2_K
    [4096 x 2048], serving-scale random wire."""
    _zipf_prefill(device, (("gate", "iq2_ks", GU), ("down", "iq2_k", DN)))


def test_zipf_prefill_on_codec_quantized_stacks(device):
    """The same prefill on stacks of N(0, 0.02) rows quantized by the package
    codec (the workloads' data), both routes against the oracle."""
    _zipf_prefill(device, (("gate", "iq2_ks", GU), ("down", "iq2_k", DN)), quantized=True, seed=515)


@pytest.mark.parametrize("member", ("iq1_s_r4", "iq2_k"))
def test_zipf_prefill_gate_in_the_other_members(device, member):
    """The gate projection of the prefill in IQ1_S_R4 and in IQ2_K (the
    fused kernel's other instantiations at 4096 wide), both routes against
    the oracle."""
    _zipf_prefill(device, (("gate", member, GU),), seed=525)
