"""GPU parity of the HIP kernels through the C ABI, against the oracle.

Mirrors the reference's kernel gate (tests/test_kernels.py):

1. the producer is **bit-exact**: its fp16 equals the oracle's float32
   dequantization rounded to fp16 (round-to-nearest-even), compared on raw
   bits, over random wire (serving and full-range scales) and converted rows;
2. the decode GEMV matches a float64 contraction of the oracle's weights:
   ``max|d| / max|ref| < 1.5e-3``, rel-L2 <= 1e-3 (the stated bar), and more
   than 99% of outputs at 0 fp16 ULP from the correctly rounded result;
3. the grouped GEMM matches a float64 contraction of the fp16 weights
   within the prefill tolerance (3e-3, reference tests/test_nn.py:132).
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

import wirepack
from mlx_iqk_amd import codec, kernels
from mlx_iqk_amd import format as fmt
from oracle import oracle

pytestmark = pytest.mark.gpu

EXPERTS = 4
OUT = 64


def _fp16_ulp(got: np.ndarray, want: np.ndarray) -> np.ndarray:
    def order(a):
        i = a.astype(np.float16).view(np.int16).astype(np.int64)
        return np.where(i < 0, np.int64(-32768) - i, i)
    return np.abs(order(got) - order(want))


def _streams(member, wire, experts, out, n, device):
    packed = fmt.pack(member, wire, n)
    shapes = fmt.component_shapes(member, experts, out, n)
    return [torch.from_numpy(np.ascontiguousarray(packed[k]).reshape(shapes[k])).to(device) for k in shapes]


def _case(member, n, seed, device, experts=EXPERTS, out=OUT, scales="serving"):
    wire = wirepack.random_wire(member, experts * out, n, seed=seed, scales=scales)
    ref = oracle.dequantize(member, wire, n).reshape(experts, out, n)
    return wire, _streams(member, wire, experts, out, n, device), ref


def _check_gemv(got: np.ndarray, want: np.ndarray, label) -> None:
    got = got.astype(np.float64)
    rel = np.max(np.abs(got - want)) / np.max(np.abs(want))
    l2 = np.linalg.norm(got - want) / np.linalg.norm(want)
    exact = float(np.mean(_fp16_ulp(got, want.astype(np.float16)) == 0))
    assert rel < 1.5e-3, (label, rel)
    assert l2 <= 1e-3, (label, l2)
    assert exact > 0.99, (label, exact)


# -- the producer is bit-exact --------------------------------------------------


@pytest.mark.parametrize("member", fmt.MEMBERS)
@pytest.mark.parametrize("n", kernels.SUPPORTED_IN_FEATURES)
@pytest.mark.parametrize("scales", ("serving", "sweep"))
def test_dequant_is_bit_identical_to_the_oracle(device, member, n, scales):
    print(f"dequant {member} n={n} scales={scales}", flush=True)
    _, streams, ref = _case(member, n, wirepack.seed_for(member, n, scales), device, scales=scales)
    got = kernels.dequant(member, streams, EXPERTS, OUT, n).cpu().numpy()
    want = ref.astype(np.float16)
    bad = int(np.sum(got.view(np.uint16) != want.view(np.uint16)))
    assert bad == 0, f"{bad} of {got.size} fp16 words differ"


@pytest.mark.parametrize("member", fmt.MEMBERS)
@pytest.mark.parametrize("n", kernels.SUPPORTED_IN_FEATURES)
def test_dequant_is_bit_identical_on_converted_rows(device, member, n):
    print(f"dequant converted {member} n={n}", flush=True)
    rng = np.random.default_rng(4242)
    rows = (rng.standard_normal((EXPERTS * OUT, n)) * 0.02).astype(np.float32)
    wire = codec.quantize(member, rows, (rng.random(n) * 0.9 + 0.1).astype(np.float32))
    streams = _streams(member, wire, EXPERTS, OUT, n, device)
    got = kernels.dequant(member, streams, EXPERTS, OUT, n).cpu().numpy()
    want = oracle.dequantize(member, wire, n).reshape(EXPERTS, OUT, n).astype(np.float16)
    assert np.array_equal(got.view(np.uint16), want.view(np.uint16))


@pytest.mark.parametrize("member", fmt.MEMBERS)
def test_dequant_writes_selected_experts_into_their_slots(device, member):
    print(f"dequant slots {member}", flush=True)
    n, experts = 2048, 6
    _, streams, ref = _case(member, n, 77, device, experts=experts, out=32)
    slot = torch.tensor([2, -1, 0, -1, 1, 9], dtype=torch.int32, device=device)  # 9 is out of range: skipped
    out = torch.full((3, 32, n), 12345, dtype=torch.int16, device=device).view(torch.float16)
    kernels.dequant(member, streams, experts, 32, n, slot_of_expert=slot, n_slots=3, out=out)
    got = out.cpu().numpy()
    for e, s in ((0, 2), (2, 0), (4, 1)):
        assert np.array_equal(got[s].view(np.uint16), ref[e].astype(np.float16).view(np.uint16)), (e, s)


def test_dequant_is_deterministic(device):
    _, streams, _ = _case("iq2_ks", 4096, 5, device)
    a = kernels.dequant("iq2_ks", streams, EXPERTS, OUT, 4096)
    b = kernels.dequant("iq2_ks", streams, EXPERTS, OUT, 4096)
    assert torch.equal(a.view(torch.int16), b.view(torch.int16))


# -- the decode GEMV ----------------------------------------------------------------


@pytest.mark.parametrize("member", fmt.MEMBERS)
@pytest.mark.parametrize("n", kernels.SUPPORTED_IN_FEATURES)
def test_gemv_matches_a_float64_reference_shared_rows(device, member, n):
    """The gate/up seam: each token's row is shared by its top_k experts."""
    print(f"gemv shared {member} n={n}", flush=True)
    _, streams, ref = _case(member, n, wirepack.seed_for(member, n, "gemv"), device)
    rng = np.random.default_rng(17)
    tokens, top_k = 8, 3
    x = rng.standard_normal((tokens, n)).astype(np.float16)
    sel = rng.integers(0, EXPERTS, size=tokens * top_k).astype(np.int32)
    got = kernels.gemv(member, torch.from_numpy(x).to(device), streams, torch.from_numpy(sel).to(device),
                       top_k, EXPERTS, OUT).cpu().numpy()
    _check_gemv(got, oracle.gemv_reference(ref, sel, x, top_k), (member, n))


@pytest.mark.parametrize("member", fmt.MEMBERS)
@pytest.mark.parametrize("n", kernels.SUPPORTED_IN_FEATURES)
def test_gemv_matches_a_float64_reference_per_pair_rows(device, member, n):
    """The down seam: one activation row per pair."""
    print(f"gemv per-pair {member} n={n}", flush=True)
    _, streams, ref = _case(member, n, wirepack.seed_for(member, n, "gemv-down"), device)
    rng = np.random.default_rng(19)
    pairs = 12
    x = rng.standard_normal((pairs, n)).astype(np.float16)
    sel = rng.integers(0, EXPERTS, size=pairs).astype(np.int32)
    got = kernels.gemv(member, torch.from_numpy(x).to(device), streams, torch.from_numpy(sel).to(device),
                       1, EXPERTS, OUT).cpu().numpy()
    _check_gemv(got, oracle.gemv_reference(ref, sel, x, 1), (member, n))


@pytest.mark.parametrize("member", fmt.MEMBERS)
@pytest.mark.parametrize("n", kernels.SUPPORTED_IN_FEATURES)
@pytest.mark.parametrize("top_k", (3, 2))
def test_gemv_large_dispatch_equals_small_dispatches(device, member, n, top_k):
    """A large dispatch takes two 16-row blocks per wavefront (shared
    activation reads): IQ1_S_R4 from 2 x 768 row workgroups, the IQ2 members at
    2048 wide from 8 x 768.  Otherwise, from 2 x 768 row workgroups, one
    workgroup serves three (top-3) or two (top-2) pairs of a token, staging
    its activations once.  A row's arithmetic is the same, so its outputs
    equal those of the same pairs in small dispatches (one block, one pair a
    workgroup) bit for bit, and meet the float64 gate; an invalid id or an
    infinite activation turns only its own pairs' rows NaN.  The IQ2 members'
    sorted form is held to the same, and the large dispatch's floor runs."""
    print(f"gemv large dispatch {member} n={n} top_k={top_k}", flush=True)
    out, tokens = 256, 256  # 256 top_k pairs x 8 row workgroups: 6144 (top-3), 4096 (top-2)
    _, streams, ref = _case(member, n, wirepack.seed_for(member, n, "large"), device, out=out)
    rng = np.random.default_rng(23)
    x = rng.standard_normal((tokens, n)).astype(np.float16)
    sel = rng.integers(0, EXPERTS, size=tokens * top_k).astype(np.int32)
    # an expert id beyond the stack and an infinite activation: NaN rows, the same in both forms
    sel[40] = EXPERTS
    x[70, n // 3] = np.inf
    nan_pairs = np.zeros(tokens * top_k, dtype=bool)
    nan_pairs[40] = True
    nan_pairs[70 * top_k:71 * top_k] = True
    xt, st = torch.from_numpy(x).to(device), torch.from_numpy(sel).to(device)
    big = kernels.gemv(member, xt, streams, st, top_k, EXPERTS, out).cpu().numpy()
    chunk = 32  # at most 96 pairs x 8 = 768 row workgroups a call
    small = np.concatenate([kernels.gemv(member, xt[t:t + chunk], streams, st[t * top_k:(t + chunk) * top_k], top_k,
                                         EXPERTS, out).cpu().numpy() for t in range(0, tokens, chunk)])
    assert np.array_equal(big.view(np.uint16), small.view(np.uint16)), member
    assert np.all(np.isnan(big[nan_pairs])) and not np.any(np.isnan(big[~nan_pairs])), member
    keep = ~nan_pairs
    with np.errstate(invalid="ignore", over="ignore"):  # the infinite token's rows, left out below
        want = oracle.gemv_reference(ref, np.where(keep, sel, 0), x, top_k)
    _check_gemv(big[keep], want[keep], (member, n))
    if member in kernels.IQ2_MEMBERS:
        order = np.argsort(sel, kind="stable")  # the invalid id sorts last
        toks = torch.from_numpy((order // top_k).astype(np.int32)).to(device)
        ys = kernels.gemv_sorted(member, xt, streams, st[torch.from_numpy(order).to(device)], toks, EXPERTS,
                                 out).cpu().numpy()
        assert np.array_equal(ys.view(np.uint16), big[order].view(np.uint16)), member
    yf = kernels.gemv(member, xt, streams, st, top_k, EXPERTS, out, floor=True).float().cpu().numpy()
    assert yf.shape == big.shape
    assert np.all(np.isnan(yf[sel >= EXPERTS])) and np.all(np.isfinite(yf[sel < EXPERTS])), member


@pytest.mark.parametrize("member", fmt.MEMBERS)
@pytest.mark.parametrize("n", kernels.SUPPORTED_IN_FEATURES)
def test_gemv_half_tile_dispatch_equals_full_tiles(device, member, n):
    """Dispatches of fewer than 768 row workgroups of 32 rows run 16-row
    workgroups (each thread stages two activation units, IQ1_S_R4 expands
    twice the grid entries); between 768 and 1536 they run the 32-row,
    one-pair form.  A row's arithmetic is the same in both, so the same pairs
    give the same bits either way, and meet the float64 gate."""
    print(f"gemv half tiles {member} n={n}", flush=True)
    out, tokens, top_k = 256, 40, 3  # 120 pairs x 8 = 960 workgroups of 32 rows; a token alone: 24
    _, streams, ref = _case(member, n, wirepack.seed_for(member, n, "half"), device, out=out)
    rng = np.random.default_rng(29)
    x = rng.standard_normal((tokens, n)).astype(np.float16)
    sel = rng.integers(0, EXPERTS, size=tokens * top_k).astype(np.int32)
    xt, st = torch.from_numpy(x).to(device), torch.from_numpy(sel).to(device)
    full = kernels.gemv(member, xt, streams, st, top_k, EXPERTS, out).cpu().numpy()
    half = np.concatenate([kernels.gemv(member, xt[t:t + 1], streams, st[t * top_k:(t + 1) * top_k], top_k,
                                        EXPERTS, out).cpu().numpy() for t in range(tokens)])
    assert np.array_equal(full.view(np.uint16), half.view(np.uint16)), member
    _check_gemv(half, oracle.gemv_reference(ref, sel, x, top_k), (member, n))
    for floor in (True, "grid"):
        yf = kernels.gemv(member, xt[:1], streams, st[:top_k], top_k, EXPERTS, out, floor=floor)
        assert torch.isfinite(yf.float()).all()


@pytest.mark.parametrize("case", range(8))
def test_gemv_dispatch_forms_agree_on_random_shapes(device, case):
    """Seeded random geometry and routing: member, width, 256-512 rows, 2-8
    experts, 1-8 pairs a token (ids repeat where a token has more pairs than
    the stack has experts), and tokens enough for 1536-8000 row
    workgroups, so the dispatch takes the large-dispatch forms (three or two
    pairs a workgroup, or two row blocks) wherever their thresholds are met.
    It equals the same pairs dispatched a token at a time (one pair a
    workgroup, one row block) bit for bit, and meets the float64 gate."""
    rng = np.random.default_rng(wirepack.seed_for("forms", case))
    member = fmt.MEMBERS[case % 3]
    n = kernels.SUPPORTED_IN_FEATURES[(case // 3) % 2]
    out = 32 * int(rng.integers(8, 17))
    experts = int(rng.integers(2, 9))
    top_k = (7, 6, 5, 1, 4, 2, 3, 8)[case]  # three, two and one pair a workgroup
    groups_per_token = top_k * out // 32
    tokens = -(-int(rng.integers(1536, 8000)) // groups_per_token)
    print(f"gemv forms {member} n={n} out={out} experts={experts} top_k={top_k} tokens={tokens}", flush=True)
    _, streams, ref = _case(member, n, wirepack.seed_for("forms", member, n, case), device, experts=experts, out=out)
    x = rng.standard_normal((tokens, n)).astype(np.float16)
    sel = np.concatenate([rng.permutation(experts)[:top_k] if top_k <= experts
                          else rng.integers(0, experts, size=top_k) for _ in range(tokens)]).astype(np.int32)
    xt, st = torch.from_numpy(x).to(device), torch.from_numpy(sel).to(device)
    big = kernels.gemv(member, xt, streams, st, top_k, experts, out).cpu().numpy()
    small = np.concatenate([kernels.gemv(member, xt[t:t + 1], streams, st[t * top_k:(t + 1) * top_k], top_k,
                                         experts, out).cpu().numpy() for t in range(tokens)])
    assert np.array_equal(big.view(np.uint16), small.view(np.uint16)), (member, n, out, top_k, tokens)
    _check_gemv(big, oracle.gemv_reference(ref, sel, x, top_k), (member, n, out, top_k))


@pytest.mark.parametrize("n", kernels.SUPPORTED_IN_FEATURES)
@pytest.mark.parametrize("out", (16, 48, 192))
def test_gemv_iq2_ks_tiles(device, n, out):
    """Row counts on both IQ2_KS paths: 64-row MFMA tiles and 16-row tiles."""
    print(f"gemv iq2_ks tiles n={n} out={out}", flush=True)
    experts = 3
    _, streams, ref = _case("iq2_ks", n, wirepack.seed_for("tiles", n, out), device, experts=experts, out=out)
    rng = np.random.default_rng(out)
    x = rng.standard_normal((5, n)).astype(np.float16)
    sel = rng.integers(0, experts, size=5).astype(np.int32)
    got = kernels.gemv("iq2_ks", torch.from_numpy(x).to(device), streams, torch.from_numpy(sel).to(device),
                       1, experts, out).cpu().numpy()
    _check_gemv(got, oracle.gemv_reference(ref, sel, x, 1), out)


@pytest.mark.parametrize("member", fmt.MEMBERS)
@pytest.mark.parametrize("n", kernels.SUPPORTED_IN_FEATURES)
def test_gemv_activations_of_wide_range(device, member, n):
    """Activations spanning fp16's range inside one sub-block: subnormals,
    exact zeros, +-65504 and values 2^-20 below their sub-block's maximum."""
    print(f"gemv wide-range {member} n={n}", flush=True)
    _, streams, ref = _case(member, n, wirepack.seed_for(member, n, "wide"), device)
    rng = np.random.default_rng(29)
    rows = 6
    mag = np.exp2(rng.uniform(-24, 6, size=(rows, n)))
    x = (mag * rng.choice([-1.0, 1.0], size=(rows, n))).astype(np.float16)
    x[0] = 0
    x[1, ::7] = 0
    x[2, 3::1024] = np.float16(65504) * np.where(np.arange(n // 1024) % 2, 1, -1)  # with 2^-24..2^6 neighbours
    x[3] = np.where(np.arange(n) % 32 == 5, np.float16(1024), np.float16(2.0 ** -10)).astype(np.float16)
    x[4] = (rng.integers(1, 1023, size=n) * 2.0 ** -24).astype(np.float16)  # subnormals only
    sel = rng.integers(0, EXPERTS, size=rows).astype(np.int32)
    with np.errstate(over="ignore"):
        got = kernels.gemv(member, torch.from_numpy(x).to(device), streams, torch.from_numpy(sel).to(device),
                           1, EXPERTS, OUT).cpu().numpy()
    want = oracle.gemv_reference(ref, sel, x, 1)
    assert np.all(got[0] == 0), member
    # Row 4's outputs are fp16 subnormals, where the output's own rounding
    # exceeds 1e-3 relative: it must land within one ULP of the rounded result.
    assert np.all(_fp16_ulp(got[4], want[4].astype(np.float16)) <= 1), member
    keep = np.nonzero((np.abs(want).max(axis=1) < 60000) & ~np.isin(np.arange(rows), (0, 4)))[0]
    assert len(keep) == rows - 2, keep
    exact = []
    for r in keep:
        g, w = got[r].astype(np.float64), want[r]
        assert np.max(np.abs(g - w)) / np.max(np.abs(w)) < 1.5e-3, (member, n, int(r))
        assert np.linalg.norm(g - w) / np.linalg.norm(w) <= 1e-3, (member, n, int(r))
        exact.append(_fp16_ulp(g, w.astype(np.float16)) == 0)
    assert np.mean(exact) > 0.95, (member, n, np.mean(exact))


@pytest.mark.parametrize("member", fmt.MEMBERS)
def test_gemv_reads_the_expert_the_index_names(device, member):
    n = 2048
    _, streams, ref = _case(member, n, 555, device)
    x = np.random.default_rng(23).standard_normal((1, n)).astype(np.float16)
    xt = torch.from_numpy(x).to(device)
    for e in range(EXPERTS):
        sel = torch.tensor([e], dtype=torch.int32, device=device)
        got = kernels.gemv(member, xt, streams, sel, 1, EXPERTS, OUT).cpu().numpy()[0].astype(np.float64)
        want = ref[e].astype(np.float64) @ x[0].astype(np.float64)
        assert np.max(np.abs(got - want)) / np.max(np.abs(want)) < 1.5e-3, e


@pytest.mark.parametrize("member", fmt.MEMBERS)
def test_gemv_marks_an_out_of_range_expert_with_nan(device, member):
    """An id beyond the stack is never dereferenced: its rows come back NaN."""
    n = 2048
    _, streams, ref = _case(member, n, 31, device)
    x = np.random.default_rng(1).standard_normal((3, n)).astype(np.float16)
    sel = np.array([1, EXPERTS + 5, 2], dtype=np.int32)
    got = kernels.gemv(member, torch.from_numpy(x).to(device), streams, torch.from_numpy(sel).to(device),
                       1, EXPERTS, OUT).cpu().numpy()
    assert np.all(np.isnan(got[1]))
    ok = oracle.gemv_reference(ref, sel[[0, 2]], x[[0, 2]], 1)
    _check_gemv(got[[0, 2]], ok, member)


@pytest.mark.parametrize("member", fmt.MEMBERS)
@pytest.mark.parametrize("n", kernels.SUPPORTED_IN_FEATURES)
def test_floor_kernels_run(device, member, n):
    _, streams, _ = _case(member, n, 9, device)
    x = torch.randn(2, n, device=device).to(torch.float16)
    sel = torch.tensor([0, 3, 1, 2], dtype=torch.int32, device=device)
    y = kernels.gemv(member, x, streams, sel, 2, EXPERTS, OUT, floor=True)
    w = kernels.dequant(member, streams, EXPERTS, OUT, n, floor=True)
    torch.cuda.synchronize()
    assert torch.isfinite(y.float()).all() and torch.isfinite(w.float()).all()


def _stream_hash(words: np.ndarray, nbytes: int, loads: int, max_waves: int) -> np.ndarray:
    """The byte-stream floor's output, restated: wavefront w folds its chunks
    (``loads`` KiB each, every ``stride``-th) as sum over lanes and loads i of
    (2i + 3)(x + 3y + 5z + 7w) of its 16-byte words, mod 2^32."""
    u = np.zeros(((nbytes + 1024 * loads - 1) // (1024 * loads)) * 256 * loads, dtype=np.uint64)
    u[:nbytes // 4] = words[:nbytes // 4]
    q = u.reshape(-1, loads, 64, 4)  # chunk, load i, lane, word
    coef = np.array([1, 3, 5, 7], dtype=np.uint64)
    per_chunk = ((q * coef).sum(axis=3) * (2 * np.arange(loads, dtype=np.uint64) + 3)[None, :, None]).sum(axis=(1, 2))
    chunks = per_chunk.size
    waves = kernels.stream_floor_words(nbytes, loads, max_waves)
    out = np.zeros(waves, dtype=np.uint64)
    for c in range(chunks):  # the grid's wavefronts stride over the chunks
        out[c % waves] += per_chunk[c]
    return (out % (1 << 32)).astype(np.uint32)


@pytest.mark.parametrize("loads,max_waves", [(4, 0), (8, 0), (16, 0), (16, 8), (8, 12), (4, 4)])
def test_stream_floor_reads_every_byte(device, loads, max_waves):
    """The byte-stream floor's output is a hash of every word it loaded (each
    chunk exactly once, whichever wavefront took it), so matching the hash
    restated on the CPU shows its load set is the span."""
    rng = np.random.default_rng(loads * 100 + max_waves)
    for nbytes in (16, 4096, 4096 * 5 + 48, 1 << 16, 3 * 16384 + 1024):
        src = rng.integers(0, 1 << 32, size=(nbytes + 16 * 1024) // 4, dtype=np.uint64).astype(np.uint32)
        got = kernels.stream_floor(torch.from_numpy(src.view(np.int32)).to(device), nbytes, loads=loads,
                                   max_waves=max_waves)
        got = got.cpu().numpy().view(np.uint32)
        want = _stream_hash(src, nbytes, loads, max_waves)
        if loads == 4 and not max_waves:
            assert np.array_equal(got, want), nbytes
        else:
            assert np.array_equal(got[:want.size], want), (nbytes, loads, max_waves)


# -- the grouped GEMM -----------------------------------------------------------------


def test_grouped_gemm_marks_rows_outside_x_with_nan(device):
    """A slot whose activation row lies beyond x is never read: its output row
    is NaN, every other row is unaffected; a y row beyond the slots is not
    stored."""
    rng = np.random.default_rng(5)
    K, N, G = 2048, 96, 3
    counts = np.array([40, 0, 30], dtype=np.int64)
    P = int(counts.sum())
    w = (rng.standard_normal((G, N, K)) * 0.02).astype(np.float16)
    x = rng.standard_normal((50, K)).astype(np.float16)
    x_rows = rng.integers(0, 50, size=P).astype(np.int32)
    x_rows[[3, 45]] = [50, 2 ** 31 - 1]
    offs = np.concatenate([[0], np.cumsum(counts)]).astype(np.int32)
    dev = {k: torch.from_numpy(v).to(device) for k, v in (("x", x), ("w", w), ("o", offs), ("r", x_rows))}
    got = kernels.grouped_gemm(dev["x"], dev["w"], dev["o"], dev["r"]).float().cpu().numpy()
    bad = np.zeros(P, dtype=bool)
    bad[[3, 45]] = True
    assert np.all(np.isnan(got[bad])) and not np.any(np.isnan(got[~bad]))
    g_of = np.repeat(np.arange(G), counts)
    want = np.stack([x[x_rows[p] % 50].astype(np.float64) @ w[g_of[p]].astype(np.float64).T for p in range(P)])
    assert np.max(np.abs(got[~bad] - want[~bad])) / np.max(np.abs(want[~bad])) < 3e-3


def test_grouped_gemm_is_deterministic(device):
    rng = np.random.default_rng(7)
    K, N = 4096, 512
    counts = np.array([300, 3, 64, 65], dtype=np.int64)
    P = int(counts.sum())
    w = torch.from_numpy((rng.standard_normal((4, N, K)) * 0.02).astype(np.float16)).to(device)
    x = torch.from_numpy(rng.standard_normal((P, K)).astype(np.float16)).to(device)
    offs = torch.from_numpy(np.concatenate([[0], np.cumsum(counts)]).astype(np.int32)).to(device)
    rows = torch.arange(P, dtype=torch.int32, device=device)
    a = kernels.grouped_gemm(x, w, offs, rows)
    b = kernels.grouped_gemm(x, w, offs, rows)
    assert torch.equal(a.view(torch.int16), b.view(torch.int16))


def test_grouped_gemm_repeats_bit_for_bit_at_the_prefill_size(device):
    """The direct-to-LDS pipeline at the 2048-token Zipf(1.1) prefill size
    (256 experts, [2048 x 4096], 12,288 sorted pairs): twenty back-to-back
    calls give identical bits (its waits are written by hand, so a missing
    one would show as calls that differ), and sampled slots match float64."""
    from mlx_iqk_amd import synth
    print("grouped gemm repeat at the prefill size", flush=True)
    E, N, K = 256, 2048, 4096
    idx = synth.zipf_routing(2048, E, 6, 1.1, 31).reshape(-1)
    order = np.argsort(idx, kind="stable")
    counts = np.bincount(idx, minlength=E)
    P = idx.size
    gen = torch.Generator(device=device).manual_seed(31)
    w = (torch.randn((E, N, K), generator=gen, device=device) * 0.02).to(torch.float16)
    x = torch.randn((2048, K), generator=gen, device=device).to(torch.float16)
    offs = torch.from_numpy(np.concatenate([[0], np.cumsum(counts)]).astype(np.int32)).to(device)
    rows = torch.from_numpy((order // 6).astype(np.int32)).to(device)
    first = kernels.grouped_gemm(x, w, offs, rows)
    out = torch.empty_like(first)
    for _ in range(20):
        kernels.grouped_gemm(x, w, offs, rows, out=out)
        assert torch.equal(out.view(torch.int16), first.view(torch.int16))
    rng = np.random.default_rng(37)
    for p in rng.choice(P, 8, replace=False):
        e = int(idx[order[p]])
        want = w[e].double() @ x[int(order[p]) // 6].double()
        got = first[p].double()
        assert float((got - want).abs().max() / want.abs().max()) < 3e-3, int(p)
    del w, x


def test_grouped_gemm_addresses_operands_beyond_4gib(device):
    """Activation rows and an expert's weights that start past 4 GiB of their
    tensors (lane addresses are 64-bit; nothing is reduced mod 2^32).  Only the
    rows the kernel reads are filled."""
    print("grouped gemm beyond 4 GiB", flush=True)
    rng = np.random.default_rng(41)
    K, N, G, P = 4096, 65536, 9, 40
    x_rows_total = 2 ** 19 + 64                                   # x: 4 GiB + 512 KiB
    x = torch.empty((x_rows_total, K), dtype=torch.float16, device=device)
    rows = (2 ** 19 + rng.permutation(64)[:P]).astype(np.int32)   # every row past byte 2^32
    xs = rng.standard_normal((P, K)).astype(np.float16)
    x[torch.from_numpy(rows.astype(np.int64)).to(device)] = torch.from_numpy(xs).to(device)
    x[0] = 0  # a dead slot of the tile reads row 0
    w = torch.empty((G, N, K), dtype=torch.float16, device=device)  # expert 8 starts at byte 2^32
    gen = torch.Generator(device=device).manual_seed(41)
    w[8] = (torch.randn((N, K), generator=gen, device=device) * 0.02).to(torch.float16)
    offs = torch.tensor([0] * 9 + [P], dtype=torch.int32, device=device)
    got = kernels.grouped_gemm(x, w, offs, torch.from_numpy(rows).to(device)).float().cpu().numpy()
    cols = np.concatenate([np.sort(rng.choice(N, 96, replace=False)), [0, N - 1]])
    w8 = w[8][torch.from_numpy(cols).to(device)].cpu().numpy()
    want = xs.astype(np.float64) @ w8.astype(np.float64).T
    rel = np.max(np.abs(got[:, cols] - want)) / np.max(np.abs(want))
    assert rel < 3e-3, rel
    del x, w


@pytest.mark.parametrize("K", (128, 96))
def test_grouped_gemm_over_more_groups_than_one_scan_round(device, K):
    """600 groups: the in-block work-list scan takes 256 a round (three rounds),
    with empty, one-slot and multi-tile groups in each; every slot against a
    float64 reference.  K = 128 takes the direct-to-LDS kernel, 96 the general
    one."""
    print(f"grouped gemm 600 groups K={K}", flush=True)
    rng = np.random.default_rng(K + 600)
    G, N = 600, 64
    counts = rng.integers(0, 4, size=G)
    counts[[3, 255, 256, 300, 511, 512, 599]] = [70, 65, 0, 64, 1, 0, 130]
    P = int(counts.sum())
    w = (rng.standard_normal((G, N, K)) * 0.05).astype(np.float16)
    xrows = 512
    x = rng.standard_normal((xrows, K)).astype(np.float16)
    x_rows = rng.integers(0, xrows, size=P).astype(np.int32)
    offs = np.concatenate([[0], np.cumsum(counts)]).astype(np.int32)
    got = kernels.grouped_gemm(torch.from_numpy(x).to(device), torch.from_numpy(w).to(device),
                               torch.from_numpy(offs).to(device),
                               torch.from_numpy(x_rows).to(device)).cpu().numpy().astype(np.float64)
    g_of = np.repeat(np.arange(G), counts)
    want = np.einsum("pk,pnk->pn", x[x_rows].astype(np.float64), w[g_of].astype(np.float64))
    rel = np.max(np.abs(got - want)) / np.max(np.abs(want))
    assert rel < 3e-3, rel


# K a multiple of 64 takes the direct-to-LDS kernel (one to many steps; at one, two and three
# steps the loads past the last step start in the prologue), other K the general one (K = 32:
# one half step, the upper chunks of every row clamped inside that row)
@pytest.mark.parametrize("K,N", [(4096, 2048), (2048, 4096), (2048, 256), (2048, 32), (4096, 272), (64, 256), (128, 64),
                                 (192, 40), (2080, 96), (96, 288), (32, 64), (32, 264)])
def test_grouped_gemm_matches_a_float64_reference(device, K, N):
    print(f"grouped gemm K={K} N={N}", flush=True)
    rng = np.random.default_rng(K + N)
    counts = np.array([0, 1, 70, 5, 0, 130, 17, 64], dtype=np.int64)  # empty, ragged, >1 M-tile
    G, P = len(counts), int(counts.sum())
    w = (rng.standard_normal((G, N, K)) * 0.02).astype(np.float16)
    xrows = 300
    x = rng.standard_normal((xrows, K)).astype(np.float16)
    x_rows = rng.integers(0, xrows, size=P).astype(np.int32)
    x_rows[[0, 1, P - 1]] = xrows - 1  # the last row of x, where a load past its row would leave x
    y_rows = rng.permutation(P).astype(np.int32)
    offs = np.concatenate([[0], np.cumsum(counts)]).astype(np.int32)
    got = kernels.grouped_gemm(torch.from_numpy(x).to(device), torch.from_numpy(w).to(device),
                               torch.from_numpy(offs).to(device), torch.from_numpy(x_rows).to(device),
                               torch.from_numpy(y_rows).to(device)).cpu().numpy().astype(np.float64)
    want = np.empty((P, N))
    g_of = np.repeat(np.arange(G), counts)
    for p in range(P):
        want[y_rows[p]] = x[x_rows[p]].astype(np.float64) @ w[g_of[p]].astype(np.float64).T
    rel = np.max(np.abs(got - want)) / np.max(np.abs(want))
    assert rel < 3e-3, rel
