"""The switch module inside a captured HIP graph (torch.cuda.CUDAGraph).

A serving loop captures a layer's projections once and replays them, so
every route of ``IqkSwitchLinear.forward`` must record without host syncs and
replay what eager execution computes: the decode GEMV, the fused prefill
(device route + fused GEMM) and the producer prefill (device route, slot
compaction in torch ops, producer, grouped GEMM).  Each replay follows new
inputs written in place and eager work with synchronizations between, and
is compared bit for bit with an eager call on the same inputs (every kernel
is deterministic).
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

import wirepack
from mlx_iqk_amd import format as fmt
from mlx_iqk_amd.nn import IqkSwitchLinear

pytestmark = pytest.mark.gpu

EXPERTS, OUT, N, TOP_K = 8, 256, 2048, 4


def _module(member, seed, device, out=OUT):
    wire = wirepack.random_wire(member, EXPERTS * out, N, seed=seed, scales="serving")
    streams = fmt.pack(member, wire, N)
    shapes = fmt.component_shapes(member, EXPERTS, out, N)
    module = IqkSwitchLinear(member, EXPERTS, out, N, device=device)
    module.load_streams({k: np.ascontiguousarray(v).reshape(shapes[k]) for k, v in streams.items()})
    return module


def _routing(rng, tokens, top_k=TOP_K):
    return np.stack([rng.choice(EXPERTS, top_k, replace=False) for _ in range(tokens)]).astype(np.int64)


@pytest.mark.parametrize("member", fmt.MEMBERS)
@pytest.mark.parametrize("route", ["decode", "decode_three_pairs", "fused", "producer"])
def test_forward_replays_from_a_graph(device, member, route):
    """decode: 1 token x top-4 (4 pairs, one pair a workgroup); decode_three_pairs:
    21 tokens x top-3 over 1024 rows (63 pairs x 32 row groups = 2016, where the
    IQ2 members serve three pairs of a token a workgroup); fused and producer:
    24 tokens x top-4 (96 pairs take the prefill route)."""
    three = route == "decode_three_pairs"
    module = _module(member, 41, device, out=1024 if three else OUT)
    module.fused_prefill = route != "producer"
    tokens, top_k = (21, 3) if three else (1 if route == "decode" else 24, TOP_K)
    prefill = route in ("fused", "producer")
    rng = np.random.default_rng(5)
    x = torch.empty(tokens, 1, 1, N, dtype=torch.float16, device=device)
    idx = torch.empty(tokens, top_k, dtype=torch.int64, device=device)

    def fill():
        x.copy_(torch.from_numpy(rng.standard_normal((tokens, 1, 1, N)).astype(np.float16)))
        idx.copy_(torch.from_numpy(_routing(rng, tokens, top_k)))

    def run():
        return module(x, idx, sorted_indices=prefill)

    fill()
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):  # warm-up off the capture stream, as torch asks
        for _ in range(2):
            run()
    torch.cuda.current_stream().wait_stream(side)
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        out = run()
    for replay in range(4):
        fill()
        want = run()
        torch.cuda.synchronize()
        graph.replay()
        torch.cuda.synchronize()
        assert out.shape == want.shape
        assert bool(torch.isfinite(want).all())
        assert torch.equal(out, want), f"replay {replay} differs from eager execution"


@pytest.mark.parametrize("member", ("iq2_ks", "iq2_k"))
@pytest.mark.parametrize("method", ("gemv_sorted", "gemv_union"))
def test_sorted_and_union_replay_from_a_graph(device, member, method):
    """The verify shapes' entry points inside a graph: 8 tokens, each routed
    to the same 3 of the experts in its own order (three runs of 8 pairs, so
    groups of three pairs hold one or two runs), a new pool and new
    activations written in place before each replay."""
    module = _module(member, 43, device)
    tokens, top_k = 8, 3
    rng = np.random.default_rng(7)
    x = torch.empty(tokens, 1, 1, N, dtype=torch.float16, device=device)
    ids = torch.empty(tokens * top_k, dtype=torch.int32, device=device)
    toks = torch.empty(tokens * top_k, dtype=torch.int32, device=device)

    def fill():
        x.copy_(torch.from_numpy(rng.standard_normal((tokens, 1, 1, N)).astype(np.float16)))
        pool = rng.choice(EXPERTS, 3, replace=False)
        idx = np.stack([rng.permutation(pool)[:top_k] for _ in range(tokens)]).reshape(-1)
        order = np.argsort(idx, kind="stable")
        ids.copy_(torch.from_numpy(idx[order].astype(np.int32)))
        toks.copy_(torch.from_numpy((order // top_k).astype(np.int32)))

    def run():
        return getattr(module, method)(x, ids, toks)

    fill()
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        for _ in range(2):
            run()
    torch.cuda.current_stream().wait_stream(side)
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        out = run()
    for replay in range(4):
        fill()
        want = run()
        torch.cuda.synchronize()
        graph.replay()
        torch.cuda.synchronize()
        assert bool(torch.isfinite(want).all())
        assert torch.equal(out, want), f"replay {replay} differs from eager execution"
