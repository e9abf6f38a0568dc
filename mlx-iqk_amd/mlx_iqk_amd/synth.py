"""Seeded synthetic expert stacks for the routed geometry.

An expert projection is a ``[out, in]`` float32 matrix drawn from N(0, 0.02)
with a Uniform(0.1, 1.0) imatrix, quantized with :mod:`mlx_iqk_amd.codec`
and relaid with :func:`mlx_iqk_amd.format.pack`.  Quantizing all 256 experts
of three projections is ~6.4 G weights of search, so a stack quantizes
``distinct`` experts and fills the rest with row-rotated copies of them: every
expert still owns its own bytes at its own address (what decode bandwidth
measures), and every row is a quantized N(0, 0.02) row.
"""

from __future__ import annotations

import zlib

import numpy as np
import torch

from . import codec
from .format import component_shapes, pack
from .kernels import stream_dtypes


def seed_for(*parts) -> int:
    return zlib.crc32("|".join(str(p) for p in parts).encode()) % (2 ** 31)


_SIGNED_VIEW = {torch.uint32: torch.int32, torch.uint16: torch.int16}


def _bits(t: torch.Tensor) -> torch.Tensor:
    """Same-width signed view: torch implements fewer kernels for uint32/uint16."""
    return t.view(_SIGNED_VIEW.get(t.dtype, t.dtype))


def quantized_rows(member: str, rows: int, n: int, seed: int, imatrix_seed: int | None = None) -> np.ndarray:
    """ik wire of ``rows`` N(0, 0.02) rows under a U(0.1, 1.0) imatrix."""
    rng = np.random.default_rng(seed)
    w = (rng.standard_normal((rows, n)) * 0.02).astype(np.float32)
    irng = np.random.default_rng(seed + 1 if imatrix_seed is None else imatrix_seed)
    imatrix = irng.uniform(0.1, 1.0, n).astype(np.float32)
    return codec.quantize(member, w, imatrix)


def expert_stack(member: str, experts: int, out: int, n: int, seed: int, device, distinct: int = 2,
                 label: str = "") -> list[torch.Tensor]:
    """Stacked relayout streams ``[experts, out, ...]`` on ``device``, kernel order.

    Expert ``e`` holds distinct tile ``e % distinct`` with its rows rotated by
    ``e // distinct`` (so no two experts share row order).
    """
    shapes = component_shapes(member, experts, out, n)
    dtypes = stream_dtypes(member)
    stacks = {k: torch.empty(shapes[k], dtype=dtypes[k], device=device) for k in shapes}
    group = 4 if member == "iq1_s_r4" else 1
    for t in range(min(distinct, experts)):
        wire = quantized_rows(member, out, n, seed_for(seed, label, member, out, n, t),
                              imatrix_seed=seed_for(seed, label, "imatrix", n))
        tile = {k: torch.from_numpy(np.ascontiguousarray(v).reshape((out,) + shapes[k][2:])).to(device)
                for k, v in pack(member, wire, n).items()}
        for e in range(t, experts, distinct):
            shift = group * ((e // distinct) % (out // group))
            for k in shapes:
                _bits(stacks[k][e]).copy_(torch.roll(_bits(tile[k]), shifts=shift, dims=0))
    return [stacks[k] for k in shapes]


def zipf_routing(tokens: int, experts: int, top_k: int, exponent: float, seed: int) -> np.ndarray:
    """``[tokens, top_k]`` expert ids, each row drawn without replacement from a
    Zipf(exponent) distribution over a seeded rank -> expert permutation."""
    rng = np.random.default_rng(seed)
    p = np.arange(1, experts + 1, dtype=np.float64) ** (-exponent)
    p /= p.sum()
    perm = rng.permutation(experts)
    out = np.empty((tokens, top_k), dtype=np.int64)
    for t in range(tokens):
        out[t] = perm[rng.choice(experts, top_k, replace=False, p=p)]
    return out


__all__ = ["expert_stack", "quantized_rows", "seed_for", "zipf_routing"]
