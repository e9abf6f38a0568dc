"""Pinning the oracle before it is trusted.

The oracle (oracle/iqk_oracle.c) restates the reference CPU dequantizers.
It is checked three independent ways, chosen so a plausible slip (a wrong
shift, a swapped nibble, a dropped offset, the wrong alphabet half, a
transposed row in the IQ1 group) fails at least one:

1. against golden vectors the reference's own compiled codec wrote
   (tests/golden/, made by tests/golden/make_golden.py from oracle/_ref);
2. against the compiled reference live, where its sources are present;
3. against closed forms: single-field blocks whose every weight is a known
   exact product, computed here in float64 from the field values.
"""

from __future__ import annotations

import hashlib
import json
import re
from pathlib import Path

import numpy as np
import pytest

import wirepack
from oracle import oracle

GOLDEN = Path(__file__).resolve().parent / "golden"
MEMBERS = ("iq2_ks", "iq2_k", "iq1_s_r4")
VALUES = np.array([-31, -13, 1, 17, -26, -8, 6, 22])
needs_ref = pytest.mark.skipif(not oracle.ref_available(), reason="reference codec not built here")


def _bits(a):
    return np.ascontiguousarray(a, dtype=np.float32).view(np.uint32)


@pytest.mark.parametrize("member", MEMBERS)
def test_oracle_matches_the_reference_golden_dequant(member):
    g = np.load(GOLDEN / f"dequant_{member}.npz")
    got = oracle.dequantize(member, g["wire"], int(g["n"]))
    assert np.array_equal(_bits(got), _bits(g["out"]))


def test_oracle_matches_the_reference_over_the_exhaustive_value_space():
    digests = json.loads((GOLDEN / "exhaustive.json").read_text())
    makers = {"iq2_ks": wirepack.exhaustive_iq2_ks, "iq2_k": wirepack.exhaustive_iq2_k,
              "iq1_s_r4": wirepack.exhaustive_iq1_s_r4}
    for member, maker in makers.items():
        d = digests[member]
        wire = maker(seed=d["seed"])
        assert hashlib.sha256(wire.tobytes()).hexdigest() == d["wire_sha256"], member
        out = oracle.dequantize(member, wire, 256)
        assert hashlib.sha256(out.tobytes()).hexdigest() == d["out_sha256"], member


@needs_ref
@pytest.mark.parametrize("member", MEMBERS)
@pytest.mark.parametrize("n", (256, 1024, 4096))
@pytest.mark.parametrize("scales", ("sweep", "serving"))
def test_oracle_matches_the_compiled_reference(member, n, scales):
    wire = wirepack.random_wire(member, 16, n, seed=wirepack.seed_for("oracle", member, n, scales), scales=scales)
    assert np.array_equal(_bits(oracle.dequantize(member, wire, n)), _bits(oracle.ref_dequantize(member, wire, n)))


def _half(v):
    return float(np.float16(v))


@pytest.mark.parametrize("code,scale,alpha", [(c, s, a) for c in range(4) for s in (0, 5, 16, 31) for a in (0, 1)])
def test_iq2_ks_closed_form(code, scale, alpha):
    d = _half(-3.0517578125e-05 * 37)
    codes = np.full((2, 256), code)
    ls = np.full((2, 8), scale)
    al = np.full((2, 8), alpha)
    # one sub-block of block 1 differs, to catch a sub-block or block mix-up
    codes[1, 96:128] = (code + 1) % 4
    ls[1, 3] = (scale + 7) % 32
    al[1, 3] = 1 - alpha
    row = wirepack.pack_iq2_ks_row(codes, ls, al, d)[None]
    out = oracle.dequantize("iq2_ks", row, 512)[0].astype(np.float64)
    want = np.full(512, d * (scale - 16) * VALUES[4 * alpha + code])
    want[256 + 96:256 + 128] = d * ((scale + 7) % 32 - 16) * VALUES[4 * (1 - alpha) + (code + 1) % 4]
    assert np.array_equal(out, want)


@pytest.mark.parametrize("code,scale,alpha", [(c, s, a) for c in range(4) for s in (0, 8, 15) for a in (0, 1)])
def test_iq2_k_closed_form(code, scale, alpha):
    d = np.array([_half(0.0123), _half(-7.5)])
    codes = np.full((2, 256), code)
    ls = np.full((2, 16), scale)
    al = np.full((2, 16), alpha)
    codes[0, 48:64] = (code + 2) % 4  # sub-block 3 of block 0
    ls[0, 3] = (scale + 3) % 16
    al[0, 3] = 1 - alpha
    row = wirepack.pack_iq2_k_row(codes, ls, al, d)[None]
    out = oracle.dequantize("iq2_k", row, 512)[0].astype(np.float64)
    want = np.concatenate([np.full(256, d[0] * (scale - 8) * VALUES[4 * alpha + code]),
                           np.full(256, d[1] * (scale - 8) * VALUES[4 * alpha + code])])
    want[48:64] = d[0] * ((scale + 3) % 16 - 8) * VALUES[4 * (1 - alpha) + (code + 2) % 4]
    assert np.array_equal(out, want)


@pytest.mark.parametrize("index", (0, 1, 1029, 1500, 2047))
@pytest.mark.parametrize("ls,neg", [(0, 0), (3, 1), (7, 0)])
def test_iq1_s_r4_closed_form(index, ls, neg):
    from mlx_iqk_amd.iq1grid import grid_codes
    code = int(grid_codes()[index])
    g = np.array([((code >> (2 * j)) & 3) - 1 for j in range(8)], dtype=np.float64)
    d = np.array([_half(0.5), _half(-0.001), _half(3.0), _half(6e-6)])
    idx = np.full((4, 8), index)
    idx[2, 5] = (index + 1) % 2048  # one sub-group of row 2 differs
    grp = wirepack.pack_iq1_s_r4_group(idx, np.full((4, 2), ls), np.full((4, 2), neg), d)
    out = oracle.dequantize("iq1_s_r4", grp.reshape(4, -1), 64).astype(np.float64)
    shift = -0.125 if neg else 0.125
    for r in range(4):
        want = np.tile(d[r] * (2 * ls + 1) * (g + shift), 8)
        if r == 2:
            c2 = int(grid_codes()[(index + 1) % 2048])
            g2 = np.array([((c2 >> (2 * j)) & 3) - 1 for j in range(8)], dtype=np.float64)
            want[40:48] = d[r] * (2 * ls + 1) * (g2 + shift)
        assert np.array_equal(out[r], want), r


@pytest.mark.parametrize("member", MEMBERS)
def test_a_flipped_code_bit_moves_exactly_its_weights(member):
    """The oracle is sensitive: one flipped wire bit changes only the weights it feeds."""
    n = 256
    wire = wirepack.random_wire(member, 4, n, seed=3, scales="serving")
    base = oracle.dequantize(member, wire, n)
    bad = wire.copy()
    byte = {"iq2_ks": 2 + 6 + 7, "iq2_k": 12 + 7, "iq1_s_r4": 8 + 5}[member]
    bad[0, byte] ^= 0x04
    moved = np.argwhere(oracle.dequantize(member, bad, n) != base)
    assert 0 < len(moved) <= 8


def test_grid_header_kats():
    from mlx_iqk_amd.iq1grid import grid_codes
    codes = grid_codes().astype(np.int64)
    assert codes.shape == (2048,)
    assert codes[1029] == 0x5555  # the all-zero entry (reference: vendor/ik_llama/iqk_iq1sr4.cpp:523)
    assert np.all(np.diff(codes) > 0)  # strictly increasing, as upstream lists them
    fields = (codes[:, None] >> (2 * np.arange(8))) & 3
    assert fields.max() == 2


@pytest.mark.skipif(not Path("/root/reference/src/mlx_iqk/iq1grid.py").is_file(), reason="reference absent")
def test_grid_header_equals_the_reference_table():
    from mlx_iqk_amd.iq1grid import grid_codes
    text = Path("/root/reference/src/mlx_iqk/iq1grid.py").read_text()
    body = text.split("KGRID_1BIT_2048 = (", 1)[1].split(")", 1)[0]
    ref = [int(v) for v in re.findall(r"\d+", body)]
    assert ref == grid_codes().astype(int).tolist()
