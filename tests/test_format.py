"""The relayout: geometry facts, pack/unpack, and bit identity with the oracle.

Mirrors the reference's format gate (tests/test_format.py): the relayout's
float32 decode must equal ik's CPU dequantizer bit for bit over the whole
decode value space and over random wire bytes.  Here "ik's dequantizer" is
the oracle (checked against the compiled reference in test_oracle.py).
"""

from __future__ import annotations

import numpy as np
import pytest

import wirepack
from mlx_iqk_amd import codec
from mlx_iqk_amd import format as fmt
from mlx_iqk_amd.iq1grid import grid_values
from oracle import oracle

WIDTHS = (256, 512, 2048, 4096)


def _bits(a):
    return np.ascontiguousarray(a, dtype=np.float32).view(np.uint32)


def _mismatches(a, b) -> int:
    return int(np.sum(_bits(a) != _bits(b)))


# -- geometry (reference: tests/test_format.py:31-101) ------------------------


def test_row_bytes_match_the_declared_budgets():
    assert fmt.ik_row_bytes("iq2_k", 256) == 76
    assert fmt.ik_row_bytes("iq2_ks", 256) == 72
    assert fmt.ik_row_bytes("iq2_k", 4096) == 76 * 16
    assert fmt.ik_row_bytes("iq2_ks", 4096) == 2 + 70 * 16
    assert fmt.ik_row_bytes("iq1_s_r4", 32) == 8
    assert fmt.ik_row_bytes("iq1_s_r4", 2048) == 386
    assert fmt.ik_row_bytes("iq1_s_r4", 4096) == 770


ROW_SIZE_FACTS = {"iq2_ks": (2, 70, 256), "iq2_k": (0, 76, 256), "iq1_s_r4": (2, 6, 32)}


@pytest.mark.parametrize("member", fmt.MEMBERS)
@pytest.mark.parametrize("n", (256, 1024, 2048, 4096, 8192))
def test_row_bytes_follow_the_struct_facts(member, n):
    meta, block, weights = ROW_SIZE_FACTS[member]
    assert fmt.ik_row_bytes(member, n) == meta + block * (n // weights)


def test_bits_per_weight():
    assert fmt.bits_per_weight("iq2_k", 4096) == 2.375
    assert fmt.bits_per_weight("iq2_ks", 4096) == 2.1875 + 16 / 4096
    assert fmt.bits_per_weight("iq2_ks", 2048) == 2.1875 + 16 / 2048
    assert fmt.bits_per_weight("iq1_s_r4", 4096) == 1.5 + 16 / 4096


@pytest.mark.parametrize("member", fmt.MEMBERS)
@pytest.mark.parametrize("n", WIDTHS)
def test_relayout_costs_exactly_what_the_member_costs(member, n):
    assert fmt.relayout_row_bytes(member, n) == fmt.ik_row_bytes(member, n)


def test_iq1_s_r4_width_and_group_guards():
    assert fmt.check_row_width(96, "iq1_s_r4") == 96
    for bad in (0, -32, 31, 100, 4001):
        with pytest.raises(fmt.IqkFormatError):
            fmt.check_row_width(bad, "iq1_s_r4")
    assert fmt.check_wire_rows("iq1_s_r4", 8) == 8
    for bad in (0, -4, 2, 6, 37):
        with pytest.raises(fmt.IqkFormatError):
            fmt.check_wire_rows("iq1_s_r4", bad)
    assert fmt.check_wire_rows("iq2_ks", 7) == 7


@pytest.mark.parametrize("bad", [0, -256, 255, 300, 4095])
def test_row_width_guard_rejects_non_multiples_of_the_block(bad):
    with pytest.raises(fmt.IqkFormatError):
        fmt.check_row_width(bad)


def test_unknown_member_is_rejected():
    with pytest.raises(fmt.IqkFormatError):
        fmt.check_member("iq3_k")


@pytest.mark.parametrize("member", ("iq2_ks", "iq2_k"))
def test_component_shapes_cover_every_weight_once(member):
    shapes = fmt.component_shapes(member, 3, 32, 2048)
    assert shapes["qs"] == (3, 32, 2048 // 16)
    assert shapes["sex"] == (3, 32, 2048 // (8 * fmt.SUB_WEIGHTS[member]))


def test_iq1_s_r4_component_shapes():
    shapes = fmt.component_shapes("iq1_s_r4", 3, 32, 2048)
    assert shapes == {"qs": (3, 32, 64), "qh": (3, 32, 64), "dv": (3, 32)}
    dt = fmt.component_dtypes("iq1_s_r4")
    assert dt["qs"].itemsize == 4 and dt["qh"].itemsize == 2 and dt["dv"] == np.float16


@pytest.mark.parametrize("member", fmt.MEMBERS)
def test_pack_rejects_a_wire_row_of_the_wrong_length(member):
    wire = np.zeros((4, fmt.ik_row_bytes(member, 2048) + 1), dtype=np.uint8)
    with pytest.raises(fmt.IqkFormatError):
        fmt.pack(member, wire, 2048)


def test_iq1_s_r4_pack_refuses_broken_groups():
    wire = wirepack.random_wire("iq1_s_r4", 8, 2048, seed=23)
    with pytest.raises(fmt.IqkFormatError):
        fmt.pack("iq1_s_r4", wire[:6], 2048)
    with pytest.raises(fmt.IqkFormatError):
        fmt.pack("iq1_s_r4", wire, 2048, chunk=6)


# -- bit identity with the oracle (reference: tests/test_format.py:168-217) ----


@pytest.mark.parametrize("member,maker,n", [
    ("iq2_ks", wirepack.exhaustive_iq2_ks, 256),
    ("iq2_k", wirepack.exhaustive_iq2_k, 256),
    ("iq1_s_r4", wirepack.exhaustive_iq1_s_r4, 256),
])
def test_exhaustive_value_space_is_bit_identical(member, maker, n):
    wire = maker(seed=5)
    got = fmt.decode_wire(member, wire, n)
    want = oracle.dequantize(member, wire, n)
    assert _mismatches(got, want) == 0
    planes = fmt.decode_planes(member, fmt.pack(member, wire, n), n)
    if member == "iq1_s_r4":
        assert wire.shape[0] == 8 * 2 * 4 * 64
        assert set(np.unique(planes["codes"])) == set(range(2048))
        assert set(np.unique(planes["values"])) == {-1, 0, 1}
        assert set(np.unique(planes["scale_index"])) == set(range(1, 16, 2))
        assert set(np.unique(planes["shift"])) == {np.float32(-0.125), np.float32(0.125)}
    else:
        lo, hi = (-16, 16) if member == "iq2_ks" else (-8, 8)
        assert set(np.unique(planes["codes"])) == {0, 1, 2, 3}
        assert set(np.unique(planes["scale_index"])) == set(range(lo, hi))
        assert set(np.unique(planes["values"])) == {int(v) for v in fmt.IQ2NL_VALUES}


@pytest.mark.parametrize("member", fmt.MEMBERS)
@pytest.mark.parametrize("n", WIDTHS)
def test_random_byte_space_is_bit_identical(member, n):
    wire = wirepack.random_wire(member, 24, n, seed=wirepack.seed_for(member, n))
    assert _mismatches(fmt.decode_wire(member, wire, n), oracle.dequantize(member, wire, n)) == 0


@pytest.mark.parametrize("member", fmt.MEMBERS)
@pytest.mark.parametrize("n", (2048, 4096))
@pytest.mark.parametrize("with_imatrix", (True, False))
def test_quantized_rows_relayout_bit_identically(member, n, with_imatrix):
    rng = np.random.default_rng(7)
    rows = rng.standard_normal((16, n)).astype(np.float32) * 0.05
    rows[3] = 0.0
    rows[5] *= 1e-4
    imatrix = rng.random(n).astype(np.float32) if with_imatrix else None
    if with_imatrix:
        imatrix[: n // 4] = 0.0  # a route-starved span: the uniform-collapse case
    wire = codec.quantize(member, rows, imatrix)
    assert _mismatches(fmt.decode_wire(member, wire, n), oracle.dequantize(member, wire, n)) == 0


# -- pack/unpack invariants (reference: tests/test_format.py:220-296) ----------


@pytest.mark.parametrize("member", fmt.MEMBERS)
def test_pack_result_is_independent_of_the_chunk_size(member):
    wire = wirepack.random_wire(member, 36, 2048, seed=13)
    whole = fmt.pack(member, wire, 2048, chunk=1024)
    chunked = fmt.pack(member, wire, 2048, chunk=8)
    assert set(whole) == set(chunked)
    for name in whole:
        assert np.array_equal(whole[name].view(np.uint8), chunked[name].view(np.uint8)), name


@pytest.mark.parametrize("member", fmt.MEMBERS)
def test_pack_is_a_permutation_not_a_rewrite(member):
    wire = wirepack.random_wire(member, 4, 2048, seed=11)
    streams = fmt.pack(member, wire, 2048)
    assert sum(int(np.asarray(v).nbytes) for v in streams.values()) == 4 * fmt.ik_row_bytes(member, 2048)
    shapes = fmt.component_shapes(member, 1, 4, 2048)
    dtypes = fmt.component_dtypes(member)
    for name, value in streams.items():
        assert value.dtype == dtypes[name]
        assert value.reshape(shapes[name]).shape == shapes[name]


@pytest.mark.parametrize("member", fmt.MEMBERS)
@pytest.mark.parametrize("n", WIDTHS)
def test_unpack_returns_the_wire_bytes_it_was_packed_from(member, n):
    wire = wirepack.random_wire(member, 24, n, seed=wirepack.seed_for(member, n, "rt"))
    back = fmt.unpack(member, fmt.pack(member, wire, n), n)
    assert back.dtype == np.uint8 and back.shape == wire.shape
    assert np.array_equal(back, wire)


@pytest.mark.parametrize("member", fmt.MEMBERS)
def test_unpack_result_is_independent_of_the_chunk_size(member):
    wire = wirepack.random_wire(member, 36, 2048, seed=19)
    streams = fmt.pack(member, wire, 2048)
    assert np.array_equal(fmt.unpack(member, streams, 2048, chunk=1024),
                          fmt.unpack(member, streams, 2048, chunk=8))


@pytest.mark.parametrize("member", fmt.MEMBERS)
def test_unpack_round_trips_quantized_rows(member):
    rng = np.random.default_rng(17)
    rows = rng.standard_normal((12, 2048)).astype(np.float32) * 0.05
    rows[2] = 0.0
    wire = codec.quantize(member, rows, rng.random(2048).astype(np.float32))
    assert np.array_equal(fmt.unpack(member, fmt.pack(member, wire, 2048), 2048), wire)


def test_relayout_code_order_on_a_single_hot_weight():
    """A single nonzero code lands at exactly its weight's k position."""
    n = 256
    for member in ("iq2_ks", "iq2_k"):
        for w in (0, 1, 15, 16, 31, 32, 63, 64, 127, 128, 200, 255):
            codes = np.zeros((1, n), dtype=np.int64)
            codes[0, w] = 3
            if member == "iq2_ks":
                wire = wirepack.pack_iq2_ks_row(codes, np.full((1, 8), 17), np.zeros((1, 8)), 1.0)[None]
            else:
                wire = wirepack.pack_iq2_k_row(codes, np.full((1, 16), 9), np.zeros((1, 16)),
                                               np.ones(1))[None]
            qs = fmt.pack(member, wire, n)["qs"].reshape(-1)
            assert (int(qs[w // 16]) >> (2 * (w % 16))) & 3 == 3, (member, w)
            got = fmt._qs_to_codes(qs[None])[0]
            assert np.flatnonzero(got).tolist() == [w], (member, w)


def test_grid_values_are_the_ternary_table():
    g = grid_values()
    assert g.shape == (2048, 8) and g.dtype == np.int8
    assert set(np.unique(g)) == {-1, 0, 1}
    assert not np.any(g[1029])  # the all-zero entry the quantizer writes for a zero block
    assert len({bytes(r) for r in g}) == 2048
