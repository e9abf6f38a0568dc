"""The product CPU codec: quantizer bytes and dequantizer floats equal the reference's.

The quantizers are pinned to the reference's own bytes -- committed golden
vectors everywhere, and the compiled reference live where its sources exist
(reference: vendor/ik_llama/iqk_iq2.cpp:205-499, iqk_iq1sr4.cpp:490-577).
"""

from __future__ import annotations

from pathlib import Path

import numpy as np
import pytest

import wirepack
from mlx_iqk_amd import codec
from mlx_iqk_amd import format as fmt
from oracle import oracle

GOLDEN = Path(__file__).resolve().parent / "golden"
needs_ref = pytest.mark.skipif(not oracle.ref_available(), reason="reference codec not built here")


@pytest.mark.parametrize("member", fmt.MEMBERS)
def test_quantizer_reproduces_the_reference_golden_bytes(member):
    g = np.load(GOLDEN / f"quantize_{member}.npz")
    assert np.array_equal(codec.quantize(member, g["rows"], g["imatrix"]), g["wire_imatrix"])
    assert np.array_equal(codec.quantize(member, g["rows"], None), g["wire_plain"])


@needs_ref
@pytest.mark.parametrize("member", fmt.MEMBERS)
@pytest.mark.parametrize("n", (2048, 4096))
def test_quantizer_matches_the_compiled_reference(member, n):
    rng = np.random.default_rng(wirepack.seed_for("codec", member, n))
    rows = (rng.standard_normal((16, n)) * 0.02).astype(np.float32)
    rows[4] = 0.0
    rows[9, : n // 2] = 0.0
    rows[11] *= 1e-5
    im = (rng.random(n) * 0.9 + 0.1).astype(np.float32)
    im[n // 3: n // 2] = 0.0
    for imatrix in (im, None):
        assert np.array_equal(codec.quantize(member, rows, imatrix), oracle.ref_quantize(member, rows, imatrix))


@pytest.mark.parametrize("member", fmt.MEMBERS)
def test_quantizer_bytes_do_not_depend_on_the_thread_count(member):
    rng = np.random.default_rng(5)
    rows = (rng.standard_normal((32, 1024)) * 0.02).astype(np.float32)
    im = rng.random(1024).astype(np.float32)
    try:
        codec.set_threads(1)
        one = codec.quantize(member, rows, im)
        codec.set_threads(7)
        many = codec.quantize(member, rows, im)
    finally:
        codec.set_threads(0)
    assert np.array_equal(one, many)


@pytest.mark.parametrize("member", fmt.MEMBERS)
@pytest.mark.parametrize("n", (256, 2048))
def test_dequantizer_matches_the_oracle(member, n):
    wire = wirepack.random_wire(member, 12, n, seed=wirepack.seed_for("deq", member, n))
    got = codec.dequantize(member, wire, n)
    want = oracle.dequantize(member, wire, n)
    assert np.array_equal(got.view(np.uint32), want.view(np.uint32))


@pytest.mark.parametrize("member", fmt.MEMBERS)
def test_dequantizer_matches_the_reference_golden(member):
    g = np.load(GOLDEN / f"dequant_{member}.npz")
    got = codec.dequantize(member, g["wire"], int(g["n"]))
    assert np.array_equal(got.view(np.uint32), g["out"].view(np.uint32))


def test_block_and_row_sizes():
    lib = codec.load()
    assert lib.iqk_block_size_iq2_k() == 76 and lib.iqk_block_size_iq2_ks() == 70
    assert lib.iqk_block_size_iq1_s_r4() == 24
    assert lib.iqk_row_size_iq1_s_r4(4096) == 770 and lib.iqk_row_size_iq1_s_r4(4001) == 0
    assert lib.iqk_row_size_iq2_ks(4096) == 1122 and lib.iqk_row_size_iq2_ks(4000) == 0
    assert lib.iqk_row_size_iq2_k(2048) == 608 and lib.iqk_row_size_iq2_k(0) == 0


def test_refused_geometry():
    with pytest.raises(fmt.IqkFormatError):
        codec.quantize("iq2_ks", np.zeros((2, 300), np.float32))
    with pytest.raises(fmt.IqkFormatError):
        codec.quantize("iq1_s_r4", np.zeros((6, 256), np.float32))
    with pytest.raises(fmt.IqkFormatError):
        codec.quantize("iq2_k", np.zeros((2, 256), np.float32), np.ones(255, np.float32))
    with pytest.raises(fmt.IqkFormatError):
        codec.dequantize("iq2_k", np.zeros((2, 75), np.uint8), 256)
    lib = codec.load()
    import ctypes
    assert lib.iqk_quantize_iq1_s_r4(None, None, 6, 256, None) == 0  # rows not a multiple of 4
    assert lib.iqk_dequantize_iq2_ks(None, None, 1, 100) != 0


def test_zero_rows_quantize_to_zero_weights():
    for member in fmt.MEMBERS:
        wire = codec.quantize(member, np.zeros((4, 256), np.float32))
        assert not np.any(codec.dequantize(member, wire, 256))
