"""IQ_K routed-expert wire format: constants, geometry, pack/unpack, reference decode.

Two layouts are in play.

**ik wire** is what ik_llama's quantizers emit (reference:
vendor/ik_llama/iqk_iq2.cpp:64-87, vendor/ik_llama/iqk_iq1sr4.cpp:72-76):

* ``IQ2_KS`` row: ``[d f16][nb x {extra u16, scales[4], qs[64]}]``; eight
  32-weight sub-blocks per 256-weight block.  Weight ``w`` of a block sits in
  qs byte ``32*(w/128) + w%32`` at bit ``2*((w/32)%4)``.
* ``IQ2_K`` block: ``{d f16, extra u16, scales[8], qs[64]}``; sixteen
  16-weight sub-blocks.  Weight ``w`` sits in qs byte
  ``32*(w/128) + 16*((w/16)%2) + w%16`` at bit ``2*((w/32)%4)``.
* ``IQ1_S_R4``: rows in groups of four, ``[4 x d f16]`` then per 32 weights a
  24-byte block ``{qs[16], qh[4] u16}`` interleaving the four rows.

**The relayout** carries exactly the same bits, re-laid k-contiguously per
output row; it is the format the GPU kernels stream (reference:
src/mlx_iqk/format.py:27-61, 352-395):

* ``qs`` (2-bit members): code ``j`` of a row in uint32 word ``j/16`` at bit
  ``2*(j%16)``.  (``IQ1_S_R4``: uint32 word ``b`` holds the four low index
  bytes of 32-weight block ``b``, byte ``i`` for 8-weight sub-group ``i``.)
* ``scl``: the wire scale bytes in k order (two 4-bit fields per byte).
* ``sch``/``sex``: one bit per sub-block, bit ``b%8`` of byte ``b/8``.
* ``qh`` (``IQ1_S_R4``): the wire ``qh`` word of the row's block.
* ``dv``: the fp16 scale per row (``IQ2_KS``, ``IQ1_S_R4``) or per 256
  weights (``IQ2_K``).

Reconstruction (the CPU dequantizer's float32 order, every product exact):

* 2-bit members: ``dl = d * float(scale_index)``; ``y = dl * float(value)``
  with ``value = IQ2NL_VALUES[4*alphabet + code]``.
* ``IQ1_S_R4``: ``dl = d * float(2*ls + 1)``; ``y = dl * (float(g) + shift)``
  with ``g`` a grid value and ``shift = +-0.125``.
"""

from __future__ import annotations

import numpy as np

from .iq1grid import grid_values

QK_K = 256
"""Weights per super-block of the two 2-bit members."""

IQ2NL_VALUES = np.array([-31, -13, 1, 17, -26, -8, 6, 22], dtype=np.int8)
"""The two 4-entry alphabets: base in 0..3, shifted (base + 5) in 4..7
(reference: vendor/ik_llama/iqk_iq2.cpp:87)."""

MEMBERS = ("iq2_ks", "iq2_k", "iq1_s_r4")
"""Routed-expert members with a relayout, a codec and kernels."""

SUB_WEIGHTS = {"iq2_ks": 32, "iq2_k": 16, "iq1_s_r4": 32}
"""Weights sharing one scale index (and one alphabet bit / shift bit)."""

WIRE_GROUP_ROWS = {"iq2_ks": 1, "iq2_k": 1, "iq1_s_r4": 4}
"""Rows one addressable ik-wire unit covers; ``IQ1_S_R4`` interleaves four."""

BLOCK_WEIGHTS = {"iq2_ks": QK_K, "iq2_k": QK_K, "iq1_s_r4": 32}
"""Weights per wire block: the row-width granularity of each member."""

IQ2_KS_BLOCK_BYTES = 70
IQ2_KS_ROW_META_BYTES = 2
IQ2_K_BLOCK_BYTES = 76
IQ1_S_R4_BLOCK_BYTES = 24
IQ1_S_R4_ROW_META_BYTES = 2
IQ1S_DELTA = 0.125
"""The per-block reconstruction shift of ``IQ1_S_R4``; ``qh`` bit 15 picks its sign."""

PACK_CHUNK_ROWS = 2048
"""Rows one pack/unpack pass holds expanded at once (one byte per weight)."""


class IqkFormatError(ValueError):
    pass


def check_member(member: str) -> str:
    if member not in MEMBERS:
        raise IqkFormatError(f"iqk routed member {member!r} not in {MEMBERS}")
    return member


def check_row_width(in_features: int, member: str = "iq2_ks") -> int:
    """Row widths the relayout defines: a positive multiple of the member's block."""
    block = BLOCK_WEIGHTS[check_member(member)]
    n = int(in_features)
    if n <= 0 or n % block:
        raise IqkFormatError(
            f"in_features {in_features} is not a positive multiple of {block} "
            f"for {member}; ik silently changes the type of such a row, so it is "
            "refused here")
    return n


def check_wire_rows(member: str, rows: int) -> int:
    group = WIRE_GROUP_ROWS[check_member(member)]
    r = int(rows)
    if r <= 0 or r % group:
        raise IqkFormatError(
            f"{member} wire rows come in groups of {group}; {rows} rows do not "
            "split into whole groups")
    return r


_BLOCK_BYTES_PER_ROW = {"iq2_ks": IQ2_KS_BLOCK_BYTES, "iq2_k": IQ2_K_BLOCK_BYTES,
                        "iq1_s_r4": IQ1_S_R4_BLOCK_BYTES // 4}
_ROW_META = {"iq2_ks": IQ2_KS_ROW_META_BYTES, "iq2_k": 0,
             "iq1_s_r4": IQ1_S_R4_ROW_META_BYTES}


def ik_row_bytes(member: str, in_features: int) -> int:
    """Bytes of one ik-wire row, as ``ggml_row_size`` charges it.

    ``IQ1_S_R4`` blocks 32 weights of four rows in 24 bytes, so a row's share
    is 6 bytes per 32 weights plus its 2-byte scale
    (reference: src/mlx_iqk/format.py:340-349).
    """
    n = check_row_width(in_features, member)
    return _ROW_META[member] + _BLOCK_BYTES_PER_ROW[member] * (n // BLOCK_WEIGHTS[member])


def component_shapes(member: str, num_experts: int, out_features: int,
                     in_features: int) -> dict[str, tuple[int, ...]]:
    """Stacked-expert shapes of every relayout stream, in kernel input order."""
    n = check_row_width(in_features, member)
    e, o = int(num_experts), int(out_features)
    if member == "iq2_ks":
        return {"qs": (e, o, n // 16), "scl": (e, o, n // 64), "sch": (e, o, n // 256),
                "sex": (e, o, n // 256), "dv": (e, o)}
    if member == "iq2_k":
        return {"qs": (e, o, n // 16), "scl": (e, o, n // 32), "sex": (e, o, n // 128),
                "dv": (e, o, n // 256)}
    return {"qs": (e, o, n // 32), "qh": (e, o, n // 32), "dv": (e, o)}


def component_dtypes(member: str) -> dict[str, np.dtype]:
    """NumPy dtype of every relayout stream."""
    check_member(member)
    if member == "iq1_s_r4":
        return {"qs": np.dtype(np.uint32), "qh": np.dtype(np.uint16),
                "dv": np.dtype(np.float16)}
    names = ("qs", "scl", "sch", "sex", "dv") if member == "iq2_ks" else \
        ("qs", "scl", "sex", "dv")
    table = {"qs": np.uint32, "dv": np.float16}
    return {name: np.dtype(table.get(name, np.uint8)) for name in names}


def bits_per_weight(member: str, in_features: int) -> float:
    return 8.0 * ik_row_bytes(member, in_features) / check_row_width(in_features, member)


def relayout_row_bytes(member: str, in_features: int) -> int:
    """Bytes of one relayout row; equal to :func:`ik_row_bytes` by construction."""
    shapes = component_shapes(member, 1, 1, in_features)
    dtypes = component_dtypes(member)
    return sum(int(np.prod(shape)) * dtypes[name].itemsize
               for name, shape in shapes.items())


# ---------------------------------------------------------------------------
# code permutation of the 2-bit members
# ---------------------------------------------------------------------------
#
# Both 2-bit wires store four 2-bit fields per qs byte (field s at bit 2s).
# Splitting a block's 64 qs bytes into the index tuple below and the field
# into s, the weight index inside the 256-block is a plain mixed-radix number:
#
#   IQ2_KS: bytes as [h (2), j (32)],          w = 128*h + 32*s + j
#   IQ2_K : bytes as [h (2), half (2), j (16)], w = 128*h + 32*s + 16*half + j
#
# so the k-ordered codes are the byte fields transposed to (h, s, ...).


def _wire_codes(member: str, qs_bytes: np.ndarray) -> np.ndarray:
    """``[rows, nb, 64]`` wire qs bytes -> ``[rows, nb*256]`` k-ordered codes."""
    rows, nb, _ = qs_bytes.shape
    fields = (qs_bytes[..., None] >> (2 * np.arange(4, dtype=np.uint8))) & 3
    if member == "iq2_ks":
        codes = fields.reshape(rows, nb, 2, 32, 4).transpose(0, 1, 2, 4, 3)
    else:
        codes = fields.reshape(rows, nb, 2, 2, 16, 4).transpose(0, 1, 2, 5, 3, 4)
    return np.ascontiguousarray(codes).reshape(rows, nb * QK_K)


def _codes_wire(member: str, codes: np.ndarray) -> np.ndarray:
    """Inverse of :func:`_wire_codes`: ``[rows, n]`` codes -> ``[rows, nb, 64]`` bytes."""
    rows, n = codes.shape
    nb = n // QK_K
    c = codes.astype(np.uint8)
    if member == "iq2_ks":
        f = c.reshape(rows, nb, 2, 4, 32).transpose(0, 1, 2, 4, 3)
    else:
        f = c.reshape(rows, nb, 2, 4, 2, 16).transpose(0, 1, 2, 4, 5, 3)
    f = f.reshape(rows, nb, 64, 4)
    shifted = f << (2 * np.arange(4, dtype=np.uint8))
    return np.bitwise_or.reduce(shifted, axis=-1).astype(np.uint8)


def _codes_to_qs(codes: np.ndarray) -> np.ndarray:
    """k-ordered 2-bit codes ``[rows, n]`` -> little-endian uint32 words ``[rows, n/16]``."""
    rows, n = codes.shape
    c = codes.astype(np.uint32).reshape(rows, n // 16, 16)
    return np.bitwise_or.reduce(c << (2 * np.arange(16, dtype=np.uint32)), axis=-1)


def _qs_to_codes(qs: np.ndarray) -> np.ndarray:
    """uint32 words ``[rows, w]`` -> codes ``[rows, 16*w]`` (uint8)."""
    rows = qs.shape[0]
    c = (np.asarray(qs, dtype=np.uint32)[..., None] >> (2 * np.arange(16, dtype=np.uint32))) & 3
    return c.astype(np.uint8).reshape(rows, -1)


def _bits_to_bytes(bits: np.ndarray) -> np.ndarray:
    return np.packbits(bits.astype(np.uint8), axis=-1, bitorder="little")


def _bytes_to_bits(planes: np.ndarray, count: int) -> np.ndarray:
    return np.unpackbits(np.ascontiguousarray(planes, dtype=np.uint8), axis=-1,
                         bitorder="little")[:, :count]


# ---------------------------------------------------------------------------
# pack: ik wire -> relayout
# ---------------------------------------------------------------------------


def _check_wire(member: str, wire: np.ndarray, n: int) -> np.ndarray:
    expect = ik_row_bytes(member, n)
    if wire.ndim != 2 or wire.shape[1] != expect:
        raise IqkFormatError(
            f"{member} rows of {n} weights are {expect} wire bytes, got {wire.shape}")
    return np.ascontiguousarray(wire, dtype=np.uint8)


def _pack_iq2_ks(wire: np.ndarray, n: int) -> dict[str, np.ndarray]:
    """(reference: src/mlx_iqk/format.py:478-517)"""
    wire = _check_wire("iq2_ks", wire, n)
    rows, nb = wire.shape[0], n // QK_K
    body = wire[:, 2:].reshape(rows, nb, IQ2_KS_BLOCK_BYTES)
    return {
        "qs": _codes_to_qs(_wire_codes("iq2_ks", body[:, :, 6:])),
        "scl": np.ascontiguousarray(body[:, :, 2:6]).reshape(rows, nb * 4),
        # extra: low byte = alphabet bits, high byte = scale high bits, both in
        # sub-block order, so each plane is one byte per block.
        "sch": np.ascontiguousarray(body[:, :, 1]),
        "sex": np.ascontiguousarray(body[:, :, 0]),
        "dv": wire[:, 0:2].copy().view(np.float16).reshape(rows),
    }


def _pack_iq2_k(wire: np.ndarray, n: int) -> dict[str, np.ndarray]:
    """(reference: src/mlx_iqk/format.py:520-554)"""
    wire = _check_wire("iq2_k", wire, n)
    rows, nb = wire.shape[0], n // QK_K
    body = wire.reshape(rows, nb, IQ2_K_BLOCK_BYTES)
    return {
        "qs": _codes_to_qs(_wire_codes("iq2_k", body[:, :, 12:])),
        "scl": np.ascontiguousarray(body[:, :, 4:12]).reshape(rows, nb * 8),
        "sex": np.ascontiguousarray(body[:, :, 2:4]).reshape(rows, nb * 2),
        "dv": np.ascontiguousarray(body[:, :, 0:2]).view(np.float16).reshape(rows, nb),
    }


def _pack_iq1_s_r4(wire: np.ndarray, n: int) -> dict[str, np.ndarray]:
    """De-interleave four-row groups (reference: src/mlx_iqk/format.py:557-588)."""
    wire = _check_wire("iq1_s_r4", wire, n)
    rows = check_wire_rows("iq1_s_r4", wire.shape[0])
    groups, nblk = rows // 4, n // 32
    g = wire.reshape(groups, 4 * ik_row_bytes("iq1_s_r4", n))
    body = g[:, 8:].reshape(groups, nblk, IQ1_S_R4_BLOCK_BYTES)
    # qs byte 4*i + k -> row k, sub-group i; qh word k -> row k.
    qs = body[:, :, :16].reshape(groups, nblk, 4, 4).transpose(0, 3, 1, 2)
    qh = np.ascontiguousarray(body[:, :, 16:]).view(np.uint16).reshape(groups, nblk, 4)
    return {
        "qs": np.ascontiguousarray(qs).reshape(rows, nblk * 4).view(np.uint32),
        "qh": np.ascontiguousarray(qh.transpose(0, 2, 1)).reshape(rows, nblk),
        "dv": np.ascontiguousarray(g[:, :8]).view(np.float16).reshape(rows),
    }


_PACK = {"iq2_ks": _pack_iq2_ks, "iq2_k": _pack_iq2_k, "iq1_s_r4": _pack_iq1_s_r4}


def pack(member: str, wire: np.ndarray, in_features: int,
         chunk: int = PACK_CHUNK_ROWS) -> dict[str, np.ndarray]:
    """Relayout ik wire rows ``[rows, ik_row_bytes]`` into the member's streams.

    Streams come back per row (``[rows, ...]``); reshape to
    :func:`component_shapes` for a stacked tensor.  The result does not depend
    on ``chunk``, which only bounds the working set
    (reference: src/mlx_iqk/format.py:612-678).
    """
    n = check_row_width(in_features, member)
    group = WIRE_GROUP_ROWS[member]
    if chunk <= 0 or chunk % group:
        raise IqkFormatError(
            f"pack chunk {chunk} is not a positive multiple of the {group}-row group")
    wire = np.asarray(wire)
    fn = _PACK[member]
    if wire.ndim == 2 and wire.shape[0] > chunk:
        check_wire_rows(member, wire.shape[0])
        parts = [fn(wire[i:i + chunk], n) for i in range(0, wire.shape[0], chunk)]
        return {k: np.concatenate([p[k] for p in parts], axis=0) for k in parts[0]}
    return fn(wire, n)


# ---------------------------------------------------------------------------
# unpack: relayout -> ik wire
# ---------------------------------------------------------------------------


def _rows2d(streams: dict[str, np.ndarray], name: str, rows: int) -> np.ndarray:
    return np.ascontiguousarray(streams[name]).reshape(rows, -1)


def _unpack_iq2_ks(streams: dict[str, np.ndarray], n: int) -> np.ndarray:
    rows = np.asarray(streams["qs"]).reshape(-1, n // 16).shape[0]
    nb = n // QK_K
    wire = np.empty((rows, ik_row_bytes("iq2_ks", n)), dtype=np.uint8)
    wire[:, 0:2] = _rows2d(streams, "dv", rows).astype(np.float16).view(np.uint8)
    body = wire[:, 2:].reshape(rows, nb, IQ2_KS_BLOCK_BYTES)
    body[:, :, 0] = _rows2d(streams, "sex", rows)
    body[:, :, 1] = _rows2d(streams, "sch", rows)
    body[:, :, 2:6] = _rows2d(streams, "scl", rows).reshape(rows, nb, 4)
    body[:, :, 6:] = _codes_wire("iq2_ks", _qs_to_codes(_rows2d(streams, "qs", rows)))
    return wire


def _unpack_iq2_k(streams: dict[str, np.ndarray], n: int) -> np.ndarray:
    rows = np.asarray(streams["qs"]).reshape(-1, n // 16).shape[0]
    nb = n // QK_K
    wire = np.empty((rows, ik_row_bytes("iq2_k", n)), dtype=np.uint8)
    body = wire.reshape(rows, nb, IQ2_K_BLOCK_BYTES)
    body[:, :, 0:2] = _rows2d(streams, "dv", rows).astype(np.float16).view(
        np.uint8).reshape(rows, nb, 2)
    body[:, :, 2:4] = _rows2d(streams, "sex", rows).reshape(rows, nb, 2)
    body[:, :, 4:12] = _rows2d(streams, "scl", rows).reshape(rows, nb, 8)
    body[:, :, 12:] = _codes_wire("iq2_k", _qs_to_codes(_rows2d(streams, "qs", rows)))
    return wire


def _unpack_iq1_s_r4(streams: dict[str, np.ndarray], n: int) -> np.ndarray:
    nblk = n // 32
    rows = check_wire_rows("iq1_s_r4", np.asarray(streams["qs"]).reshape(-1, nblk).shape[0])
    groups = rows // 4
    row_bytes = ik_row_bytes("iq1_s_r4", n)
    g = np.empty((groups, 4 * row_bytes), dtype=np.uint8)
    g[:, :8] = _rows2d(streams, "dv", rows).astype(np.float16).view(np.uint8).reshape(groups, 8)
    body = g[:, 8:].reshape(groups, nblk, IQ1_S_R4_BLOCK_BYTES)
    qs = _rows2d(streams, "qs", rows).astype(np.uint32).view(np.uint8).reshape(groups, 4, nblk, 4)
    body[:, :, :16] = qs.transpose(0, 2, 3, 1).reshape(groups, nblk, 16)
    qh = _rows2d(streams, "qh", rows).astype(np.uint16).reshape(groups, 4, nblk)
    body[:, :, 16:] = np.ascontiguousarray(qh.transpose(0, 2, 1)).view(np.uint8).reshape(
        groups, nblk, 8)
    return g.reshape(rows, row_bytes)


_UNPACK = {"iq2_ks": _unpack_iq2_ks, "iq2_k": _unpack_iq2_k, "iq1_s_r4": _unpack_iq1_s_r4}


def unpack(member: str, streams: dict[str, np.ndarray], in_features: int,
           chunk: int = PACK_CHUNK_ROWS) -> np.ndarray:
    """Inverse of :func:`pack`: per-row streams back to ik wire rows
    (reference: src/mlx_iqk/format.py:744-772)."""
    n = check_row_width(in_features, member)
    group = WIRE_GROUP_ROWS[member]
    if chunk <= 0 or chunk % group:
        raise IqkFormatError(
            f"unpack chunk {chunk} is not a positive multiple of the {group}-row group")
    words = n // 16 if member != "iq1_s_r4" else n // 32
    rows = np.asarray(streams["qs"]).reshape(-1, words).shape[0]
    fn = _UNPACK[member]
    if rows <= chunk:
        return fn(streams, n)
    per_row = {k: np.ascontiguousarray(v).reshape(rows, -1) for k, v in streams.items()}
    return np.concatenate(
        [fn({k: v[i:i + chunk] for k, v in per_row.items()}, n)
         for i in range(0, rows, chunk)], axis=0)


# ---------------------------------------------------------------------------
# reference decode of the relayout
# ---------------------------------------------------------------------------


def _decode_planes_iq1_s_r4(streams: dict[str, np.ndarray], n: int) -> dict[str, np.ndarray]:
    nblk = n // 32
    qs = np.ascontiguousarray(streams["qs"]).reshape(-1, nblk).astype(np.uint32)
    rows = qs.shape[0]
    qh = np.ascontiguousarray(streams["qh"]).reshape(rows, nblk).astype(np.int64)
    low = qs.view(np.uint8).reshape(rows, nblk, 4).astype(np.int64)
    high = (qh[:, :, None] >> (3 * np.arange(4))) & 7
    index = (low | (high << 8)).reshape(rows, nblk * 4)
    scale_index = 2 * ((qh >> 12) & 7) + 1
    shift = np.where(qh & 0x8000, np.float32(-IQ1S_DELTA), np.float32(IQ1S_DELTA))
    d = np.asarray(streams["dv"]).reshape(rows, 1).astype(np.float32)
    dl = d * scale_index.astype(np.float32)
    values = grid_values()[index].reshape(rows, n).astype(np.int64)
    gv = values.astype(np.float32) + np.repeat(shift, 32, axis=1).astype(np.float32)
    weights = np.repeat(dl, 32, axis=1) * gv
    return {"codes": index, "values": values, "scale_index": scale_index,
            "sub_scale": dl, "shift": shift, "weights": weights.astype(np.float32)}


def decode_planes(member: str, streams: dict[str, np.ndarray],
                  in_features: int) -> dict[str, np.ndarray]:
    """Integer planes and the float32 reconstruction of relayout rows.

    ``weights`` follows the CPU dequantizer's chain: ``dl = d * float(idx)``
    then ``y = dl * float(value)`` (``IQ1_S_R4``: ``dl * (float(g) + shift)``)
    (reference: src/mlx_iqk/format.py:819-882).
    """
    n = check_row_width(in_features, member)
    if member == "iq1_s_r4":
        return _decode_planes_iq1_s_r4(streams, n)
    sub = SUB_WEIGHTS[member]
    nsub = n // sub
    qs = np.ascontiguousarray(streams["qs"]).reshape(-1, n // 16)
    rows = qs.shape[0]
    codes = _qs_to_codes(qs).astype(np.int64)
    scl = np.ascontiguousarray(streams["scl"]).reshape(rows, -1).astype(np.int64)
    nib = np.stack([scl & 0xF, scl >> 4], axis=-1).reshape(rows, nsub)
    alpha = _bytes_to_bits(np.ascontiguousarray(streams["sex"]).reshape(rows, -1),
                           nsub).astype(np.int64)
    if member == "iq2_ks":
        hi = _bytes_to_bits(np.ascontiguousarray(streams["sch"]).reshape(rows, -1),
                            nsub).astype(np.int64)
        scale_index = (nib | (hi << 4)) - 16
        d = np.asarray(streams["dv"]).reshape(rows, 1).astype(np.float32)
        d = np.repeat(d, nsub, axis=1)
    else:
        scale_index = nib - 8
        d = np.asarray(streams["dv"]).reshape(rows, n // QK_K).astype(np.float32)
        d = np.repeat(d, QK_K // sub, axis=1)
    dl = d * scale_index.astype(np.float32)
    values = IQ2NL_VALUES.astype(np.int64)[np.repeat(alpha, sub, axis=1) * 4 + codes]
    weights = np.repeat(dl, sub, axis=1) * values.astype(np.float32)
    return {"codes": codes, "values": values, "scale_index": scale_index,
            "sub_scale": dl, "weights": weights.astype(np.float32)}


def decode(member: str, streams: dict[str, np.ndarray], in_features: int) -> np.ndarray:
    """Float32 reference dequantization of relayout rows, ``[rows, n]``."""
    return decode_planes(member, streams, in_features)["weights"]


def decode_wire(member: str, wire: np.ndarray, in_features: int) -> np.ndarray:
    """Pack ik wire rows and decode them: the whole build-time path."""
    return decode(member, pack(member, wire, in_features), in_features)


__all__ = [
    "BLOCK_WEIGHTS", "IQ1S_DELTA", "IQ1_S_R4_BLOCK_BYTES", "IQ2NL_VALUES",
    "IQ2_KS_BLOCK_BYTES", "IQ2_K_BLOCK_BYTES", "MEMBERS", "PACK_CHUNK_ROWS", "QK_K",
    "SUB_WEIGHTS", "WIRE_GROUP_ROWS", "IqkFormatError", "bits_per_weight",
    "check_member", "check_row_width", "check_wire_rows", "component_dtypes",
    "component_shapes", "decode", "decode_planes", "decode_wire", "ik_row_bytes",
    "pack", "relayout_row_bytes", "unpack",
]
