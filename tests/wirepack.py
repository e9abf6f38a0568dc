"""Independent packers into the ik block layouts, for the bit-exactness gates.

They build ``block_iq2_ks`` / ``block_iq2_k`` / ``block_iq1_s_r4`` bytes
straight from field values (codes, scale indices, alphabet bits, grid
indices), writing each weight's field where the ik encoders put it
(reference: vendor/ik_llama/iqk_iq2.cpp:330-336, 485-489;
vendor/ik_llama/iqk_iq1sr4.cpp:552-572).  They do not use the package's
format module, so a test that checks the package's decode against them
cannot pass because both share a mistake (the reference keeps the same
separation, tests/wirepack.py:1-10).
"""

from __future__ import annotations

import zlib

import numpy as np

QK = 256


def seed_for(*parts) -> int:
    """A stable seed from any label (Python's str hash is salted per process)."""
    return zlib.crc32("|".join(str(p) for p in parts).encode()) % (2 ** 31)


def finite_half(rng: np.random.Generator, size) -> np.ndarray:
    """Random finite fp16 values over the whole sign/exponent range."""
    bits = rng.integers(0, 1 << 16, size=size, dtype=np.uint32).astype(np.uint16)
    nonfinite = (bits & 0x7C00) == 0x7C00
    bits = np.where(nonfinite, bits & 0xBFFF, bits).astype(np.uint16)
    return bits.view(np.float16)


def serving_half(rng: np.random.Generator, size) -> np.ndarray:
    """Scales of the magnitude a converted expert row carries, subnormals included."""
    mag = rng.random(size) * 8e-4 + 2e-5
    return (mag * np.where(rng.random(size) < 0.5, -1.0, 1.0)).astype(np.float16)


def tiny_half(rng: np.random.Generator, size) -> np.ndarray:
    """Subnormal fp16 scales (either sign), mantissas log-uniform so many are a
    few ulps of 2^-24: a large share of decoded weights come out subnormal (or
    round to zero), and none overflows."""
    e = rng.integers(0, 10, size=size)
    bits = rng.integers(1 << e, 1 << (e + 1), dtype=np.int64) | np.where(rng.random(size) < 0.5, 0x8000, 0)
    return bits.astype(np.uint16).view(np.float16)


def _scales(rng, size, mode):
    if mode == "sweep":
        return finite_half(rng, size)
    if mode == "serving":
        return serving_half(rng, size)
    if mode == "tiny":
        return tiny_half(rng, size)
    raise ValueError(mode)


def pack_iq2_ks_row(codes: np.ndarray, ls: np.ndarray, alpha: np.ndarray, d: float) -> np.ndarray:
    """One IQ2_KS row from fields: codes [nb, 256] (0..3), ls [nb, 8] (0..31,
    offset-16 scale index), alpha [nb, 8] (0/1); d the fp16 row scale."""
    nb = codes.shape[0]
    row = np.zeros(2 + 70 * nb, dtype=np.uint8)
    row[:2] = np.array([d], dtype=np.float16).view(np.uint8)
    for b in range(nb):
        blk = row[2 + 70 * b: 2 + 70 * (b + 1)]
        extra = 0
        for sb in range(8):
            v = int(ls[b, sb])
            blk[2 + sb // 2] |= (v & 15) << (4 * (sb % 2))
            extra |= ((v >> 4) & 1) << (8 + sb)
            extra |= (int(alpha[b, sb]) & 1) << sb
        blk[0], blk[1] = extra & 0xFF, extra >> 8
        for w in range(QK):
            sb = w // 32
            blk[6 + 32 * (sb // 4) + w % 32] |= int(codes[b, w]) << (2 * (sb % 4))
    return row


def pack_iq2_k_row(codes: np.ndarray, ls: np.ndarray, alpha: np.ndarray, d: np.ndarray) -> np.ndarray:
    """One IQ2_K row: codes [nb, 256], ls [nb, 16] (0..15, offset-8), alpha [nb, 16],
    d [nb] fp16 block scales."""
    nb = codes.shape[0]
    row = np.zeros(76 * nb, dtype=np.uint8)
    for b in range(nb):
        blk = row[76 * b: 76 * (b + 1)]
        blk[:2] = np.array([d[b]], dtype=np.float16).view(np.uint8)
        extra = 0
        for sb in range(16):
            blk[4 + sb // 2] |= (int(ls[b, sb]) & 15) << (4 * (sb % 2))
            extra |= (int(alpha[b, sb]) & 1) << sb
        blk[2], blk[3] = extra & 0xFF, extra >> 8
        for w in range(QK):
            ib32 = w // 32
            blk[12 + 32 * (ib32 // 4) + 16 * ((w // 16) % 2) + w % 16] |= int(codes[b, w]) << (2 * (ib32 % 4))
    return row


def pack_iq1_s_r4_group(index: np.ndarray, ls: np.ndarray, neg: np.ndarray, d: np.ndarray) -> np.ndarray:
    """One four-row IQ1_S_R4 group: index [4, n/8] grid indices (0..2047),
    ls [4, n/32] (0..7), neg [4, n/32] (1 = shift -0.125), d [4] fp16."""
    nblk = index.shape[1] // 4
    grp = np.zeros(8 + 24 * nblk, dtype=np.uint8)
    grp[:8] = np.asarray(d, dtype=np.float16).view(np.uint8)
    for ib in range(nblk):
        blk = grp[8 + 24 * ib: 8 + 24 * (ib + 1)]
        for k in range(4):
            h = (int(ls[k, ib]) & 7) << 12 | (int(neg[k, ib]) & 1) << 15
            for i in range(4):
                g = int(index[k, 4 * ib + i])
                blk[4 * i + k] = g & 0xFF
                h |= (g >> 8) << (3 * i)
            blk[16 + 2 * k], blk[17 + 2 * k] = h & 0xFF, h >> 8
    return grp


def exhaustive_iq2_ks(seed: int = 0) -> np.ndarray:
    """Every (scale index, alphabet, code) triple at every position: 32 x 2 x 4
    rows of one 256-weight block, codes rotated so each position sees each code."""
    rng = np.random.default_rng(seed)
    w = np.arange(QK)
    rows = []
    for s in range(32):
        for a in range(2):
            for rot in range(4):
                rows.append(pack_iq2_ks_row(((w + rot) % 4)[None], np.full((1, 8), s), np.full((1, 8), a),
                                            finite_half(rng, 1)[0]))
    return np.stack(rows)


def exhaustive_iq2_k(seed: int = 0) -> np.ndarray:
    """Every (scale index, alphabet, code) triple at every position: 16 x 2 x 4 rows."""
    rng = np.random.default_rng(seed)
    w = np.arange(QK)
    rows = []
    for s in range(16):
        for a in range(2):
            for rot in range(4):
                rows.append(pack_iq2_k_row(((w + rot) % 4)[None], np.full((1, 16), s), np.full((1, 16), a),
                                           finite_half(rng, 1)))
    return np.stack(rows)


def exhaustive_iq1_s_r4(seed: int = 0) -> np.ndarray:
    """Every grid index at every block position under every (scale, shift sign):
    rows of 256 weights (32 indices each); 64 rows cover the 2048 indices, four
    rotations move each index through the four positions of its block."""
    rng = np.random.default_rng(seed)
    idx = np.arange(2048).reshape(64, 32)
    groups = []
    for s in range(8):
        for neg in range(2):
            for rot in range(4):
                block = np.roll(idx, rot, axis=1)
                for g in range(16):
                    groups.append(pack_iq1_s_r4_group(block[4 * g: 4 * g + 4], np.full((4, 8), s),
                                                      np.full((4, 8), neg), finite_half(rng, 4)))
    wire = np.stack(groups)  # [groups, 4 * row_bytes]
    return wire.reshape(-1, 2 + 6 * 256 // 32)


def random_wire(member: str, rows: int, n: int, seed: int, scales: str = "sweep") -> np.ndarray:
    """Uniformly random wire rows; every field of every member is legal over its
    whole byte space, only the fp16 scales are drawn (``sweep`` = all finite fp16,
    ``serving`` = converted-row magnitudes, ``tiny`` = subnormal fp16)."""
    rng = np.random.default_rng(seed)
    if member == "iq1_s_r4":
        assert rows % 4 == 0
        rb = 2 + 6 * (n // 32)
        out = rng.integers(0, 256, size=(rows, rb), dtype=np.uint8)
        g = out.reshape(rows // 4, 4 * rb)
        g[:, :8] = _scales(rng, (rows // 4, 4), scales).view(np.uint8).reshape(rows // 4, 8)
        return out
    nb = n // QK
    if member == "iq2_k":
        out = rng.integers(0, 256, size=(rows, nb, 76), dtype=np.uint8)
        out[:, :, :2] = _scales(rng, (rows, nb), scales).view(np.uint8).reshape(rows, nb, 2)
        return out.reshape(rows, 76 * nb)
    out = rng.integers(0, 256, size=(rows, 2 + 70 * nb), dtype=np.uint8)
    out[:, :2] = _scales(rng, rows, scales).view(np.uint8).reshape(rows, 2)
    return out
