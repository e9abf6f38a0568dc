"""The IQ1_S ternary grid, the one lookup table ``IQ1_S_R4`` decodes from.

The 2048 packed code words live in one place, ``csrc/iq1s_grid.h``, which the
CPU codec and the HIP kernels compile in; this module reads the same file so
the Python decode, the CPU codec and the GPU kernels cannot disagree about a
single entry.

Entry ``k`` packs eight positions at two bits each (position ``i`` in bits
``2i..2i+1``); the decoded value of position ``i`` is ``field - 1``, one of
-1, 0, +1 (reference: src/mlx_iqk/iq1grid.py:199-212,
vendor/ik_llama/iqk_iq1sr4.cpp:257-265).
"""

from __future__ import annotations

import re
from functools import lru_cache
from pathlib import Path

import numpy as np

NGRID_IQ1S = 2048
"""Grid entries; an index is 11 bits and every value is legal."""

ZERO_INDEX = 1029
"""The grid entry whose eight values are all zero (code word 0x5555)."""

GRID_HEADER = Path(__file__).resolve().parents[1] / "csrc" / "iq1s_grid.h"


@lru_cache(maxsize=1)
def _codes() -> np.ndarray:
    text = GRID_HEADER.read_text()
    body = text.split("iqk_iq1s_grid_codes[IQK_IQ1S_GRID_SIZE] = {", 1)[1]
    body = body.split("};", 1)[0]
    words = [int(tok, 16) for tok in re.findall(r"0x[0-9a-fA-F]+", body)]
    if len(words) != NGRID_IQ1S:
        raise RuntimeError(f"{GRID_HEADER} holds {len(words)} grid words, not 2048")
    out = np.array(words, dtype=np.uint16)
    out.setflags(write=False)
    return out


def grid_codes() -> np.ndarray:
    """The packed grid code words as ``uint16 [2048]`` (read-only)."""
    return _codes()


@lru_cache(maxsize=1)
def _values() -> np.ndarray:
    codes = _codes().astype(np.int32)[:, None]
    fields = (codes >> (2 * np.arange(8, dtype=np.int32))[None, :]) & 3
    out = (fields - 1).astype(np.int8)
    out.setflags(write=False)
    return out


def grid_values() -> np.ndarray:
    """The decode table as ``int8 [2048, 8]``, every value in -1, 0, +1."""
    return _values()


__all__ = ["GRID_HEADER", "NGRID_IQ1S", "ZERO_INDEX", "grid_codes", "grid_values"]
