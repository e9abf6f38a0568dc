"""Write the golden vectors under tests/golden/ from the reference's own codec.

Run in a container that has the reference sources (``make -C oracle ref``
builds them into oracle/_ref from /root/reference/vendor/ik_llama):

    python tests/golden/make_golden.py

Each fixture is data only -- inputs and the reference's outputs:

* ``quantize_<member>.npz``: seeded float rows (with zero and tiny rows), an
  imatrix with a zeroed span, and the reference quantizer's wire bytes with
  and without the imatrix;
* ``dequant_<member>.npz``: random wire over the whole fp16 scale range and
  the reference dequantizer's float32 output;
* ``exhaustive.json``: sha256 of the reference dequantizer's float32 output
  over each member's exhaustive enumeration (tests/wirepack.py), too large to
  store whole.
"""

from __future__ import annotations

import hashlib
import json
import sys
from pathlib import Path

import numpy as np

HERE = Path(__file__).resolve().parent
ROOT = HERE.parents[1]
sys.path.insert(0, str(ROOT))
sys.path.insert(0, str(ROOT / "tests"))

import wirepack  # noqa: E402
from oracle import oracle  # noqa: E402

MEMBERS = ("iq2_ks", "iq2_k", "iq1_s_r4")
N = {"iq2_ks": 512, "iq2_k": 512, "iq1_s_r4": 256}


def quantize_fixture(member: str) -> dict:
    n = N[member]
    rng = np.random.default_rng(wirepack.seed_for("golden-quantize", member))
    rows = (rng.standard_normal((8, n)) * 0.02).astype(np.float32)
    rows[1] = 0.0
    rows[2] *= 1e-4
    imatrix = (rng.random(n) * 0.9 + 0.1).astype(np.float32)
    imatrix[: n // 8] = 0.0
    return {
        "rows": rows, "imatrix": imatrix,
        "wire_imatrix": oracle.ref_quantize(member, rows, imatrix),
        "wire_plain": oracle.ref_quantize(member, rows, None),
    }


def dequant_fixture(member: str) -> dict:
    n = N[member]
    wire = wirepack.random_wire(member, 8, n, seed=wirepack.seed_for("golden-dequant", member), scales="sweep")
    return {"wire": wire, "n": np.array(n), "out": oracle.ref_dequantize(member, wire, n)}


def exhaustive_digests() -> dict:
    makers = {"iq2_ks": wirepack.exhaustive_iq2_ks, "iq2_k": wirepack.exhaustive_iq2_k,
              "iq1_s_r4": wirepack.exhaustive_iq1_s_r4}
    out = {}
    for member, maker in makers.items():
        wire = maker(seed=5)
        ref = oracle.ref_dequantize(member, wire, 256)
        out[member] = {"seed": 5, "rows": int(wire.shape[0]),
                       "wire_sha256": hashlib.sha256(wire.tobytes()).hexdigest(),
                       "out_sha256": hashlib.sha256(ref.tobytes()).hexdigest()}
    return out


def main() -> None:
    if not oracle.ref_available():
        oracle.build(with_ref=True)
    for member in MEMBERS:
        np.savez_compressed(HERE / f"quantize_{member}.npz", **quantize_fixture(member))
        np.savez_compressed(HERE / f"dequant_{member}.npz", **dequant_fixture(member))
    (HERE / "exhaustive.json").write_text(json.dumps(exhaustive_digests(), indent=2, sort_keys=True) + "\n")
    print("golden vectors written to", HERE)


if __name__ == "__main__":
    main()
