"""Build recipes for the two native libraries of this package.

* ``libiqk_codec.so`` -- the CPU codec (quantizers and dequantizers), g++.
* ``libiqk_hip.so``   -- the gfx950 kernels behind the C ABI, hipcc.

Both land in ``mlx_iqk_amd/_lib/`` beside the Python sources, so the built
files travel with the source tree.  ``python -m mlx_iqk_amd.build`` builds
both.
"""

from __future__ import annotations

import os
import shutil
import subprocess
import sys
from pathlib import Path

PACKAGE = Path(__file__).resolve().parent
PROJECT = PACKAGE.parent
CSRC = PROJECT / "csrc"
INCLUDE = PROJECT.parent / "include"
LIBDIR = PACKAGE / "_lib"

CODEC_LIB = LIBDIR / "libiqk_codec.so"
HIP_LIB = LIBDIR / "libiqk_hip.so"

HIP_SOURCES = ("iqk_abi.hip", "iqk_gemv.hip", "iqk_gemv_mfma.hip", "iqk_dequant.hip", "iqk_gemm.hip")
OFFLOAD_ARCH = "gfx950"


def _hipcc() -> str:
    for cand in (os.environ.get("HIPCC"), "/opt/rocm/bin/hipcc", shutil.which("hipcc")):
        if cand and Path(cand).exists():
            return cand
    raise RuntimeError("hipcc not found (set HIPCC or install ROCm)")


def _run(cmd: list[str]) -> None:
    proc = subprocess.run(cmd, capture_output=True, text=True)
    if proc.returncode != 0:
        raise RuntimeError(f"build failed: {' '.join(cmd)}\n{proc.stdout}\n{proc.stderr}")


def codec_command(out: Path = CODEC_LIB) -> list[str]:
    # Plain IEEE single precision: no -ffast-math, no -mfma, so the quantizers'
    # float rounding is the reference's.
    return ["g++", "-O2", "-std=c++17", "-fPIC", "-shared", "-pthread", f"-I{INCLUDE}",
            "-o", str(out), str(CSRC / "codec" / "iqk_codec.cpp")]


def hip_command(out: Path = HIP_LIB) -> list[str]:
    return [_hipcc(), f"--offload-arch={OFFLOAD_ARCH}", "-O3", "-fPIC", "-shared", "-std=c++17",
            # packed fp32 VALU ops stay off: hand the compiler no v_pk_*_f32
            "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
            f"-I{INCLUDE}", "-o", str(out)] + [str(CSRC / "hip" / s) for s in HIP_SOURCES]


def build_codec() -> Path:
    LIBDIR.mkdir(parents=True, exist_ok=True)
    tmp = CODEC_LIB.with_suffix(".so.tmp")
    _run(codec_command(tmp))
    tmp.replace(CODEC_LIB)
    return CODEC_LIB


def build_hip() -> Path:
    LIBDIR.mkdir(parents=True, exist_ok=True)
    tmp = HIP_LIB.with_suffix(".so.tmp")
    _run(hip_command(tmp))
    tmp.replace(HIP_LIB)
    return HIP_LIB


def build_all() -> None:
    build_codec()
    build_hip()


if __name__ == "__main__":
    build_all()
    print(f"built {CODEC_LIB}\nbuilt {HIP_LIB}", file=sys.stderr)
