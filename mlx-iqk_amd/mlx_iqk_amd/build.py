"""Build recipes for the two native libraries of this package.

* ``libiqk_codec.so`` -- the CPU codec (quantizers and dequantizers), g++.
* ``libiqk_hip.so``   -- the gfx950 kernels behind the C ABI, hipcc.

Both land in ``mlx_iqk_amd/_lib/`` beside the Python sources, so the built
files travel with the source tree.  ``python -m mlx_iqk_amd.build`` builds
both.
"""

from __future__ import annotations

import hashlib
import os
import shutil
import subprocess
import sys
import sysconfig
import tempfile
from pathlib import Path

PACKAGE = Path(__file__).resolve().parent
PROJECT = PACKAGE.parent
CSRC = PROJECT / "csrc"
INCLUDE = PROJECT.parent / "include"
LIBDIR = PACKAGE / "_lib"

CODEC_LIB = LIBDIR / "libiqk_codec.so"
HIP_LIB = LIBDIR / "libiqk_hip.so"
LAUNCH_EXT = LIBDIR / ("_iqk_launch" + (sysconfig.get_config_var("EXT_SUFFIX") or ".so"))

# Source -> extra hipcc flags.  The MFMA decode GEMV folds each accumulator
# right after its MFMA chain, so its MFMA results go straight to VGPRs.
HIP_SOURCES = {
    "iqk_abi.hip": (),
    "iqk_gemv.hip": (),
    "iqk_gemv_mfma.hip": ("-mllvm", "-amdgpu-mfma-vgpr-form"),
    "iqk_dequant.hip": (),
    "iqk_gemm.hip": (),
    "iqk_fused_gemm.hip": (),
    "iqk_pack.hip": (),
    "iqk_floor.hip": (),
    "iqk_route.hip": (),
}
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


def hip_source_files() -> list[Path]:
    """Every file the kernel library is compiled from."""
    return sorted([*(CSRC / "hip").glob("*.hip"), *(CSRC / "hip").glob("*.h"), CSRC / "iq1s_grid.h",
                   INCLUDE / "iqk_hip.h"])


def hip_source_hash() -> str:
    """A digest of the kernel library's sources and compile flags.  It is
    compiled into the library (``iqk_hip_source_hash``), so a loader can tell a
    library built from other sources -- a stale build -- from a current one."""
    h = hashlib.sha256()
    for f in hip_source_files():
        h.update(f.name.encode() + b"\0" + f.read_bytes() + b"\0")
    h.update(repr(sorted(HIP_SOURCES.items())).encode() + OFFLOAD_ARCH.encode())
    return h.hexdigest()[:16]


def hip_object_command(source: str, obj: Path, source_hash: str = "") -> list[str]:
    return [_hipcc(), f"--offload-arch={OFFLOAD_ARCH}", "-O3", "-fPIC", "-std=c++17",
            # packed fp32 VALU ops stay off: hand the compiler no v_pk_*_f32
            "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
            f'-DIQK_SOURCE_HASH="{source_hash or hip_source_hash()}"',
            *HIP_SOURCES[source], f"-I{INCLUDE}", "-c", "-o", str(obj), str(CSRC / "hip" / source)]


def hip_link_command(objects: list[Path], out: Path) -> list[str]:
    return [_hipcc(), f"--offload-arch={OFFLOAD_ARCH}", "-shared", "-fPIC", "-o", str(out)] + [str(o) for o in objects]


def build_codec() -> Path:
    LIBDIR.mkdir(parents=True, exist_ok=True)
    tmp = CODEC_LIB.with_suffix(".so.tmp")
    _run(codec_command(tmp))
    tmp.replace(CODEC_LIB)
    return CODEC_LIB


def build_hip() -> Path:
    """Compile every source to an object (in parallel, in a temporary
    directory) and link them into ``libiqk_hip.so``."""
    LIBDIR.mkdir(parents=True, exist_ok=True)
    tmp = HIP_LIB.with_suffix(".so.tmp")
    with tempfile.TemporaryDirectory(prefix="iqk_hip_") as work:
        objects = [Path(work) / (Path(s).stem + ".o") for s in HIP_SOURCES]
        digest = hip_source_hash()
        procs = [(cmd, subprocess.Popen(cmd, stdout=subprocess.PIPE, stderr=subprocess.PIPE, text=True))
                 for cmd in (hip_object_command(s, o, digest) for s, o in zip(HIP_SOURCES, objects))]
        failures = []
        for cmd, proc in procs:
            out, err = proc.communicate()
            if proc.returncode != 0:
                failures.append(f"{' '.join(cmd)}\n{out}\n{err}")
        if failures:
            raise RuntimeError("build failed: " + "\n".join(failures))
        _run(hip_link_command(objects, tmp))
    tmp.replace(HIP_LIB)
    return HIP_LIB


def launch_command(out: Path = LAUNCH_EXT, source_hash: str = "") -> list[str]:
    """The CPython binding of the decode launch path, linked against the
    kernel library beside it (found through $ORIGIN)."""
    return ["gcc", "-O2", "-shared", "-fPIC", f"-I{sysconfig.get_paths()['include']}", f"-I{INCLUDE}",
            f'-DIQK_SOURCE_HASH="{source_hash or hip_source_hash()}"', "-o", str(out),
            str(CSRC / "launch" / "iqk_launch.c"), f"-L{LIBDIR}", "-liqk_hip", "-Wl,-rpath,$ORIGIN"]


def build_launch() -> Path:
    LIBDIR.mkdir(parents=True, exist_ok=True)
    tmp = LAUNCH_EXT.with_suffix(".so.tmp")
    _run(launch_command(tmp))
    tmp.replace(LAUNCH_EXT)
    return LAUNCH_EXT


def build_all() -> None:
    build_codec()
    build_hip()
    build_launch()


if __name__ == "__main__":
    build_all()
    print(f"built {CODEC_LIB}\nbuilt {HIP_LIB}", file=sys.stderr)
