"""The host-side C/C++ under AddressSanitizer and UndefinedBehaviorSanitizer.

Builds tests/sanitize/harness.cpp with the package codec
(csrc/codec/iqk_codec.cpp) and the C oracle (oracle/iqk_oracle.c), all with
``-fsanitize=address,undefined``, into a temporary directory, and runs it on
the CPU: every quantizer and dequantizer over ordinary, degenerate and
extreme rows and over random wire, on four worker threads, with the codec's
dequantization checked against the oracle's bit for bit.  Any sanitizer
report aborts the harness, so the test needs its exit status 0 and a clean
stderr.
"""

from __future__ import annotations

import os
import shutil
import subprocess
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parents[1]
SAN = ["-fsanitize=address,undefined", "-fno-sanitize-recover=all", "-fno-omit-frame-pointer", "-g", "-O1"]


@pytest.fixture(scope="module")
def harness(tmp_path_factory):
    if not shutil.which("g++") or not shutil.which("gcc"):
        pytest.skip("no host compiler")
    work = tmp_path_factory.mktemp("sanitize")
    oracle_obj = work / "iqk_oracle.o"
    exe = work / "harness"
    steps = [
        ["gcc", *SAN, "-std=c11", "-c", "-o", str(oracle_obj), str(ROOT / "oracle" / "iqk_oracle.c")],
        ["g++", *SAN, "-std=c++17", "-pthread", f"-I{ROOT / 'include'}", "-o", str(exe),
         str(ROOT / "tests" / "sanitize" / "harness.cpp"),
         str(ROOT / "mlx-iqk_amd" / "csrc" / "codec" / "iqk_codec.cpp"), str(oracle_obj), "-lm"],
    ]
    for cmd in steps:
        proc = subprocess.run(cmd, capture_output=True, text=True)
        assert proc.returncode == 0, f"{' '.join(cmd)}\n{proc.stderr}"
    return exe


def test_codec_and_oracle_run_clean_under_asan_and_ubsan(harness):
    env = dict(os.environ, ASAN_OPTIONS="detect_leaks=0:abort_on_error=0:halt_on_error=1",
               UBSAN_OPTIONS="print_stacktrace=1:halt_on_error=1")
    proc = subprocess.run([str(harness)], capture_output=True, text=True, env=env, timeout=600)
    assert proc.returncode == 0, proc.stdout + proc.stderr
    assert "runtime error" not in proc.stderr and "Sanitizer" not in proc.stderr, proc.stderr
    assert "0 failure(s)" in proc.stdout
