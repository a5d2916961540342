"""The append kernel's 4-bit quantiser (quantize4_tab in adaptq_amd/csrc/quant.hpp,
one table lookup) equals the reference's binary search (quantize<4>) on every
float bit pattern, and the oracle's quantize_fast on a stride of them: the
header is compiled for the host by tests/cpp/quant_exhaustive.cpp (~3 s on 8
threads)."""
import os
import shutil
import subprocess

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def test_quantize4_table_equals_binary_search_everywhere(tmp_path):
    if not shutil.which("g++"):
        pytest.skip("no g++")
    exe = tmp_path / "quant_exhaustive"
    r = subprocess.run(["g++", "-std=c++17", "-O2", "-pthread",
                        os.path.join(ROOT, "tests", "cpp", "quant_exhaustive.cpp"),
                        "-x", "c", os.path.join(ROOT, "oracle", "oracle.c"), "-lm", "-o", str(exe)],
                       capture_output=True, text=True)
    assert r.returncode == 0, r.stderr
    r = subprocess.run([str(exe)], capture_output=True, text=True, timeout=300)
    assert r.returncode == 0 and "mismatches 0" in r.stdout, r.stdout
