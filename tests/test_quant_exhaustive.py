"""The append kernels' quantisers (the 4-bit cell lookup quantize_g4 and the
sign-split quantize_ss2/3 in adaptq_amd/csrc/quant.hpp) equal the reference's
binary search (quantize<B>) on every float bit pattern (every finite one for
the sign-split forms; NaN takes its code before the cell lookup, as the wide
append kernel does), and the oracle's quantize_fast on a stride of them; the
2-bit quantiser of the values before the scalings (quantize_bd2) equals
quantize<2> of the twice-rounded scaled value on every finite float for every
padded size up to 128: the header is compiled for the host by
tests/cpp/quant_exhaustive.cpp (~50 s on 8 threads)."""
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
