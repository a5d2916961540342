"""The sparse-V kernels' exponential (aq::expf_ref, adaptq_amd/csrc/expf_ref.hpp,
a restatement of glibc 2.35's expf) equals the host libm's expf -- the one the
reference's softmax calls -- on every float in [-104, 89] and the special
values: the header is compiled for the host by tests/cpp/expf_check.cpp
(FMA contraction off, as in the kernels' build; ~5 s on 8 threads)."""
import os
import shutil
import subprocess

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def test_expf_ref_equals_libm_everywhere(tmp_path):
    if not shutil.which("g++"):
        pytest.skip("no g++")
    exe = tmp_path / "expf_check"
    r = subprocess.run(["g++", "-std=c++17", "-O2", "-mfma", "-ffp-contract=off", "-pthread",
                        os.path.join(ROOT, "tests", "cpp", "expf_check.cpp"), "-lm", "-o", str(exe)],
                       capture_output=True, text=True)
    assert r.returncode == 0, r.stderr
    r = subprocess.run([str(exe)], capture_output=True, text=True, timeout=300)
    assert r.returncode == 0 and " 0 mismatches" in r.stdout, r.stdout
