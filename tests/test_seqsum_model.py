"""The segment algorithm of chain_sum_block (adaptq_amd/csrc/seqsum.hpp: the
reference's left-to-right fp32 sums of the sparse-V selection,
attention.cpp:422-426 and :454-472, computed by a whole block) run on the host
with the kernels' own per-term functions (seqsum_terms.hpp), against the
plain fp32 chain: the count of terms added before the stop and the sum's bits
must be equal on every sequence of tests/cpp/seqsum_check.cpp (softmax sums,
sorted-probability quad sums with mass stops, stops at reached values,
tie-heavy, subnormal, zero and wide-range terms), for 1 to 8 terms a thread
and in chunks of 8,192 terms (chain_sum_long); with a planted 3-5% error in
the prefix the walk's checks must send sums to the redo and still give the
chain's bits."""
import os
import shutil
import subprocess

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def test_seqsum_model_equals_chain(tmp_path):
    if not shutil.which("g++"):
        pytest.skip("no g++")
    exe = tmp_path / "seqsum_check"
    r = subprocess.run(["g++", "-std=c++17", "-O2", "-ffp-contract=off",
                        os.path.join(ROOT, "tests", "cpp", "seqsum_check.cpp"), "-o", str(exe)],
                       capture_output=True, text=True)
    assert r.returncode == 0, r.stderr
    r = subprocess.run([str(exe)], capture_output=True, text=True, timeout=300)
    assert r.returncode == 0 and " 0 mismatches" in r.stdout, r.stdout
    # the planted misprediction reached the redo
    redone = int(r.stdout.split(" segments, ")[1].split(" redone")[0])
    assert redone > 0, r.stdout
