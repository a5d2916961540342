"""The HIP IKernelBackend (include/adaptq/kernel.h, adaptq::select_kernel_backend)
driven through the interface by tests/cpp/kernel_backend_check.cpp, as the
reference's V2 runtime would call it.  Bar: fwht_forward/inverse bit-exact
with the oracle and with the reference's scalar backend; kdot_batch and
vaccum_batch within float32 rounding (1e-5 of the largest magnitude) of the
float64 model and of the reference's scalar backend."""
import os
import subprocess

import numpy as np
import pytest

import kb_cases
from bind import KernelRef

pytestmark = pytest.mark.gpu
ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def _close(got, want):
    return np.max(np.abs(got - want)) <= 1e-5 * max(1.0, float(np.max(np.abs(want))))


def test_hip_kernel_backend(oracle, tmp_path):
    exe = tmp_path / "kernel_backend_check"
    lib_dir = os.path.join(ROOT, "adaptq_amd")
    r = subprocess.run(["g++", "-std=c++17", "-O1", "-I", os.path.join(ROOT, "include"),
                        os.path.join(ROOT, "tests", "cpp", "kernel_backend_check.cpp"),
                        "-L", lib_dir, "-ladaptq", f"-Wl,-rpath,{lib_dir}", "-o", str(exe)],
                       capture_output=True, text=True)
    assert r.returncode == 0, r.stderr
    cs = kb_cases.cases()
    kb_cases.write_inputs(tmp_path / "in.bin", cs)
    r = subprocess.run([str(exe), str(tmp_path / "in.bin"), str(tmp_path / "out.bin")],
                       capture_output=True, text=True, timeout=120)
    print(r.stdout, r.stderr)
    assert r.returncode == 0, r.stdout + r.stderr
    assert "backend hip-gfx950" in r.stdout and f"cases {len(cs)}" in r.stdout
    outs = kb_cases.read_outputs(tmp_path / "out.bin", cs)
    ref = KernelRef() if KernelRef.available else None
    for c, o in zip(cs, outs):
        tag = (c["bits"], c["p"], c["n"])
        lg, acc = kb_cases.model(c, oracle)
        assert _close(o["logits"], lg), tag
        assert _close(o["acc"], acc), tag
        assert np.array_equal(o["fwd"].view(np.uint32),
                              oracle.fwht_forward(c["x"], c["D"]).view(np.uint32)), tag
        assert np.array_equal(o["inv"].view(np.uint32),
                              oracle.fwht_inverse(c["x"], c["D"]).view(np.uint32)), tag
        if ref is not None:
            assert _close(o["logits"], ref.kdot(c["q"], c["rows"], c["scales"], c["bits"])), tag
            assert _close(o["acc"], ref.vaccum(c["rows"], c["scales"], c["w"], c["p"], c["bits"])), tag
            assert np.array_equal(o["fwd"].view(np.uint32),
                                  ref.fwht(c["x"], c["D"], True).view(np.uint32)), tag
