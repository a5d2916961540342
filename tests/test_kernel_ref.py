"""The kernel-backend model (tests/kb_cases.py, codes decoded by the oracle) and
the oracle's transforms against the reference's own scalar IKernelBackend
(kernels/scalar/kdot_scalar.cpp, compiled in place into oracle/_ref): the
FWHTs bit for bit, kdot/vaccum within float32 rounding of the float64 model.
CPU only; the GPU backend is compared with both in test_gpu_kernel_backend.py."""
import numpy as np
import pytest

import kb_cases
from bind import KernelRef

pytestmark = pytest.mark.skipif(not KernelRef.available,
                                reason="oracle/_ref/libkernel_ref.so not built")


def test_reference_scalar_backend_matches_model(oracle):
    ref = KernelRef()
    for c in kb_cases.cases():
        if c["n"] == 1000 and c["p"] == 256:
            continue  # keep the CPU suite short; the GPU test covers it
        lg, acc = kb_cases.model(c, oracle)
        got = ref.kdot(c["q"], c["rows"], c["scales"], c["bits"])
        assert np.max(np.abs(got - lg)) <= 1e-5 * max(1.0, np.max(np.abs(lg))), (c["bits"], c["p"], c["n"])
        gv = ref.vaccum(c["rows"], c["scales"], c["w"], c["p"], c["bits"])
        assert np.max(np.abs(gv - acc)) <= 1e-5 * max(1.0, np.max(np.abs(acc))), (c["bits"], c["p"], c["n"])
        f = ref.fwht(c["x"], c["D"], True)
        i = ref.fwht(c["x"], c["D"], False)
        assert np.array_equal(f.view(np.uint32), oracle.fwht_forward(c["x"], c["D"]).view(np.uint32))
        assert np.array_equal(i.view(np.uint32), oracle.fwht_inverse(c["x"], c["D"]).view(np.uint32))
