"""The C-ABI library without a GPU: it loads, exports every function that
include/*.h declares, and its argument validation answers with the
reference's return codes and error strings (core/adaptq_c_api.cpp:15-281)
before any device call is made.  No compute call is issued here."""
import ctypes as C
import glob
import os
import re

import numpy as np
import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


@pytest.fixture(scope="module")
def lib():
    from adaptq_amd import _lib
    return _lib.lib


def declared_functions():
    names = set()
    for h in glob.glob(os.path.join(ROOT, "include", "*.h")):
        text = open(h).read()
        text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
        text = re.sub(r"//[^\n]*", "", text)
        for m in re.finditer(r"\b(adaptq_[a-z_0-9]+)\s*\(", text):
            names.add(m.group(1))
    return names


# C++-linkage declarations (adaptq_backend.h) are exported under their
# Itanium-mangled names, as in the reference's build.
MANGLED = {"adaptq_make_vtable": "_Z18adaptq_make_vtableP14IAdaptQBackend"}


def test_exports_every_declared_symbol(lib):
    names = declared_functions()
    assert len(names) >= 17 + 8
    missing = [n for n in sorted(names) if not hasattr(lib, MANGLED.get(n, n))]
    assert not missing, missing


def test_signature_table_covers_header():
    from adaptq_amd import _lib
    # adaptq_make_vtable has C++ linkage (a struct by value): not bound through ctypes
    names = declared_functions() - {"adaptq_make_vtable"}
    assert names <= set(_lib.SIGNATURES), names - set(_lib.SIGNATURES)


def test_version_and_features(lib):
    from adaptq_amd import _lib
    assert lib.adaptq_version().decode()
    f = lib.adaptq_features()
    assert f & _lib.FEAT_HYBRID and f & _lib.FEAT_SPARSE_V and f & _lib.FEAT_HIP
    assert not f & _lib.FEAT_AVX2


@pytest.mark.parametrize("args", [
    (0, 4, 2, 16), (-1, 4, 2, 16), (64, 5, 2, 16), (64, 4, 1, 16), (64, 4, 2, -1),
    (64, 8, 2, 16), (64, 4, 17, 16),
])
def test_create_rejects_invalid(lib, args):
    dim, kb, vb, cap = args
    assert lib.adaptq_create(dim, kb, vb, cap, 0, 0.0, 0) is None
    assert lib.adaptq_last_error() == b"adaptq_create: invalid dimensions or capacity"
    assert lib.adaptq_create(64, 4, 2, 16, 0, 0.0, -1) is None


def test_mha_create_rejects_invalid(lib):
    assert lib.adaptq_mha_create(0, 64, 4, 2, 16, 0, 0.0, 0) is None
    assert lib.adaptq_last_error() == b"adaptq_mha_create: invalid parameters"
    assert lib.adaptq_mha_create(4, 64, 4, 3 + 2, 16, 0, 0.0, 0) is None


def test_null_handles(lib):
    f = np.zeros(64, np.float32)
    fp = f.ctypes.data_as(C.POINTER(C.c_float))
    lib.adaptq_destroy(None)
    lib.adaptq_mha_destroy(None)
    assert lib.adaptq_compute(None, fp, fp) == -1
    assert lib.adaptq_last_error() == b"adaptq_compute: null handle"
    assert lib.adaptq_compute_batch(None, fp, 1, fp) == -1
    assert lib.adaptq_last_error() == b"adaptq_compute_batch: null handle"
    lib.adaptq_append(None, fp, fp, 0)
    assert lib.adaptq_last_error() == b"adaptq_append: null handle"
    lib.adaptq_reset(None)
    assert lib.adaptq_last_error() == b"adaptq_reset: null handle"
    assert lib.adaptq_kv_bytes(None) == 0
    assert lib.adaptq_last_error() == b"adaptq_kv_bytes: null handle"
    assert lib.adaptq_mha_compute(None, 0, fp, fp) == -1
    assert lib.adaptq_last_error() == b"adaptq_mha_compute: null handle"
    assert lib.adaptq_mha_compute_batch(None, 0, fp, 1, fp) == -1
    lib.adaptq_mha_append(None, 0, fp, fp, 0)
    assert lib.adaptq_last_error() == b"adaptq_mha_append: null handle"
    lib.adaptq_mha_reset(None)
    assert lib.adaptq_mha_total_kv_bytes(None) == 0
    assert lib.adaptq_flush(None) == -1
    assert lib.adaptq_mha_head(None, 0) is None
    assert lib.adaptq_plan_create(None, 0) is None
    lib.adaptq_plan_destroy(None)
    assert lib.adaptq_plan_compute_device(None, None, None, None) == -1
    assert lib.adaptq_plan_append_device(None, None, None, 1, 0, None) == -1
    assert lib.adaptq_plan_compute_device_static(None, None, None, None) == -1
    assert lib.adaptq_plan_workspace_bytes(None) == -1
    assert lib.adaptq_last_error() == b"adaptq_plan_workspace_bytes: null handle"


def test_error_is_thread_local(lib):
    import threading
    lib.adaptq_compute(None, None, None)
    seen = []
    t = threading.Thread(target=lambda: seen.append(lib.adaptq_last_error()))
    t.start()
    t.join()
    assert seen == [b""]
    assert lib.adaptq_last_error() == b"adaptq_compute: null handle"


def test_pybind_module_loads():
    import importlib
    m = importlib.import_module("adaptq_amd.adaptq_py")
    assert hasattr(m, "MHAContext")
    with pytest.raises(RuntimeError, match="invalid parameters"):
        m.MHAContext(0, 64, 4, 2, 16)  # rejected before any device call


def test_llama_adapter_header_compiles():
    """include/adapter_llamacpp.h builds as llama.cpp would include it, and a
    program using it links against libadaptq.so (run on the GPU in
    test_gpu_ggml.py)."""
    import shutil
    import subprocess
    import tempfile
    if not shutil.which("g++"):
        pytest.skip("no g++")
    src = os.path.join(ROOT, "tests", "cpp", "llama_adapter_check.cpp")
    with tempfile.TemporaryDirectory() as d:
        r = subprocess.run(["g++", "-std=c++17", "-I", os.path.join(ROOT, "include"), src,
                            "-L", os.path.join(ROOT, "adaptq_amd"), "-ladaptq",
                            "-o", os.path.join(d, "check")], capture_output=True, text=True)
    assert r.returncode == 0, r.stderr
