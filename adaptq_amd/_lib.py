"""ctypes binding of libadaptq.so (the C ABI in include/adaptq.h).

Loading the library does not touch the GPU; the first context creation does.
If the library has not been built, importing this module raises ImportError:
there is no CPU fallback.
"""
from __future__ import annotations

import ctypes as C
import os

_HERE = os.path.dirname(os.path.abspath(__file__))
# ADAPTQ_AMD_LIB names another build of the same ABI (bench.py --clock-stamps
# sets it to the timing library, libadaptq_clk.so)
LIB_PATH = os.environ.get("ADAPTQ_AMD_LIB") or os.path.join(_HERE, "libadaptq.so")

_f = C.POINTER(C.c_float)
_u8 = C.POINTER(C.c_uint8)
_ip = C.POINTER(C.c_int)

# name -> (restype, argtypes); every symbol declared in include/adaptq.h.
SIGNATURES = {
    "adaptq_last_error": (C.c_char_p, []),
    "adaptq_create": (C.c_void_p, [C.c_int, C.c_int, C.c_int, C.c_int, C.c_uint64, C.c_float,
                                   C.c_int]),
    "adaptq_destroy": (None, [C.c_void_p]),
    "adaptq_append": (None, [C.c_void_p, _f, _f, C.c_int]),
    "adaptq_compute": (C.c_int, [C.c_void_p, _f, _f]),
    "adaptq_compute_batch": (C.c_int, [C.c_void_p, _f, C.c_int, _f]),
    "adaptq_reset": (None, [C.c_void_p]),
    "adaptq_kv_bytes": (C.c_size_t, [C.c_void_p]),
    "adaptq_mha_create": (C.c_void_p, [C.c_int, C.c_int, C.c_int, C.c_int, C.c_int, C.c_uint64,
                                       C.c_float, C.c_int]),
    "adaptq_mha_destroy": (None, [C.c_void_p]),
    "adaptq_mha_append": (None, [C.c_void_p, C.c_int, _f, _f, C.c_int]),
    "adaptq_mha_compute": (C.c_int, [C.c_void_p, C.c_int, _f, _f]),
    "adaptq_mha_compute_batch": (C.c_int, [C.c_void_p, C.c_int, _f, C.c_int, _f]),
    "adaptq_mha_reset": (None, [C.c_void_p]),
    "adaptq_mha_total_kv_bytes": (C.c_size_t, [C.c_void_p]),
    "adaptq_features": (C.c_uint, []),
    "adaptq_version": (C.c_char_p, []),
    # extensions
    "adaptq_flush": (C.c_int, [C.c_void_p]),
    "adaptq_ring_info": (C.c_int, [C.c_void_p, _ip, _ip, _ip, _ip, _ip, _ip]),
    "adaptq_read_slots": (C.c_int, [C.c_void_p, C.c_int, C.c_int, _u8, _u8, _f, _f]),
    "adaptq_sparse_weights": (C.c_int, [C.c_void_p, _f, _f]),
    "adaptq_mha_head": (C.c_void_p, [C.c_void_p, C.c_int]),
    "adaptq_mha_append_all": (C.c_int, [C.c_void_p, _f, _f, C.c_int]),
    "adaptq_mha_compute_all": (C.c_int, [C.c_void_p, _f, _f]),
    "adaptq_mha_append_all_device": (C.c_int, [C.c_void_p, C.c_void_p, C.c_void_p, C.c_int,
                                               C.c_int, C.c_void_p]),
    "adaptq_mha_compute_all_device": (C.c_int, [C.c_void_p, C.c_void_p, C.c_void_p,
                                                C.c_void_p]),
    "adaptq_ggml_append_f32": (C.c_int, [C.c_void_p, C.c_void_p, C.c_void_p, C.c_int, C.c_int,
                                         C.c_int, C.c_size_t, C.c_size_t, C.c_size_t, C.c_size_t,
                                         C.c_int]),
    "adaptq_ggml_attn_f32": (C.c_int, [C.c_void_p, C.c_void_p, C.c_int, C.c_int, C.c_int,
                                       C.c_size_t, C.c_size_t, C.c_void_p, C.c_size_t,
                                       C.c_size_t]),
    "adaptq_ggml_append_f32_device": (C.c_int, [C.c_void_p, C.c_void_p, C.c_void_p, C.c_int,
                                                C.c_int, C.c_int, C.c_size_t, C.c_size_t,
                                                C.c_size_t, C.c_size_t, C.c_int, C.c_void_p]),
    "adaptq_ggml_attn_f32_device": (C.c_int, [C.c_void_p, C.c_void_p, C.c_int, C.c_int, C.c_int,
                                              C.c_size_t, C.c_size_t, C.c_void_p, C.c_size_t,
                                              C.c_size_t, C.c_void_p]),
    "adaptq_snapshot_save": (C.c_int, [C.POINTER(C.c_void_p), C.c_int, C.c_char_p]),
    "adaptq_snapshot_load": (C.c_int, [C.POINTER(C.c_void_p), C.c_int, C.c_char_p]),
    "adaptq_plan_create": (C.c_void_p, [C.POINTER(C.c_void_p), C.c_int]),
    "adaptq_plan_destroy": (None, [C.c_void_p]),
    "adaptq_plan_append_device": (C.c_int, [C.c_void_p, C.c_void_p, C.c_void_p, C.c_int,
                                            C.c_int, C.c_void_p]),
    "adaptq_plan_compute_device": (C.c_int, [C.c_void_p, C.c_void_p, C.c_void_p, C.c_void_p]),
    "adaptq_plan_compute_device_static": (C.c_int, [C.c_void_p, C.c_void_p, C.c_void_p,
                                                    C.c_void_p]),
    "adaptq_plan_workspace_bytes": (C.c_longlong, [C.c_void_p]),
    "adaptq_mha_append_compute_all_device": (C.c_int, [C.c_void_p, C.c_void_p, C.c_void_p, C.c_int,
                                                       C.c_void_p, C.c_void_p, C.c_void_p]),
}

FEAT_AVX2, FEAT_HYBRID, FEAT_SPARSE_V, FEAT_HIP = 1, 2, 4, 8


def load(path: str = LIB_PATH) -> C.CDLL:
    if not os.path.exists(path):
        raise ImportError(
            f"{path} is not built; run `python -m adaptq_amd.build` "
            "(the HIP library is required: there is no CPU fallback)")
    lib = C.CDLL(path)
    for name, (res, args) in SIGNATURES.items():
        fn = getattr(lib, name)
        fn.restype = res
        fn.argtypes = args
    return lib


lib = load()


def last_error() -> str:
    return lib.adaptq_last_error().decode()


def fptr(a):
    return a.ctypes.data_as(_f)


def u8ptr(a):
    return a.ctypes.data_as(_u8)
