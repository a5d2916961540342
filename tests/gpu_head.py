"""Test helpers over the C ABI (adaptq_amd._lib): a thin ctypes head wrapper
with the same surface as oracle/bind.py's OracleHead, plus comparison utils."""
from __future__ import annotations

import ctypes as C
import os

import numpy as np

from adaptq_amd import _lib

L = _lib.lib


def err() -> str:
    return _lib.last_error()


class GpuHead:
    def __init__(self, dim, k_bits, v_bits, cap, seed, v_mass=0.0, hyb=0):
        self.dim = dim
        self.h = L.adaptq_create(dim, k_bits, v_bits, cap, seed, v_mass, hyb)
        assert self.h, err()

    @classmethod
    def wrap(cls, handle, dim):
        self = cls.__new__(cls)
        self.dim, self.h = dim, handle
        self._borrowed = True
        return self

    def __del__(self):
        if getattr(self, "h", None) and not getattr(self, "_borrowed", False):
            L.adaptq_destroy(self.h)
            self.h = None

    def append(self, k, v, pos=0):
        k = np.ascontiguousarray(k, np.float32)
        v = np.ascontiguousarray(v, np.float32)
        L.adaptq_append(self.h, _lib.fptr(k), _lib.fptr(v), pos)

    def compute(self, q):
        q = np.ascontiguousarray(q, np.float32)
        out = np.zeros(self.dim, np.float32)
        n = L.adaptq_compute(self.h, _lib.fptr(q), _lib.fptr(out))
        assert n >= 0, err()
        return out, n

    def compute_batch(self, qs):
        qs = np.ascontiguousarray(qs, np.float32)
        outs = np.zeros((qs.shape[0], self.dim), np.float32)
        n = L.adaptq_compute_batch(self.h, _lib.fptr(qs), qs.shape[0], _lib.fptr(outs))
        assert n >= 0, err()
        return outs, n

    def reset(self):
        L.adaptq_reset(self.h)

    def kv_bytes(self):
        return L.adaptq_kv_bytes(self.h)

    def info(self):
        vals = [C.c_int() for _ in range(6)]
        assert L.adaptq_ring_info(self.h, *[C.byref(v) for v in vals]) == 0, err()
        keys = ["head", "size", "cap", "padded", "k_pb", "v_pb"]
        return {k: v.value for k, v in zip(keys, vals)}

    def read_slots(self, first, count):
        i = self.info()
        kc = np.zeros((count, i["k_pb"]), np.uint8)
        vc = np.zeros((count, i["v_pb"]), np.uint8)
        ks = np.zeros(count, np.float32)
        vs = np.zeros(count, np.float32)
        rc = L.adaptq_read_slots(self.h, first, count, _lib.u8ptr(kc), _lib.u8ptr(vc),
                                 _lib.fptr(ks), _lib.fptr(vs))
        assert rc == 0, err()
        return kc, vc, ks, vs


# Worst errors seen per test (nodeid without parameters): every rel_err call
# records its norm-wise error and elementwise statistics; conftest prints the
# ledger at the end of the session and writes it to $AQ_PARITY_LOG if set.
ERROR_LEDGER: dict = {}


def _record(y, r, ne):
    node = os.environ.get("PYTEST_CURRENT_TEST", "").split(" ")[0]
    if not node or y.size == 0:
        return
    key = node.split("[")[0]
    d = np.abs(y - r)
    scale = float(np.max(np.abs(r)))
    # elementwise relative error over the elements that carry the output
    # (|r| >= 1e-3 max|r|); near-zero elements make it meaningless
    big = np.abs(r) >= 1e-3 * scale if scale > 0 else np.zeros(r.shape, bool)
    er = d[big] / np.abs(r[big]) if big.any() else np.zeros(1)
    e = ERROR_LEDGER.setdefault(key, {"calls": 0, "elements": 0, "norm_max": 0.0,
                                      "abs_max": 0.0, "elem_rel_max": 0.0,
                                      "elem_rel_median_max": 0.0})
    e["calls"] += 1
    e["elements"] += int(y.size)
    e["norm_max"] = max(e["norm_max"], ne)
    e["abs_max"] = max(e["abs_max"], float(np.max(d)))
    e["elem_rel_max"] = max(e["elem_rel_max"], float(np.max(er)))
    e["elem_rel_median_max"] = max(e["elem_rel_median_max"], float(np.median(er)))


def rel_err(y, r):
    """Norm-wise relative error max|y - r| / max(max|r|, 1e-30)."""
    y = np.asarray(y, np.float64)
    r = np.asarray(r, np.float64)
    ne = float(np.max(np.abs(y - r)) / max(float(np.max(np.abs(r))), 1e-30))
    _record(y, r, ne)
    return ne


def same_bits(a, b):
    a = np.ascontiguousarray(a)
    b = np.ascontiguousarray(b)
    return a.shape == b.shape and a.tobytes() == b.tobytes()


class DeviceBuffer:
    """Device memory through the HIP runtime libadaptq.so is linked against."""

    _hip = None

    @classmethod
    def hip(cls):
        if cls._hip is None:
            h = C.CDLL("libamdhip64.so.7")
            h.hipMalloc.argtypes = [C.POINTER(C.c_void_p), C.c_size_t]
            h.hipFree.argtypes = [C.c_void_p]
            h.hipMemcpy.argtypes = [C.c_void_p, C.c_void_p, C.c_size_t, C.c_int]
            h.hipDeviceSynchronize.argtypes = []
            cls._hip = h
        return cls._hip

    def __init__(self, nbytes):
        self.nbytes = nbytes
        self.ptr = C.c_void_p()
        rc = self.hip().hipMalloc(C.byref(self.ptr), nbytes)
        assert rc == 0, rc

    def upload(self, a):
        a = np.ascontiguousarray(a)
        assert a.nbytes <= self.nbytes
        assert self.hip().hipMemcpy(self.ptr, a.ctypes.data, a.nbytes, 1) == 0  # H2D

    def download(self, shape, dtype=np.float32):
        out = np.empty(shape, dtype)
        assert self.hip().hipMemcpy(out.ctypes.data, self.ptr, out.nbytes, 2) == 0  # D2H
        return out

    def __del__(self):
        if getattr(self, "ptr", None) and self.ptr.value:
            self.hip().hipFree(self.ptr)
            self.ptr = None


def sync():
    assert DeviceBuffer.hip().hipDeviceSynchronize() == 0
