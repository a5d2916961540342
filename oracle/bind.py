"""ctypes bindings for the test-only checkers in oracle/.

TEST INFRASTRUCTURE ONLY: imported by tests/, __graft_entry__.smoke() and
bench.py's cpu_baseline leg, never by the product package.

- ``Oracle``: our plain-C restatement (oracle/liboracle.so).
- ``Ref``: the reference's own hot path compiled in place from
  /root/reference (oracle/_ref/libadaptq_ref.so, built by oracle/Makefile);
  absent on machines where it was never built.
"""
from __future__ import annotations

import ctypes as C
import os
import subprocess

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
ORACLE_SO = os.path.join(HERE, "liboracle.so")
REF_SO = os.path.join(HERE, "_ref", "libadaptq_ref.so")

_f = C.POINTER(C.c_float)
_u8 = C.POINTER(C.c_uint8)
_i8 = C.POINTER(C.c_int8)
_ip = C.POINTER(C.c_int)


def fptr(a):
    return a.ctypes.data_as(_f)


def u8ptr(a):
    return a.ctypes.data_as(_u8)


def i8ptr(a):
    return a.ctypes.data_as(_i8)


def build_oracle(with_ref: bool = False) -> None:
    """Compile liboracle.so (and the reference build when asked)."""
    targets = ["oracle"] + (["ref"] if with_ref else [])
    subprocess.run(["make", "-s", "-C", HERE] + targets, check=True)


def packed_bytes(p: int, bits: int) -> int:
    return p * 4 if bits == 16 else (p * bits + 7) // 8


def next_pow2(n: int) -> int:
    p = 1
    while p < n:
        p <<= 1
    return p


class Oracle:
    """The CPU restatement (oracle/oracle.c)."""

    def __init__(self, path: str = ORACLE_SO):
        if not os.path.exists(path):
            build_oracle()
        L = self.lib = C.CDLL(path)
        L.orc_next_pow2.argtypes = [C.c_int]
        L.orc_next_pow2.restype = C.c_int
        L.orc_rademacher.argtypes = [_i8, C.c_int, C.c_uint64]
        L.orc_fwht_forward.argtypes = [_f, _i8, C.c_int]
        L.orc_fwht_inverse.argtypes = [_f, _i8, C.c_int]
        L.orc_quantize_fast.argtypes = [C.c_float, C.c_int]
        L.orc_quantize_fast.restype = C.c_int
        L.orc_codebook.argtypes = [C.c_int, _f]
        L.orc_pack.argtypes = [_u8, C.c_int, C.c_int, _u8]
        L.orc_unpack.argtypes = [_u8, C.c_int, C.c_int, _u8]
        L.orc_quantize_vec.argtypes = [_f, C.c_int, C.c_int, _i8, C.c_int, _u8, _u8]
        L.orc_quantize_vec.restype = C.c_float
        L.orc_head_create.argtypes = [C.c_int, C.c_int, C.c_int, C.c_int, C.c_uint64,
                                      C.c_float, C.c_int]
        L.orc_head_create.restype = C.c_void_p
        L.orc_head_destroy.argtypes = [C.c_void_p]
        L.orc_head_append.argtypes = [C.c_void_p, _f, _f, C.c_int]
        L.orc_head_compute.argtypes = [C.c_void_p, _f, _f]
        L.orc_head_compute.restype = C.c_int
        L.orc_head_compute_sel.argtypes = [C.c_void_p, _f, _f, _f]
        L.orc_head_compute_sel.restype = C.c_int
        L.orc_head_compute_batch.argtypes = [C.c_void_p, _f, C.c_int, _f]
        L.orc_head_compute_batch.restype = C.c_int
        L.orc_head_reset.argtypes = [C.c_void_p]
        L.orc_head_kv_bytes.argtypes = [C.c_void_p]
        L.orc_head_kv_bytes.restype = C.c_size_t
        L.orc_head_info.argtypes = [C.c_void_p] + [_ip] * 7
        L.orc_head_read_slots.argtypes = [C.c_void_p, C.c_int, C.c_int, _u8, _u8, _f, _f]
        L.orc_head_signs.argtypes = [C.c_void_p]
        L.orc_head_signs.restype = C.c_void_p
        L.orc_mha_seed.argtypes = [C.c_uint64, C.c_int]
        L.orc_mha_seed.restype = C.c_uint64

    # codec ---------------------------------------------------------------
    def rademacher(self, n: int, seed: int) -> np.ndarray:
        D = np.empty(n, np.int8)
        self.lib.orc_rademacher(i8ptr(D), n, seed)
        return D

    def fwht_forward(self, x: np.ndarray, D: np.ndarray) -> np.ndarray:
        y = np.ascontiguousarray(x, np.float32).copy()
        self.lib.orc_fwht_forward(fptr(y), i8ptr(D), y.size)
        return y

    def fwht_inverse(self, x: np.ndarray, D: np.ndarray) -> np.ndarray:
        y = np.ascontiguousarray(x, np.float32).copy()
        self.lib.orc_fwht_inverse(fptr(y), i8ptr(D), y.size)
        return y

    def quantize_fast(self, v: float, bits: int) -> int:
        return self.lib.orc_quantize_fast(v, bits)

    def codebook(self, bits: int) -> np.ndarray:
        cb = np.zeros(1 << bits, np.float32)
        self.lib.orc_codebook(bits, fptr(cb))
        return cb

    def pack(self, idx: np.ndarray, bits: int) -> np.ndarray:
        idx = np.ascontiguousarray(idx, np.uint8)
        out = np.zeros(packed_bytes(idx.size, bits), np.uint8)
        self.lib.orc_pack(u8ptr(idx), idx.size, bits, u8ptr(out))
        return out

    def unpack(self, packed: np.ndarray, p: int, bits: int) -> np.ndarray:
        packed = np.ascontiguousarray(packed, np.uint8)
        out = np.zeros(p, np.uint8)
        self.lib.orc_unpack(u8ptr(packed), p, bits, u8ptr(out))
        return out

    def quantize_vec(self, x: np.ndarray, D: np.ndarray, bits: int):
        x = np.ascontiguousarray(x, np.float32)
        p = D.size
        packed = np.zeros(packed_bytes(p, bits), np.uint8)
        idx = np.zeros(p, np.uint8)
        s = self.lib.orc_quantize_vec(fptr(x), x.size, p, i8ptr(D), bits, u8ptr(packed),
                                      u8ptr(idx))
        return packed, np.float32(s), idx

    def mha_seed(self, base: int, i: int) -> int:
        return self.lib.orc_mha_seed(base, i)

    def head(self, dim, k_bits, v_bits, cap, seed, v_mass=0.0, hyb=0) -> "OracleHead":
        return OracleHead(self, dim, k_bits, v_bits, cap, seed, v_mass, hyb)


class OracleHead:
    def __init__(self, o: Oracle, dim, k_bits, v_bits, cap, seed, v_mass, hyb):
        self.o, self.L = o, o.lib
        self.dim, self.k_bits, self.v_bits, self.cap = dim, k_bits, v_bits, cap
        self.p = next_pow2(dim)
        self.h = self.L.orc_head_create(dim, k_bits, v_bits, cap, seed, v_mass, hyb)

    def __del__(self):
        if getattr(self, "h", None):
            self.L.orc_head_destroy(self.h)
            self.h = None

    def append(self, k, v, pos=0):
        k = np.ascontiguousarray(k, np.float32)
        v = np.ascontiguousarray(v, np.float32)
        self.L.orc_head_append(self.h, fptr(k), fptr(v), pos)

    def compute(self, q):
        q = np.ascontiguousarray(q, np.float32)
        out = np.zeros(self.dim, np.float32)
        n = self.L.orc_head_compute(self.h, fptr(q), fptr(out))
        return out, n

    def sparse_weights(self, q):
        """Sparse-V selection of one query: per-token weights (p * vscale) *
        isp in ring order (oldest first), 0 for tokens left out."""
        q = np.ascontiguousarray(q, np.float32)
        out = np.zeros(self.dim, np.float32)
        n = self.info()["size"]
        w = np.full(max(n, 1), np.nan, np.float32)
        self.L.orc_head_compute_sel(self.h, fptr(q), fptr(out), fptr(w))
        return w[:n]

    def compute_batch(self, qs):
        qs = np.ascontiguousarray(qs, np.float32)
        nq = qs.shape[0]
        outs = np.zeros((nq, self.dim), np.float32)
        n = self.L.orc_head_compute_batch(self.h, fptr(qs), nq, fptr(outs))
        return outs, n

    def reset(self):
        self.L.orc_head_reset(self.h)

    def kv_bytes(self):
        return self.L.orc_head_kv_bytes(self.h)

    def info(self):
        vals = [C.c_int() for _ in range(7)]
        self.L.orc_head_info(self.h, *[C.byref(v) for v in vals])
        keys = ["head", "size", "cap", "padded", "k_pb", "v_pb", "raw_count"]
        return {k: v.value for k, v in zip(keys, vals)}

    def read_slots(self, first, count):
        i = self.info()
        kc = np.zeros((count, i["k_pb"]), np.uint8)
        vc = np.zeros((count, i["v_pb"]), np.uint8)
        ks = np.zeros(count, np.float32)
        vs = np.zeros(count, np.float32)
        self.L.orc_head_read_slots(self.h, first, count, u8ptr(kc), u8ptr(vc), fptr(ks),
                                   fptr(vs))
        return kc, vc, ks, vs

    def signs(self):
        ptr = self.L.orc_head_signs(self.h)
        return np.ctypeslib.as_array(C.cast(ptr, _i8), shape=(self.p,)).copy()


class Ref:
    """The reference's own hot path, compiled in place (oracle/_ref)."""

    available = os.path.exists(REF_SO)

    def __init__(self, path: str = REF_SO):
        L = self.lib = C.CDLL(path)
        L.refx_rademacher.argtypes = [_i8, C.c_int, C.c_uint64]
        L.refx_fwht_forward.argtypes = [_f, _i8, C.c_int]
        L.refx_fwht_inverse.argtypes = [_f, _i8, C.c_int]
        L.refx_quantize_fast.argtypes = [C.c_float, C.c_int]
        L.refx_quantize_fast.restype = C.c_int
        L.refx_pack.argtypes = [_u8, C.c_int, C.c_int, _u8]
        L.refx_quantize_into.argtypes = [C.c_int, C.c_uint64, C.c_int, _f, _u8]
        L.refx_quantize_into.restype = C.c_float
        L.refx_head_create.argtypes = [C.c_int, C.c_int, C.c_int, C.c_int, C.c_uint64,
                                       C.c_float, C.c_int]
        L.refx_head_create.restype = C.c_void_p
        L.refx_head_destroy.argtypes = [C.c_void_p]
        L.refx_head_append.argtypes = [C.c_void_p, _f, _f, C.c_int]
        L.refx_head_compute.argtypes = [C.c_void_p, _f, _f]
        L.refx_head_compute.restype = C.c_int
        L.refx_head_reset.argtypes = [C.c_void_p]
        L.refx_head_info.argtypes = [C.c_void_p] + [_ip] * 5
        L.refx_head_read_slots.argtypes = [C.c_void_p, C.c_int, C.c_int, _u8, _u8, _f, _f]
        # the reference's C ABI (include/adaptq.h)
        L.adaptq_create.argtypes = [C.c_int, C.c_int, C.c_int, C.c_int, C.c_uint64,
                                    C.c_float, C.c_int]
        L.adaptq_create.restype = C.c_void_p
        L.adaptq_destroy.argtypes = [C.c_void_p]
        L.adaptq_append.argtypes = [C.c_void_p, _f, _f, C.c_int]
        L.adaptq_compute.argtypes = [C.c_void_p, _f, _f]
        L.adaptq_compute.restype = C.c_int
        L.adaptq_kv_bytes.argtypes = [C.c_void_p]
        L.adaptq_kv_bytes.restype = C.c_size_t
        L.adaptq_version.restype = C.c_char_p
        L.adaptq_reset.argtypes = [C.c_void_p]
        L.refx_append_rows.argtypes = [C.c_void_p, _f, _f, C.c_int, C.c_int]
        L.refx_compute_reps.argtypes = [C.c_void_p, _f, _f, C.c_int]
        L.refx_compute_reps.restype = C.c_int

    def rademacher(self, n: int, seed: int) -> np.ndarray:
        D = np.empty(n, np.int8)
        self.lib.refx_rademacher(i8ptr(D), n, seed)
        return D

    def fwht_forward(self, x, D):
        y = np.ascontiguousarray(x, np.float32).copy()
        self.lib.refx_fwht_forward(fptr(y), i8ptr(D), y.size)
        return y

    def fwht_inverse(self, x, D):
        y = np.ascontiguousarray(x, np.float32).copy()
        self.lib.refx_fwht_inverse(fptr(y), i8ptr(D), y.size)
        return y

    def quantize_fast(self, v, bits):
        return self.lib.refx_quantize_fast(v, bits)

    def quantize_into(self, x, seed, bits):
        x = np.ascontiguousarray(x, np.float32)
        p = next_pow2(x.size)
        out = np.zeros(packed_bytes(p, bits), np.uint8)
        s = self.lib.refx_quantize_into(x.size, seed, bits, fptr(x), u8ptr(out))
        return out, np.float32(s)

    def head(self, dim, k_bits, v_bits, cap, seed, v_mass=0.0, hyb=0) -> "RefHead":
        return RefHead(self, dim, k_bits, v_bits, cap, seed, v_mass, hyb)


class RefHead:
    def __init__(self, r: Ref, dim, k_bits, v_bits, cap, seed, v_mass, hyb):
        self.L = r.lib
        self.dim = dim
        self.h = self.L.refx_head_create(dim, k_bits, v_bits, cap, seed, v_mass, hyb)

    def __del__(self):
        if getattr(self, "h", None):
            self.L.refx_head_destroy(self.h)
            self.h = None

    def append(self, k, v, pos=0):
        k = np.ascontiguousarray(k, np.float32)
        v = np.ascontiguousarray(v, np.float32)
        self.L.refx_head_append(self.h, fptr(k), fptr(v), pos)

    def compute(self, q):
        q = np.ascontiguousarray(q, np.float32)
        out = np.zeros(self.dim, np.float32)
        n = self.L.refx_head_compute(self.h, fptr(q), fptr(out))
        return out, n

    def reset(self):
        self.L.refx_head_reset(self.h)

    def info(self):
        vals = [C.c_int() for _ in range(5)]
        self.L.refx_head_info(self.h, *[C.byref(v) for v in vals])
        return dict(zip(["head", "size", "k_pb", "v_pb", "raw_floats"], [v.value for v in vals]))

    def read_slots(self, first, count):
        i = self.info()
        kc = np.zeros((count, i["k_pb"]), np.uint8)
        vc = np.zeros((count, i["v_pb"]), np.uint8)
        ks = np.zeros(count, np.float32)
        vs = np.zeros(count, np.float32)
        self.L.refx_head_read_slots(self.h, first, count, u8ptr(kc), u8ptr(vc), fptr(ks),
                                    fptr(vs))
        return kc, vc, ks, vs


SNAP_REF_SO = os.path.join(HERE, "_ref", "libsnapshot_ref.so")


class SnapshotRef:
    """The reference's SessionSnapshot::load/save (replay/session_snapshot.cpp),
    compiled in place into oracle/_ref/libsnapshot_ref.so and opened with lazy
    binding (its capture() needs the unbuilt V2 runtime and is never called)."""

    available = os.path.exists(SNAP_REF_SO)

    def __init__(self, path: str = SNAP_REF_SO):
        L = self.lib = C.CDLL(path, mode=os.RTLD_LAZY)
        L.snapref_load.argtypes = [C.c_char_p, C.c_char_p, C.c_int]
        L.snapref_load.restype = C.c_void_p
        L.snapref_free.argtypes = [C.c_void_p]
        L.snapref_info.argtypes = [C.c_void_p, _ip]
        L.snapref_head.argtypes = [C.c_void_p, C.c_int, _ip, C.POINTER(C.POINTER(C.c_uint8)),
                                   C.POINTER(C.POINTER(C.c_float)),
                                   C.POINTER(C.POINTER(C.c_uint8))]
        L.snapref_head.restype = C.c_int
        L.snapref_save.argtypes = [C.c_void_p, C.c_char_p, C.c_char_p, C.c_int]
        L.snapref_save.restype = C.c_int

    def load(self, path: str) -> dict:
        """The file as the reference reads it; raises ValueError with the
        reference's exception text when it refuses the file."""
        err = C.create_string_buffer(512)
        h = self.lib.snapref_load(path.encode(), err, 512)
        if not h:
            raise ValueError(err.value.decode())
        try:
            info = np.zeros(7, np.int32)
            self.lib.snapref_info(h, info.ctypes.data_as(_ip))
            keys = ["n_layers", "n_heads", "dim", "bits", "n_tokens", "n_blocks", "flags"]
            out = {k: int(v) for k, v in zip(keys, info)}
            heads = []
            for i in range(out["n_blocks"]):
                ints = np.zeros(4, np.int32)
                d, s, t = C.POINTER(C.c_uint8)(), C.POINTER(C.c_float)(), C.POINTER(C.c_uint8)()
                assert self.lib.snapref_head(h, i, ints.ctypes.data_as(_ip), C.byref(d),
                                             C.byref(s), C.byref(t)) == 0
                layer, head, n, sb = (int(x) for x in ints)
                heads.append(dict(
                    layer=layer, head=head, cache_size=n, slot_bytes=sb,
                    data=np.ctypeslib.as_array(d, (2 * n * sb,)).copy() if n * sb else np.zeros(0, np.uint8),
                    scales=np.ctypeslib.as_array(s, (2 * n,)).copy() if n else np.zeros(0, np.float32),
                    tags=np.ctypeslib.as_array(t, (2 * n,)).copy() if n else np.zeros(0, np.uint8)))
            out["heads"] = heads
            return out
        finally:
            self.lib.snapref_free(h)

    def resave(self, src: str, dst: str) -> None:
        """load(src) then save(dst), both by the reference."""
        err = C.create_string_buffer(512)
        h = self.lib.snapref_load(src.encode(), err, 512)
        if not h:
            raise ValueError(err.value.decode())
        try:
            if self.lib.snapref_save(h, dst.encode(), err, 512) != 0:
                raise ValueError(err.value.decode())
        finally:
            self.lib.snapref_free(h)


KERNEL_REF_SO = os.path.join(HERE, "_ref", "libkernel_ref.so")


class KernelRef:
    """The reference's scalar IKernelBackend (kernels/scalar/kdot_scalar.cpp),
    compiled in place into oracle/_ref/libkernel_ref.so."""

    available = os.path.exists(KERNEL_REF_SO)

    def __init__(self, path: str = KERNEL_REF_SO):
        L = self.lib = C.CDLL(path)
        L.kref_kdot.argtypes = [_f, _u8, _f, C.c_int, C.c_int, C.c_int, _f]
        L.kref_vaccum.argtypes = [_u8, _f, _f, C.c_int, C.c_int, C.c_int, _f]
        L.kref_fwht.argtypes = [_f, _i8, C.c_int, C.c_int]

    def kdot(self, q, rows, scales, bits):
        q = np.ascontiguousarray(q, np.float32)
        rows = np.ascontiguousarray(rows, np.uint8)
        scales = np.ascontiguousarray(scales, np.float32)
        out = np.zeros(len(scales), np.float32)
        self.lib.kref_kdot(fptr(q), u8ptr(rows), fptr(scales), len(scales), q.size, bits, fptr(out))
        return out

    def vaccum(self, rows, scales, w, padded, bits):
        rows = np.ascontiguousarray(rows, np.uint8)
        scales = np.ascontiguousarray(scales, np.float32)
        w = np.ascontiguousarray(w, np.float32)
        acc = np.zeros(padded, np.float32)
        self.lib.kref_vaccum(u8ptr(rows), fptr(scales), fptr(w), len(scales), padded, bits, fptr(acc))
        return acc

    def fwht(self, x, D, forward):
        y = np.ascontiguousarray(x, np.float32).copy()
        self.lib.kref_fwht(fptr(y), i8ptr(np.ascontiguousarray(D, np.int8)), y.size, int(forward))
        return y
