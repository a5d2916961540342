"""Host-buffer paths after asynchronous flushes.  Staged host appends are
quantised by launches the call does not wait for (rows and queries go through
pinned memory); every later observer must still see them: ring inspection,
a plan decode on another stream, an MHA decode after uneven per-head staging,
and destroy while a flush may still run."""
import ctypes as C

import numpy as np
import pytest

from adaptq_amd import _lib
from gpu_head import DeviceBuffer, GpuHead, err, rel_err, same_bits, sync

pytestmark = pytest.mark.gpu
L = _lib.lib


def _mha(H, dim, cap, seed, vm=0.0, hyb=0):
    m = L.adaptq_mha_create(H, dim, 4, 2, cap, seed, vm, hyb)
    assert m, err()
    return m


def _heads(m, H, dim):
    return [GpuHead.wrap(L.adaptq_mha_head(m, h), dim) for h in range(H)]


def _oracles(oracle, m, H, dim, cap, vm=0.0, hyb=0):
    # per-head seeds of the MHA: base ^ (h * 0xDEADBEEFCAFE) (c_api.cpp:160)
    base = 11
    return [oracle.head(dim, 4, 2, cap, (base ^ (h * 0xDEADBEEFCAFE)) & (2**64 - 1), vm, hyb)
            for h in range(H)]


def test_auto_flush_then_inspect_and_plan(oracle):
    H, dim, cap, n = 3, 64, 2048, 1100  # 1024 staged tokens flush by themselves
    rng = np.random.default_rng(5)
    m = _mha(H, dim, cap, 11)
    refs = _oracles(oracle, m, H, dim, cap)
    K = rng.standard_normal((n, H, dim)).astype(np.float32)
    V = rng.standard_normal((n, H, dim)).astype(np.float32)
    for t in range(n):
        assert L.adaptq_mha_append_all(m, _lib.fptr(K[t]), _lib.fptr(V[t]), t) == 0, err()
        for h in range(H):
            refs[h].append(K[t, h], V[t, h], t)
    heads = _heads(m, H, dim)
    for g, o in zip(heads, refs):
        for a, b in zip(g.read_slots(0, n), o.read_slots(0, n)):
            assert same_bits(a, b)
    # more staged tokens, then a plan decode on the null stream
    for t in range(n, n + 5):
        K1 = rng.standard_normal((H, dim)).astype(np.float32)
        assert L.adaptq_mha_append_all(m, _lib.fptr(K1), _lib.fptr(K1), t) == 0, err()
        for h in range(H):
            refs[h].append(K1[h], K1[h], t)
    plan = L.adaptq_plan_create((C.c_void_p * H)(*[g.h for g in heads]), H)
    assert plan, err()
    q = rng.standard_normal((H, dim)).astype(np.float32)
    dq, do = DeviceBuffer(q.nbytes), DeviceBuffer(q.nbytes)
    dq.upload(q)
    assert L.adaptq_plan_compute_device(plan, dq.ptr, do.ptr, None) == 0, err()
    sync()
    y = do.download((H, dim))
    for h in range(H):
        assert rel_err(y[h], refs[h].compute(q[h])[0]) <= 1e-4
    L.adaptq_plan_destroy(plan)
    L.adaptq_mha_destroy(m)


@pytest.mark.parametrize("vm,hyb", [(0.0, 0), (0.95, 0), (0.95, 512)])
def test_uneven_staging_then_mha_compute(oracle, vm, hyb):
    H, dim, cap = 4, 64, 4096
    rng = np.random.default_rng(6)
    m = _mha(H, dim, cap, 11, vm, hyb)
    refs = _oracles(oracle, m, H, dim, cap, vm, hyb)
    heads = _heads(m, H, dim)
    out = np.zeros((H, dim), np.float32)
    for step in range(4):
        # whole-MHA tokens, then a few extra tokens on some heads only
        n_all = [700, 1, 2, 300][step]
        for t in range(n_all):
            K = rng.standard_normal((H, dim)).astype(np.float32)
            V = rng.standard_normal((H, dim)).astype(np.float32)
            assert L.adaptq_mha_append_all(m, _lib.fptr(K), _lib.fptr(V), t) == 0, err()
            for h in range(H):
                refs[h].append(K[h], V[h], t)
        for h in range(step % H):
            k = rng.standard_normal(dim).astype(np.float32)
            heads[h].append(k, k, 0)
            refs[h].append(k, k, 0)
        q = rng.standard_normal((H, dim)).astype(np.float32)
        assert L.adaptq_mha_compute_all(m, _lib.fptr(q), _lib.fptr(out)) >= 0, err()
        for h in range(H):
            assert rel_err(out[h], refs[h].compute(q[h])[0]) <= 1e-4, (step, h)
    L.adaptq_mha_destroy(m)


def test_destroy_right_after_staging():
    # the flush queued by 1024 staged tokens may still run when destroy comes
    dim = 128
    rng = np.random.default_rng(7)
    for _ in range(3):
        h = L.adaptq_create(dim, 4, 4, 4096, 3, 0.0, 0)
        assert h, err()
        x = rng.standard_normal(dim).astype(np.float32)
        for t in range(1030):
            L.adaptq_append(h, _lib.fptr(x), _lib.fptr(x), t)
        L.adaptq_destroy(h)
    m = _mha(8, dim, 2048, 3)
    X = rng.standard_normal((8, dim)).astype(np.float32)
    for t in range(1024):
        assert L.adaptq_mha_append_all(m, _lib.fptr(X), _lib.fptr(X), t) == 0
    L.adaptq_mha_destroy(m)
    sync()
