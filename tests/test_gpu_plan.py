"""Batched device-pointer path (adaptq_plan_*): one append launch and one
decode launch for many heads must give the same ring bytes as per-token host
appends and the same outputs as the oracle."""
import ctypes as C

import numpy as np
import pytest

from adaptq_amd import _lib
from gpu_head import DeviceBuffer, GpuHead, err, rel_err, same_bits, sync

pytestmark = pytest.mark.gpu
L = _lib.lib


@pytest.mark.parametrize("dim,kb,vb,cap,n", [(128, 4, 2, 300, 350), (64, 3, 2, 512, 200),
                                             (64, 16, 2, 128, 128), (128, 4, 4, 64, 64)])
def test_plan_append_and_compute(oracle, dim, kb, vb, cap, n):
    print(f"plan dim={dim} k{kb}v{vb} cap={cap} n={n}", flush=True)
    H = 6
    rng = np.random.default_rng(dim + n)
    heads = [GpuHead(dim, kb, vb, cap, 100 + i) for i in range(H)]
    refs = [oracle.head(dim, kb, vb, cap, 100 + i) for i in range(H)]
    # a few host appends first, so the plan starts from a non-empty ring
    pre = rng.standard_normal((H, 5, 2, dim)).astype(np.float32)
    for i in range(H):
        for t in range(5):
            heads[i].append(pre[i, t, 0], pre[i, t, 1], t)
            refs[i].append(pre[i, t, 0], pre[i, t, 1], t)
    k = rng.standard_normal((H, n, dim)).astype(np.float32)
    v = rng.standard_normal((H, n, dim)).astype(np.float32)
    dk, dv = DeviceBuffer(k.nbytes), DeviceBuffer(v.nbytes)
    dk.upload(k)
    dv.upload(v)
    arr = (C.c_void_p * H)(*[h.h for h in heads])
    plan = L.adaptq_plan_create(arr, H)
    assert plan, err()
    assert L.adaptq_plan_append_device(plan, dk.ptr, dv.ptr, n, 0, None) == 0, err()
    sync()
    for i in range(H):
        for t in range(n):
            refs[i].append(k[i, t], v[i, t], t)
    for g, o in zip(heads, refs):
        gi, oi = g.info(), o.info()
        assert (gi["head"], gi["size"]) == (oi["head"], oi["size"])
        for x, y in zip(g.read_slots(0, oi["size"]), o.read_slots(0, oi["size"])):
            assert same_bits(x, y)
    q = rng.standard_normal((H, dim)).astype(np.float32)
    dq, do = DeviceBuffer(q.nbytes), DeviceBuffer(q.nbytes)
    dq.upload(q)
    assert L.adaptq_plan_compute_device(plan, dq.ptr, do.ptr, None) == 0, err()
    sync()
    y = do.download((H, dim))
    r = np.stack([o.compute(q[i])[0] for i, o in enumerate(refs)])
    assert rel_err(y, r) <= 1e-4
    L.adaptq_plan_destroy(plan)


def test_plan_rejects_mixed_shapes():
    a = GpuHead(64, 4, 2, 16, 1)
    b = GpuHead(128, 4, 2, 16, 1)
    arr = (C.c_void_p * 2)(a.h, b.h)
    assert not L.adaptq_plan_create(arr, 2)
    assert "differ" in err()


def test_plan_empty_rings_give_zeros():
    H, dim = 3, 64
    heads = [GpuHead(dim, 4, 2, 32, i) for i in range(H)]
    arr = (C.c_void_p * H)(*[h.h for h in heads])
    plan = L.adaptq_plan_create(arr, H)
    q = np.ones((H, dim), np.float32)
    dq, do = DeviceBuffer(q.nbytes), DeviceBuffer(q.nbytes)
    dq.upload(q)
    do.upload(np.full((H, dim), 7.0, np.float32))
    assert L.adaptq_plan_compute_device(plan, dq.ptr, do.ptr, None) == 0, err()
    sync()
    assert np.all(do.download((H, dim)) == 0)
    L.adaptq_plan_destroy(plan)


# Sparse-V (v_mass > 0) and hybrid (raw mirror) branches through one plan:
# heads hold different numbers of tokens, outputs match the oracle per head.
# Above 8,192 tokens the launch sorts over many blocks per head; heads at or
# below it in the same launch are selected inside the select kernel.
@pytest.mark.parametrize("dim,kb,vb,cap,vm,hyb,sizes", [
    (64, 4, 2, 4096, 0.95, 0, [2048, 1500, 3000, 7]),
    (128, 3, 2, 2048, 0.9, 0, [1025, 1280, 600]),
    (64, 4, 2, 12000, 0.95, 0, [9000, 100, 5000, 8193]),
    (128, 4, 4, 10000, 0.95, 0, [10000, 3000, 8192]),
    (64, 4, 2, 1024, 0.95, 512, [512, 300, 1, 64]),
    (128, 16, 2, 256, 0.95, 256, [200, 256]),
])
def test_plan_compute_sparse_and_hybrid(oracle, dim, kb, vb, cap, vm, hyb, sizes):
    print(f"plan branch dim={dim} k{kb}v{vb} v_mass={vm} hyb={hyb} sizes={sizes}", flush=True)
    H = len(sizes)
    rng = np.random.default_rng(dim + len(sizes))
    heads = [GpuHead(dim, kb, vb, cap, 200 + i, vm, hyb) for i in range(H)]
    refs = [oracle.head(dim, kb, vb, cap, 200 + i, vm, hyb) for i in range(H)]
    for i, n in enumerate(sizes):
        kv = rng.standard_normal((n, 2, dim)).astype(np.float32)
        for t in range(n):
            heads[i].append(kv[t, 0], kv[t, 1], t)
            refs[i].append(kv[t, 0], kv[t, 1], t)
    arr = (C.c_void_p * H)(*[h.h for h in heads])
    plan = L.adaptq_plan_create(arr, H)
    assert plan, err()
    for _ in range(2):
        q = (3 * rng.standard_normal((H, dim))).astype(np.float32)
        dq, do = DeviceBuffer(q.nbytes), DeviceBuffer(q.nbytes)
        dq.upload(q)
        assert L.adaptq_plan_compute_device(plan, dq.ptr, do.ptr, None) == 0, err()
        sync()
        y = do.download((H, dim))
        for i, o in enumerate(refs):
            r = o.compute(q[i])[0]
            assert rel_err(y[i], r) <= 1e-4, (i, rel_err(y[i], r))
    L.adaptq_plan_destroy(plan)


def test_plan_rejects_mixed_branches():
    # head 0 keeps its raw mirror (hybrid branch), head 1 has evicted (sparse-V)
    dim = 64
    a, b = GpuHead(dim, 4, 2, 8, 1, 0.95, 8), GpuHead(dim, 4, 2, 8, 2, 0.95, 8)
    x = np.ones(dim, np.float32)
    for t in range(4):
        a.append(x, x, t)
    for t in range(9):
        b.append(x, x, t)
    arr = (C.c_void_p * 2)(a.h, b.h)
    plan = L.adaptq_plan_create(arr, 2)
    assert plan, err()
    dq, do = DeviceBuffer(2 * dim * 4), DeviceBuffer(2 * dim * 4)
    dq.upload(np.ones((2, dim), np.float32))
    assert L.adaptq_plan_compute_device(plan, dq.ptr, do.ptr, None) == -1
    assert "different branches" in err()
    L.adaptq_plan_destroy(plan)


# More contexts than one launch's grid holds (items go in the grid's y
# dimension, at most 65,535): the decode runs in chunks of items; sampled heads
# on both sides of the chunk boundary match the oracle.
@pytest.mark.parametrize("vm", [0.0, 0.95])
def test_plan_more_items_than_one_grid(oracle, vm):
    H, dim, cap, n = 65600, 64, 8, 3
    print(f"plan of {H} contexts, v_mass={vm}", flush=True)
    rng = np.random.default_rng(17)
    hs = [L.adaptq_create(dim, 4, 2, cap, i, vm, 0) for i in range(H)]
    assert all(hs), err()
    try:
        plan = L.adaptq_plan_create((C.c_void_p * H)(*hs), H)
        assert plan, err()
        k = rng.standard_normal((H, n, dim)).astype(np.float32)
        v = rng.standard_normal((H, n, dim)).astype(np.float32)
        q = rng.standard_normal((H, dim)).astype(np.float32)
        dk, dv, dq, do = (DeviceBuffer(x.nbytes) for x in (k, v, q, q))
        dk.upload(k)
        dv.upload(v)
        dq.upload(q)
        assert L.adaptq_plan_append_device(plan, dk.ptr, dv.ptr, n, 0, None) == 0, err()
        assert L.adaptq_plan_compute_device(plan, dq.ptr, do.ptr, None) == 0, err()
        sync()
        y = do.download((H, dim))
        assert np.isfinite(y).all()
        for h in (0, 65534, 65535, 65536, H - 1):
            o = oracle.head(dim, 4, 2, cap, h, vm, 0)
            for t in range(n):
                o.append(k[h, t], v[h, t], t)
            g = GpuHead.wrap(hs[h], dim)
            for a, b in zip(g.read_slots(0, n), o.read_slots(0, n)):
                assert same_bits(a, b), h
            assert rel_err(y[h], o.compute(q[h])[0]) <= 1e-4, h
        L.adaptq_plan_destroy(plan)
    finally:
        for x in hs:
            L.adaptq_destroy(x)


def test_plan_rejects_duplicate_contexts():
    a, b = GpuHead(64, 4, 2, 16, 1), GpuHead(64, 4, 2, 16, 2)
    arr = (C.c_void_p * 3)(a.h, b.h, a.h)
    assert not L.adaptq_plan_create(arr, 3)
    assert "more than once" in err()


# Single-token appends (decode steps) and 64..128-token appends advance the
# ring state inside the V-side launch; longer ones with a separate kernel.
# Every length keeps the ring equal to per-token host appends.
@pytest.mark.parametrize("n_tok", [1, 2, 63, 64, 128, 129, 300])
def test_plan_append_lengths_keep_ring_state(oracle, n_tok):
    H, dim, cap = 5, 64, 200
    rng = np.random.default_rng(n_tok)
    heads = [GpuHead(dim, 4, 2, cap, 50 + i, 0.0, 96) for i in range(H)]
    refs = [oracle.head(dim, 4, 2, cap, 50 + i, 0.0, 96) for i in range(H)]
    plan = L.adaptq_plan_create((C.c_void_p * H)(*[h.h for h in heads]), H)
    assert plan, err()
    for step in range(3):
        k = rng.standard_normal((H, n_tok, dim)).astype(np.float32)
        v = rng.standard_normal((H, n_tok, dim)).astype(np.float32)
        dk, dv = DeviceBuffer(k.nbytes), DeviceBuffer(v.nbytes)
        dk.upload(k)
        dv.upload(v)
        assert L.adaptq_plan_append_device(plan, dk.ptr, dv.ptr, n_tok, 0, None) == 0, err()
        sync()
        for i in range(H):
            for t in range(n_tok):
                refs[i].append(k[i, t], v[i, t], t)
    for g, o in zip(heads, refs):
        gi, oi = g.info(), o.info()
        assert (gi["head"], gi["size"]) == (oi["head"], oi["size"])
        for x, y in zip(g.read_slots(0, oi["size"]), o.read_slots(0, oi["size"])):
            assert same_bits(x, y)
    q = rng.standard_normal((H, dim)).astype(np.float32)
    dq, do = DeviceBuffer(q.nbytes), DeviceBuffer(q.nbytes)
    dq.upload(q)
    assert L.adaptq_plan_compute_device(plan, dq.ptr, do.ptr, None) == 0, err()
    sync()
    y = do.download((H, dim))
    for i, o in enumerate(refs):
        assert rel_err(y[i], o.compute(q[i])[0]) <= 1e-4
    L.adaptq_plan_destroy(plan)
