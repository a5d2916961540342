"""The allocation-free plan decode (adaptq_plan_compute_device_static: the
workspace in the library's static device scratch) against the allocating one
(adaptq_plan_compute_device) through the C ABI: two calls in a row, the
second with a smaller input, on a dense plan whose rings need a split-K
workspace and on sparse-V plans through each selection path; outputs
bit-identical (the same kernels and split plan run on both).  Calls from two
host threads on two streams, whose decodes would race on the shared scratch
if they overlapped on the GPU, give the same bits.  Also the refusals: a
workspace above the scratch's size, and staged host appends; and the
workspace query."""
import ctypes as C
import threading

import numpy as np
import pytest

from adaptq_amd import _lib
from gpu_head import GpuHead, err

pytestmark = pytest.mark.gpu
L = _lib.lib


def _plan(heads):
    p = L.adaptq_plan_create((C.c_void_p * len(heads))(*[h.h for h in heads]), len(heads))
    assert p, err()
    return p


def _fill(torch, heads, n, seed):
    g = torch.Generator(device="cuda")
    g.manual_seed(seed)
    dim = heads[0].dim
    k = torch.randn(len(heads), n, dim, generator=g, device="cuda")
    v = torch.randn(len(heads), n, dim, generator=g, device="cuda")
    p = _plan(heads)
    assert L.adaptq_plan_append_device(p, C.c_void_p(k.data_ptr()), C.c_void_p(v.data_ptr()), n, 0,
                                       None) == 0, err()
    return p


def _both(torch, plan, n_ctx, dim, seed):
    g = torch.Generator(device="cuda")
    g.manual_seed(seed)
    q = torch.randn(n_ctx, dim, generator=g, device="cuda")
    a = torch.full((n_ctx, dim), float("nan"), device="cuda")
    b = torch.full((n_ctx, dim), float("nan"), device="cuda")
    assert L.adaptq_plan_compute_device(plan, C.c_void_p(q.data_ptr()), C.c_void_p(a.data_ptr()),
                                        None) == 0, err()
    assert L.adaptq_plan_compute_device_static(plan, C.c_void_p(q.data_ptr()),
                                               C.c_void_p(b.data_ptr()), None) == 0, err()
    torch.cuda.synchronize()
    a, b = a.cpu().numpy(), b.cpu().numpy()
    assert np.isfinite(b).all()
    assert a.tobytes() == b.tobytes()


@pytest.mark.parametrize("dim,kb,vb,vm,sizes", [
    (128, 4, 2, 0.0, [(4, 20000), (2, 3000)]),   # dense, split-K partials in the scratch
    (64, 4, 2, 0.95, [(3, 5000), (2, 1500)]),    # sparse-V, selection workspace in the scratch
    (64, 3, 2, 0.95, [(2, 10000), (1, 9000)]),   # sparse-V with the per-item radix sort
    (64, 2, 2, 0.95, [(1, 70000), (1, 66000)]),  # sparse-V, the sort with superblock sums
])
def test_static_matches_allocating(dim, kb, vb, vm, sizes):
    import torch
    for i, (n_ctx, n) in enumerate(sizes):
        print(f"no-alloc decode d{dim} K{kb}V{vb} v_mass={vm}: {n_ctx} contexts x {n} tokens",
              flush=True)
        heads = [GpuHead(dim, kb, vb, n, 100 * i + h, vm, 0) for h in range(n_ctx)]
        plan = _fill(torch, heads, n, 7 + i)
        need = L.adaptq_plan_workspace_bytes(plan)
        assert 0 <= need <= 8 << 20, (need, err())
        _both(torch, plan, n_ctx, dim, 11 + i)
        L.adaptq_plan_destroy(plan)


def test_static_calls_from_two_streams():
    """Two host threads, each with its own stream and plan (a dense plan with
    split-K partials, a sparse-V plan), issue static decodes back to back
    without synchronising; every output equals the allocating call's bits."""
    import torch
    print("no-alloc decode: two threads, two streams, 6 calls each", flush=True)
    da = [GpuHead(128, 4, 2, 20000, 300 + h, 0.0, 0) for h in range(4)]
    db = [GpuHead(64, 4, 2, 5000, 400 + h, 0.95, 0) for h in range(3)]
    pa, pb = _fill(torch, da, 20000, 5), _fill(torch, db, 5000, 6)
    assert L.adaptq_plan_workspace_bytes(pa) > 0 and L.adaptq_plan_workspace_bytes(pb) > 0
    reps = 6
    g = torch.Generator(device="cuda")
    g.manual_seed(9)
    jobs = []
    for plan, n_ctx, dim in ((pa, 4, 128), (pb, 3, 64)):
        qs = [torch.randn(n_ctx, dim, generator=g, device="cuda") for _ in range(reps)]
        want = []
        for q in qs:
            a = torch.empty(n_ctx, dim, device="cuda")
            assert L.adaptq_plan_compute_device(plan, C.c_void_p(q.data_ptr()),
                                                C.c_void_p(a.data_ptr()), None) == 0, err()
            want.append(a)
        outs = [torch.full((n_ctx, dim), float("nan"), device="cuda") for _ in range(reps)]
        jobs.append((plan, qs, outs, want))
    torch.cuda.synchronize()
    streams = [torch.cuda.Stream(), torch.cuda.Stream()]
    start = threading.Barrier(2)
    rcs = [[], []]

    def run(i):
        plan, qs, outs, _ = jobs[i]
        sp = C.c_void_p(streams[i].cuda_stream)
        start.wait()
        for q, o in zip(qs, outs):
            rcs[i].append(L.adaptq_plan_compute_device_static(plan, C.c_void_p(q.data_ptr()),
                                                              C.c_void_p(o.data_ptr()), sp))

    ths = [threading.Thread(target=run, args=(i,)) for i in range(2)]
    for t in ths:
        t.start()
    for t in ths:
        t.join()
    torch.cuda.synchronize()
    assert rcs == [[0] * reps, [0] * reps], (rcs, err())
    for i, (_, _, outs, want) in enumerate(jobs):
        for r, (o, w) in enumerate(zip(outs, want)):
            assert o.cpu().numpy().tobytes() == w.cpu().numpy().tobytes(), (i, r)
    L.adaptq_plan_destroy(pa)
    L.adaptq_plan_destroy(pb)


def test_static_refuses_oversized_workspace():
    import torch
    print("no-alloc decode: workspace above the scratch", flush=True)
    # d1024 contexts take the generic kernel: 4 * (1024 + 4) bytes each, and
    # 2,100 of them exceed the 8 MiB scratch (empty rings: nothing launches)
    heads = [GpuHead(1024, 4, 2, 1, h) for h in range(2100)]
    plan = _plan(heads)
    q = torch.zeros(2100, 1024, device="cuda")
    out = torch.zeros(2100, 1024, device="cuda")
    assert L.adaptq_plan_workspace_bytes(plan) > 8 << 20
    assert L.adaptq_plan_compute_device_static(plan, C.c_void_p(q.data_ptr()),
                                               C.c_void_p(out.data_ptr()), None) == -1
    assert "static scratch" in err()
    L.adaptq_plan_destroy(plan)


def test_static_refuses_staged_host_appends():
    import torch
    print("no-alloc decode: staged host appends", flush=True)
    g = GpuHead(64, 4, 2, 64, 3)
    g.append(np.ones(64, np.float32), np.ones(64, np.float32), 0)
    plan = _plan([g])
    q = torch.zeros(1, 64, device="cuda")
    out = torch.zeros(1, 64, device="cuda")
    assert L.adaptq_plan_compute_device_static(plan, C.c_void_p(q.data_ptr()),
                                               C.c_void_p(out.data_ptr()), None) == -1
    assert "staged" in err()
    assert L.adaptq_plan_workspace_bytes(plan) == -1 and "staged" in err()
    assert L.adaptq_flush(g.h) == 0, err()
    assert L.adaptq_plan_compute_device_static(plan, C.c_void_p(q.data_ptr()),
                                               C.c_void_p(out.data_ptr()), None) == 0, err()
    torch.cuda.synchronize()
    L.adaptq_plan_destroy(plan)


def test_static_refuses_graph_capture():
    """Under HIP graph capture the call refuses (its ordering event cannot be
    waited on inside a capture) and queues nothing."""
    import torch
    print("no-alloc decode: refused under graph capture", flush=True)
    heads = [GpuHead(64, 4, 2, 256, 500 + h, 0.0, 0) for h in range(2)]
    plan = _fill(torch, heads, 256, 12)
    q = torch.randn(2, 64, device="cuda")
    out = torch.zeros(2, 64, device="cuda")
    x = torch.ones(16, device="cuda")
    torch.cuda.synchronize()
    s = torch.cuda.Stream()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.stream(s):
        graph.capture_begin()
        x.mul_(2.0)  # the graph is not empty
        rc = L.adaptq_plan_compute_device_static(plan, C.c_void_p(q.data_ptr()),
                                                 C.c_void_p(out.data_ptr()),
                                                 C.c_void_p(s.cuda_stream))
        msg = err()
        graph.capture_end()
    torch.cuda.synchronize()
    assert rc == -1 and "graph capture" in msg, (rc, msg)
    # outside the capture the call works as before
    assert L.adaptq_plan_compute_device_static(plan, C.c_void_p(q.data_ptr()),
                                               C.c_void_p(out.data_ptr()), None) == 0, err()
    torch.cuda.synchronize()
    assert np.isfinite(out.cpu().numpy()).all()
    L.adaptq_plan_destroy(plan)
