"""Ordering between callers' streams and the library's own stream.

Device-form calls queue kernels on the caller's stream; host-form calls,
resets, flushes and inspection use the library stream.  Each case keeps the
caller's stream busy with a bounded spin kernel (torch.cuda._sleep) before
the device-form call, then makes the other kind of call at once, without any
synchronisation by the caller, and checks the result against the oracle: the
library must order the two itself.
"""
import ctypes as C

import numpy as np
import pytest

from adaptq_amd import _lib
from golden import inputs as I
from gpu_head import GpuHead, err, rel_err, same_bits

pytestmark = pytest.mark.gpu
L = _lib.lib
TOL = 1e-4


def busy(torch):
    """Keep torch's current stream busy for a few milliseconds (bounded)."""
    if hasattr(torch.cuda, "_sleep"):
        torch.cuda._sleep(20_000_000)
    else:
        a = torch.randn(4096, 4096, device="cuda")
        for _ in range(4):
            a = a @ a * 1e-3


@pytest.mark.parametrize("side_stream", [False, True])
def test_torch_reset_after_queued_forward(oracle, side_stream):
    """The advisor's case: forward() on GPU tensors queued behind other work,
    reset_cache() at once, then a new sequence: its output must be the
    oracle's over the new sequence only."""
    import torch
    from adaptq_amd.torch_adapter import AdaptQAttention
    print(f"torch reset after queued forward, side_stream={side_stream}", flush=True)
    H, dim, seed = 4, 64, 42
    rng = np.random.default_rng(11)
    mod = AdaptQAttention(dim, H, k_bits=4, v_bits=2, capacity=256, seed=seed)
    stream = torch.cuda.Stream() if side_stream else torch.cuda.current_stream()
    seq1 = rng.standard_normal((40, 3, H, dim)).astype(np.float32)
    seq2 = rng.standard_normal((30, 3, H, dim)).astype(np.float32)
    with torch.cuda.stream(stream):
        d1, d2 = torch.from_numpy(seq1).cuda(), torch.from_numpy(seq2).cuda()
        torch.cuda.synchronize()
        busy(torch)
        for t in range(seq1.shape[0]):
            mod(d1[t, 0:1], d1[t, 1:2], d1[t, 2:3])
        mod.reset_cache()  # no synchronisation in between
        for t in range(seq2.shape[0]):
            out = mod(d2[t, 0:1], d2[t, 1:2], d2[t, 2:3])
        y = out.cpu().numpy()[0]
    refs = [oracle.head(dim, 4, 2, 256, I.mha_seed(seed, h), 0.95, 512) for h in range(H)]
    for t in range(seq2.shape[0]):
        for h in range(H):
            refs[h].append(seq2[t, 1, h], seq2[t, 2, h], t)
    for h in range(H):
        r, n = refs[h].compute(seq2[-1, 0, h])
        assert n == seq2.shape[0]
        assert rel_err(y[h], r) <= TOL, (h, rel_err(y[h], r))


def test_host_compute_after_queued_device_append(oracle):
    """plan_append_device on a busy caller stream, then adaptq_compute (the
    library stream) at once: the decode must see the appended tokens."""
    import torch
    print("host compute after queued device append", flush=True)
    dim, n0, n1 = 128, 300, 200
    rng = np.random.default_rng(12)
    g = GpuHead(dim, 4, 2, 1024, 5)
    o = oracle.head(dim, 4, 2, 1024, 5)
    kv0 = rng.standard_normal((n0, 2, dim)).astype(np.float32)
    for t in range(n0):
        g.append(kv0[t, 0], kv0[t, 1], t)
        o.append(kv0[t, 0], kv0[t, 1], t)
    kv1 = rng.standard_normal((2, n1, dim)).astype(np.float32)
    plan = L.adaptq_plan_create((C.c_void_p * 1)(g.h), 1)
    assert plan, err()
    side = torch.cuda.Stream()
    with torch.cuda.stream(side):
        kd = torch.from_numpy(kv1[0]).cuda()
        vd = torch.from_numpy(kv1[1]).cuda()
        torch.cuda.synchronize()
        busy(torch)
        assert L.adaptq_plan_append_device(plan, C.c_void_p(kd.data_ptr()), C.c_void_p(vd.data_ptr()),
                                           n1, n0, C.c_void_p(side.cuda_stream)) == 0, err()
    for t in range(n1):
        o.append(kv1[0, t], kv1[1, t], n0 + t)
    q = rng.standard_normal(dim).astype(np.float32)
    y, n = g.compute(q)  # no synchronisation of `side`
    r, nr = o.compute(q)
    assert n == nr == n0 + n1
    assert rel_err(y, r) <= TOL
    torch.cuda.synchronize()
    L.adaptq_plan_destroy(plan)


def test_read_slots_after_queued_device_append(oracle):
    """mha_append_all_device on a busy stream, then read_slots at once: the
    ring bytes must include the appended tokens."""
    import torch
    print("read_slots after queued device append", flush=True)
    H, dim, n = 3, 64, 150
    rng = np.random.default_rng(13)
    m = L.adaptq_mha_create(H, dim, 4, 2, 256, 9, 0.0, 0)
    assert m, err()
    K = rng.standard_normal((H, n, dim)).astype(np.float32)
    V = rng.standard_normal((H, n, dim)).astype(np.float32)
    side = torch.cuda.Stream()
    with torch.cuda.stream(side):
        kd, vd = torch.from_numpy(K).cuda(), torch.from_numpy(V).cuda()
        torch.cuda.synchronize()
        busy(torch)
        assert L.adaptq_mha_append_all_device(m, C.c_void_p(kd.data_ptr()), C.c_void_p(vd.data_ptr()),
                                              n, 0, C.c_void_p(side.cuda_stream)) == 0, err()
    for h in range(H):
        gh = GpuHead.wrap(L.adaptq_mha_head(m, h), dim)
        o = oracle.head(dim, 4, 2, 256, I.mha_seed(9, h))
        for t in range(n):
            o.append(K[h, t], V[h, t], t)
        for a, b in zip(gh.read_slots(0, n), o.read_slots(0, n)):
            assert same_bits(a, b), h
    torch.cuda.synchronize()
    L.adaptq_mha_destroy(m)


def test_device_compute_after_host_appends(oracle):
    """Host appends staged then flushed on the library stream, followed at
    once by a device-form decode on a caller stream: the caller's stream must
    wait for the flush."""
    import torch
    print("device compute after host appends", flush=True)
    H, dim, n = 4, 128, 700
    rng = np.random.default_rng(14)
    m = L.adaptq_mha_create(H, dim, 4, 4, 1024, 21, 0.0, 0)
    assert m, err()
    K = rng.standard_normal((n, H, dim)).astype(np.float32)
    V = rng.standard_normal((n, H, dim)).astype(np.float32)
    refs = [oracle.head(dim, 4, 4, 1024, I.mha_seed(21, h)) for h in range(H)]
    for t in range(n):
        assert L.adaptq_mha_append_all(m, _lib.fptr(K[t]), _lib.fptr(V[t]), t) == 0, err()
        for h in range(H):
            refs[h].append(K[t, h], V[t, h], t)
    q = rng.standard_normal((H, dim)).astype(np.float32)
    side = torch.cuda.Stream()
    with torch.cuda.stream(side):
        qd = torch.from_numpy(q).cuda()
        od = torch.full((H, dim), float("nan"), device="cuda")
        assert L.adaptq_mha_compute_all_device(m, C.c_void_p(qd.data_ptr()),
                                               C.c_void_p(od.data_ptr()),
                                               C.c_void_p(side.cuda_stream)) == n, err()
        y = od.cpu().numpy()
    for h in range(H):
        r, _ = refs[h].compute(q[h])
        assert rel_err(y[h], r) <= TOL, h
    L.adaptq_mha_destroy(m)


def test_host_reset_then_device_append(oracle):
    """adaptq_mha_reset (library stream) followed at once by a device-form
    append on a caller stream and a host decode."""
    import torch
    print("reset then device append", flush=True)
    H, dim, n = 2, 64, 80
    rng = np.random.default_rng(15)
    m = L.adaptq_mha_create(H, dim, 3, 2, 128, 4, 0.0, 0)
    assert m, err()
    K = rng.standard_normal((H, 2 * n, dim)).astype(np.float32)
    V = rng.standard_normal((H, 2 * n, dim)).astype(np.float32)
    side = torch.cuda.Stream()
    with torch.cuda.stream(side):
        kd, vd = torch.from_numpy(K).cuda(), torch.from_numpy(V).cuda()
        torch.cuda.synchronize()
        s = C.c_void_p(side.cuda_stream)
        busy(torch)
        assert L.adaptq_mha_append_all_device(m, C.c_void_p(kd.data_ptr()), C.c_void_p(vd.data_ptr()),
                                              2 * n, 0, s) == 0, err()
        L.adaptq_mha_reset(m)
        k2 = kd[:, :n].contiguous()
        v2 = vd[:, n:].contiguous()
        assert L.adaptq_mha_append_all_device(m, C.c_void_p(k2.data_ptr()), C.c_void_p(v2.data_ptr()),
                                              n, 0, s) == 0, err()
    q = rng.standard_normal((H, dim)).astype(np.float32)
    out = np.zeros((H, dim), np.float32)
    assert L.adaptq_mha_compute_all(m, _lib.fptr(q), _lib.fptr(out)) == n, err()
    for h in range(H):
        o = oracle.head(dim, 3, 2, 128, I.mha_seed(4, h))
        for t in range(n):
            o.append(K[h, t], V[h, n + t], t)
        r, _ = o.compute(q[h])
        assert rel_err(out[h], r) <= TOL, h
    torch.cuda.synchronize()
    L.adaptq_mha_destroy(m)
