"""Whole-MHA batches (adaptq_mha_append_all / _compute_all and their device
forms), the vectorised Engine and the torch module, against per-head calls
and the oracle.  Bar: ring codes and scales identical to per-head appends;
outputs within 1e-4 of the oracle in every branch (dense, hybrid, sparse-V)."""
import ctypes as C

import numpy as np
import pytest

from adaptq_amd import _lib
from golden import inputs as I
from gpu_head import GpuHead, err, rel_err, same_bits

pytestmark = pytest.mark.gpu
L = _lib.lib
TOL = 1e-4


def _mha(H, dim, kb, vb, cap, seed, vm, hyb):
    m = L.adaptq_mha_create(H, dim, kb, vb, cap, seed, vm, hyb)
    assert m, err()
    return m


@pytest.mark.parametrize("dim,kb,vb,vm,hyb,n", [
    (128, 4, 2, 0.0, 0, 700), (64, 4, 2, 0.95, 512, 300), (64, 4, 2, 0.95, 512, 900),
    (96, 3, 2, 0.0, 0, 400), (64, 16, 2, 0.95, 512, 600), (128, 4, 4, 0.5, 0, 1100),
])
def test_append_all_compute_all(oracle, dim, kb, vb, vm, hyb, n):
    print(f"batch dim={dim} k{kb}v{vb} vm={vm} hyb={hyb} n={n}", flush=True)
    H, cap, seed = 5, 1024, 77
    rng = np.random.default_rng(dim + n)
    K = rng.standard_normal((n, H, dim)).astype(np.float32)
    V = rng.standard_normal((n, H, dim)).astype(np.float32)
    q = rng.standard_normal((H, dim)).astype(np.float32)
    mb = _mha(H, dim, kb, vb, cap, seed, vm, hyb)    # whole-MHA calls
    mh = _mha(H, dim, kb, vb, cap, seed, vm, hyb)    # per-head calls
    refs = [oracle.head(dim, kb, vb, cap, I.mha_seed(seed, h), vm, hyb) for h in range(H)]
    for t in range(n):
        assert L.adaptq_mha_append_all(mb, _lib.fptr(K[t]), _lib.fptr(V[t]), t) == 0, err()
        for h in range(H):
            L.adaptq_mha_append(mh, h, _lib.fptr(np.ascontiguousarray(K[t, h])),
                                _lib.fptr(np.ascontiguousarray(V[t, h])), t)
            refs[h].append(K[t, h], V[t, h], t)
    out = np.zeros((H, dim), np.float32)
    got = L.adaptq_mha_compute_all(mb, _lib.fptr(q), _lib.fptr(out))
    assert got == min(n, cap), err()
    for h in range(H):
        r, _ = refs[h].compute(q[h])
        assert rel_err(out[h], r) <= TOL, h
        gb = GpuHead.wrap(L.adaptq_mha_head(mb, h), dim)
        gh = GpuHead.wrap(L.adaptq_mha_head(mh, h), dim)
        for a, b in zip(gb.read_slots(0, gb.info()["size"]), gh.read_slots(0, gh.info()["size"])):
            assert same_bits(a, b)
    L.adaptq_mha_destroy(mb)
    L.adaptq_mha_destroy(mh)


def test_compute_all_falls_back_when_heads_differ(oracle):
    dim, H = 64, 3
    m = _mha(H, dim, 4, 2, 256, 5, 0.0, 0)
    refs = [oracle.head(dim, 4, 2, 256, I.mha_seed(5, h)) for h in range(H)]
    rng = np.random.default_rng(1)
    for t in range(50):
        h = t % H if t >= 30 else None
        kv = rng.standard_normal((H, 2, dim)).astype(np.float32)
        for i in range(H):
            if h is None or i == h:
                L.adaptq_mha_append(m, i, _lib.fptr(np.ascontiguousarray(kv[i, 0])),
                                    _lib.fptr(np.ascontiguousarray(kv[i, 1])), t)
                refs[i].append(kv[i, 0], kv[i, 1], t)
    q = rng.standard_normal((H, dim)).astype(np.float32)
    out = np.zeros((H, dim), np.float32)
    assert L.adaptq_mha_compute_all(m, _lib.fptr(q), _lib.fptr(out)) > 0, err()
    for i in range(H):
        assert rel_err(out[i], refs[i].compute(q[i])[0]) <= TOL
    L.adaptq_mha_destroy(m)


def test_device_forms_with_torch(oracle):
    import torch
    dim, H, T = 128, 4, 600
    dev = torch.device("cuda:0")
    for vm, hyb in [(0.0, 0), (0.95, 512)]:
        print(f"device forms vm={vm} hyb={hyb}", flush=True)
        m = _mha(H, dim, 4, 2, 2048, 11, vm, hyb)
        refs = [oracle.head(dim, 4, 2, 2048, I.mha_seed(11, h), vm, hyb) for h in range(H)]
        g = torch.Generator(device="cpu").manual_seed(3)
        K = torch.randn(H, T, dim, generator=g)
        V = torch.randn(H, T, dim, generator=g)
        q = torch.randn(H, dim, generator=g)
        for h in range(H):
            for t in range(T):
                refs[h].append(K[h, t].numpy(), V[h, t].numpy(), t)
        s = torch.cuda.current_stream()
        # 400 tokens in one launch, then 200 one at a time
        kd, vd = K[:, :400].contiguous().to(dev), V[:, :400].contiguous().to(dev)
        assert L.adaptq_mha_append_all_device(m, C.c_void_p(kd.data_ptr()), C.c_void_p(vd.data_ptr()),
                                              400, 0, C.c_void_p(s.cuda_stream)) == 0, err()
        for t in range(400, T):
            kt, vt = K[:, t].contiguous().to(dev), V[:, t].contiguous().to(dev)
            assert L.adaptq_mha_append_all_device(m, C.c_void_p(kt.data_ptr()),
                                                  C.c_void_p(vt.data_ptr()), 1, t,
                                                  C.c_void_p(s.cuda_stream)) == 0, err()
        qd = q.to(dev)
        od = torch.empty_like(qd)
        n = L.adaptq_mha_compute_all_device(m, C.c_void_p(qd.data_ptr()), C.c_void_p(od.data_ptr()),
                                            C.c_void_p(s.cuda_stream))
        assert n == T, err()
        torch.cuda.synchronize()
        out = od.cpu().numpy()
        for h in range(H):
            assert rel_err(out[h], refs[h].compute(q[h].numpy())[0]) <= TOL, (vm, h)
        L.adaptq_mha_destroy(m)


def test_engine_vectorised_matches_oracle(oracle):
    from adaptq_amd.core import Engine
    dim, H = 64, 6
    eng = Engine(dim=dim, heads=H, k_bits=3, v_bits=2, capacity=800, seed=9)
    refs = [oracle.head(dim, 3, 2, 800, I.mha_seed(9, h), 0.95, 512) for h in range(H)]
    rng = np.random.default_rng(2)
    for t in range(1000):  # hybrid branch, then (after 512) sparse-V, then eviction
        k = rng.standard_normal((H, dim)).astype(np.float32)
        v = rng.standard_normal((H, dim)).astype(np.float32)
        eng.append(k, v)
        for h in range(H):
            refs[h].append(k[h], v[h], t)
        if t in (200, 700, 999):
            q = rng.standard_normal((H, dim)).astype(np.float32)
            out = eng.compute(q)
            for h in range(H):
                assert rel_err(out[h], refs[h].compute(q[h])[0]) <= TOL, (t, h)


@pytest.mark.parametrize("on_gpu", [True, False])
def test_torch_module(oracle, on_gpu):
    import torch
    from adaptq_amd.torch_adapter import AdaptQAttention
    dim, H = 64, 4
    mod = AdaptQAttention(dim=dim, heads=H, k_bits=4, v_bits=2, capacity=1024, seed=42)
    refs = [oracle.head(dim, 4, 2, 1024, I.mha_seed(42, h), 0.95, 512) for h in range(H)]
    dev = torch.device("cuda:0") if on_gpu else torch.device("cpu")
    g = torch.Generator(device="cpu").manual_seed(5)
    for t in range(600):
        q, k, v = (torch.randn(1, H, dim, generator=g) for _ in range(3))
        out = mod(q.to(dev), k.to(dev), v.to(dev))
        for h in range(H):
            refs[h].append(k[0, h].numpy(), v[0, h].numpy(), t)
        if t in (10, 599):
            assert out.device == dev and out.shape == (1, H, dim)
            o = out.cpu().numpy()[0]
            for h in range(H):
                assert rel_err(o[h], refs[h].compute(q[0, h].numpy())[0]) <= TOL, (t, h)
    mod.reset_cache()
    assert mod.engine.kv_bytes == 0
    with pytest.raises(ValueError):
        mod(torch.zeros(2, H, dim), torch.zeros(2, H, dim), torch.zeros(2, H, dim))
