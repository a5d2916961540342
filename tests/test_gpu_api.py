"""Behavioural contracts of the reference's C ABI (tests/unit/test_api.cpp
and core/adaptq_c_api.cpp), on the GPU build: return codes, error strings,
empty caches, reset, capacity 0, contexts above 65536 tokens, degenerate
inputs, hybrid-mirror invalidation on the first eviction, several handles
used from several threads."""
import ctypes as C
import threading

import numpy as np
import pytest

from adaptq_amd import _lib
from gpu_head import GpuHead, err, rel_err

pytestmark = pytest.mark.gpu
L = _lib.lib
fp = _lib.fptr


def test_create_accepts_all_bits_and_sets_no_error():
    """test_api.cpp:25-29, :111-116.  Like the reference, a successful create
    leaves the thread's last error as it was (empty on a fresh thread)."""
    print("api: create", flush=True)
    seen = []

    def work():
        for kb in (2, 3, 4, 16):
            for vb in (2, 3, 4, 16):
                h = L.adaptq_create(128, kb, vb, 1024, 42, 0.0, 0)
                seen.append((bool(h), err(), L.adaptq_kv_bytes(h) if h else -1))
                L.adaptq_destroy(h)
        m = L.adaptq_mha_create(4, 128, 4, 2, 1024, 0, 0.0, 0)
        seen.append((bool(m), err(), 0))
        L.adaptq_mha_destroy(m)

    t = threading.Thread(target=work)
    t.start()
    t.join()
    assert seen == [(True, "", 0)] * 17


def test_null_buffers_on_live_handles():
    print("api: null buffers", flush=True)
    h = L.adaptq_create(64, 4, 2, 16, 42, 0.0, 0)
    q = np.ones(64, np.float32)
    out = np.zeros(64, np.float32)
    L.adaptq_append(h, None, fp(q), 0)
    assert err() == "adaptq_append: null key"
    L.adaptq_append(h, fp(q), None, 0)
    assert err() == "adaptq_append: null val"
    assert L.adaptq_compute(h, None, fp(out)) == -1 and err() == "adaptq_compute: null query"
    assert L.adaptq_compute(h, fp(q), None) == -1 and err() == "adaptq_compute: null out"
    assert L.adaptq_compute_batch(h, None, 1, fp(out)) == -1
    assert err() == "adaptq_compute_batch: null queries"
    assert L.adaptq_compute_batch(h, fp(q), 1, None) == -1
    assert err() == "adaptq_compute_batch: null outs"
    assert L.adaptq_compute_batch(h, fp(q), -1, fp(out)) == -1
    assert err() == "adaptq_compute_batch: negative num_queries"
    assert L.adaptq_compute_batch(h, None, 0, None) == 0
    L.adaptq_destroy(h)

    m = L.adaptq_mha_create(2, 64, 4, 2, 16, 0, 0.0, 0)
    L.adaptq_mha_append(m, 0, None, fp(q), 0)
    assert err() == "adaptq_mha_append: null key"
    L.adaptq_mha_append(m, 0, fp(q), None, 0)
    assert err() == "adaptq_mha_append: null val"
    L.adaptq_mha_append(m, 2, fp(q), fp(q), 0)
    assert err() == "adaptq_mha_append: head_idx out of range"
    L.adaptq_mha_append(m, -1, fp(q), fp(q), 0)
    assert err() == "adaptq_mha_append: head_idx out of range"
    assert L.adaptq_mha_compute(m, 2, fp(q), fp(out)) == -1
    assert err() == "adaptq_mha_compute: head_idx out of range"
    assert L.adaptq_mha_compute(m, 0, None, fp(out)) == -1
    assert err() == "adaptq_mha_compute: null query"
    assert L.adaptq_mha_compute_batch(m, 0, fp(q), -1, fp(out)) == -1
    assert err() == "adaptq_mha_compute_batch: negative num_queries"
    assert L.adaptq_mha_compute_batch(m, 5, fp(q), 1, fp(out)) == -1
    assert err() == "adaptq_mha_compute_batch: head_idx out of range"
    assert L.adaptq_mha_compute_batch(m, 0, None, 0, None) == 0
    L.adaptq_mha_append(m, 1, fp(q), fp(q), 0)
    assert err() == ""  # success clears the message
    assert L.adaptq_mha_compute(m, 1, fp(q), fp(out)) == 1
    L.adaptq_mha_destroy(m)


def test_empty_append_compute_reset():
    print("api: empty/reset", flush=True)
    g = GpuHead(64, 4, 2, 32, 42)
    out, n = g.compute(np.ones(64, np.float32))
    assert n == 0 and not out.any()
    rng = np.random.default_rng(0)
    for t in range(2):
        g.append(rng.standard_normal(64), rng.standard_normal(64), t)
    assert g.kv_bytes() == 2 * (32 + 16)
    out, n = g.compute(rng.standard_normal(64))
    assert n == 2 and np.linalg.norm(out) > 1e-10
    g.reset()
    assert g.kv_bytes() == 0 and err() == ""
    out, n = g.compute(np.ones(64, np.float32))
    assert n == 0 and not out.any()


def test_capacity_zero():
    print("api: capacity 0", flush=True)
    g = GpuHead(64, 4, 2, 0, 42)
    g.append(np.ones(64, np.float32), np.ones(64, np.float32), 0)
    out, n = g.compute(np.ones(64, np.float32))
    assert n == 0 and not out.any() and g.kv_bytes() == 0


def test_contexts_above_65536_tokens(oracle):
    """test_api.cpp:303-330: 65535, 65536, 65537 and 100000 cached tokens."""
    print("api: 100000 tokens", flush=True)
    dim = 64
    g = GpuHead(dim, 4, 2, 100005, 42)
    o = oracle.head(dim, 4, 2, 100005, 42)
    rng = np.random.default_rng(5)
    q = rng.standard_normal(dim).astype(np.float32)
    cur = 0
    for target in (65535, 65536, 65537, 100000):
        kv = rng.standard_normal((target - cur, 2, dim)).astype(np.float32)
        for t in range(target - cur):
            g.append(kv[t, 0], kv[t, 1], cur + t)
            o.append(kv[t, 0], kv[t, 1], cur + t)
        cur = target
        y, n = g.compute(q)
        r, m = o.compute(q)
        assert n == m == target
        assert rel_err(y, r) <= 1e-4


def test_degenerate_inputs(oracle):
    """test_api.cpp:334-361: zeros, NaN and +-1e38 rows neither crash nor
    disturb the other rows' codes; outputs equal the oracle's (NaN included)."""
    print("api: degenerate inputs", flush=True)
    g = GpuHead(64, 4, 2, 128, 42)
    o = oracle.head(64, 4, 2, 128, 42)
    rows = [(np.zeros(64), np.zeros(64)), (np.full(64, np.nan), np.full(64, np.nan)),
            (np.full(64, 1e38), np.full(64, -1e38))]
    for t, (k, v) in enumerate(rows):
        g.append(k, v, t)
        o.append(k, v, t)
    y, n = g.compute(np.zeros(64, np.float32))
    r, m = o.compute(np.zeros(64, np.float32))
    assert n == m == 3
    assert np.array_equal(np.isnan(y), np.isnan(r))
    fin = ~np.isnan(r)
    assert np.allclose(y[fin], r[fin], rtol=1e-4, atol=1e-30)


def test_hybrid_mirror_invalidated_on_first_eviction(oracle):
    """attention.cpp:338-366, :491-523: the fp32 branch serves n <= hybrid
    until the ring first evicts; after that the packed path serves."""
    print("api: hybrid invalidation", flush=True)
    dim, cap, hyb = 64, 40, 64
    g = GpuHead(dim, 4, 2, cap, 3, 0.0, hyb)
    o = oracle.head(dim, 4, 2, cap, 3, 0.0, hyb)
    rng = np.random.default_rng(2)
    q = rng.standard_normal(dim).astype(np.float32)
    for t in range(cap + 5):
        k, v = rng.standard_normal((2, dim)).astype(np.float32)
        g.append(k, v, t)
        o.append(k, v, t)
        if t in (10, cap - 1, cap, cap + 4):
            y, _ = g.compute(q)
            r, _ = o.compute(q)
            assert rel_err(y, r) <= 1e-4, t
    g.reset()
    o.reset()
    for t in range(5):  # reset restores the mirror
        k, v = rng.standard_normal((2, dim)).astype(np.float32)
        g.append(k, v, t)
        o.append(k, v, t)
    assert rel_err(g.compute(q)[0], o.compute(q)[0]) <= 1e-4


def test_handles_from_several_threads(oracle):
    """Independent handles are usable concurrently (adaptq.h:12)."""
    print("api: threads", flush=True)
    dim, n, T = 64, 400, 4
    rng = np.random.default_rng(8)
    data = rng.standard_normal((T, n, 2, dim)).astype(np.float32)
    qs = rng.standard_normal((T, dim)).astype(np.float32)
    results = [None] * T
    errors = []

    def work(i):
        try:
            g = GpuHead(dim, 4, 2, 256, 50 + i)
            for t in range(n):
                g.append(data[i, t, 0], data[i, t, 1], t)
                if t % 97 == 0:
                    g.compute(qs[i])
            results[i] = g.compute(qs[i])[0]
        except Exception as e:  # surfaced below
            errors.append(repr(e))

    threads = [threading.Thread(target=work, args=(i,)) for i in range(T)]
    for t in threads:
        t.start()
    for t in threads:
        t.join()
    assert not errors, errors
    for i in range(T):
        o = oracle.head(dim, 4, 2, 256, 50 + i)
        for t in range(n):
            o.append(data[i, t, 0], data[i, t, 1], t)
        assert rel_err(results[i], o.compute(qs[i])[0]) <= 1e-4


def test_read_slots_bounds():
    g = GpuHead(64, 4, 2, 8, 1)
    kc = np.zeros((4, 32), np.uint8)
    assert L.adaptq_read_slots(g.h, 6, 4, _lib.u8ptr(kc), None, None, None) == -1
    assert err() == "adaptq_read_slots: slot range out of bounds"
    assert L.adaptq_mha_head(None, 0) is None
