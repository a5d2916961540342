"""The decode step with its append in the decode launch (launch_decode_step:
dense decodes at padded 64 with quantised K and V, one block per head).

The fused launch must leave the same ring bytes and give the same outputs as
the append launch followed by the decode launch, and both must match the
oracle (attention.cpp:338-366 then :480-660).  Covered: the device-form step
(adaptq_mha_append_compute_all_device) against the two device-form calls,
bit for bit, over every K/V width pair at dim 64 and 48, across ring wraps,
with NaN, zero and tiny step rows; the host forms the reference's API uses
(adaptq_append + adaptq_compute, adaptq_mha_append + adaptq_mha_compute_all)
against the oracle; and the steps the fused launch declines (hybrid mirror
branch, sparse-V, heads of different ring sizes) falling back correctly.
"""
import ctypes as C

import numpy as np
import pytest

from adaptq_amd import _lib
from gpu_head import GpuHead, err, rel_err

pytestmark = pytest.mark.gpu
L = _lib.lib


def mha_heads(m, n_heads, dim):
    return [GpuHead.wrap(L.adaptq_mha_head(m, h), dim) for h in range(n_heads)]


def ring_bytes(heads):
    out = []
    for hd in heads:
        inf = hd.info()
        out.append((inf["head"], inf["size"]) + tuple(a.tobytes() for a in hd.read_slots(0, inf["cap"])))
    return out


def step_rows(rng, n_heads, dim, special=None):
    k = rng.standard_normal((n_heads, dim)).astype(np.float32)
    v = rng.standard_normal((n_heads, dim)).astype(np.float32)
    if special == "nan":
        k[0, 5] = np.nan
        v[1 % n_heads, 2] = np.nan
    elif special == "zero":
        k[0] = 0.0
        v[0] = 0.0
    elif special == "tiny":
        k[0] *= np.float32(1e-8)
        v[-1] *= np.float32(1e-8)
    return k, v


@pytest.mark.parametrize("dim", [64, 48])
@pytest.mark.parametrize("kb,vb", [(4, 2), (3, 2), (2, 2), (4, 4), (3, 3), (2, 4), (4, 3)])
def test_device_step_matches_two_calls(torch_dev, dim, kb, vb):
    torch = torch_dev
    print(f"fused step d{dim} K{kb}V{vb}", flush=True)
    nh, cap, n0, steps = 4, 300, 280, 40  # the steps wrap the ring
    rng = np.random.default_rng(dim * 100 + kb * 10 + vb)
    ma = L.adaptq_mha_create(nh, dim, kb, vb, cap, 11, 0.0, 0)
    mb = L.adaptq_mha_create(nh, dim, kb, vb, cap, 11, 0.0, 0)
    assert ma and mb, err()
    bulk_k = torch.from_numpy(rng.standard_normal((nh, n0, dim)).astype(np.float32)).cuda()
    bulk_v = torch.from_numpy(rng.standard_normal((nh, n0, dim)).astype(np.float32)).cuda()
    for m in (ma, mb):
        assert L.adaptq_mha_append_all_device(m, C.c_void_p(bulk_k.data_ptr()),
                                              C.c_void_p(bulk_v.data_ptr()), n0, 0, None) == 0, err()
    oa = torch.empty(nh, dim, device="cuda")
    ob = torch.empty(nh, dim, device="cuda")
    for s in range(steps):
        special = {3: "nan", 7: "zero", 11: "tiny"}.get(s)
        k, v = step_rows(rng, nh, dim, special)
        q = rng.standard_normal((nh, dim)).astype(np.float32)
        kd, vd, qd = (torch.from_numpy(x).cuda() for x in (k, v, q))
        na = L.adaptq_mha_append_compute_all_device(ma, C.c_void_p(kd.data_ptr()),
                                                    C.c_void_p(vd.data_ptr()), n0 + s,
                                                    C.c_void_p(qd.data_ptr()),
                                                    C.c_void_p(oa.data_ptr()), None)
        assert na == min(n0 + s + 1, cap), (na, err())
        assert L.adaptq_mha_append_all_device(mb, C.c_void_p(kd.data_ptr()),
                                              C.c_void_p(vd.data_ptr()), 1, n0 + s, None) == 0
        assert L.adaptq_mha_compute_all_device(mb, C.c_void_p(qd.data_ptr()),
                                               C.c_void_p(ob.data_ptr()), None) == na, err()
        torch.cuda.synchronize()
        ya, yb = oa.cpu().numpy(), ob.cpu().numpy()
        assert ya.tobytes() == yb.tobytes() or (np.isnan(ya).any() and
                                                np.array_equal(np.isnan(ya), np.isnan(yb))), s
    assert ring_bytes(mha_heads(ma, nh, dim)) == ring_bytes(mha_heads(mb, nh, dim))
    L.adaptq_mha_destroy(ma)
    L.adaptq_mha_destroy(mb)


@pytest.mark.parametrize("kb,vb", [(4, 2), (3, 2)])
def test_host_forms_match_oracle(oracle, kb, vb):
    """The reference's per-step calls: adaptq_append then adaptq_compute on a
    context, and adaptq_mha_append per head then adaptq_mha_compute_all."""
    print(f"host-form steps K{kb}V{vb}", flush=True)
    dim, nh, cap, n0, steps = 64, 3, 128, 100, 60
    rng = np.random.default_rng(kb * 7 + vb)
    g = GpuHead(dim, kb, vb, cap, 5)
    o = oracle.head(dim, kb, vb, cap, 5)
    m = L.adaptq_mha_create(nh, dim, kb, vb, cap, 9, 0.0, 0)
    om = [oracle.head(dim, kb, vb, cap, oracle.mha_seed(9, h)) for h in range(nh)]
    for t in range(n0 + steps):
        k, v = step_rows(rng, nh, dim, {n0 + 2: "nan", n0 + 5: "tiny"}.get(t))
        g.append(k[0], v[0], t)
        o.append(k[0], v[0], t)
        for h in range(nh):
            L.adaptq_mha_append(m, h, _lib.fptr(np.ascontiguousarray(k[h])),
                                _lib.fptr(np.ascontiguousarray(v[h])), t)
            om[h].append(k[h], v[h], t)
        if t >= n0:
            q = rng.standard_normal((nh, dim)).astype(np.float32)
            y, n = g.compute(q[0])
            r, nr = o.compute(q[0])
            assert n == nr
            if np.isnan(r).any():
                assert np.array_equal(np.isnan(y), np.isnan(r))
            else:
                assert rel_err(y, r) <= 1e-4, t
            out = np.zeros((nh, dim), np.float32)
            assert L.adaptq_mha_compute_all(m, _lib.fptr(q), _lib.fptr(out)) == nr, err()
            for h in range(nh):
                rh, _ = om[h].compute(q[h])
                if not np.isnan(rh).any():
                    assert rel_err(out[h], rh) <= 1e-4, (t, h)
    kc, vc, ks, vs = g.read_slots(0, cap)
    okc, ovc, oks, ovs = o.read_slots(0, cap)
    assert kc.tobytes() == okc.tobytes() and vc.tobytes() == ovc.tobytes()
    assert ks.tobytes() == oks.tobytes() and vs.tobytes() == ovs.tobytes()
    assert g.info()["head"] == o.info()["head"]
    for h in range(nh):
        hd = GpuHead.wrap(L.adaptq_mha_head(m, h), dim)
        assert [a.tobytes() for a in hd.read_slots(0, cap)] == \
            [a.tobytes() for a in om[h].read_slots(0, cap)], h
    L.adaptq_mha_destroy(m)


@pytest.mark.parametrize("vm,hyb", [(0.0, 8), (0.95, 0), (0.95, 8)])
def test_declined_steps_match_oracle(oracle, vm, hyb):
    """Steps the fused launch does not take: the hybrid mirror branch (the
    first hyb tokens, and the mirror writes of the steps after it), sparse-V;
    each decoded step against the oracle, ring bytes at the end."""
    print(f"declined steps v_mass={vm} hyb={hyb}", flush=True)
    dim, cap = 64, 40
    rng = np.random.default_rng(int(vm * 100) + hyb)
    g = GpuHead(dim, 4, 2, cap, 3, vm, hyb)
    o = oracle.head(dim, 4, 2, cap, 3, vm, hyb)
    for t in range(70):  # through the hybrid threshold and past the wrap
        k, v = step_rows(rng, 1, dim)
        g.append(k[0], v[0], t)
        o.append(k[0], v[0], t)
        q = rng.standard_normal(dim).astype(np.float32)
        y, n = g.compute(q)
        r, nr = o.compute(q)
        assert n == nr
        assert rel_err(y, r) <= 1e-4, t
    assert [a.tobytes() for a in g.read_slots(0, cap)] == [a.tobytes() for a in o.read_slots(0, cap)]
    assert g.info()["head"] == o.info()["head"]


def test_uneven_heads_fall_back(oracle, torch_dev):
    """Heads whose rings differ in size: the device step appends, then reports
    that the decode needs adaptq_mha_compute_all; the host form decodes head
    by head."""
    torch = torch_dev
    print("uneven heads", flush=True)
    dim, nh, cap = 64, 2, 64
    rng = np.random.default_rng(4)
    m = L.adaptq_mha_create(nh, dim, 4, 2, cap, 1, 0.0, 0)
    om = [oracle.head(dim, 4, 2, cap, oracle.mha_seed(1, h)) for h in range(nh)]
    k, v = step_rows(rng, nh, dim)
    L.adaptq_mha_append(m, 0, _lib.fptr(k[0]), _lib.fptr(v[0]), 0)  # head 0 only
    om[0].append(k[0], v[0], 0)
    k, v = step_rows(rng, nh, dim)
    q = rng.standard_normal((nh, dim)).astype(np.float32)
    kd, vd, qd = (torch.from_numpy(x).cuda() for x in (k, v, q))
    od = torch.empty(nh, dim, device="cuda")
    rc = L.adaptq_mha_append_compute_all_device(m, C.c_void_p(kd.data_ptr()), C.c_void_p(vd.data_ptr()),
                                                1, C.c_void_p(qd.data_ptr()), C.c_void_p(od.data_ptr()),
                                                None)
    assert rc == -1 and "differ" in err()
    torch.cuda.synchronize()
    for h in range(nh):
        om[h].append(k[h], v[h], 1)
    out = np.zeros((nh, dim), np.float32)
    assert L.adaptq_mha_compute_all(m, _lib.fptr(q), _lib.fptr(out)) == 2, err()
    for h in range(nh):
        assert rel_err(out[h], om[h].compute(q[h])[0]) <= 1e-4
    L.adaptq_mha_destroy(m)
