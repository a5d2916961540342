"""BASELINE configurations 1-4 end to end on the GPU, through the C ABI's MHA
entry points, against the reference's own outputs (tests/golden/, written
from the reference build) and the CPU oracle.

Bar: ring state, codes and scales bit-exact (SHA-256 over every slot);
attention outputs within 1e-4 norm-wise relative error.  Both the pure
packed-KV decode (v_mass 0, hybrid 0) and the Python Engine defaults
(v_mass 0.95, hybrid 512: hybrid fp32 and sparse-V branches) are covered.
"""
import ctypes as C
import hashlib
import os

import numpy as np
import pytest

from adaptq_amd import _lib
from golden import inputs as I
from gpu_head import GpuHead, err, rel_err, same_bits

pytestmark = pytest.mark.gpu
L = _lib.lib
GOLD = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")
MODES = [(0.0, 0), (0.95, 512)]
TOL = 1e-4


def load(name):
    return np.load(os.path.join(GOLD, name))


class Mha:
    def __init__(self, n_heads, dim, kb, vb, cap, base, vm, hyb):
        self.dim = dim
        self.m = L.adaptq_mha_create(n_heads, dim, kb, vb, cap, base, vm, hyb)
        assert self.m, err()
        self.heads = [GpuHead.wrap(L.adaptq_mha_head(self.m, h), dim) for h in range(n_heads)]

    def append(self, h, k, v, pos):
        k = np.ascontiguousarray(k, np.float32)
        v = np.ascontiguousarray(v, np.float32)
        L.adaptq_mha_append(self.m, h, _lib.fptr(k), _lib.fptr(v), pos)

    def compute(self, h, q):
        q = np.ascontiguousarray(q, np.float32)
        out = np.zeros(self.dim, np.float32)
        n = L.adaptq_mha_compute(self.m, h, _lib.fptr(q), _lib.fptr(out))
        assert n >= 0, err()
        return out, n

    def __del__(self):
        if getattr(self, "m", None):
            L.adaptq_mha_destroy(self.m)
            self.m = None


def ring_sha(head):
    inf = head.info()
    kc, vc, ks, vs = head.read_slots(0, inf["size"])
    h = hashlib.sha256()
    for a in (kc, vc, ks, vs):
        h.update(np.ascontiguousarray(a).tobytes())
    return h.hexdigest()


@pytest.mark.parametrize("vm,hyb", MODES)
def test_config1(vm, hyb):
    print(f"config1 v_mass={vm} hyb={hyb}", flush=True)
    c = I.CONFIG1
    g = load("config1.npz")
    K, V, q = I.config1_inputs()
    m = Mha(c["n_heads"], c["dim"], c["k_bits"], c["v_bits"], c["cap"], 42, vm, hyb)
    for t in range(c["n"]):
        for h in range(c["n_heads"]):
            m.append(h, K[t, h], V[t, h], t)
    out = np.stack([m.compute(h, q[h])[0] for h in range(c["n_heads"])])
    assert rel_err(out, g[f"out_vm{int(vm * 100)}_h{hyb}"]) <= TOL
    assert L.adaptq_mha_total_kv_bytes(m.m) == 393216
    for h, hd in enumerate(m.heads):
        inf = hd.info()
        assert [inf["head"], inf["size"]] == list(g[f"head{h}_state"])
        assert ring_sha(hd) == str(g[f"head{h}_sha"])
        kc, vc, ks, vs = hd.read_slots(inf["size"] - 64, 64)
        assert same_bits(kc, g[f"head{h}_kc_last"]) and same_bits(vs, g[f"head{h}_vs_last"])


@pytest.mark.parametrize("vm,hyb", MODES)
def test_config2(vm, hyb):
    print(f"config2 v_mass={vm} hyb={hyb}", flush=True)
    c = I.CONFIG2
    g = load("config2.npz")
    ref = g[f"out_vm{int(vm * 100)}_h{hyb}"]
    for layer in range(c["n_layers"]):
        kb, vb, base, K, V, q = I.config2_layer(layer)
        m = Mha(c["n_heads"], c["dim"], kb, vb, c["cap"], base, vm, hyb)
        for t in range(c["n"]):
            for h in range(c["n_heads"]):
                m.append(h, K[t, h], V[t, h], t)
        for h in range(c["n_heads"]):
            out, n = m.compute(h, q[h])
            assert n == c["n"]
            assert rel_err(out, ref[layer, h]) <= TOL, (layer, h)
        if vm == 0.0:
            assert ring_sha(m.heads[0]) == str(g[f"ring_sha_l{layer}"]), layer


@pytest.mark.parametrize("vm,hyb", MODES)
def test_config3_decode_steps(vm, hyb):
    """Bulk append, then 256 steps of (append one token, compute) per head."""
    print(f"config3 v_mass={vm} hyb={hyb}", flush=True)
    c = I.CONFIG3
    g = load("config3.npz")
    steps = list(g["steps"])
    ref = g[f"out_vm{int(vm * 100)}_h{hyb}"]
    for layer in range(c["n_layers"]):
        kb, vb, base, K, V, Q = I.config3_layer(layer)
        m = Mha(c["n_heads"], c["dim"], kb, vb, c["cap"], base, vm, hyb)
        for t in range(c["bulk"]):
            for h in range(c["n_heads"]):
                m.append(h, K[t, h], V[t, h], t)
        for s in range(c["steps"]):
            for h in range(c["n_heads"]):
                t = c["bulk"] + s
                m.append(h, K[t, h], V[t, h], t)
                out, n = m.compute(h, Q[s, h])
                assert n == t + 1
                if s in steps:
                    assert rel_err(out, ref[steps.index(s), layer, h]) <= TOL, (layer, h, s)


def test_config4_wrap_and_queries(oracle):
    """40000 appends into capacity 32768: 7232 evictions, head = 7232."""
    print("config4 wrap", flush=True)
    c = I.CONFIG4
    g = load("config4.npz")
    Q = I.config4_queries()
    for vm, hyb in MODES:
        m = Mha(c["n_heads"], c["dim"], c["k_bits"], c["v_bits"], c["cap"], 7, vm, hyb)
        for ch in range((c["n"] + c["chunk"] - 1) // c["chunk"]):
            K, V = I.config4_chunk(ch)
            for t in range(K.shape[0]):
                for h in range(c["n_heads"]):
                    m.append(h, K[t, h], V[t, h], ch * c["chunk"] + t)
        tag = f"vm{int(vm * 100)}_h{hyb}"
        for h in range(c["n_heads"]):
            qs = np.ascontiguousarray(Q[:, h])
            outs = np.zeros((c["n_queries"], c["dim"]), np.float32)
            n = L.adaptq_mha_compute_batch(m.m, h, _lib.fptr(qs), c["n_queries"],
                                           _lib.fptr(outs))
            assert n == c["cap"], err()
            assert rel_err(outs[:8], g[f"out_{tag}"][:, h]) <= TOL, (h, tag)
            if vm == 0.0:
                hd = m.heads[h]
                inf = hd.info()
                assert [inf["head"], inf["size"]] == list(g[f"head{h}_state"])
                assert ring_sha(hd) == str(g[f"head{h}_sha"])
                if h < 2:
                    kc, vc, ks, vs = hd.read_slots(7200, 64)
                    assert same_bits(kc, g[f"head{h}_kc_wrap"])
                    assert same_bits(vc, g[f"head{h}_vc_wrap"])
        if vm == 0.0:
            # the remaining 56 queries of one head against the oracle
            o = oracle.head(c["dim"], c["k_bits"], c["v_bits"], c["cap"], I.mha_seed(7, 3))
            for ch in range((c["n"] + c["chunk"] - 1) // c["chunk"]):
                K, V = I.config4_chunk(ch)
                for t in range(K.shape[0]):
                    o.append(K[t, 3], V[t, 3], 0)
            r, _ = o.compute_batch(np.ascontiguousarray(Q[8:, 3]))
            outs = np.zeros((56, c["dim"]), np.float32)
            qs = np.ascontiguousarray(Q[8:, 3])
            assert L.adaptq_mha_compute_batch(m.m, 3, _lib.fptr(qs), 56, _lib.fptr(outs)) == c["cap"]
            assert rel_err(outs, r) <= TOL
        assert L.adaptq_mha_total_kv_bytes(m.m) == 33554432
        del m
