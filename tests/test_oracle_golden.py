"""The CPU oracle (oracle/oracle.c) against the reference's own outputs.

The fixtures in tests/golden/ were written by tests/golden/make_golden.py from
the reference's hot-path sources compiled in place (oracle/_ref).  Codes,
scales, signs and FWHT outputs must match bit for bit; attention outputs are
held to 1e-6 norm-wise relative error (the oracle follows the reference's
AVX2 summation order, so most match exactly).
"""
import os

import numpy as np
import pytest

from golden import inputs as I

GOLD = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")
MODES = [(0.0, 0), (0.95, 512)]


def load(name):
    return np.load(os.path.join(GOLD, name))


def rel(y, r):
    return float(np.max(np.abs(y - r)) / max(float(np.max(np.abs(r))), 1e-30))


def bits_equal(a, b):
    a, b = np.asarray(a), np.asarray(b)
    return a.shape == b.shape and a.tobytes() == b.tobytes()


def test_rademacher(oracle):
    g = load("rademacher.npz")
    plus = np.unpackbits(g["plus"], axis=1)
    for s, n, row in zip(g["seeds"], g["dims"], plus):
        D = oracle.rademacher(int(n), int(s))
        assert np.array_equal(D > 0, row[:n].astype(bool)), f"seed {int(s):#x}"
        assert set(np.unique(D)) <= {-1, 1}


def test_fwht(oracle):
    g = load("fwht.npz")
    for p in (64, 128, 256):
        D = g[f"D{p}"]
        for x, fwd, inv in zip(g[f"x{p}"], g[f"fwd{p}"], g[f"inv{p}"]):
            assert bits_equal(oracle.fwht_forward(x, D), fwd)
            assert bits_equal(oracle.fwht_inverse(x, D), inv)


@pytest.mark.parametrize("bits", [2, 3, 4])
def test_quantize_fast(oracle, bits):
    g = load("quantize_fast.npz")
    got = np.array([oracle.quantize_fast(float(v), bits) for v in g["vals"]], np.uint8)
    assert np.array_equal(got, g[f"idx{bits}"])
    got = np.array([oracle.quantize_fast(float(v), bits) for v in g[f"edge_vals{bits}"]], np.uint8)
    assert np.array_equal(got, g[f"edge_idx{bits}"])
    # every threshold was located: 2^bits - 1 index changes, each seen as a
    # (below, at, above) triple
    assert len(g[f"edge_vals{bits}"]) == 3 * ((1 << bits) - 1)


@pytest.mark.parametrize("dim", [64, 128, 96, 48])
@pytest.mark.parametrize("bits", [2, 3, 4])
def test_codec(oracle, dim, bits):
    g = load("codec.npz")
    D = oracle.rademacher(oracle.lib.orc_next_pow2(dim), 0x5EED + dim)
    codes, scales = g[f"codes_d{dim}_b{bits}"], g[f"scales_d{dim}_b{bits}"]
    k = 0
    for fam in I.FAMILIES:
        for x in I.codec_inputs(dim, fam):
            c, s, _ = oracle.quantize_vec(x, D, bits)
            assert bits_equal(c, codes[k]), f"{fam} vector {k}: codes differ"
            assert bits_equal(np.float32(s), scales[k]), f"{fam} vector {k}: scale differs"
            k += 1


def _ring_check(head, g, h, sl=None):
    inf = head.info()
    assert [inf["head"], inf["size"]] == list(g[f"head{h}_state"])
    kc, vc, ks, vs = head.read_slots(0, inf["size"])
    import hashlib
    hh = hashlib.sha256()
    for a in (kc, vc, ks, vs):
        hh.update(np.ascontiguousarray(a).tobytes())
    assert hh.hexdigest() == str(g[f"head{h}_sha"])


def test_config1(oracle):
    c = I.CONFIG1
    g = load("config1.npz")
    K, V, q = I.config1_inputs()
    for vm, hyb in MODES:
        heads = [oracle.head(c["dim"], c["k_bits"], c["v_bits"], c["cap"],
                             oracle.mha_seed(42, h), vm, hyb) for h in range(c["n_heads"])]
        for t in range(c["n"]):
            for h, hd in enumerate(heads):
                hd.append(K[t, h], V[t, h], t)
        out = np.stack([hd.compute(q[h])[0] for h, hd in enumerate(heads)])
        ref = g[f"out_vm{int(vm * 100)}_h{hyb}"]
        assert rel(out, ref) <= 1e-6
        if vm == 0.0:
            for h, hd in enumerate(heads):
                _ring_check(hd, g, h)
                kc, vc, ks, vs = hd.read_slots(0, 64)
                assert bits_equal(kc, g[f"head{h}_kc_first"])
                assert bits_equal(vs, g[f"head{h}_vs_first"])


def test_config2(oracle):
    c = I.CONFIG2
    g = load("config2.npz")
    for vm, hyb in MODES:
        ref = g[f"out_vm{int(vm * 100)}_h{hyb}"]
        for layer in range(c["n_layers"]):
            kb, vb, base, K, V, q = I.config2_layer(layer)
            for h in range(c["n_heads"]):
                hd = oracle.head(c["dim"], kb, vb, c["cap"], oracle.mha_seed(base, h), vm, hyb)
                for t in range(c["n"]):
                    hd.append(K[t, h], V[t, h], t)
                out, n = hd.compute(q[h])
                assert n == c["n"]
                assert rel(out, ref[layer, h]) <= 1e-6, (layer, h, vm, hyb)


def test_config3(oracle):
    c = I.CONFIG3
    g = load("config3.npz")
    steps = list(g["steps"])
    for vm, hyb in MODES:
        ref = g[f"out_vm{int(vm * 100)}_h{hyb}"]
        for layer in range(0, c["n_layers"], 3):  # every third layer keeps the CPU suite short
            kb, vb, base, K, V, Q = I.config3_layer(layer)
            for h in range(c["n_heads"]):
                hd = oracle.head(c["dim"], kb, vb, c["cap"], oracle.mha_seed(base, h), vm, hyb)
                for t in range(c["bulk"]):
                    hd.append(K[t, h], V[t, h], t)
                for s in range(max(steps) + 1):
                    hd.append(K[c["bulk"] + s, h], V[c["bulk"] + s, h], c["bulk"] + s)
                    if s in steps:
                        out, _ = hd.compute(Q[s, h])
                        assert rel(out, ref[steps.index(s), layer, h]) <= 1e-6, (layer, h, s)


def test_config4_wrap(oracle):
    """Ring wraparound: 40000 appends into capacity 32768 (7232 evictions)."""
    c = I.CONFIG4
    g = load("config4.npz")
    Q = I.config4_queries()
    heads = [oracle.head(c["dim"], c["k_bits"], c["v_bits"], c["cap"], oracle.mha_seed(7, h))
             for h in range(2)]
    for ch in range((c["n"] + c["chunk"] - 1) // c["chunk"]):
        K, V = I.config4_chunk(ch)
        for t in range(K.shape[0]):
            for h, hd in enumerate(heads):
                hd.append(K[t, h], V[t, h], ch * c["chunk"] + t)
    for h, hd in enumerate(heads):
        _ring_check(hd, g, h)
        kc, vc, ks, vs = hd.read_slots(7200, 64)
        assert bits_equal(kc, g[f"head{h}_kc_wrap"])
        assert bits_equal(vc, g[f"head{h}_vc_wrap"])
        assert bits_equal(ks, g[f"head{h}_ks_wrap"])
        out, n = hd.compute(Q[0, h])
        assert n == c["cap"]
        assert rel(out, g["out_vm0_h0"][0, h]) <= 1e-6
