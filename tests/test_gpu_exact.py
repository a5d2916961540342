"""The GPU's outputs against exact attention, beside the reference's own.

An fp32 decode of a packed ring approximates the float64 softmax attention
over the dequantised ring (tests/golden/exact64.py).  The reference's AVX2
path and its scalar path (attention.cpp:606-659) each sit some distance from
that exact value; tests/golden/ref_flavours.json records those distances for
configs 1-4 and two rings at padded 512 and 1024 (v_mass 0, hybrid 0),
measured on the reference build by
tests/golden/ref_flavours.py.  Here the library decodes the same rings and
its distance to the exact value, norm-wise (max|y - x| / max|x|) and
elementwise (max |y - x| / |x| over entries with |x| >= 1e-3 max|x|), worst
over the config's heads, must not exceed the farther of the reference's two
paths (its AVX2 path and its scalar path, which differ only in the order of
the key dot products): within the reference's own spread.  The rings are
bit-exact with the reference's (tests/test_gpu_configs.py), so the exact
value is the same for all three.
"""
import json
import os

import numpy as np
import pytest

from adaptq_amd import _lib
from golden import exact64 as X
from golden import inputs as I
from gpu_head import err
from test_gpu_configs import Mha

pytestmark = pytest.mark.gpu
L = _lib.lib
GOLD = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")
REF_EXACT = json.load(open(os.path.join(GOLD, "ref_flavours.json")))["exact"]


def ref_bar(tag):
    """The farther of the reference's AVX2 and scalar paths from exact."""
    a, b = REF_EXACT["base"][tag], REF_EXACT["scalar"][tag]
    return {"norm_max": max(a["norm_max"], b["norm_max"]),
            "elem_max": max(a["elem_max"], b["elem_max"]),
            "avx2": (a["norm_max"], a["elem_max"]), "scalar": (b["norm_max"], b["elem_max"])}


def cfg_heads(name):
    """(mha, [(head index, query, seed, kb, vb)]) with the rings filled as
    tests/golden/ref_flavours.py fills the reference's."""
    if name == "config1":
        c = I.CONFIG1
        K, V, q = I.config1_inputs()
        m = Mha(c["n_heads"], c["dim"], c["k_bits"], c["v_bits"], c["cap"], 42, 0.0, 0)
        for t in range(c["n"]):
            for h in range(c["n_heads"]):
                m.append(h, K[t, h], V[t, h], t)
        yield m, [(h, q[h], I.mha_seed(42, h), c["k_bits"], c["v_bits"])
                  for h in range(c["n_heads"])]
    elif name == "config2":
        c = I.CONFIG2
        for layer in range(c["n_layers"]):
            kb, vb, base, K, V, q = I.config2_layer(layer)
            m = Mha(c["n_heads"], c["dim"], kb, vb, c["cap"], base, 0.0, 0)
            for t in range(c["n"]):
                for h in range(c["n_heads"]):
                    m.append(h, K[t, h], V[t, h], t)
            yield m, [(h, q[h], I.mha_seed(base, h), kb, vb) for h in range(c["n_heads"])]
    elif name == "config3":
        c = I.CONFIG3
        for layer in range(c["n_layers"]):
            kb, vb, base, K, V, Q = I.config3_layer(layer)
            m = Mha(c["n_heads"], c["dim"], kb, vb, c["cap"], base, 0.0, 0)
            for t in range(c["bulk"] + 1):
                for h in range(c["n_heads"]):
                    m.append(h, K[t, h], V[t, h], t)
            yield m, [(h, Q[0, h], I.mha_seed(base, h), kb, vb) for h in range(c["n_heads"])]
    elif name in I.WIDE:
        c = I.WIDE[name]
        K, V, q = I.wide_inputs(name)
        base = c["base_seed"]
        m = Mha(c["n_heads"], c["dim"], c["k_bits"], c["v_bits"], c["cap"], base, 0.0, 0)
        for t in range(c["n"]):
            for h in range(c["n_heads"]):
                m.append(h, K[t, h], V[t, h], t)
        yield m, [(h, q[h], I.mha_seed(base, h), c["k_bits"], c["v_bits"])
                  for h in range(c["n_heads"])]
    else:
        c = I.CONFIG4
        Q = I.config4_queries()
        m = Mha(c["n_heads"], c["dim"], c["k_bits"], c["v_bits"], c["cap"], 7, 0.0, 0)
        for ch in range((c["n"] + c["chunk"] - 1) // c["chunk"]):
            K, V = I.config4_chunk(ch)
            for t in range(K.shape[0]):
                for h in range(c["n_heads"]):
                    m.append(h, K[t, h], V[t, h], ch * c["chunk"] + t)
        yield m, [(h, Q[qi, h], I.mha_seed(7, h), c["k_bits"], c["v_bits"])
                  for qi in range(8) for h in range(c["n_heads"])]


@pytest.mark.parametrize("name", ["config1", "config2", "config3", "config4", "wide512", "wide1000"])
def test_distance_to_exact_within_reference_spread(oracle, name):
    print(f"{name}: GPU and reference against exact attention", flush=True)
    cb = {b: oracle.codebook(b).astype(np.float64) for b in (2, 3, 4)}
    worst = [0.0, 0.0]
    rings = {}
    for m, items in cfg_heads(name):
        for h, q, seed, kb, vb in items:
            out, n = m.compute(h, q)
            assert n > 0, err()
            key = (id(m), h)
            if key not in rings:
                hd = m.heads[h]
                rings[key] = hd.read_slots(0, hd.info()["size"])
            p = m.heads[h].info()["padded"]
            x = X.attention(*rings[key], oracle.rademacher(p, seed), kb, vb, m.dim, q, cb)
            ne, ee = X.stats(out, x)
            worst = [max(worst[0], ne), max(worst[1], ee)]
        rings.clear()
    ref = ref_bar(f"{name}_vm0_h0")
    print(f"{name}: to exact, GPU norm-wise {worst[0]:.3e} elementwise {worst[1]:.3e}; "
          f"reference AVX2 {ref['avx2'][0]:.3e} / {ref['avx2'][1]:.3e}, "
          f"scalar {ref['scalar'][0]:.3e} / {ref['scalar'][1]:.3e}", flush=True)
    assert worst[0] <= ref["norm_max"], (worst, ref)
    assert worst[1] <= ref["elem_max"], (worst, ref)


def test_config4_batch_distance_to_exact(oracle):
    """Config 4's 64 queries in one compute_batch (the multi-query kernel):
    the first 8 against exact attention, beside the reference's figure."""
    print("config4 compute_batch against exact attention", flush=True)
    c = I.CONFIG4
    Q = I.config4_queries()
    cb = {b: oracle.codebook(b).astype(np.float64) for b in (2, 3, 4)}
    (m, _items), = list(cfg_heads("config4"))
    worst = [0.0, 0.0]
    for h in range(c["n_heads"]):
        qs = np.ascontiguousarray(Q[:, h])
        outs = np.zeros((c["n_queries"], c["dim"]), np.float32)
        assert L.adaptq_mha_compute_batch(m.m, h, _lib.fptr(qs), c["n_queries"],
                                          _lib.fptr(outs)) == c["cap"], err()
        hd = m.heads[h]
        ring = hd.read_slots(0, hd.info()["size"])
        D = oracle.rademacher(128, I.mha_seed(7, h))
        for qi in range(8):
            x = X.attention(*ring, D, c["k_bits"], c["v_bits"], c["dim"], Q[qi, h], cb)
            ne, ee = X.stats(outs[qi], x)
            worst = [max(worst[0], ne), max(worst[1], ee)]
    ref = ref_bar("config4_vm0_h0")
    print(f"config4 batch: to exact, GPU norm-wise {worst[0]:.3e} elementwise {worst[1]:.3e}; "
          f"reference AVX2 {ref['avx2'][0]:.3e} / {ref['avx2'][1]:.3e}, "
          f"scalar {ref['scalar'][0]:.3e} / {ref['scalar'][1]:.3e}", flush=True)
    assert worst[0] <= ref["norm_max"], (worst, ref)
    assert worst[1] <= ref["elem_max"], (worst, ref)
