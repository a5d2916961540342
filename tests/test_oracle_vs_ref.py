"""The CPU oracle against the reference's own code on random cases.

Runs only where oracle/_ref was built (the development container, which has
/root/reference); elsewhere the golden fixtures stand in for it.  Codes and
scales must be identical; outputs within 1e-6 norm-wise relative error.
"""
import numpy as np
import pytest

from golden import inputs as I


@pytest.mark.parametrize("seed", range(6))
def test_codec_fuzz(oracle, ref, seed):
    rng = np.random.default_rng(seed)
    for _ in range(40):
        dim = int(rng.choice([1, 2, 3, 7, 31, 48, 64, 96, 100, 128, 200, 256, 513, 1024]))
        bits = int(rng.choice([2, 3, 4]))
        fam = I.FAMILIES[int(rng.integers(len(I.FAMILIES)))]
        with np.errstate(over="ignore"):
            x = I.codec_inputs(dim, fam)[int(rng.integers(8))] * np.float32(rng.lognormal(0, 3))
        s64 = int(rng.integers(0, 2**63))
        c_ref, s_ref = ref.quantize_into(x, s64, bits)
        D = oracle.rademacher(oracle.lib.orc_next_pow2(dim), s64)
        c, s, _ = oracle.quantize_vec(x, D, bits)
        assert c.tobytes() == c_ref.tobytes(), (dim, bits, fam)
        assert np.float32(s).tobytes() == np.float32(s_ref).tobytes(), (dim, bits, fam)


@pytest.mark.parametrize("case", range(8))
def test_head_fuzz(oracle, ref, case):
    rng = np.random.default_rng(100 + case)
    dim = int(rng.choice([32, 64, 96, 128]))
    kb = int(rng.choice([2, 3, 4, 16]))
    vb = int(rng.choice([2, 3, 4, 16]))
    if kb != 16 and vb == 16:
        vb = 2  # the reference's scalar path dereferences a null V codebook here
    cap = int(rng.integers(1, 700))
    n = int(rng.integers(1, 900))
    vm = float(rng.choice([0.0, 0.5, 0.95]))
    hyb = int(rng.choice([0, 16, 512]))
    seed = int(rng.integers(0, 2**63))
    o = oracle.head(dim, kb, vb, cap, seed, vm, hyb)
    r = ref.head(dim, kb, vb, cap, seed, vm, hyb)
    K = rng.standard_normal((n, dim)).astype(np.float32)
    V = rng.standard_normal((n, dim)).astype(np.float32)
    for t in range(n):
        o.append(K[t], V[t], t)
        r.append(K[t], V[t], t)
    oi, ri = o.info(), r.info()
    assert (oi["head"], oi["size"]) == (ri["head"], ri["size"])
    a, b = o.read_slots(0, oi["size"]), r.read_slots(0, ri["size"])
    for x, y in zip(a, b):
        assert x.tobytes() == y.tobytes()
    for _ in range(2):
        q = (2 * rng.standard_normal(dim)).astype(np.float32)
        yo, no = o.compute(q)
        yr, nr = r.compute(q)
        assert no == nr
        assert np.max(np.abs(yo - yr)) <= 1e-6 * max(float(np.max(np.abs(yr))), 1e-30)


@pytest.mark.parametrize("case", range(6))
def test_sparse_selection_reproduces_reference(oracle, ref, case):
    """The oracle's sparse-V selection weights (the checker of the GPU's
    selection) rebuild the reference build's own output: the V rows of the
    selected tokens, weighted as reported and summed in float64, then the
    inverse FWHT and signs, give the reference's compute() to 1e-5, while
    every weight is (p_t * vscale_t) / sqrt(p) of a token the reference's
    softmax ranks at or above the cut."""
    rng = np.random.default_rng(300 + case)
    dim = int(rng.choice([64, 128]))
    kb, vb = int(rng.choice([2, 3, 4])), int(rng.choice([2, 3, 4]))
    n = int(rng.integers(200, 3000))
    vm = float(rng.choice([0.5, 0.95, 0.999]))
    seed = int(rng.integers(0, 2**63))
    o = oracle.head(dim, kb, vb, n, seed, vm, 0)
    r = ref.head(dim, kb, vb, n, seed, vm, 0)
    K = rng.standard_normal((n, dim)).astype(np.float32)
    V = rng.standard_normal((n, dim)).astype(np.float32)
    for t in range(n):
        o.append(K[t], V[t], t)
        r.append(K[t], V[t], t)
    p = o.info()["padded"]
    kc, vc, ks, vs = o.read_slots(0, n)  # no wrap: slot t holds token t
    cbk = oracle.codebook(kb).astype(np.float64)
    cbv = oracle.codebook(vb).astype(np.float64)
    kcodes = np.stack([oracle.unpack(kc[t], p, kb) for t in range(n)]).astype(np.int64)
    codes = np.stack([oracle.unpack(vc[t], p, vb) for t in range(n)]).astype(np.int64)
    D = o.signs().astype(np.float64)
    H = np.array([[(-1) ** bin(i & j).count("1") for j in range(p)] for i in range(p)], np.float64)
    for _ in range(2):
        q = (2 * rng.standard_normal(dim)).astype(np.float32)
        w = o.sparse_weights(q).astype(np.float64)
        yr, _ = r.compute(q)
        acc = (w[:, None] * cbv[codes]).sum(axis=0)
        y = (H @ acc / np.sqrt(p) * D)[:dim]
        assert np.max(np.abs(y - yr)) <= 1e-5 * np.max(np.abs(yr)), (case, vm)
        # float64 probabilities from the closed form (logit_t = kscale_t *
        # (H (D q)) . CB_K[codes_t] / (sqrt(dim) p)): the selection is a
        # prefix of the descending order, up to float32 rounding
        qp = np.zeros(p)
        qp[:dim] = q
        lg = ks.astype(np.float64) * (cbk[kcodes] @ (H @ (D * qp))) / (np.sqrt(dim) * p)
        pr = np.exp(lg - lg.max())
        pr /= pr.sum()
        sel = np.flatnonzero(w)
        left = np.setdiff1d(np.arange(n), sel)
        assert sel.size > 0
        if left.size:
            assert pr[sel].min() >= pr[left].max() * (1 - 1e-4), (case, vm)
        # and a selected token's weight is its probability times vscale / sqrt(p)
        np.testing.assert_allclose(w[sel], pr[sel] * vs[sel] / np.sqrt(p), rtol=1e-4)
