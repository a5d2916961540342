"""The CPU oracle pinned by mathematics, independently of the golden fixtures.

Each check is chosen so that a plausible slip in the oracle (a dropped term,
a swapped butterfly sign, a transposed index, a wrong scale) fails it:

* FWHT: small-integer inputs keep every butterfly exact in fp32, so the
  forward transform must equal the exact integer Sylvester-Hadamard product
  rounded once by the fp32 scale; round trip and linearity.
* Rademacher signs: the xorshift64 closed form of reference core/fwht.cpp:21-27.
* Quantiser: monotone, all 2^b levels reachable, NaN -> the centroid below
  zero, and every decision threshold is the fp32 midpoint of neighbouring
  centroids (codebook.cpp:67-100), located to the ulp in the golden sweep.
* Packing: the closed-form MSB-first layouts of quantizer.cpp:156-209.
* kv_bytes: the closed forms of the reference README (README.md:152-158).
* Attention: float64 softmax attention over the closed-form dequantised ring
  (x_hat = scale * D . (H c) / p), for the dense, K16, V16 and hybrid paths.
"""
import os

import numpy as np
import pytest
from scipy.linalg import hadamard

GOLD = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")


def _scale(p):
    return np.float32(np.float32(1.0) / np.sqrt(np.float32(p)))


# ------------------------------------------------------------------ FWHT
@pytest.mark.parametrize("p", [2, 4, 8, 16, 64, 128, 256, 1024])
def test_fwht_exact_small_integers(oracle, p):
    rng = np.random.default_rng(p)
    H = hadamard(p).astype(np.int64)
    for seed in range(3):
        D = oracle.rademacher(p, 77 + seed)
        x = rng.integers(-50, 51, p).astype(np.float32)
        want_fwd = (H @ (D.astype(np.int64) * x.astype(np.int64))).astype(np.float32) * _scale(p)
        assert np.array_equal(oracle.fwht_forward(x, D), want_fwd)
        want_inv = D.astype(np.float32) * ((H @ x.astype(np.int64)).astype(np.float32) * _scale(p))
        assert np.array_equal(oracle.fwht_inverse(x, D), want_inv)


@pytest.mark.parametrize("p", [64, 128, 512])
def test_fwht_round_trip_and_linearity(oracle, p):
    rng = np.random.default_rng(3)
    D = oracle.rademacher(p, 5)
    x = rng.standard_normal(p).astype(np.float32)
    y = rng.standard_normal(p).astype(np.float32)
    assert np.max(np.abs(oracle.fwht_inverse(oracle.fwht_forward(x, D), D) - x)) < 1e-5
    lhs = oracle.fwht_forward(2 * x + 3 * y, D).astype(np.float64)
    rhs = 2 * oracle.fwht_forward(x, D).astype(np.float64) + 3 * oracle.fwht_forward(y, D)
    assert np.max(np.abs(lhs - rhs)) < 1e-4
    # orthonormal: norms preserved
    assert abs(np.linalg.norm(oracle.fwht_forward(x, D)) / np.linalg.norm(x) - 1) < 1e-5


# ------------------------------------------------------------ Rademacher
def _xorshift_signs(n, seed):
    s = seed if seed != 0 else 0xDEADBEEFCAFE1234
    out = np.empty(n, np.int8)
    m = (1 << 64) - 1
    for i in range(n):
        s ^= (s << 13) & m
        s ^= s >> 7
        s ^= (s << 17) & m
        out[i] = 1 if s & 1 else -1
    return out


@pytest.mark.parametrize("seed", [0, 1, 42, 7 ^ 0xDEADBEEFCAFE, (1 << 64) - 1])
def test_rademacher_closed_form(oracle, seed):
    assert np.array_equal(oracle.rademacher(256, seed), _xorshift_signs(256, seed))


# ------------------------------------------------------------- quantiser
@pytest.mark.parametrize("bits", [2, 3, 4])
def test_quantizer_structure(oracle, bits):
    g = np.load(os.path.join(GOLD, "quantize_fast.npz"))
    vals = np.sort(g["vals"][:16001])
    idx = np.array([oracle.quantize_fast(float(v), bits) for v in vals])
    assert np.all(np.diff(idx) >= 0)
    assert set(idx) == set(range(1 << bits))
    assert oracle.quantize_fast(float("nan"), bits) == (1 << (bits - 1)) - 1
    assert oracle.quantize_fast(-0.0, bits) == oracle.quantize_fast(0.0, bits) == 1 << (bits - 1)
    # thresholds: the first float of each level is the fp32 midpoint of the
    # neighbouring centroids (the middle threshold is exactly 0)
    cb = oracle.codebook(bits)
    assert np.all(np.diff(cb) > 0) and np.allclose(cb, -cb[::-1])
    firsts = g[f"edge_vals{bits}"][1::3]  # (below, at, above) triples
    mids = [(np.float32(0.0) if k == (1 << (bits - 1)) - 1 else (cb[k] + cb[k + 1]) * np.float32(0.5))
            for k in range((1 << bits) - 1)]
    assert np.array_equal(firsts, np.array(mids, np.float32))


def _pack_closed_form(idx, bits):
    if bits == 4:
        return (idx[0::2] << 4 | idx[1::2]).astype(np.uint8)
    if bits == 2:
        return (idx[0::4] << 6 | idx[1::4] << 4 | idx[2::4] << 2 | idx[3::4]).astype(np.uint8)
    out = []
    for g in range(len(idx) // 8):
        w = 0
        for k in range(8):
            w |= int(idx[8 * g + k]) << (21 - 3 * k)
        out += [(w >> 16) & 255, (w >> 8) & 255, w & 255]
    return np.array(out, np.uint8)


@pytest.mark.parametrize("bits", [2, 3, 4])
@pytest.mark.parametrize("p", [8, 64, 128, 1024])
def test_pack_layout(oracle, bits, p):
    rng = np.random.default_rng(p + bits)
    idx = rng.integers(0, 1 << bits, p).astype(np.uint8)
    packed = oracle.pack(idx, bits)
    assert np.array_equal(packed, _pack_closed_form(idx.astype(np.int64), bits))
    assert np.array_equal(oracle.unpack(packed, p, bits), idx)


def test_kv_bytes_closed_form(oracle):
    """README.md:152-158: dim 64, 14 heads, context 512."""
    rng = np.random.default_rng(0)
    k = rng.standard_normal((512, 64)).astype(np.float32)
    for (kb, vb), want in [((16, 16), 3670016), ((4, 2), 344064), ((3, 2), 286720)]:
        h = oracle.head(64, kb, vb, 512, 1)
        for t in range(512):
            h.append(k[t], k[t], t)
        assert 14 * h.kv_bytes() == want


# ------------------------------------------------------------- attention
def _dequant(codes, scales, D, bits, p, oracle):
    if bits == 16:
        return codes.view(np.float32).reshape(len(scales), p).astype(np.float64)
    cb = oracle.codebook(bits).astype(np.float64)
    H = hadamard(p).astype(np.float64)
    rows = []
    for c, s in zip(codes, scales):
        y = cb[oracle.unpack(c, p, bits)]
        rows.append(float(s) * D * (H @ y) / p)
    return np.array(rows)


def _attention64(head, oracle, q, dim, kb, vb):
    inf = head.info()
    p = inf["padded"]
    kc, vc, ks, vs = head.read_slots(0, inf["size"])
    D = head.signs().astype(np.float64)
    K = _dequant(kc, ks, D, kb, p, oracle)
    V = _dequant(vc, vs, D, vb, p, oracle)
    qp = np.zeros(p)
    qp[:dim] = q
    logits = K @ qp / np.sqrt(dim)
    w = np.exp(logits - logits.max())
    w /= w.sum()
    return (w @ V)[:dim]


@pytest.mark.parametrize("dim,kb,vb", [
    (64, 4, 2), (128, 4, 2), (64, 3, 2), (128, 4, 4), (64, 2, 3), (96, 4, 2), (48, 3, 4),
    (64, 16, 2), (64, 4, 16), (64, 16, 16),
])
def test_attention_float64(oracle, dim, kb, vb):
    rng = np.random.default_rng(dim * 10 + kb + vb)
    n, cap = 300, 256  # wraps: slots hold tokens 44..299
    h = oracle.head(dim, kb, vb, cap, 1234)
    K = rng.standard_normal((n, dim)).astype(np.float32)
    V = rng.standard_normal((n, dim)).astype(np.float32)
    for t in range(n):
        h.append(K[t], V[t], t)
    for _ in range(3):
        q = (2 * rng.standard_normal(dim)).astype(np.float32)
        out, m = h.compute(q)
        assert m == cap
        want = _attention64(h, oracle, q.astype(np.float64), dim, kb, vb)
        assert np.max(np.abs(out - want)) / np.max(np.abs(want)) < 2e-5


def test_hybrid_is_exact_attention(oracle):
    rng = np.random.default_rng(9)
    dim, n = 64, 100
    h = oracle.head(dim, 4, 2, 512, 3, 0.95, 128)
    K = rng.standard_normal((n, dim)).astype(np.float32)
    V = rng.standard_normal((n, dim)).astype(np.float32)
    for t in range(n):
        h.append(K[t], V[t], t)
    q = rng.standard_normal(dim).astype(np.float32)
    out, _ = h.compute(q)
    logits = K.astype(np.float64) @ q / np.sqrt(dim)
    w = np.exp(logits - logits.max())
    want = (w / w.sum()) @ V.astype(np.float64)
    assert np.max(np.abs(out - want)) / np.max(np.abs(want)) < 2e-6


def test_empty_and_reset(oracle):
    h = oracle.head(64, 4, 2, 16, 1)
    out, n = h.compute(np.ones(64, np.float32))
    assert n == 0 and not out.any()
    for t in range(20):
        h.append(np.ones(64, np.float32), np.ones(64, np.float32), t)
    assert h.info()["size"] == 16 and h.info()["head"] == 4
    h.reset()
    assert h.info()["size"] == 0 and h.kv_bytes() == 0
