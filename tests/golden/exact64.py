"""float64 softmax attention over a dequantised ring: the exact value that a
head's fp32 decode approximates (test helper; no reference code).

A ring row of b-bit codes c with scale s stands for the vector
s * D * (H CB_b[c]) / p (H the p x p Sylvester-Hadamard matrix, D the head's
signs), which is what the reference's rotated-domain decode computes with
(attention.cpp:373-474 with fwht_inverse, fwht.cpp:106-134); fp32 rows (16
bits) stand for themselves.  Codes are MSB-first (quantizer.cpp:156-225).
"""
from __future__ import annotations

import numpy as np
from scipy.linalg import hadamard


def unpack_rows(codes, p, bits):
    """[n][p] codes of packed rows."""
    c = codes.astype(np.uint32)
    if bits == 4:
        return np.stack([c >> 4, c & 15], axis=2).reshape(len(c), p)
    if bits == 2:
        return np.stack([(c >> 6) & 3, (c >> 4) & 3, (c >> 2) & 3, c & 3],
                        axis=2).reshape(len(c), p)
    g = c.reshape(len(c), -1, 3)
    w = (g[:, :, 0] << 16) | (g[:, :, 1] << 8) | g[:, :, 2]
    return np.stack([(w >> (21 - 3 * k)) & 7 for k in range(8)], axis=2).reshape(len(c), p)


def dequant(codes, scales, D, bits, p, cb):
    if bits == 16:
        return codes.view(np.float32).reshape(len(scales), p).astype(np.float64)
    Y = cb[bits][unpack_rows(codes, p, bits)]
    return (Y @ hadamard(p).astype(np.float64)) * D[None, :] / p * \
        scales.astype(np.float64)[:, None]


def attention(kc, vc, ks, vs, D, kb, vb, dim, q, cb):
    """Exact softmax(K^ q / sqrt(dim)) V^ over the ring rows given (any slot
    order), first dim entries.  D: the head's signs (+-1, length p); cb:
    {bits: float64 codebook}."""
    p = len(D)
    D = np.asarray(D, np.float64)
    K = dequant(kc, ks, D, kb, p, cb)
    V = dequant(vc, vs, D, vb, p, cb)
    qp = np.zeros(p)
    qp[:dim] = np.asarray(q, np.float64)
    lg = K @ qp / np.sqrt(dim)
    w = np.exp(lg - lg.max())
    return ((w / w.sum()) @ V)[:dim]


def stats(y, r):
    """(norm-wise max|y - r| / max|r|, elementwise max |y - r| / |r| over
    entries with |r| >= 1e-3 max|r|)."""
    y = np.asarray(y, np.float64)
    r = np.asarray(r, np.float64)
    scale = float(np.max(np.abs(r)))
    d = np.abs(y - r)
    norm = float(np.max(d) / max(scale, 1e-30))
    big = np.abs(r) >= 1e-3 * scale if scale > 0 else np.zeros(r.shape, bool)
    elem = float(np.max(d[big] / np.abs(r[big]))) if big.any() else 0.0
    return norm, elem


def tie_bound(kc, vc, ks, vs, D, vb, dim, cb, weights, kind, groups=97):
    """Per-entry bound on how far two sparse-V decodes of one ring can differ
    when they order exactly tied probabilities differently (attention.cpp:
    448-473 sorts with an unstable std::sort).  Both take the same number of
    tokens (the mass walk adds the same sequence of values) and differ only in
    which members of the tie group T at the cut they take: at most
    m = min(taken, left) tokens of T each way, each contributing p* V^_t to
    the output (V^ the dequantised rows, scales included).  Returns
    (bound [dim], m, p*): |y - y'|_j <= 2 m p* max_{t in T} |V^_{t,j}|.
    weights: per-token weights (p_t vscale_t / sqrt(p), 0 if not taken) of
    one decode, ring order; kind "zero" (every probability tied) or "rep"
    (token t carries key t mod groups)."""
    p = len(D)
    V = dequant(vc, vs, np.asarray(D, np.float64), vb, p, cb)[:, :dim]
    n = len(weights)
    taken = weights != 0
    if kind == "zero":
        T = np.ones(n, bool)
    else:
        g = np.arange(n) % groups
        mixed = [k for k in range(groups) if taken[g == k].any() and (~taken[g == k]).any()]
        if not mixed:
            return np.zeros(dim), 0, 0.0
        assert len(mixed) == 1, mixed
        T = g == mixed[0]
    m = int(min((taken & T).sum(), (~taken & T).sum()))
    t0 = np.flatnonzero(taken & T)[0]
    pstar = float(weights[t0]) / (float(vs[t0]) / np.sqrt(p)) * (1 + 1e-6)
    return 2 * m * pstar * np.max(np.abs(V[T]), axis=0), m, pstar
