"""Sparse-V under exact probability ties at the mass cut, on the CPU: the
oracle's decode (ties taken oldest first, the order the GPU kernels use)
against the reference build's (tests/golden/ties.npz, written from
oracle/_ref by tests/golden/make_golden.py).

The reference orders the selection with an unstable std::sort
(attention.cpp:451-453); which of several tokens with the same probability
it takes at the cut depends on the C++ standard library's sort, not on the
data.  So where a tie group straddles the cut the two decodes take different
members of it and their outputs differ; every other token, the number taken
and the weights of the tokens both take are the same.  Bar: per entry,
|y - y_ref| <= 2 m p* max_{t in T} |V^_t| + 1e-4 max|y_ref| (tie group T at the
cut, m = min(taken, left) of its members, p* their probability: see
tests/golden/exact64.tie_bound).  The cases cover every selection path's
length (2,048 / 5,000 / 20,000 / 70,000 tokens), with a zero query (every
probability tied) and with repeated keys.
"""
import os

import numpy as np
import pytest

from golden import exact64 as X
from golden import inputs as I

GOLD = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")


@pytest.mark.parametrize("n,kind", I.TIE_CASES)
def test_oracle_within_tie_bound(oracle, n, kind):
    c = I.TIE_SHAPE
    ref = np.load(os.path.join(GOLD, "ties.npz"))[f"out_{kind}{n}"]
    K, V, q, seed = I.tie_inputs(n, kind)
    h = oracle.head(c["dim"], c["k_bits"], c["v_bits"], n, seed, c["v_mass"], 0)
    for t in range(n):
        h.append(K[t], V[t], t)
    y, m_n = h.compute(q)
    assert m_n == n
    w = h.sparse_weights(q)
    kc, vc, ks, vs = h.read_slots(0, n)
    cb = {b: oracle.codebook(b).astype(np.float64) for b in (2, 3, 4)}
    bound, m, pstar = X.tie_bound(kc, vc, ks, vs, h.signs(), c["v_bits"], c["dim"], cb, w, kind)
    d = np.abs(y.astype(np.float64) - ref)
    tol = bound + 1e-4 * np.max(np.abs(ref))
    print(f"{kind}{n}: taken {int((w != 0).sum())}, straddling members m={m}, p*={pstar:.3e}; "
          f"max|y - y_ref| / max|y_ref| = {np.max(d) / np.max(np.abs(ref)):.2e}, "
          f"worst share of the bound {np.max(d / tol):.2f}")
    assert m > 0  # the case does tie at the cut
    assert np.all(d <= tol)
