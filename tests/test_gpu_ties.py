"""Sparse-V under exact probability ties at the mass cut, on the GPU, against
the reference build's outputs (tests/golden/ties.npz) and the oracle.

The library takes tied tokens oldest first at the cut, as the oracle does
(same per-token weights, bit for bit); the reference's unstable std::sort
(attention.cpp:451-453) takes members of the tie group in an order set by
its C++ standard library.  Bar against the reference, per entry:
|y - y_ref| <= 2 m p* max_{t in T} |V^_t| + 1e-4 max|y_ref| (tie group T at the
cut, m = min(taken, left) of its members, p* their probability;
tests/golden/exact64.tie_bound); against the oracle: weights bit-identical,
outputs within 1e-4 norm-wise.  One case per selection path's length.
"""
import os

import numpy as np
import pytest

from adaptq_amd import _lib
from golden import exact64 as X
from golden import inputs as I
from gpu_head import GpuHead, err, rel_err

pytestmark = pytest.mark.gpu
L = _lib.lib
GOLD = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")


@pytest.mark.parametrize("n,kind", I.TIE_CASES)
def test_ties_at_the_cut(oracle, n, kind):
    print(f"ties {kind}{n}", flush=True)
    c = I.TIE_SHAPE
    ref = np.load(os.path.join(GOLD, "ties.npz"))[f"out_{kind}{n}"]
    K, V, q, seed = I.tie_inputs(n, kind)
    g = GpuHead(c["dim"], c["k_bits"], c["v_bits"], n, seed, c["v_mass"], 0)
    o = oracle.head(c["dim"], c["k_bits"], c["v_bits"], n, seed, c["v_mass"], 0)
    for t in range(n):
        g.append(K[t], V[t], t)
        o.append(K[t], V[t], t)
    y = np.zeros(c["dim"], np.float32)
    assert L.adaptq_compute(g.h, _lib.fptr(q), _lib.fptr(y)) == n, err()
    w = np.full(n, np.nan, np.float32)
    assert L.adaptq_sparse_weights(g.h, _lib.fptr(q), _lib.fptr(w)) == n, err()
    wo = o.sparse_weights(q)
    assert w.tobytes() == wo.tobytes()
    assert rel_err(y, o.compute(q)[0]) <= 1e-4
    kc, vc, ks, vs = g.read_slots(0, n)
    cb = {b: oracle.codebook(b).astype(np.float64) for b in (2, 3, 4)}
    bound, m, pstar = X.tie_bound(kc, vc, ks, vs, o.signs(), c["v_bits"], c["dim"], cb, w, kind)
    d = np.abs(y.astype(np.float64) - ref)
    tol = bound + 1e-4 * np.max(np.abs(ref))
    print(f"{kind}{n}: m={m}, max|y - y_ref| / max|y_ref| = {np.max(d) / np.max(np.abs(ref)):.2e},"
          f" worst share of the bound {np.max(d / tol):.2f}", flush=True)
    assert m > 0
    assert np.all(d <= tol)
