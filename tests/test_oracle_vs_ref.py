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
