"""The Python Engine (adaptq_amd.core.Engine over the pybind11 MHAContext)
with the reference's own Engine-level contracts (tests/test_la_policy.py,
tests/test_asymmetric_engine.py): shapes, cosine floors against the dense
K16/V16 engine, kv_bytes relations, reset.  Outputs are also held to the
oracle at 1e-4."""
import numpy as np
import pytest

from golden import inputs as I
from gpu_head import rel_err

pytestmark = pytest.mark.gpu


def Engine(*a, **k):
    from adaptq_amd.core import Engine as E
    return E(*a, **k)


@pytest.mark.parametrize("k_bits,v_bits,min_cos", [
    (4, 4, 0.90), (4, 2, 0.85), (3, 2, 0.75), (16, 2, 0.85), (16, 16, 0.999),
])
def test_cosine_vs_dense(k_bits, v_bits, min_cos):
    """test_la_policy.py:193-230."""
    print(f"engine cosine k{k_bits}v{v_bits}", flush=True)
    dim, heads, seq_len = 64, 4, 32
    rng = np.random.default_rng(7)
    ks = [rng.standard_normal((heads, dim)).astype(np.float32) for _ in range(seq_len)]
    vs = [rng.standard_normal((heads, dim)).astype(np.float32) for _ in range(seq_len)]
    q = rng.standard_normal((heads, dim)).astype(np.float32)

    def run(kb, vb):
        eng = Engine(dim=dim, heads=heads, k_bits=kb, v_bits=vb, capacity=256, seed=42)
        for k, v in zip(ks, vs):
            eng.append(k, v)
        return eng.compute(q)

    dense, out = run(16, 16), run(k_bits, v_bits)
    sims = [float(dense[h] @ out[h] / (np.linalg.norm(dense[h]) * np.linalg.norm(out[h])))
            for h in range(heads)]
    assert np.mean(sims) >= min_cos


def test_engine_matches_oracle(oracle):
    """Engine defaults (v_mass 0.95, hybrid 512) beyond the hybrid threshold:
    the sparse-V branch, head seeds base ^ i*0xDEADBEEFCAFE."""
    print("engine vs oracle", flush=True)
    dim, heads, n = 64, 3, 700
    eng = Engine(dim=dim, heads=heads, k_bits=4, v_bits=2, capacity=1024, seed=42)
    refs = [oracle.head(dim, 4, 2, 1024, I.mha_seed(42, h), 0.95, 512) for h in range(heads)]
    rng = np.random.default_rng(1)
    for t in range(n):
        k = rng.standard_normal((heads, dim)).astype(np.float32)
        v = rng.standard_normal((heads, dim)).astype(np.float32)
        eng.append(k, v)
        for h in range(heads):
            refs[h].append(k[h], v[h], t)
        if t in (100, n - 1):  # hybrid branch, then sparse-V
            q = rng.standard_normal((heads, dim)).astype(np.float32)
            out = eng.compute(q)
            for h in range(heads):
                assert rel_err(out[h], refs[h].compute(q[h])[0]) <= 1e-4


def test_kv_bytes_relations():
    """test_la_policy.py:159-185."""
    def nbytes(kb, vb, seq):
        eng = Engine(dim=64, heads=4, k_bits=kb, v_bits=vb, capacity=256)
        rng = np.random.default_rng(0)
        for _ in range(seq):
            eng.append(rng.standard_normal((4, 64)).astype(np.float32),
                       rng.standard_normal((4, 64)).astype(np.float32))
        return eng.kv_bytes

    assert nbytes(16, 16, 128) / nbytes(4, 2, 128) >= 2.0
    assert nbytes(4, 2, 128) == 2 * nbytes(4, 2, 64) == 4 * 128 * (32 + 16)


def test_reset_and_shapes():
    """test_la_policy.py:243-267."""
    eng = Engine(dim=64, heads=2, k_bits=4, v_bits=2, capacity=32, seed=42)
    rng = np.random.default_rng(0)
    for _ in range(10):
        eng.append(rng.standard_normal((2, 64)).astype(np.float32),
                   rng.standard_normal((2, 64)).astype(np.float32))
    assert eng.kv_bytes > 0 and eng.pos == 10
    eng.reset()
    assert eng.pos == 0 and eng.kv_bytes == 0
    assert np.allclose(eng.compute(rng.standard_normal((2, 64)).astype(np.float32)), 0.0)
    with pytest.raises(ValueError):
        eng.append(np.zeros((3, 64), np.float32), np.zeros((3, 64), np.float32))
    with pytest.raises(ValueError):
        eng.compute(np.zeros((2, 32), np.float32))


def test_pybind_compute_batch_matches_single():
    from adaptq_amd import adaptq_py
    ctx = adaptq_py.MHAContext(2, 128, 4, 2, 512, 9, 0.0, 0)
    rng = np.random.default_rng(4)
    for t in range(300):
        for h in range(2):
            ctx.append(h, rng.standard_normal(128).astype(np.float32),
                       rng.standard_normal(128).astype(np.float32), t)
    qs = rng.standard_normal((5, 128)).astype(np.float32)
    outs = np.asarray(ctx.compute_batch(1, qs)).reshape(5, 128)
    for i in range(5):
        assert rel_err(outs[i], ctx.compute(1, qs[i])) <= 1e-6
    assert ctx.n_heads == 2 and ctx.head_dim == 128
