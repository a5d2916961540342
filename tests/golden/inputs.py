"""Deterministic inputs of the BASELINE configurations and of the codec fixtures.

Shared by make_golden.py (which runs the reference build to write the expected
values) and by the tests (which regenerate the same inputs and compare).
Every generator is a pure function of its arguments: numpy's PCG64 stream is
platform independent, so the GPU box regenerates bit-identical inputs.

Configurations (BASELINE.json "configs", numbered 1-5 there):
  1  one MHA, 4 heads, d64, K4/V2, capacity 2048, seed 42, 2048 N(0,1) tokens
  2  24 layers x 14 heads, d64, context 512, layer 0 K16/V2, layers 1-23
     K4/V2, seed 42^layer, two outlier channels (3, 17) x20 in K, V and q
  3  22 layers x 4 heads, d64, layer 0 K16/V2, layers 1-21 K3/V2, Student-t(4)
     scaled to unit variance, 1024-token bulk append then 256 steps of
     (append one token, compute)
  4  8 heads, d128, K4/V4, capacity 32768, seed 7, 40000 appended tokens
     (7232 evictions), 64 queries
"""
from __future__ import annotations

import numpy as np

MHA_SEED_MULT = 0xDEADBEEFCAFE
U64 = (1 << 64) - 1


def mha_seed(base: int, i: int) -> int:
    """Seed of head i of an MHA (reference core/adaptq_c_api.cpp:160)."""
    return (base ^ (i * MHA_SEED_MULT)) & U64


def _normal(rng, shape):
    return rng.standard_normal(shape, dtype=np.float32)


def _student_t(rng, shape):
    # Student-t(4) has variance 2: divide by sqrt(2) for unit variance
    return (rng.standard_t(4, shape) / np.sqrt(2.0)).astype(np.float32)


# ---------------------------------------------------------------- config 1
CONFIG1 = dict(n_heads=4, dim=64, k_bits=4, v_bits=2, cap=2048, base_seed=42, n=2048)


def config1_inputs():
    rng = np.random.default_rng(42)
    K = _normal(rng, (2048, 4, 64))
    V = _normal(rng, (2048, 4, 64))
    q = _normal(rng, (4, 64))
    return K, V, q


# ---------------------------------------------------------------- config 2
CONFIG2 = dict(n_layers=24, n_heads=14, dim=64, cap=512, n=512, outliers=(3, 17))


def config2_layer(layer: int):
    """(k_bits, v_bits, base_seed, K[512,14,64], V, q[14,64]) of one layer."""
    rng = np.random.default_rng([2, layer])
    K = _normal(rng, (512, 14, 64))
    V = _normal(rng, (512, 14, 64))
    q = _normal(rng, (14, 64))
    for a in (K, V, q):
        a[..., list(CONFIG2["outliers"])] *= np.float32(20.0)
    kb = 16 if layer == 0 else 4
    return kb, 2, 42 ^ layer, K, V, q


# ---------------------------------------------------------------- config 3
CONFIG3 = dict(n_layers=22, n_heads=4, dim=64, cap=1280, bulk=1024, steps=256)


def config3_layer(layer: int):
    """(k_bits, v_bits, base_seed, K[1280,4,64], V, Q[256,4,64]) of one layer.

    Tokens 0..1023 are the bulk append; token 1024+s is appended at step s,
    before the step's query Q[s] is computed."""
    rng = np.random.default_rng([3, layer])
    K = _student_t(rng, (1280, 4, 64))
    V = _student_t(rng, (1280, 4, 64))
    Q = _student_t(rng, (256, 4, 64))
    kb = 16 if layer == 0 else 3
    return kb, 2, 42 ^ layer, K, V, Q


# ---------------------------------------------------------------- config 4
CONFIG4 = dict(n_heads=8, dim=128, k_bits=4, v_bits=4, cap=32768, base_seed=7, n=40000,
               n_queries=64, chunk=4096)


def config4_chunk(c: int):
    """Tokens [c*4096, min((c+1)*4096, 40000)) as (K[t,8,128], V[t,8,128])."""
    lo = c * CONFIG4["chunk"]
    hi = min(lo + CONFIG4["chunk"], CONFIG4["n"])
    rng = np.random.default_rng([4, c])
    K = _normal(rng, (hi - lo, 8, 128))
    V = _normal(rng, (hi - lo, 8, 128))
    return K, V


def config4_queries():
    rng = np.random.default_rng([4, 1000])
    return _normal(rng, (64, 8, 128))


# Padded 512 and 1024 (the library's wide decode kernel): N(0,1) rings, the
# second wrapped (1,300 tokens into 1,024 slots).
WIDE = {
    "wide512": dict(n_heads=4, dim=512, k_bits=4, v_bits=2, cap=2048, base_seed=51, n=2048),
    "wide1000": dict(n_heads=2, dim=1000, k_bits=3, v_bits=4, cap=1024, base_seed=52, n=1300),
}


def wide_inputs(name: str):
    """(K[n,h,dim], V[n,h,dim], q[h,dim]) of a WIDE case."""
    c = WIDE[name]
    rng = np.random.default_rng([5, c["dim"]])
    K = _normal(rng, (c["n"], c["n_heads"], c["dim"]))
    V = _normal(rng, (c["n"], c["n_heads"], c["dim"]))
    q = _normal(rng, (c["n_heads"], c["dim"]))
    return K, V, q


# ---------------------------------------------------------- codec families
FAMILIES = ["normal", "student_t", "outliers", "zeros", "huge", "tiny", "nan", "inf",
            "negzero", "mixed"]


def codec_inputs(dim: int, family: str, n: int = 8) -> np.ndarray:
    """n vectors of length dim for the quantiser fixtures."""
    rng = np.random.default_rng([5, dim, FAMILIES.index(family)])
    x = _normal(rng, (n, dim))
    if family == "student_t":
        x = _student_t(rng, (n, dim))
    elif family == "outliers":
        x[:, [3 % dim, 17 % dim]] *= np.float32(20.0)
    elif family == "zeros":
        x[:] = 0.0
    elif family == "huge":
        x = np.sign(x).astype(np.float32) * np.float32(1e38)
    elif family == "tiny":
        x = (np.sign(x) * np.float32(1e-38)).astype(np.float32)
        x[:, ::3] = np.float32(1e-45)  # smallest subnormal
    elif family == "nan":
        x[:, ::7] = np.nan
    elif family == "inf":
        x[:, 5 % dim] = np.inf
    elif family == "negzero":
        x[:] = -0.0
        x[:, 1 % dim] = np.float32(1e-3)
    elif family == "mixed" and n >= 4:
        x[0] = 0.0
        x[1, :] = np.float32(1e7)
        x[2] *= np.float32(1e-20)
        x[3, ::2] = -0.0
    return np.ascontiguousarray(x, np.float32)


# ------------------------------------------------- sparse-V ties at the cut
# Rings whose probabilities tie exactly at the mass cut, one per selection
# path (fused <= 3,072 tokens, in-LDS sort <= 8,192, per-item radix sort
# above, with superblock sums past 65,536): "zero" decodes a zero query (every
# logit 0, every probability 1/n); "rep" repeats 97 key vectors (equal codes
# and scales, so equal probabilities within each group of keys).
TIE_CASES = [(n, kind) for n in (2048, 5000, 20000, 70000) for kind in ("zero", "rep")]
TIE_SHAPE = dict(dim=64, k_bits=4, v_bits=2, v_mass=0.95)


def tie_inputs(n: int, kind: str):
    """(K [n][64], V [n][64], q [64], seed of the head's signs)."""
    rng = np.random.default_rng([6, n, ("zero", "rep").index(kind)])
    dim = TIE_SHAPE["dim"]
    if kind == "zero":
        K = _normal(rng, (n, dim))
    else:
        K = _normal(rng, (97, dim))[np.arange(n) % 97]
    V = _normal(rng, (n, dim))
    q = np.zeros(dim, np.float32) if kind == "zero" else _normal(rng, (dim,))
    return np.ascontiguousarray(K), V, q, 1000 + n
