"""Sparse-V selection compared exactly with the oracle (attention.cpp:448-473).

The output bound (1e-4 norm-wise) cannot see a token that one side takes at
the mass cut and the other leaves out: its weight is below the cut mass.  Here
the library's per-token selection weights (adaptq_sparse_weights: (p_t *
vscale_t) / sqrt(p) for selected tokens, 0 otherwise, in ring order) are
compared with the oracle's, token by token: the selected set must be the same,
and the weights the same bits.  The cases cover every selection code path:
the fused one-block kernel (rings up to 3,072 tokens at padded 64/128), the
in-LDS radix sort of the select kernel (up to 8,192 tokens), the per-item
multi-block radix sort plus cut kernel above that (up to 65,536 tokens: a
wrapped 32,768-token ring, exact ties across sort blocks, every probability
equal) and, above it, the same sort with superblock sums (a plain and a
wrapped ring of 70,000 tokens, a wrapped ring of 300,000), at v_mass 0.95 /
0.999 / 0.9999 and with peaked queries.
"""
import numpy as np
import pytest

from adaptq_amd import _lib
from golden import inputs as I
from gpu_head import GpuHead, err

pytestmark = pytest.mark.gpu
L = _lib.lib


def gpu_weights(head, q, n):
    q = np.ascontiguousarray(q, np.float32)
    w = np.full(n, np.nan, np.float32)
    got = L.adaptq_sparse_weights(head.h, _lib.fptr(q), _lib.fptr(w))
    assert got == n, (got, err())
    return w


def check_selection(g, o, q, label):
    n = o.info()["size"]
    wg = gpu_weights(g, q, n)
    wo = o.sparse_weights(q)
    sel_g, sel_o = wg != 0, wo != 0
    only_g = np.flatnonzero(sel_g & ~sel_o)
    only_o = np.flatnonzero(sel_o & ~sel_g)
    print(f"{label}: n={n} selected gpu={int(sel_g.sum())} oracle={int(sel_o.sum())}", flush=True)
    assert only_g.size == 0 and only_o.size == 0, (label, only_g[:8], only_o[:8])
    diff = np.flatnonzero(wg.view(np.uint32) != wo.view(np.uint32))
    if diff.size:
        ulps = np.abs(wg.view(np.int32)[diff].astype(np.int64) - wo.view(np.int32)[diff])
        print(f"{label}: {diff.size} weights differ, at most {int(ulps.max())} ulp", flush=True)
    assert diff.size == 0, (label, diff[:8], wg[diff[:4]], wo[diff[:4]])


def fill(dim, kb, vb, cap, seed, n_tok, v_mass, oracle, rng, family="normal"):
    g = GpuHead(dim, kb, vb, cap, seed, v_mass, 0)
    o = oracle.head(dim, kb, vb, cap, seed, v_mass, 0)
    if family == "normal":
        kv = rng.standard_normal((n_tok, 2, dim)).astype(np.float32)
    else:  # Student-t(4) scaled to unit variance
        kv = (rng.standard_t(4, size=(n_tok, 2, dim)) / np.sqrt(2.0)).astype(np.float32)
    for t in range(n_tok):
        g.append(kv[t, 0], kv[t, 1], t)
        o.append(kv[t, 0], kv[t, 1], t)
    return g, o


def test_config1_selection(oracle):
    """Config 1 under Engine defaults (4 heads d64 K4/V2, 2,048 tokens): the
    fused kernel at padded 64."""
    c = I.CONFIG1
    K, V, q = I.config1_inputs()
    for h in range(c["n_heads"]):
        seed = I.mha_seed(42, h)
        g = GpuHead(c["dim"], c["k_bits"], c["v_bits"], c["cap"], seed, 0.95, 0)
        o = oracle.head(c["dim"], c["k_bits"], c["v_bits"], c["cap"], seed, 0.95, 0)
        for t in range(c["n"]):
            g.append(K[t, h], V[t, h], t)
            o.append(K[t, h], V[t, h], t)
        check_selection(g, o, q[h], f"config1 head {h}")


@pytest.mark.parametrize("dim,kb,vb,n_tok,v_mass,peak", [
    (64, 4, 2, 1000, 0.95, 1.0),      # fused, one token per thread
    (128, 4, 4, 2500, 0.999, 1.0),    # fused after the logits kernel (padded 128)
    (64, 3, 2, 3072, 0.9999, 1.0),    # fused at its size limit, 3-bit K
    (64, 4, 2, 5000, 0.95, 6.0),      # in-LDS sort, peaked query
    (128, 2, 3, 8192, 0.999, 1.0),    # in-LDS sort at its size limit
    (64, 4, 4, 9000, 0.95, 1.0),      # item sort, 5 blocks a pass
    (128, 4, 2, 12000, 0.9999, 3.0),  # item sort, peaked
    (64, 2, 2, 65536, 0.95, 1.0),     # item sort at its size limit
    (32, 4, 2, 600, 0.95, 1.0),       # padded 32: K rows in XOR order, codes read a byte at a time
    (200, 4, 3, 700, 0.95, 3.0),      # padded 256: 16-byte row loads in the logits kernel
    (512, 3, 4, 1200, 0.95, 1.0),     # padded 512, 3-bit K: 48-byte chunks
    (1000, 2, 2, 900, 0.99, 1.0),     # padded 1024, 2-bit K
])
def test_selection_paths(oracle, dim, kb, vb, n_tok, v_mass, peak):
    rng = np.random.default_rng(1000 + n_tok)
    g, o = fill(dim, kb, vb, n_tok, 17, n_tok, v_mass, oracle, rng)
    for j in range(3):
        q = (rng.standard_normal(dim) * peak).astype(np.float32)
        check_selection(g, o, q, f"d{dim} K{kb}V{vb} n={n_tok} v_mass={v_mass} q{j}")


def test_wrapped_long_ring_selection(oracle):
    """Config 4's ring under Engine defaults (d128 K4/V4, capacity 32,768,
    40,000 tokens: 7,232 evictions): the per-item radix sort over a wrapped
    ring."""
    rng = np.random.default_rng(7)
    g, o = fill(128, 4, 4, 32768, 7, 40000, 0.95, oracle, rng)
    assert g.info()["head"] == o.info()["head"] == 7232
    for j in range(2):
        q = rng.standard_normal(128).astype(np.float32)
        check_selection(g, o, q, f"config4 ring q{j}")


def test_item_sort_ties(oracle):
    """Exact ties spread over every sort block: 10,000 tokens whose K rows
    repeat 97 vectors (equal codes and scales, so equal probabilities), and
    a zero query, where every probability is equal (no sort pass runs)."""
    rng = np.random.default_rng(11)
    n = 10000
    g = GpuHead(64, 4, 2, n, 23, 0.95, 0)
    o = oracle.head(64, 4, 2, n, 23, 0.95, 0)
    base = rng.standard_normal((97, 64)).astype(np.float32)
    vals = rng.standard_normal((n, 64)).astype(np.float32)
    for t in range(n):
        g.append(base[t % 97], vals[t], t)
        o.append(base[t % 97], vals[t], t)
    for j in range(2):
        q = rng.standard_normal(64).astype(np.float32)
        check_selection(g, o, q, f"repeated keys q{j}")
    check_selection(g, o, np.zeros(64, np.float32), "zero query")


def test_superblock_sort_selection(oracle):
    """A ring of 70,000 tokens: 35 sort blocks, the scatter reading two
    superblocks' sums."""
    rng = np.random.default_rng(70)
    g, o = fill(64, 2, 2, 70000, 29, 70000, 0.95, oracle, rng)
    q = rng.standard_normal(64).astype(np.float32)
    check_selection(g, o, q, "n=70000")


def test_superblock_sort_wrapped_selection(oracle):
    """A wrapped ring above 32 sort blocks (capacity 66,000, 70,000 tokens
    appended: 4,000 evictions)."""
    rng = np.random.default_rng(66)
    g, o = fill(64, 4, 2, 66000, 31, 70000, 0.95, oracle, rng)
    assert g.info()["head"] == o.info()["head"] == 4000
    q = rng.standard_normal(64).astype(np.float32)
    check_selection(g, o, q, "cap=66000 n=70000 wrapped")


def test_student_t_selection(oracle):
    """Config 3's data (Student-t(4), d64 K3/V2, 1,025 tokens)."""
    rng = np.random.default_rng(3)
    g, o = fill(64, 3, 2, 1280, 5, 1025, 0.95, oracle, rng, family="t")
    for j in range(3):
        q = (rng.standard_t(4, size=64) / np.sqrt(2.0)).astype(np.float32)
        check_selection(g, o, q, f"config3 shape q{j}")


def test_not_sparse_is_an_error():
    g = GpuHead(64, 4, 2, 64, 1, 0.0, 0)
    g.append(np.ones(64, np.float32), np.ones(64, np.float32), 0)
    w = np.zeros(1, np.float32)
    q = np.ones(64, np.float32)
    assert L.adaptq_sparse_weights(g.h, _lib.fptr(q), _lib.fptr(w)) == -1
    assert "sparse-V" in err()


def test_many_superblocks_wrapped_selection(oracle):
    """A wrapped ring of 300,000 tokens (capacity 300,000, 310,000 appended):
    147 sort blocks in 5 superblocks."""
    rng = np.random.default_rng(300)
    g, o = fill(64, 2, 2, 300000, 37, 310000, 0.95, oracle, rng)
    assert g.info()["head"] == o.info()["head"] == 10000
    q = (2.0 * rng.standard_normal(64)).astype(np.float32)
    check_selection(g, o, q, "cap=300000 n=310000 wrapped")
