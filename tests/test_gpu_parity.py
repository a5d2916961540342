"""GPU parity against the oracle (oracle/oracle.c) on seeded inputs.

Bar: packed codes, scales and ring state bit-exact; attention outputs within
1e-4 norm-wise relative error (max|y - r| / max|r|), as BASELINE.json's
north star states.
"""
import numpy as np
import pytest

from gpu_head import GpuHead, rel_err, same_bits

pytestmark = pytest.mark.gpu

TOL = 1e-4


def _inputs(rng, n, dim, family):
    k = rng.standard_normal((n, dim)).astype(np.float32)
    v = rng.standard_normal((n, dim)).astype(np.float32)
    if family == "student_t":
        k = (rng.standard_t(4, (n, dim)) / np.sqrt(2)).astype(np.float32)
        v = (rng.standard_t(4, (n, dim)) / np.sqrt(2)).astype(np.float32)
    elif family == "outliers":
        k[:, [3, 17 % dim]] *= 20
        v[:, [3, 17 % dim]] *= 20
    elif family == "tiny":
        k *= np.float32(1e-20)
        v *= np.float32(1e-7)
    elif family == "huge":
        k *= np.float32(1e18)
        v *= np.float32(-3e17)
    return k, v


def _fill(heads, k, v):
    for t in range(k.shape[0]):
        for h in heads:
            h.append(k[t], v[t], t)


def _ring_equal(g, o):
    gi, oi = g.info(), o.info()
    assert (gi["head"], gi["size"]) == (oi["head"], oi["size"])
    n = oi["cap"]
    if n == 0:
        return
    a = g.read_slots(0, oi["size"])
    b = o.read_slots(0, oi["size"])
    for x, y, what in zip(a, b, ["k codes", "v codes", "k scale", "v scale"]):
        assert same_bits(x, y), f"{what} differ in {int((x != y).any(axis=-1).sum()) if x.ndim > 1 else int((x.view(np.uint32) != y.view(np.uint32)).sum())} slots"


@pytest.mark.parametrize("dim,kb,vb", [
    (64, 4, 2), (128, 4, 2), (64, 3, 2), (128, 3, 3), (64, 2, 2), (128, 2, 4),
    (64, 16, 2), (128, 4, 16), (96, 4, 2), (32, 3, 4), (256, 4, 2), (48, 2, 3),
])
@pytest.mark.parametrize("family", ["normal", "student_t", "outliers", "tiny", "huge"])
def test_append_bit_exact(oracle, dim, kb, vb, family):
    print(f"append parity dim={dim} k{kb}v{vb} {family}", flush=True)
    rng = np.random.default_rng(dim * 1000 + kb * 10 + vb)
    cap, n = 96, 150  # wraps the ring
    seed = int(rng.integers(0, 2**63))
    k, v = _inputs(rng, n, dim, family)
    g = GpuHead(dim, kb, vb, cap, seed)
    o = oracle.head(dim, kb, vb, cap, seed)
    _fill([g, o], k, v)
    _ring_equal(g, o)


@pytest.mark.parametrize("dim,kb,vb", [(128, 4, 2), (64, 2, 3), (128, 3, 4), (32, 4, 4)])
def test_append_clamp_paths(oracle, dim, kb, vb):
    """The append kernel skips sigma and the +-3 sigma clamp for a wave whose
    rows all have sum x^2 >= 1e-10 (provably inert there) and runs the
    reference's steps for any other wave.  Waves of 64 consecutive tokens:
    all normal rows (skip); one tiny row among normal ones; rows just above
    and below the bound; denormal-scale rows; single-spike rows (all FWHT
    outputs equal in magnitude); rows that rotate to a single value far
    above 3 sigma (where the clamp acts).  Codes and scales bit-exact."""
    print(f"append clamp paths dim={dim} k{kb}v{vb}", flush=True)
    rng = np.random.default_rng(dim + kb * 7 + vb)
    n = 6 * 64
    k = rng.standard_normal((n, dim)).astype(np.float32)
    v = rng.standard_normal((n, dim)).astype(np.float32)
    k[64 + 17] *= np.float32(1e-7)                       # one tiny row in a normal wave
    v[64 + 40] *= np.float32(1e-30)
    b = np.sqrt(1e-10 / dim)                              # rows around s = 1e-10
    k[128:192] *= np.float32(b) * np.linspace(0.98, 1.02, 64, dtype=np.float32)[:, None]
    v[128:192] *= np.float32(b) * np.linspace(1.02, 0.98, 64, dtype=np.float32)[:, None]
    k[192:256] *= np.float32(1e-20)                       # squares underflow
    v[192:256] *= np.float32(3e-23)
    k[256:320] = 0.0                                      # single spikes
    v[256:320] = 0.0
    for t in range(256, 320):
        k[t, t % dim] = np.float32(rng.uniform(0.1, 5.0))
        v[t, (3 * t) % dim] = np.float32(-rng.uniform(0.1, 5.0))
    seed = int(rng.integers(0, 2**63))
    g = GpuHead(dim, kb, vb, n, seed)
    o = oracle.head(dim, kb, vb, n, seed)
    # rows D . h_j (a Hadamard row under the head's signs) rotate to one
    # value sqrt(p) and zeros: far above 3 sigma, where the clamp acts
    D = o.signs().astype(np.float32)[:dim]
    idx = np.arange(dim)
    for t in range(320, 384):
        hj = np.array([(-1) ** bin(i & (t % dim)).count("1") for i in idx], np.float32)
        hv = np.array([(-1) ** bin(i & ((5 * t) % dim)).count("1") for i in idx], np.float32)
        k[t] = D * hj * np.float32(rng.uniform(0.5, 2.0))
        v[t] = D * hv * np.float32(-rng.uniform(0.5, 2.0))
    _fill([g, o], k, v)
    _ring_equal(g, o)


@pytest.mark.parametrize("dim,kb,vb", [(128, 4, 2), (128, 2, 4), (64, 4, 2), (64, 2, 2),
                                       (32, 4, 4), (96, 4, 2), (128, 3, 2)])
def test_bulk_append_kernel_rows(oracle, dim, kb, vb):
    """The lane-per-vector append kernel (a whole-MHA flush of 48 heads x 384
    tokens, above the one-wave kernel's 16,384 vectors).  It codes 2- and
    4-bit values before the scalings by 1/sqrt(p) and sqrt(p), against
    thresholds moved through both roundings, and clamps codes rather than
    values on the sigma path.  Waves of 64 tokens per head: normal rows; one
    tiny row among normal ones; rows around the s = 1e-10 bound; single
    spikes; Hadamard rows far above 3 sigma; rows whose rotation cancels to
    exact and signed zeros and denormal values (x0 = +-x1 under the head's
    signs plus one tiny entry), where v = fl(fl(b / sqrt p) * sqrt p) is -0
    for tiny negative b.  Codes and scales bit-exact for every head."""
    from adaptq_amd import _lib
    from golden import inputs as I
    from gpu_head import err
    L = _lib.lib
    print(f"bulk append kernel dim={dim} k{kb}v{vb}", flush=True)
    H, T, seed = 48, 6 * 64, 1234 + dim
    rng = np.random.default_rng(dim * 31 + kb * 5 + vb)
    refs = [oracle.head(dim, kb, vb, T, I.mha_seed(seed, h)) for h in range(H)]
    K = rng.standard_normal((T, H, dim)).astype(np.float32)
    V = rng.standard_normal((T, H, dim)).astype(np.float32)
    tiny = np.array([1e-45, -1e-45, 3e-45, -4e-45, 1e-42, -1e-40, 7e-39, -2e-38, 1e-36,
                     -1e-30, 0.0, -0.0], np.float32)
    b = np.sqrt(1e-10 / dim)
    idx = np.arange(dim)
    for h in range(H):
        D = refs[h].signs().astype(np.float32)[:dim]
        K[64 + h % 64, h] *= np.float32(1e-7)
        V[64 + (h * 7) % 64, h] *= np.float32(1e-30)
        K[128:192, h] *= np.float32(b) * np.linspace(0.98, 1.02, 64, dtype=np.float32)[:, None]
        V[128:192, h] *= np.float32(b) * np.linspace(1.02, 0.98, 64, dtype=np.float32)[:, None]
        for t in range(192, 256):  # spikes, or Hadamard rows (one value far above 3 sigma)
            if t % 2:
                K[t, h] = 0.0
                V[t, h] = 0.0
                K[t, h, t % dim] = np.float32(rng.uniform(0.1, 5.0))
                V[t, h, (3 * t) % dim] = np.float32(-rng.uniform(0.1, 5.0))
            else:
                hj = np.array([(-1) ** bin(i & (t % dim)).count("1") for i in idx], np.float32)
                K[t, h] = D * hj * np.float32(rng.uniform(0.5, 2.0))
                V[t, h] = D * hj[::-1].copy() * np.float32(-rng.uniform(0.5, 2.0))
        for t in range(256, T):  # cancellations to zeros and denormals
            for X, off in ((K, 0), (V, 5)):
                a = np.float32(rng.uniform(0.5, 2.0)) * (1 if t % 3 else -1)
                x = np.zeros(dim, np.float32)
                x[0] = a
                x[1] = a * D[0] * D[1] * (1 if (t + off) % 4 else -1)
                x[2] = tiny[(t + off + h) % len(tiny)]
                if (t + h) % 5 == 0:
                    x[3:] = np.float32(-0.0)
                X[t, h] = x
    m = L.adaptq_mha_create(H, dim, kb, vb, T, seed, 0.0, 0)
    assert m, err()
    for t in range(T):
        assert L.adaptq_mha_append_all(m, _lib.fptr(np.ascontiguousarray(K[t])),
                                       _lib.fptr(np.ascontiguousarray(V[t])), t) == 0, err()
        for h in range(H):
            refs[h].append(K[t, h], V[t, h], t)
    # the whole-MHA call flushes the staged rows of all heads in one launch
    q = rng.standard_normal((H, dim)).astype(np.float32)
    out = np.zeros((H, dim), np.float32)
    assert L.adaptq_mha_compute_all(m, _lib.fptr(q), _lib.fptr(out)) == T, err()
    for h in range(H):
        _ring_equal(GpuHead.wrap(L.adaptq_mha_head(m, h), dim), refs[h])
    for h in (0, 17, H - 1):
        assert rel_err(out[h], refs[h].compute(q[h])[0]) <= TOL, h
    L.adaptq_mha_destroy(m)


@pytest.mark.parametrize("dim,kb,vb", [(128, 4, 2), (64, 2, 4), (32, 2, 2)])
def test_bulk_append_lanes_over_heads(oracle, dim, kb, vb):
    """The lane-per-vector append kernel with fewer than 64 tokens per head
    (400 heads x 48 tokens: lanes run over (head, token) pairs, so a wave mixes
    heads): normal rows, tiny rows, and rows whose rotation cancels to zeros
    and denormal values.  Codes and scales bit-exact for every head."""
    from adaptq_amd import _lib
    from golden import inputs as I
    from gpu_head import err
    L = _lib.lib
    print(f"bulk append lanes over heads dim={dim} k{kb}v{vb}", flush=True)
    H, T, seed = 400, 48, 99 + dim
    rng = np.random.default_rng(dim * 17 + kb + vb)
    refs = [oracle.head(dim, kb, vb, T, I.mha_seed(seed, h)) for h in range(H)]
    K = rng.standard_normal((T, H, dim)).astype(np.float32)
    V = rng.standard_normal((T, H, dim)).astype(np.float32)
    tiny = np.array([1e-45, -1e-45, -3e-45, 1e-40, -7e-39, 0.0, -0.0], np.float32)
    for h in range(0, H, 3):
        D = refs[h].signs().astype(np.float32)[:dim]
        for t in range(h % 5, T, 4):
            for X, off in ((K, 0), (V, 3)):
                x = np.zeros(dim, np.float32)
                x[0] = np.float32(rng.uniform(0.5, 2.0))
                x[1] = x[0] * D[0] * D[1] * (1 if (t + off) % 2 else -1)
                x[2] = tiny[(t + off + h) % len(tiny)]
                X[t, h] = x
        K[(h * 7) % T, h] *= np.float32(1e-7)
        V[(h * 11) % T, h] *= np.float32(1e-30)
    m = L.adaptq_mha_create(H, dim, kb, vb, T, seed, 0.0, 0)
    assert m, err()
    for t in range(T):
        assert L.adaptq_mha_append_all(m, _lib.fptr(np.ascontiguousarray(K[t])),
                                       _lib.fptr(np.ascontiguousarray(V[t])), t) == 0, err()
        for h in range(H):
            refs[h].append(K[t, h], V[t, h], t)
    q = rng.standard_normal((H, dim)).astype(np.float32)
    out = np.zeros((H, dim), np.float32)
    assert L.adaptq_mha_compute_all(m, _lib.fptr(q), _lib.fptr(out)) == T, err()
    for h in range(H):
        _ring_equal(GpuHead.wrap(L.adaptq_mha_head(m, h), dim), refs[h])
    L.adaptq_mha_destroy(m)


def test_append_special_values(oracle):
    dim, cap = 64, 32
    rows = [np.zeros(dim, np.float32), np.full(dim, np.nan, np.float32),
            np.full(dim, 1e38, np.float32), np.full(dim, -1e38, np.float32),
            np.full(dim, 1e-38, np.float32), np.full(dim, -0.0, np.float32),
            np.full(dim, np.inf, np.float32)]
    x = np.zeros(dim, np.float32)
    x[5] = 1e-38
    rows.append(x)
    x = np.zeros(dim, np.float32)
    x[0] = 1e7
    rows.append(x)
    for kb, vb in [(4, 2), (3, 3), (2, 4)]:
        print(f"special values k{kb}v{vb}", flush=True)
        g = GpuHead(dim, kb, vb, cap, 42)
        o = oracle.head(dim, kb, vb, cap, 42)
        for i, r in enumerate(rows):
            for h in (g, o):
                h.append(r, r[::-1].copy(), i)
        _ring_equal(g, o)


DECODE_CASES = [
    # dim, kb, vb, cap, n
    (64, 4, 2, 2048, 2048),
    (128, 4, 2, 1024, 1500),
    (128, 4, 4, 512, 700),
    (64, 3, 2, 1280, 1100),
    (128, 2, 3, 300, 300),
    (64, 16, 2, 512, 512),
    (64, 16, 16, 256, 200),
    (128, 4, 16, 256, 256),
    (96, 4, 2, 256, 300),
    (256, 3, 2, 200, 260),
    (32, 2, 2, 100, 77),
    # padded 256 through the LUT kernel (nibble K table at 2/4 bits, pair
    # table at 3 bits), every quantised K/V pair: a wrapped ring over several
    # splits, a ring shorter than one tile, an unpadded dim
    (256, 4, 2, 3000, 5000),
    (256, 4, 3, 300, 300),
    (256, 4, 4, 100, 40),
    (256, 2, 2, 700, 700),
    (256, 2, 3, 500, 600),
    (256, 2, 4, 256, 256),
    (256, 3, 3, 512, 512),
    (256, 3, 4, 1000, 1000),
    (200, 4, 2, 600, 777),
    # padded 256 with fp32 keys or values (the reference's layer-0 K16 policy
    # at head dim 256) through the LUT kernel
    (256, 16, 2, 1500, 2000),
    (256, 16, 4, 300, 200),
    (256, 4, 16, 700, 700),
    (256, 16, 16, 256, 300),
    (200, 16, 3, 400, 400),
    # padded 512 and 1024 through the wide kernel (quantised K and V): a
    # wrapped ring over several splits, unpadded dims, every K width, a ring
    # shorter than one step of the block's waves
    (512, 4, 2, 3000, 4100),
    (300, 3, 3, 700, 700),
    (512, 2, 4, 1500, 1500),
    (1024, 4, 4, 2000, 2600),
    (1000, 2, 3, 600, 600),
    (600, 3, 2, 300, 13),
    # fp32 keys there take the row-dot kernel (one token a thread): every V
    # width, a wrapped ring, a ring of exactly one block's tokens, a dim that
    # is not a multiple of 4
    (512, 16, 2, 300, 300),
    (1024, 16, 16, 600, 700),
    (700, 16, 4, 900, 1000),
    (512, 16, 3, 256, 256),
    (602, 16, 16, 300, 257),
]


@pytest.mark.parametrize("dim,kb,vb,cap,n", DECODE_CASES)
def test_decode_dense(oracle, dim, kb, vb, cap, n):
    print(f"decode dense dim={dim} k{kb}v{vb} cap={cap} n={n}", flush=True)
    rng = np.random.default_rng(n + dim)
    seed = 42 + dim
    k, v = _inputs(rng, n, dim, "normal")
    g = GpuHead(dim, kb, vb, cap, seed)
    o = oracle.head(dim, kb, vb, cap, seed)
    _fill([g, o], k, v)
    for _ in range(3):
        q = rng.standard_normal(dim).astype(np.float32)
        y, ny = g.compute(q)
        r, nr = o.compute(q)
        assert ny == nr
        assert rel_err(y, r) <= TOL, rel_err(y, r)


@pytest.mark.parametrize("dim,kb,vb,hyb,n", [
    (64, 4, 2, 512, 512), (128, 4, 4, 64, 40), (96, 3, 2, 128, 100), (64, 16, 2, 16, 10),
    (256, 4, 2, 512, 500), (256, 3, 3, 64, 64),
    # the mirror at padded 512 and 1024: the row-dot kernel
    (512, 4, 2, 512, 400), (602, 3, 4, 300, 257), (1024, 2, 2, 64, 40),
])
def test_decode_hybrid(oracle, dim, kb, vb, hyb, n):
    print(f"decode hybrid dim={dim} k{kb}v{vb} hyb={hyb} n={n}", flush=True)
    rng = np.random.default_rng(7 * n + dim)
    k, v = _inputs(rng, n, dim, "normal")
    g = GpuHead(dim, kb, vb, 1024, 9, 0.95, hyb)
    o = oracle.head(dim, kb, vb, 1024, 9, 0.95, hyb)
    _fill([g, o], k, v)
    q = rng.standard_normal(dim).astype(np.float32)
    y, _ = g.compute(q)
    r, _ = o.compute(q)
    assert rel_err(y, r) <= TOL


# Sort in LDS (n <= 16384) and in the workspace (above); quad sums staged in
# one and in several chunks (n/4 above 4096); peaked queries (qs 20: the cut
# falls after a few quads) and flat ones; v_mass near 1 (the single-token tail
# runs); ragged n.  At padded 64 up to 3,072 tokens the one-block kernel runs
# (1, 2 and 4 tokens per thread; a wrapped ring; 3-bit V at the size limit).
@pytest.mark.parametrize("dim,kb,vb,cap,n,vm,qs", [
    (64, 4, 2, 2048, 2048, 0.95, 3), (128, 4, 4, 512, 700, 0.95, 3), (64, 3, 2, 600, 513, 0.7, 3),
    (128, 2, 3, 9000, 9000, 0.95, 3), (64, 4, 2, 100, 7, 0.5, 3), (64, 4, 2, 17000, 17001, 0.95, 3),
    (64, 2, 4, 3000, 2999, 0.95, 20), (128, 4, 2, 20000, 20000, 0.999, 1),
    (64, 4, 3, 5000, 4998, 0.9999, 0.5), (64, 4, 2, 1500, 2600, 0.95, 3),
    (64, 3, 3, 3072, 3072, 0.9, 3),
])
def test_decode_sparse_v(oracle, dim, kb, vb, cap, n, vm, qs):
    print(f"decode sparse dim={dim} k{kb}v{vb} n={n} v_mass={vm} qscale={qs}", flush=True)
    rng = np.random.default_rng(3 * n + dim)
    k, v = _inputs(rng, n, dim, "normal")
    g = GpuHead(dim, kb, vb, cap, 5, vm, 0)
    o = oracle.head(dim, kb, vb, cap, 5, vm, 0)
    _fill([g, o], k, v)
    for _ in range(2):
        q = (qs * rng.standard_normal(dim)).astype(np.float32)
        y, _ = g.compute(q)
        r, _ = o.compute(q)
        assert rel_err(y, r) <= TOL


def test_compute_batch(oracle):
    dim, kb, vb, cap, n = 128, 4, 4, 4096, 5000
    rng = np.random.default_rng(11)
    k, v = _inputs(rng, n, dim, "normal")
    g = GpuHead(dim, kb, vb, cap, 7)
    o = oracle.head(dim, kb, vb, cap, 7)
    _fill([g, o], k, v)
    qs = rng.standard_normal((16, dim)).astype(np.float32)
    y, ny = g.compute_batch(qs)
    r, nr = o.compute_batch(qs)
    assert ny == nr == cap
    assert rel_err(y, r) <= TOL
