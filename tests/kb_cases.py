"""Cases for the kernel-backend tests (IKernelBackend): inputs, the file
format read by tests/cpp/kernel_backend_check.cpp, and a float64 model of
kdot_batch / vaccum_batch (kernels/scalar/kdot_scalar.cpp semantics) over
codes decoded by the oracle."""
import numpy as np


def row_bytes(p, bits):
    return (p * bits + 7) // 8


def cases():
    out = []
    rng = np.random.default_rng(11)
    for bits in (2, 3, 4):
        for p in (8, 64, 128, 256):
            for n in (1, 37, 1000):
                q = rng.standard_normal(p).astype(np.float32)
                rows = rng.integers(0, 256, (n, row_bytes(p, bits)), np.uint8)
                scales = (rng.random(n) + 0.5).astype(np.float32)
                w = rng.random(n).astype(np.float32)
                w[rng.random(n) < 0.2] = 0.0
                D = np.where(rng.random(p) < 0.5, 1, -1).astype(np.int8)
                x = rng.standard_normal(p).astype(np.float32)
                out.append(dict(bits=bits, p=p, n=n, q=q, rows=rows, scales=scales, w=w, D=D, x=x))
    return out


def write_inputs(path, cs):
    with open(path, "wb") as f:
        for c in cs:
            f.write(np.array([c["bits"], c["p"], c["n"]], "<i4").tobytes())
            for k in ("q", "rows", "scales", "w", "D", "x"):
                f.write(c[k].tobytes())


def read_outputs(path, cs):
    data = np.fromfile(path, np.float32)
    res, off = [], 0
    for c in cs:
        n, p = c["n"], c["p"]
        parts = []
        for size in (n, p, p, p):
            parts.append(data[off:off + size])
            off += size
        res.append(dict(zip(("logits", "acc", "fwd", "inv"), parts)))
    assert off == data.size
    return res


def model(c, oracle):
    """float64 kdot logits and vaccum acc for case c (codes via the oracle)."""
    cb = oracle.codebook(c["bits"]).astype(np.float64)
    codes = np.stack([oracle.unpack(r, c["p"], c["bits"]) for r in c["rows"]]).astype(np.int64)
    vals = cb[codes]                                       # [n][p]
    logits = (vals @ c["q"].astype(np.float64)) * c["scales"] / c["p"]
    acc = (c["w"].astype(np.float64) * c["scales"]) @ vals
    return logits, acc
