"""ggml operator forms (adaptq_ggml_append_f32 / _attn_f32 and their device
forms) and the llama.cpp adapter class, against per-head calls and the oracle.

Tensors follow ggml's layout: f32 [head_dim, n_heads, n] with byte strides
nb1 (between heads) and nb2 (between tokens or queries); the tests pad both so
a stride mistake reads or writes the wrong row.  Bar: ring codes and scales
identical to per-head appends; outputs within 1e-4 of the oracle; padding of
the destination untouched."""
import ctypes as C
import os
import subprocess

import numpy as np
import pytest

from adaptq_amd import _lib
from golden import inputs as I
from gpu_head import GpuHead, err, rel_err, same_bits

pytestmark = pytest.mark.gpu
L = _lib.lib
TOL = 1e-4
ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


class GgmlTensor:
    """A [dim, heads, n] f32 tensor in a padded buffer (ggml byte strides)."""

    def __init__(self, dim, heads, n, pad1=8, pad2=16, fill=0.0):
        self.dim, self.heads, self.n = dim, heads, n
        self.nb1 = (dim + pad1) * 4
        self.nb2 = self.nb1 * heads + pad2 * 4
        self.buf = np.full(self.nb2 // 4 * n, fill, np.float32)

    def view(self):  # [n, heads, dim] view of the data
        return np.lib.stride_tricks.as_strided(
            self.buf, (self.n, self.heads, self.dim), (self.nb2, self.nb1, 4), writeable=True)

    def ptr(self):
        return _lib.fptr(self.buf)

    def padding_mask(self):
        m = np.ones(self.buf.shape, bool)
        idx = (np.arange(self.n)[:, None, None] * (self.nb2 // 4)
               + np.arange(self.heads)[None, :, None] * (self.nb1 // 4)
               + np.arange(self.dim)[None, None, :])
        m[idx.ravel()] = False
        return m


def _mha(H, dim, kb, vb, cap, seed, vm, hyb):
    m = L.adaptq_mha_create(H, dim, kb, vb, cap, seed, vm, hyb)
    assert m, err()
    return m


@pytest.mark.parametrize("vm,hyb,n_tok", [(0.0, 0, 300), (0.95, 512, 300), (0.95, 512, 700),
                                         (0.0, 0, 1100)])
def test_ggml_host_forms(oracle, vm, hyb, n_tok):
    print(f"ggml host vm={vm} hyb={hyb} n={n_tok}", flush=True)
    H, dim, kb, vb, cap, seed, nq = 4, 64, 4, 2, 1024, 21, 3
    rng = np.random.default_rng(n_tok)
    K, V = GgmlTensor(dim, H, n_tok), GgmlTensor(dim, H, n_tok, pad1=4, pad2=3)
    K.view()[:] = rng.standard_normal((n_tok, H, dim)).astype(np.float32)
    V.view()[:] = rng.standard_normal((n_tok, H, dim)).astype(np.float32)
    mg = _mha(H, dim, kb, vb, cap, seed, vm, hyb)   # ggml forms
    mh = _mha(H, dim, kb, vb, cap, seed, vm, hyb)   # per-head calls
    refs = [oracle.head(dim, kb, vb, cap, I.mha_seed(seed, h), vm, hyb) for h in range(H)]
    # one token at a time, then the rest in one call (a prompt burst)
    first = 40
    for t in range(first):
        sub = lambda T: T.buf[t * (T.nb2 // 4):]
        assert L.adaptq_ggml_append_f32(mg, _lib.fptr(sub(K)), _lib.fptr(sub(V)), dim, H, 1,
                                        K.nb1, K.nb2, V.nb1, V.nb2, t) == 0, err()
    rest = lambda T: T.buf[first * (T.nb2 // 4):]
    assert L.adaptq_ggml_append_f32(mg, _lib.fptr(rest(K)), _lib.fptr(rest(V)), dim, H,
                                    n_tok - first, K.nb1, K.nb2, V.nb1, V.nb2, first) == 0, err()
    kv, vv = K.view(), V.view()
    for t in range(n_tok):
        for h in range(H):
            k, v = np.ascontiguousarray(kv[t, h]), np.ascontiguousarray(vv[t, h])
            L.adaptq_mha_append(mh, h, _lib.fptr(k), _lib.fptr(v), t)
            refs[h].append(k, v, t)
    Q = GgmlTensor(dim, H, nq, pad1=0, pad2=0)
    Q.view()[:] = rng.standard_normal((nq, H, dim)).astype(np.float32)
    Dst = GgmlTensor(dim, H, nq, pad1=2, pad2=5, fill=7.0)
    n = L.adaptq_ggml_attn_f32(mg, Q.ptr(), dim, H, nq, Q.nb1, Q.nb2, Dst.ptr(), Dst.nb1, Dst.nb2)
    assert n == min(n_tok, cap), err()
    assert np.all(Dst.buf[Dst.padding_mask()] == 7.0)
    out, qv = Dst.view(), Q.view()
    for h in range(H):
        for j in range(nq):
            r, _ = refs[h].compute(np.ascontiguousarray(qv[j, h]))
            assert rel_err(out[j, h], r) <= TOL, (h, j)
        gg = GpuHead.wrap(L.adaptq_mha_head(mg, h), dim)
        gh = GpuHead.wrap(L.adaptq_mha_head(mh, h), dim)
        for a, b in zip(gg.read_slots(0, gg.info()["size"]), gh.read_slots(0, gh.info()["size"])):
            assert same_bits(a, b)
    L.adaptq_mha_destroy(mg)
    L.adaptq_mha_destroy(mh)


def test_ggml_attn_falls_back_when_heads_differ(oracle):
    """Per-head appends leave heads of different sizes: the host form works
    head by head (all queries of a head at once); the device form refuses."""
    import torch
    H, dim = 3, 64
    m = _mha(H, dim, 4, 2, 256, 5, 0.0, 0)
    refs = [oracle.head(dim, 4, 2, 256, I.mha_seed(5, h)) for h in range(H)]
    rng = np.random.default_rng(4)
    for h in range(H):
        for t in range(20 + 10 * h):
            k, v = rng.standard_normal((2, dim)).astype(np.float32)
            L.adaptq_mha_append(m, h, _lib.fptr(k), _lib.fptr(v), t)
            refs[h].append(k, v, t)
    Q = GgmlTensor(dim, H, 2, pad1=1, pad2=1)
    Q.view()[:] = rng.standard_normal((2, H, dim)).astype(np.float32)
    Dst = GgmlTensor(dim, H, 2)
    assert L.adaptq_ggml_attn_f32(m, Q.ptr(), dim, H, 2, Q.nb1, Q.nb2, Dst.ptr(), Dst.nb1,
                                  Dst.nb2) > 0, err()
    for h in range(H):
        for j in range(2):
            assert rel_err(Dst.view()[j, h], refs[h].compute(np.ascontiguousarray(Q.view()[j, h]))[0]) <= TOL
    dq = torch.zeros(2 * H * dim, device="cuda")
    do = torch.zeros_like(dq)
    s = torch.cuda.current_stream().cuda_stream
    assert L.adaptq_ggml_attn_f32_device(m, C.c_void_p(dq.data_ptr()), dim, H, 2, dim * 4,
                                         H * dim * 4, C.c_void_p(do.data_ptr()), dim * 4,
                                         H * dim * 4, C.c_void_p(s)) == -1
    assert "differ" in err()
    L.adaptq_mha_destroy(m)


@pytest.mark.parametrize("vm,hyb", [(0.0, 0), (0.95, 512)])
def test_ggml_device_forms(oracle, vm, hyb):
    import torch
    print(f"ggml device vm={vm} hyb={hyb}", flush=True)
    H, dim, kb, vb, cap, seed, T, nq = 4, 128, 4, 2, 2048, 3, 600, 2
    dev = torch.device("cuda:0")
    g = torch.Generator(device="cpu").manual_seed(8)
    # padded ggml buffers: [T][H][dim + 4] with 16 floats after each token
    nb1, nb2 = (dim + 4) * 4, ((dim + 4) * H + 16) * 4
    kbuf = torch.zeros(T * nb2 // 4)
    vbuf = torch.zeros(T * nb2 // 4)
    kv = kbuf.as_strided((T, H, dim), (nb2 // 4, nb1 // 4, 1))
    vv = vbuf.as_strided((T, H, dim), (nb2 // 4, nb1 // 4, 1))
    kv.copy_(torch.randn(T, H, dim, generator=g))
    vv.copy_(torch.randn(T, H, dim, generator=g))
    m = _mha(H, dim, kb, vb, cap, seed, vm, hyb)
    refs = [oracle.head(dim, kb, vb, cap, I.mha_seed(seed, h), vm, hyb) for h in range(H)]
    for t in range(T):
        for h in range(H):
            refs[h].append(kv[t, h].numpy(), vv[t, h].numpy(), t)
    kd, vd = kbuf.to(dev), vbuf.to(dev)
    s = torch.cuda.current_stream().cuda_stream
    # 450 tokens in one launch, then single tokens
    assert L.adaptq_ggml_append_f32_device(m, C.c_void_p(kd.data_ptr()), C.c_void_p(vd.data_ptr()),
                                           dim, H, 450, nb1, nb2, nb1, nb2, 0, C.c_void_p(s)) == 0, err()
    for t in range(450, T):
        off = t * nb2
        assert L.adaptq_ggml_append_f32_device(
            m, C.c_void_p(kd.data_ptr() + off), C.c_void_p(vd.data_ptr() + off), dim, H, 1,
            nb1, nb2, nb1, nb2, t, C.c_void_p(s)) == 0, err()
    q = torch.randn(nq, H, dim, generator=g)
    qd = q.to(dev)
    dbuf = torch.full((nq * (H * (dim + 2) + 8),), 5.0, device=dev)
    dn1, dn2 = (dim + 2) * 4, (H * (dim + 2) + 8) * 4
    n = L.adaptq_ggml_attn_f32_device(m, C.c_void_p(qd.data_ptr()), dim, H, nq, dim * 4,
                                      H * dim * 4, C.c_void_p(dbuf.data_ptr()), dn1, dn2,
                                      C.c_void_p(s))
    assert n == T, err()
    torch.cuda.synchronize()
    host = dbuf.cpu()
    out = host.as_strided((nq, H, dim), (dn2 // 4, dn1 // 4, 1)).numpy()
    mask = torch.ones_like(host, dtype=torch.bool)
    mask.as_strided((nq, H, dim), (dn2 // 4, dn1 // 4, 1)).fill_(False)
    assert torch.all(host[mask] == 5.0)
    for h in range(H):
        for j in range(nq):
            assert rel_err(out[j, h], refs[h].compute(q[j, h].numpy())[0]) <= TOL, (vm, h, j)
    L.adaptq_mha_destroy(m)


def test_ggml_argument_errors():
    m = _mha(2, 64, 4, 2, 64, 1, 0.0, 0)
    x = np.zeros(2 * 64 * 4, np.float32)
    p = _lib.fptr(x)
    assert L.adaptq_ggml_append_f32(m, p, p, 32, 2, 1, 256, 512, 256, 512, 0) == -1
    assert "shape" in err()
    assert L.adaptq_ggml_append_f32(m, p, p, 64, 3, 1, 256, 512, 256, 512, 0) == -1
    assert L.adaptq_ggml_attn_f32(m, p, 64, 2, 1, 258, 512, p, 256, 512) == -1
    assert "multiples of 4" in err()
    assert L.adaptq_ggml_attn_f32(m, p, 64, 2, -1, 256, 512, p, 256, 512) == -1
    assert L.adaptq_ggml_append_f32(m, None, p, 64, 2, 1, 256, 512, 256, 512, 0) == -1
    assert L.adaptq_ggml_append_f32(None, p, p, 64, 2, 1, 256, 512, 256, 512, 0) == -1
    # zero tokens / queries are no-ops; an empty cache attends to zeros
    assert L.adaptq_ggml_append_f32(m, p, p, 64, 2, 0, 256, 512, 256, 512, 0) == 0
    out = np.full(2 * 64, 3.0, np.float32)
    assert L.adaptq_ggml_attn_f32(m, p, 64, 2, 1, 256, 512, _lib.fptr(out), 256, 512) == 0
    assert np.all(out == 0.0)
    L.adaptq_mha_destroy(m)


def test_llama_adapter_cpp(tmp_path):
    """The C++ adapter header compiled and run as llama.cpp would use it."""
    exe = tmp_path / "llama_adapter_check"
    src = os.path.join(ROOT, "tests", "cpp", "llama_adapter_check.cpp")
    lib_dir = os.path.join(ROOT, "adaptq_amd")
    r = subprocess.run(["g++", "-std=c++17", "-O1", "-I", os.path.join(ROOT, "include"), src,
                        "-L", lib_dir, "-ladaptq", f"-Wl,-rpath,{lib_dir}", "-o", str(exe)],
                       capture_output=True, text=True)
    assert r.returncode == 0, r.stderr
    r = subprocess.run([str(exe)], capture_output=True, text=True, timeout=120)
    print(r.stdout, r.stderr)
    assert r.returncode == 0 and "OK" in r.stdout, r.stdout + r.stderr
    assert "[AdapTQ/llama.cpp] KV:" in r.stderr
