"""BASELINE configs[4] -- the headline -- at its full size, generated and
launched exactly as bench.py does: 2,048 MHAs (one per sequence and layer,
base seed = sequence * 32 + layer) of 8 heads = 16,384 contexts, d128, K4/V2,
8,192 tokens each, N(0,1) K/V times a per-head log-normal(0, 0.5) scale from
torch's generator seeded 42, appended through plans of 1,024 contexts, then
one batched decode launch of all 16,384 heads through one plan.

Checked: for sampled heads across the stack (first, last, both sides of every
chunk boundary sampled), every ring byte and scale bit-exact against the
oracle, and the output within 1e-4 norm-wise of the oracle's, with the
norm-wise and elementwise errors printed; for every head, the output finite
and inside the bound |out_j| <= max|CB_V| * max_t ||v_t|| that any decode of
its ring obeys."""
import ctypes as C

import numpy as np
import pytest

from adaptq_amd import _lib
from golden import inputs as I
from gpu_head import GpuHead, err, rel_err, same_bits

pytestmark = pytest.mark.gpu
L = _lib.lib

N_SEQ, N_LAYER, HEADS, N, DIM, KB, VB = 64, 32, 8, 8192, 128, 4, 2
H = N_SEQ * N_LAYER * HEADS
CHUNK = 1024
SAMPLES = (0, 1, 1023, 1024, 5000, 8191, 8192, 12345, 16382, 16383)


def test_config5_full_headline_launch(oracle):
    import torch
    print(f"config5 full size: {H} heads x {N} tokens d{DIM} K{KB}/V{VB}", flush=True)
    dev = torch.device("cuda:0")
    n_eng = N_SEQ * N_LAYER
    mhas, ctxs = [], []
    for e in range(n_eng):
        m = L.adaptq_mha_create(HEADS, DIM, KB, VB, N, e, 0.0, 0)
        assert m, err()
        mhas.append(m)
        ctxs += [L.adaptq_mha_head(m, i) for i in range(HEADS)]
    plan = L.adaptq_plan_create((C.c_void_p * H)(*ctxs), H)
    assert plan, err()
    stream = C.c_void_p(torch.cuda.current_stream().cuda_stream)
    g = torch.Generator(device=dev)
    g.manual_seed(42)
    scales = torch.exp(0.5 * torch.randn(H, generator=g, device=dev))
    sampled = {}
    for c0 in range(0, H, CHUNK):
        sub = L.adaptq_plan_create((C.c_void_p * CHUNK)(*ctxs[c0:c0 + CHUNK]), CHUNK)
        assert sub, err()
        k = torch.randn(CHUNK, N, DIM, generator=g, device=dev) * scales[c0:c0 + CHUNK, None, None]
        v = torch.randn(CHUNK, N, DIM, generator=g, device=dev) * scales[c0:c0 + CHUNK, None, None]
        assert L.adaptq_plan_append_device(sub, C.c_void_p(k.data_ptr()), C.c_void_p(v.data_ptr()),
                                           N, 0, stream) == 0, err()
        torch.cuda.synchronize()
        for h in SAMPLES:
            if c0 <= h < c0 + CHUNK:
                sampled[h] = (k[h - c0].cpu().numpy(), v[h - c0].cpu().numpy())
        L.adaptq_plan_destroy(sub)
        del k, v
    print("appended", flush=True)
    q = torch.randn(H, DIM, generator=g, device=dev)
    out = torch.full((H, DIM), float("nan"), device=dev)
    assert L.adaptq_plan_compute_device(plan, C.c_void_p(q.data_ptr()),
                                        C.c_void_p(out.data_ptr()), stream) == 0, err()
    torch.cuda.synchronize()
    y = out.cpu().numpy()
    qh = q.cpu().numpy()
    assert np.isfinite(y).all()
    vmax = 1.5104 * scales.cpu().numpy() * 2.0 * np.sqrt(DIM)
    assert (np.abs(y).max(axis=1) <= vmax).all()

    worst_norm, worst_elem = 0.0, 0.0
    for h in SAMPLES:
        kh, vh = sampled[h]
        e, i = divmod(h, HEADS)
        o = oracle.head(DIM, KB, VB, N, I.mha_seed(e, i))
        for t in range(N):
            o.append(kh[t], vh[t], t)
        gh = GpuHead.wrap(ctxs[h], DIM)
        gi, oi = gh.info(), o.info()
        assert (gi["head"], gi["size"]) == (oi["head"], oi["size"]) == (0, N)
        for a, b in zip(gh.read_slots(0, N), o.read_slots(0, N)):
            assert same_bits(a, b), f"head {h}: ring bytes differ"
        r, nr = o.compute(qh[h])
        assert nr == N
        ne = rel_err(y[h], r)
        big = np.abs(r) >= 1e-3 * np.abs(r).max()
        ee = float(np.max(np.abs(y[h][big] - r[big]) / np.abs(r[big])))
        med = float(np.median(np.abs(y[h][big] - r[big]) / np.abs(r[big])))
        print(f"head {h}: norm-wise {ne:.2e}, elementwise max {ee:.2e} median {med:.2e} "
              f"(entries >= 1e-3 max|r|)", flush=True)
        worst_norm, worst_elem = max(worst_norm, ne), max(worst_elem, ee)
        assert ne <= 1e-4, (h, ne)
    print(f"worst over {len(SAMPLES)} sampled heads: norm-wise {worst_norm:.2e}, "
          f"elementwise {worst_elem:.2e}", flush=True)
    L.adaptq_plan_destroy(plan)
    for m in mhas:
        L.adaptq_mha_destroy(m)
