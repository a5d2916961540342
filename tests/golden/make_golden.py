"""Write the golden fixtures of tests/golden/ from the reference's own code.

Runs oracle/_ref/libadaptq_ref.so: the reference's hot-path sources compiled
in place from /root/reference by oracle/Makefile (target ``ref``).  It needs
that build, so it runs in the development container only; the fixtures it
writes are committed and travel with the repository.

    make -C oracle ref && python tests/golden/make_golden.py

Each file holds inputs (or the name of the deterministic generator in
inputs.py that makes them) and the reference's outputs:

  rademacher.npz     sign vectors D for the seeds of configs 1-5 and seed 0
  fwht.npz           fwht_forward / fwht_inverse at p = 64, 128, 256
  quantize_fast.npz  codebook index of a dense value sweep, bits 2/3/4
  codec.npz          packed codes + scale of quantize_into over dims
                     {64, 128, 96, 48} x bits {2,3,4} x inputs.FAMILIES
  config1.npz        ring state/hashes/edge slots and outputs of config 1
  config2.npz        outputs of config 2 (all 24 layers x 14 heads)
  config3.npz        outputs of config 3 at steps 0, 1, 127, 255
  config4.npz        ring state around the wrap point and 8 query outputs
  ties.npz           sparse-V outputs of inputs.TIE_CASES (probabilities tied
                     exactly at the mass cut)

Outputs are given for (v_mass, hybrid_thresh) = (0, 0) -- pure packed-KV
decode -- and (0.95, 512), the Python Engine defaults.
"""
from __future__ import annotations

import hashlib
import os
import sys

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(os.path.dirname(HERE))
sys.path.insert(0, os.path.join(ROOT, "oracle"))
sys.path.insert(0, HERE)

from bind import Ref, next_pow2  # noqa: E402
import inputs as I  # noqa: E402

MODES = [(0.0, 0), (0.95, 512)]


def sha(*arrays) -> str:
    h = hashlib.sha256()
    for a in arrays:
        h.update(np.ascontiguousarray(a).tobytes())
    return h.hexdigest()


def ring_digest(head) -> dict:
    inf = head.info()
    kc, vc, ks, vs = head.read_slots(0, inf["size"])
    return dict(head=inf["head"], size=inf["size"], sha=sha(kc, vc, ks, vs), kc=kc, vc=vc,
                ks=ks, vs=vs)


def save(name, **arrays):
    path = os.path.join(HERE, name)
    np.savez_compressed(path, **arrays)
    print(f"wrote {name}: {os.path.getsize(path) // 1024} KiB")


def gen_rademacher(r: Ref):
    seeds, dims = [0], [64]
    seeds += [I.mha_seed(42, i) for i in range(4)]
    dims += [64] * 4
    for layer in range(24):
        seeds += [I.mha_seed(42 ^ layer, i) for i in range(14)]
        dims += [64] * 14
    for layer in range(22):
        seeds += [I.mha_seed(42 ^ layer, i) for i in range(4)]
        dims += [64] * 4
    seeds += [I.mha_seed(7, i) for i in range(8)]
    dims += [128] * 8
    for e in (0, 1, 2047):  # config 5: engine seed = sequence*32 + layer
        seeds += [I.mha_seed(e, i) for i in range(8)]
        dims += [128] * 8
    seeds += [1, 2, 0xFFFFFFFFFFFFFFFF, 0x8000000000000000]
    dims += [1024, 256, 128, 64]
    plus = np.zeros((len(seeds), 1024), np.uint8)
    for k, (s, n) in enumerate(zip(seeds, dims)):
        D = r.rademacher(n, s)
        plus[k, :n] = D > 0
    save("rademacher.npz", seeds=np.array(seeds, np.uint64), dims=np.array(dims, np.int32),
         plus=np.packbits(plus, axis=1))


def gen_fwht(r: Ref):
    out = {}
    rng = np.random.default_rng(11)
    for p in (64, 128, 256):
        D = r.rademacher(p, 1000 + p)
        x = rng.standard_normal((6, p), dtype=np.float32)
        x[0] = np.arange(p, dtype=np.float32) - p / 2  # small integers: exact stages
        x[1] = 0.0
        x[1, 3] = 1.0
        out[f"D{p}"] = D
        out[f"x{p}"] = x
        out[f"fwd{p}"] = np.stack([r.fwht_forward(v, D) for v in x])
        out[f"inv{p}"] = np.stack([r.fwht_inverse(v, D) for v in x])
    save("fwht.npz", **out)


def ordered(x) -> int:
    """Integer with the same order as the float32 x."""
    u = int(np.float32(x).view(np.uint32))
    return u if u < 0x80000000 else -(u & 0x7FFFFFFF)


def unordered(k: int) -> np.float32:
    u = k if k >= 0 else (-k) | 0x80000000
    return np.array([u], np.uint32).view(np.float32)[0]


def gen_quantize_fast(r: Ref):
    vals = np.linspace(-4.0, 4.0, 16001, dtype=np.float32)
    extra = np.array([0.0, -0.0, np.inf, -np.inf, np.nan, 1e-45, -1e-45, 3.4e38, -3.4e38],
                     np.float32)
    # thresholds and their float neighbours, found from the sweep's index changes
    vals = np.concatenate([vals, extra])
    out = {"vals": vals}
    for b in (2, 3, 4):
        idx = np.array([r.quantize_fast(float(v), b) for v in vals], np.uint8)
        near = []
        for i in np.nonzero(np.diff(idx[:16001].astype(int)))[0]:
            lo, hi = ordered(vals[i]), ordered(vals[i + 1])
            while hi - lo > 1:  # bisect on the float order to the exact threshold
                mid = (lo + hi) // 2
                if r.quantize_fast(float(unordered(mid)), b) == idx[i]:
                    lo = mid
                else:
                    hi = mid
            near += [unordered(lo), unordered(hi), unordered(hi + 1)]
        near = np.array(near, np.float32)
        out[f"edge_vals{b}"] = near
        out[f"edge_idx{b}"] = np.array([r.quantize_fast(float(v), b) for v in near], np.uint8)
        out[f"idx{b}"] = idx
    save("quantize_fast.npz", **out)


def gen_codec(r: Ref):
    out = {}
    for dim in (64, 128, 96, 48):
        seed = 0x5EED + dim
        for b in (2, 3, 4):
            codes, scales = [], []
            for fam in I.FAMILIES:
                for v in I.codec_inputs(dim, fam):
                    c, s = r.quantize_into(v, seed, b)
                    codes.append(c)
                    scales.append(s)
            out[f"codes_d{dim}_b{b}"] = np.stack(codes)
            out[f"scales_d{dim}_b{b}"] = np.array(scales, np.float32)
    out["families"] = np.array(I.FAMILIES)
    save("codec.npz", **out)


def gen_config1(r: Ref):
    c = I.CONFIG1
    K, V, q = I.config1_inputs()
    out = {"input_sha": sha(K, V, q)}
    for vm, hyb in MODES:
        heads = [r.head(c["dim"], c["k_bits"], c["v_bits"], c["cap"], I.mha_seed(42, h), vm, hyb)
                 for h in range(c["n_heads"])]
        for t in range(c["n"]):
            for h, hd in enumerate(heads):
                hd.append(K[t, h], V[t, h], t)
        tag = f"vm{int(vm * 100)}_h{hyb}"
        out[f"out_{tag}"] = np.stack([hd.compute(q[h])[0] for h, hd in enumerate(heads)])
        if vm == 0.0:
            for h, hd in enumerate(heads):
                d = ring_digest(hd)
                out[f"head{h}_state"] = np.array([d["head"], d["size"]], np.int32)
                out[f"head{h}_sha"] = d["sha"]
                for key in ("kc", "vc", "ks", "vs"):
                    out[f"head{h}_{key}_first"] = d[key][:64]
                    out[f"head{h}_{key}_last"] = d[key][-64:]
    save("config1.npz", **out)


def gen_config2(r: Ref):
    c = I.CONFIG2
    out = {}
    shas = []
    for vm, hyb in MODES:
        outs = np.zeros((c["n_layers"], c["n_heads"], c["dim"]), np.float32)
        for layer in range(c["n_layers"]):
            kb, vb, base, K, V, q = I.config2_layer(layer)
            if vm == 0.0:
                shas.append(sha(K, V, q))
            for h in range(c["n_heads"]):
                hd = r.head(c["dim"], kb, vb, c["cap"], I.mha_seed(base, h), vm, hyb)
                for t in range(c["n"]):
                    hd.append(K[t, h], V[t, h], t)
                outs[layer, h] = hd.compute(q[h])[0]
                if vm == 0.0 and h == 0:
                    out[f"ring_sha_l{layer}"] = ring_digest(hd)["sha"]
        out[f"out_vm{int(vm * 100)}_h{hyb}"] = outs
    out["input_sha"] = np.array(shas)
    save("config2.npz", **out)


CONFIG3_STEPS = (0, 1, 127, 255)


def gen_config3(r: Ref):
    c = I.CONFIG3
    out = {}
    for vm, hyb in MODES:
        outs = np.zeros((len(CONFIG3_STEPS), c["n_layers"], c["n_heads"], c["dim"]), np.float32)
        for layer in range(c["n_layers"]):
            kb, vb, base, K, V, Q = I.config3_layer(layer)
            for h in range(c["n_heads"]):
                hd = r.head(c["dim"], kb, vb, c["cap"], I.mha_seed(base, h), vm, hyb)
                for t in range(c["bulk"]):
                    hd.append(K[t, h], V[t, h], t)
                for s in range(c["steps"]):
                    hd.append(K[c["bulk"] + s, h], V[c["bulk"] + s, h], c["bulk"] + s)
                    if s in CONFIG3_STEPS:
                        outs[CONFIG3_STEPS.index(s), layer, h] = hd.compute(Q[s, h])[0]
        out[f"out_vm{int(vm * 100)}_h{hyb}"] = outs
    out["steps"] = np.array(CONFIG3_STEPS, np.int32)
    save("config3.npz", **out)


def gen_config4(r: Ref):
    c = I.CONFIG4
    Q = I.config4_queries()
    out = {}
    for vm, hyb in MODES:
        heads = [r.head(c["dim"], c["k_bits"], c["v_bits"], c["cap"], I.mha_seed(7, h), vm, hyb)
                 for h in range(c["n_heads"])]
        for ch in range((c["n"] + c["chunk"] - 1) // c["chunk"]):
            K, V = I.config4_chunk(ch)
            for t in range(K.shape[0]):
                for h, hd in enumerate(heads):
                    hd.append(K[t, h], V[t, h], ch * c["chunk"] + t)
        tag = f"vm{int(vm * 100)}_h{hyb}"
        out[f"out_{tag}"] = np.stack([np.stack([hd.compute(Q[qi, h])[0] for h, hd in
                                                enumerate(heads)]) for qi in range(8)])
        if vm == 0.0:
            for h, hd in enumerate(heads):
                d = ring_digest(hd)
                out[f"head{h}_state"] = np.array([d["head"], d["size"]], np.int32)
                out[f"head{h}_sha"] = d["sha"]
                if h < 2:
                    for key in ("kc", "vc", "ks", "vs"):
                        out[f"head{h}_{key}_wrap"] = d[key][7200:7264]
    save("config4.npz", **out)


def gen_ties(r: Ref):
    c = I.TIE_SHAPE
    out = {}
    for n, kind in I.TIE_CASES:
        K, V, q, seed = I.tie_inputs(n, kind)
        hd = r.head(c["dim"], c["k_bits"], c["v_bits"], n, seed, c["v_mass"], 0)
        for t in range(n):
            hd.append(K[t], V[t], t)
        out[f"out_{kind}{n}"] = hd.compute(q)[0]
    save("ties.npz", **out)


def main():
    if not Ref.available:
        sys.exit("oracle/_ref/libadaptq_ref.so is missing: run `make -C oracle ref` "
                 "(needs /root/reference)")
    r = Ref()
    only = sys.argv[1:]  # generator names, e.g. gen_ties; default: all
    for fn in (gen_rademacher, gen_fwht, gen_quantize_fast, gen_codec, gen_config1,
               gen_config2, gen_config3, gen_config4, gen_ties):
        if not only or fn.__name__ in only:
            fn(r)


if __name__ == "__main__":
    main()
