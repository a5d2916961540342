"""The reference's own numerical spread across its build flavours.

Runs the reference's hot-path sources compiled in place under four flavours
(oracle/Makefile targets `ref` and `flavours`):

  base    -std=c++17 -O3 -ffp-contract=off (oracle/_ref/libadaptq_ref.so, the
          flavour every golden fixture comes from)
  gnu     -std=gnu++17 -O3 -fopenmp: CMake's flags (CMakeLists.txt:4, :17);
          GCC's default in GNU mode contracts a*b+c to FMA where the target
          allows it
  native  -std=c++17 -O3 -fopenmp -march=native: setup.py's (setup.py:25, :38),
          the flavour the pip package's Engine uses
  scalar  base with __builtin_cpu_supports defined to 0: AttentionHead::compute
          takes its scalar path (attention.cpp:635-659) instead of the AVX2
          one (:606-633)

and writes tests/golden/ref_flavours.json:

  codec    per flavour, over the codec fixture inputs (inputs.codec_inputs:
           dims 64/128/96/48 x bits 2/3/4 x every family): vectors whose
           packed codes differ from base, and whose scales differ
  rings    per flavour, configs 1-4: ring slots (K or V codes or scales)
           that differ from base
  outputs  per flavour, configs 1-4 in both (v_mass, hybrid) modes against
           base: the worst norm-wise error max|y - r| / max|r| per head, and
           the worst elementwise relative error over entries with |r| >=
           1e-3 max|r| (the statistics of tests/gpu_head.py)
  floor    scalar against base, configs 1-4 with v_mass = 0 and hybrid 0
           (the scalar path ignores v_mass): the same two statistics -- the
           reference's own AVX2-vs-scalar spread on the same inputs
  exact    base and scalar against float64 softmax attention over the same
           dequantised ring (K^ = scale D H CB[codes] / p, fp32 keys as
           stored), configs 1-4 with v_mass = 0 and hybrid 0: how far the
           reference's own fp32 results sit from the exact value
  The WIDE cases of inputs.py (padded 512 and 1024) add to rings, outputs,
  floor and exact with v_mass 0 and hybrid 0.

    make -C oracle ref flavours && python tests/golden/ref_flavours.py
"""
from __future__ import annotations

import json
import os
import sys

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(os.path.dirname(HERE))
sys.path.insert(0, os.path.join(ROOT, "oracle"))
sys.path.insert(0, HERE)

from bind import Oracle, Ref  # noqa: E402
import exact64 as X  # noqa: E402
import inputs as I  # noqa: E402

REF_DIR = os.path.join(ROOT, "oracle", "_ref")
FLAVOURS = {f: os.path.join(REF_DIR, f"libadaptq_ref_{f}.so") for f in ("gnu", "native", "scalar")}
FLAVOURS["base"] = os.path.join(REF_DIR, "libadaptq_ref.so")
MODES = [(0.0, 0), (0.95, 512)]


stats = X.stats


def codec(refs):
    res = {}
    for dim in (64, 128, 96, 48):
        seed = 0x5EED + dim
        for b in (2, 3, 4):
            for fam in I.FAMILIES:
                for v in I.codec_inputs(dim, fam):
                    got = {f: r.quantize_into(v, seed, b) for f, r in refs.items()}
                    c0, s0 = got["base"]
                    for f, (c, s) in got.items():
                        e = res.setdefault(f, {"vectors": 0, "codes_differ": 0, "scales_differ": 0})
                        e["vectors"] += 1
                        e["codes_differ"] += int(c.tobytes() != c0.tobytes())
                        e["scales_differ"] += int(np.float32(s).tobytes() != np.float32(s0).tobytes())
    return res


def heads_of(cfg_name, r, vm, hyb):
    """(label, head, query) of every head of a config, rings filled."""
    out = []
    if cfg_name == "config1":
        c = I.CONFIG1
        K, V, q = I.config1_inputs()
        hs = [r.head(c["dim"], c["k_bits"], c["v_bits"], c["cap"], I.mha_seed(42, h), vm, hyb)
              for h in range(c["n_heads"])]
        for t in range(c["n"]):
            for h, hd in enumerate(hs):
                hd.append(K[t, h], V[t, h], t)
        out = [(f"h{h}", hd, q[h], (c["k_bits"], c["v_bits"], I.mha_seed(42, h)))
               for h, hd in enumerate(hs)]
    elif cfg_name == "config2":
        c = I.CONFIG2
        for layer in range(c["n_layers"]):
            kb, vb, base, K, V, q = I.config2_layer(layer)
            for h in range(c["n_heads"]):
                hd = r.head(c["dim"], kb, vb, c["cap"], I.mha_seed(base, h), vm, hyb)
                for t in range(c["n"]):
                    hd.append(K[t, h], V[t, h], t)
                out.append((f"l{layer}h{h}", hd, q[h], (kb, vb, I.mha_seed(base, h))))
    elif cfg_name == "config3":
        c = I.CONFIG3
        for layer in range(c["n_layers"]):
            kb, vb, base, K, V, Q = I.config3_layer(layer)
            for h in range(c["n_heads"]):
                hd = r.head(c["dim"], kb, vb, c["cap"], I.mha_seed(base, h), vm, hyb)
                for t in range(c["bulk"] + 1):  # the bulk, then step 0's token
                    hd.append(K[t, h], V[t, h], t)
                out.append((f"l{layer}h{h}", hd, Q[0, h], (kb, vb, I.mha_seed(base, h))))
    elif cfg_name in I.WIDE:
        c = I.WIDE[cfg_name]
        K, V, q = I.wide_inputs(cfg_name)
        base = c["base_seed"]
        hs = [r.head(c["dim"], c["k_bits"], c["v_bits"], c["cap"], I.mha_seed(base, h), vm, hyb)
              for h in range(c["n_heads"])]
        for t in range(c["n"]):
            for h, hd in enumerate(hs):
                hd.append(K[t, h], V[t, h], t)
        out = [(f"h{h}", hd, q[h], (c["k_bits"], c["v_bits"], I.mha_seed(base, h)))
               for h, hd in enumerate(hs)]
    else:
        c = I.CONFIG4
        Q = I.config4_queries()
        hs = [r.head(c["dim"], c["k_bits"], c["v_bits"], c["cap"], I.mha_seed(7, h), vm, hyb)
              for h in range(c["n_heads"])]
        for ch in range((c["n"] + c["chunk"] - 1) // c["chunk"]):
            K, V = I.config4_chunk(ch)
            for t in range(K.shape[0]):
                for h, hd in enumerate(hs):
                    hd.append(K[t, h], V[t, h], ch * c["chunk"] + t)
        out = [(f"h{h}q{qi}", hd, Q[qi, h], (c["k_bits"], c["v_bits"], I.mha_seed(7, h)))
               for qi in range(8) for h, hd in enumerate(hs)]
    return out


def exact(ref, hd, q, kb, vb, seed, cb):
    """float64 attention over the dequantised ring of reference head hd."""
    inf = hd.info()
    p = 1
    while p < hd.dim:
        p <<= 1
    kc, vc, ks, vs = hd.read_slots(0, inf["size"])
    return X.attention(kc, vc, ks, vs, ref.rademacher(p, seed), kb, vb, hd.dim, q, cb)


def ring_diff(a, b):
    ia, ib = a.info(), b.info()
    assert ia["size"] == ib["size"]
    ka, va, sa, ta = a.read_slots(0, ia["size"])
    kb, vb, sb, tb = b.read_slots(0, ib["size"])
    diff = (np.any(ka != kb, axis=1) | np.any(va != vb, axis=1) |
            (sa.view(np.uint32) != sb.view(np.uint32)) | (ta.view(np.uint32) != tb.view(np.uint32)))
    return int(diff.sum()), int(diff.size)


def configs(refs):
    cb = {b: Oracle().codebook(b).astype(np.float64) for b in (2, 3, 4)}
    rings, outs, floor, ex = {}, {}, {}, {}
    for cfg in ("config1", "config2", "config3", "config4") + tuple(I.WIDE):
        print(cfg, flush=True)
        for vm, hyb in (MODES if cfg.startswith("config") else MODES[:1]):
            tag = f"{cfg}_vm{int(vm * 100)}_h{hyb}"
            per = {f: heads_of(cfg, r, vm, hyb) for f, r in refs.items() if f != "scalar" or vm == 0.0}
            base = per["base"]
            ys0 = [hd.compute(q)[0] for _, hd, q, _ in base]
            if vm == 0.0:
                xs = [exact(refs["base"], hd, q, *m, cb) for _, hd, q, m in base]
                ys1 = [hd.compute(q)[0] for _, hd, q, _ in per["scalar"]]
                for f, ys in (("base", ys0), ("scalar", ys1)):
                    st = [stats(y, x) for y, x in zip(ys, xs)]
                    ex.setdefault(f, {})[tag] = {"norm_max": max(t[0] for t in st),
                                                 "elem_max": max(t[1] for t in st),
                                                 "heads": len(st)}
            for f, hs in per.items():
                if f == "base":
                    continue
                ys = [hd.compute(q)[0] for _, hd, q, _ in hs]
                st = [stats(y, y0) for y, y0 in zip(ys, ys0)]
                entry = {"norm_max": max(s[0] for s in st), "elem_max": max(s[1] for s in st),
                         "heads": len(st)}
                if f == "scalar":
                    if hyb == 0:
                        floor[tag] = entry
                    continue
                outs.setdefault(f, {})[tag] = entry
                if vm == 0.0:
                    nd = [ring_diff(hd, hd0) for (_, hd, _, _), (_, hd0, _, _) in zip(hs, base)]
                    rings.setdefault(f, {})[cfg] = {"slots_differ": sum(x[0] for x in nd),
                                                    "slots": sum(x[1] for x in nd)}
    return rings, outs, floor, ex


def main():
    missing = [p for p in FLAVOURS.values() if not os.path.exists(p)]
    if missing:
        sys.exit(f"missing {missing}: run `make -C oracle ref flavours` (needs /root/reference)")
    refs = {f: Ref(p) for f, p in FLAVOURS.items()}
    res = {"codec": codec(refs)}
    res["rings"], res["outputs"], res["floor"], res["exact"] = configs(refs)
    path = os.path.join(HERE, "ref_flavours.json")
    with open(path, "w") as f:
        json.dump(res, f, indent=1, sort_keys=True)
    print(json.dumps(res, indent=1, sort_keys=True))


if __name__ == "__main__":
    main()
