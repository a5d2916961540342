"""Packed-ring snapshots (adaptq_snapshot_save / _load, AQSS v2): the library's
file equals tests/aqss.py's bytes built from the rings read back through
adaptq_read_slots (logical order), the reference's own loader reads it and its
re-save is byte-identical, and loading restores rings that decode as before."""
import ctypes as C

import numpy as np
import pytest

import aqss
from adaptq_amd import _lib
from bind import SnapshotRef
from gpu_head import GpuHead, err, rel_err, same_bits

pytestmark = pytest.mark.gpu
L = _lib.lib


def _layers(n_layers, H, dim, kb, vb, cap, seed=3, vm=0.0, hyb=0):
    ms = [L.adaptq_mha_create(H, dim, kb, vb, cap, seed + l, vm, hyb) for l in range(n_layers)]
    assert all(ms), err()
    return ms


def _arr(ms):
    return (C.c_void_p * len(ms))(*ms)


def _logical(head: GpuHead):
    """Cached tokens oldest first: (k rows, v rows, k scales, v scales)."""
    i = head.info()
    n, cap = i["size"], i["cap"]
    slots = [(i["head"] - n + cap + t) % cap for t in range(n)]
    kc, vc, ks, vs = head.read_slots(0, cap) if cap else (None,) * 4
    if n == 0:
        return (np.zeros((0, i["k_pb"]), np.uint8), np.zeros((0, i["v_pb"]), np.uint8),
                np.zeros(0, np.float32), np.zeros(0, np.float32))
    return kc[slots], vc[slots], ks[slots], vs[slots]


def _expected_bytes(ms, H, dim, kb, vb):
    blocks, n_tok = [], 0
    for layer, m in enumerate(ms):
        for h in range(H):
            g = GpuHead.wrap(L.adaptq_mha_head(m, h), dim)
            kr, vr, ks, vs = _logical(g)
            i = g.info()
            n_tok = max(n_tok, len(ks))
            blocks.append(aqss.head_block(layer, h, kr, vr, ks, vs, kb, vb, max(i["k_pb"], i["v_pb"])))
    return aqss.snapshot(len(ms), H, dim, kb, n_tok, blocks)


def _fill(ms, H, dim, sizes, rng):
    for layer, m in enumerate(ms):
        for h in range(H):
            for t in range(sizes[layer][h]):
                k, v = rng.standard_normal((2, dim)).astype(np.float32)
                L.adaptq_mha_append(m, h, _lib.fptr(k), _lib.fptr(v), t)


@pytest.mark.parametrize("dim,kb,vb", [(64, 4, 2), (128, 4, 4), (96, 3, 2), (64, 2, 16)])
def test_snapshot_round_trip(tmp_path, dim, kb, vb):
    print(f"snapshot d{dim} k{kb}v{vb}", flush=True)
    H, cap = 3, 256
    sizes = [[400, 37, 256], [100, 0, 1]]  # wrapped, partial, exactly full, empty
    rng = np.random.default_rng(dim + kb)
    ms = _layers(2, H, dim, kb, vb, cap)
    _fill(ms, H, dim, sizes, rng)
    path = tmp_path / "s.aqss"
    assert L.adaptq_snapshot_save(_arr(ms), 2, str(path).encode()) == 0, err()
    data = path.read_bytes()
    assert data == _expected_bytes(ms, H, dim, kb, vb)

    if SnapshotRef.available:
        ref = SnapshotRef()
        snap = ref.load(str(path))
        assert (snap["n_layers"], snap["n_heads"], snap["dim"], snap["bits"]) == (2, H, dim, kb)
        assert [h["cache_size"] for h in snap["heads"]] == [min(s, cap) for l in sizes for s in l]
        ref.resave(str(path), str(tmp_path / "r.aqss"))
        assert (tmp_path / "r.aqss").read_bytes() == data

    qs = rng.standard_normal((2, H, dim)).astype(np.float32)
    before = np.zeros_like(qs)
    for layer, m in enumerate(ms):
        for h in range(H):
            L.adaptq_mha_compute(m, h, _lib.fptr(qs[layer, h]), _lib.fptr(before[layer, h]))

    fresh = _layers(2, H, dim, kb, vb, cap)
    _fill(fresh, H, dim, [[5, 5, 5], [5, 5, 5]], rng)  # replaced by the load
    assert L.adaptq_snapshot_load(_arr(fresh), 2, str(path).encode()) == 0, err()
    for layer in range(2):
        for h in range(H):
            a = GpuHead.wrap(L.adaptq_mha_head(ms[layer], h), dim)
            b = GpuHead.wrap(L.adaptq_mha_head(fresh[layer], h), dim)
            n = min(sizes[layer][h], cap)
            assert b.info()["size"] == n and b.info()["head"] == n % cap
            for x, y in zip(_logical(a), _logical(b)):
                assert same_bits(x, y)
            out = np.zeros(dim, np.float32)
            assert L.adaptq_mha_compute(fresh[layer], h, _lib.fptr(qs[layer, h]), _lib.fptr(out)) == n
            assert rel_err(out, before[layer, h]) <= 1e-5 if n else not out.any()
    path2 = tmp_path / "s2.aqss"
    assert L.adaptq_snapshot_save(_arr(fresh), 2, str(path2).encode()) == 0, err()
    assert path2.read_bytes() == data
    # appends continue after the restored tokens
    k, v = rng.standard_normal((2, dim)).astype(np.float32)
    L.adaptq_mha_append(fresh[1], 1, _lib.fptr(k), _lib.fptr(v), 0)
    assert GpuHead.wrap(L.adaptq_mha_head(fresh[1], 1), dim).info()["size"] == 1
    for m in ms + fresh:
        L.adaptq_mha_destroy(m)


def test_snapshot_reference_rejects_fp32_keys(tmp_path):
    """bits = 16 is written for fp32 keys; the reference's loader accepts only
    2..4 (session_snapshot.cpp:304-305), this library's accepts it."""
    if not SnapshotRef.available:
        pytest.skip("oracle/_ref/libsnapshot_ref.so not built")
    ms = _layers(1, 2, 64, 16, 2, 64)
    _fill(ms, 2, 64, [[10, 3]], np.random.default_rng(0))
    path = tmp_path / "f.aqss"
    assert L.adaptq_snapshot_save(_arr(ms), 1, str(path).encode()) == 0, err()
    with pytest.raises(ValueError, match="invalid bits"):
        SnapshotRef().load(str(path))
    assert L.adaptq_snapshot_load(_arr(ms), 1, str(path).encode()) == 0, err()
    L.adaptq_mha_destroy(ms[0])


def test_snapshot_load_refusals_change_nothing(tmp_path):
    H, dim, cap = 2, 64, 128
    src = _layers(2, H, dim, 4, 2, cap)
    _fill(src, H, dim, [[50, 60], [70, 80]], np.random.default_rng(5))
    path = tmp_path / "ok.aqss"
    assert L.adaptq_snapshot_save(_arr(src), 2, str(path).encode()) == 0, err()
    good = path.read_bytes()
    dst = _layers(2, H, dim, 4, 2, cap)
    _fill(dst, H, dim, [[7, 8], [9, 10]], np.random.default_rng(6))
    snap_before = tmp_path / "before.aqss"
    assert L.adaptq_snapshot_save(_arr(dst), 2, str(snap_before).encode()) == 0

    def refused(blob, msg, layers=dst, n=2):
        bad = tmp_path / "bad.aqss"
        bad.write_bytes(blob)
        assert L.adaptq_snapshot_load(_arr(layers), n, str(bad).encode()) == -1
        assert msg in err(), err()

    refused(b"XXXX" + good[4:], "magic")
    refused(good[:40], "truncated")
    refused(good[:-1], "truncated")
    refused(good[:4] + (3).to_bytes(4, "little") + good[8:], "version")
    refused(good, "shape", layers=dst[:1], n=1)
    other = _layers(2, H, 128, 4, 2, cap)
    refused(good, "shape", layers=other)
    small = _layers(2, H, dim, 4, 2, 32)
    refused(good, "cache size", layers=small)
    v3 = _layers(2, H, dim, 4, 3, cap)
    refused(good, "tags", layers=v3)  # 3-bit V rows are 24 B: slot bytes stay 32, the tags differ
    assert L.adaptq_snapshot_load(_arr(dst), 2, b"/nonexistent/x.aqss") == -1
    after = tmp_path / "after.aqss"
    assert L.adaptq_snapshot_save(_arr(dst), 2, str(after).encode()) == 0
    assert after.read_bytes() == snap_before.read_bytes()
    for m in src + dst + other + small + v3:
        L.adaptq_mha_destroy(m)
