"""The AQSS v2 snapshot layout, pinned against the reference's own loader and
saver (replay/session_snapshot.cpp compiled in place into oracle/_ref).  CPU
only: the bytes come from tests/aqss.py, which the GPU tests then compare with
the library's writer."""
import numpy as np
import pytest

import aqss
from bind import SnapshotRef

pytestmark = pytest.mark.skipif(not SnapshotRef.available,
                                reason="oracle/_ref/libsnapshot_ref.so not built")


def _blocks(rng, n_layers, n_heads, sizes, k_pb, v_pb, kb, vb):
    out, raw = [], []
    sb = max(k_pb, v_pb)
    for layer in range(n_layers):
        for head in range(n_heads):
            n = sizes[layer * n_heads + head]
            kr = rng.integers(0, 256, (n, k_pb), np.uint8)
            vr = rng.integers(0, 256, (n, v_pb), np.uint8)
            ks = rng.random(n, np.float32) + 0.5
            vs = rng.random(n, np.float32) + 0.5
            out.append(aqss.head_block(layer, head, kr, vr, ks, vs, kb, vb, sb))
            raw.append((kr, vr, ks, vs))
    return out, raw


def test_reference_loads_the_layout(tmp_path):
    rng = np.random.default_rng(0)
    sizes = [5, 0, 17, 3]
    blocks, raw = _blocks(rng, 2, 2, sizes, 32, 16, 4, 2)
    path = tmp_path / "a.aqss"
    path.write_bytes(aqss.snapshot(2, 2, 64, 4, max(sizes), blocks))
    snap = SnapshotRef().load(str(path))
    assert (snap["n_layers"], snap["n_heads"], snap["dim"], snap["bits"], snap["n_tokens"],
            snap["n_blocks"], snap["flags"]) == (2, 2, 64, 4, 17, 4, 0)
    for i, h in enumerate(snap["heads"]):
        kr, vr, ks, vs = raw[i]
        n = sizes[i]
        assert (h["layer"], h["head"], h["cache_size"], h["slot_bytes"]) == (i // 2, i % 2, n, 32)
        data = h["data"].reshape(2 * n, 32) if n else np.zeros((0, 32), np.uint8)
        assert np.array_equal(data[:n, :32], kr)
        assert np.array_equal(data[n:, :16], vr) and not data[n:, 16:].any()
        assert np.array_equal(h["scales"], np.concatenate([ks, vs]))
        assert list(h["tags"]) == [4] * n + [2] * n


def test_reference_resave_is_byte_identical(tmp_path):
    rng = np.random.default_rng(1)
    blocks, _ = _blocks(rng, 1, 3, [9, 1, 4], 64, 32, 4, 2)
    src, dst = tmp_path / "s.aqss", tmp_path / "d.aqss"
    src.write_bytes(aqss.snapshot(1, 3, 128, 4, 9, blocks))
    SnapshotRef().resave(str(src), str(dst))
    assert dst.read_bytes() == src.read_bytes()


@pytest.mark.parametrize("mutate,msg", [
    (lambda b: b"XXXX" + b[4:], "invalid magic"),
    (lambda b: b[:60], "exceeds remaining"),
    (lambda b: b[:-3], "exceeds remaining"),
    (lambda b: b[:8] + (3).to_bytes(4, "little") + b[12:], "inconsistent head count"),
])
def test_reference_refusals(tmp_path, mutate, msg):
    rng = np.random.default_rng(2)
    blocks, _ = _blocks(rng, 1, 2, [3, 2], 32, 16, 4, 2)
    path = tmp_path / "bad.aqss"
    path.write_bytes(mutate(aqss.snapshot(1, 2, 64, 4, 3, blocks)))
    with pytest.raises(ValueError, match=msg):
        SnapshotRef().load(str(path))
