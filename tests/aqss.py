"""AQSS v2 snapshot bytes written independently of the library (test helper).

Follows the layout documented in reference replay/session_snapshot.h:16-40
and written by session_snapshot.cpp:205-255, so tests can compare it with the
reference's own loader (test_snapshot_format.py) and with the library's
writer (test_gpu_snapshot.py)."""
import struct

import numpy as np

MAGIC = 0x41515353
TAG = {2: 0x02, 3: 0x03, 4: 0x04, 16: 0xFF}


def head_block(layer, head, k_rows, v_rows, k_scales, v_scales, k_bits, v_bits, slot_bytes):
    """One head: k_rows/v_rows (n, row bytes) uint8 in logical order."""
    n = len(k_scales)
    out = [struct.pack("<iiii", layer, head, n, slot_bytes), struct.pack("<Q", 2 * n * slot_bytes)]
    for rows in (k_rows, v_rows):
        pad = np.zeros((n, slot_bytes), np.uint8)
        if n:
            pad[:, :rows.shape[1]] = rows
        out.append(pad.tobytes())
    out.append(struct.pack("<i", 2 * n))
    out.append(np.concatenate([np.asarray(k_scales, np.float32),
                               np.asarray(v_scales, np.float32)]).astype("<f4").tobytes())
    out.append(struct.pack("<i", 2 * n))
    out.append(bytes([TAG[k_bits]] * n + [TAG[v_bits]] * n))
    return b"".join(out)


def snapshot(n_layers, n_heads, dim, bits, n_tokens, blocks, flags=0, tail=b""):
    hdr = struct.pack("<IIiiiiiiQ", MAGIC, 2, n_layers, n_heads, dim, bits, n_tokens,
                      n_layers * n_heads, flags)
    return hdr + b"".join(blocks) + tail
