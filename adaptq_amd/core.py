"""Python API mirroring the reference's adaptq/core.py:9-83.

``Engine(dim, heads, k_bits=4, v_bits=4, capacity=4096, seed=42, v_mass=0.95,
hybrid_thresh=512)`` with ``append(k, v)``, ``compute(q)``, ``reset()`` and the
``kv_bytes`` property, over the pybind11 module ``adaptq_py.MHAContext`` built
from adaptq_amd/csrc/adapter_python.cpp.  Same defaults, shapes and errors as
the reference; the ring buffers live in GPU memory.

Where the reference loops over heads in Python (adaptq/core.py:45-74), this
Engine makes one call for all heads (``MHAContext.append_all`` /
``compute_all``): one append launch and one decode launch per step.
"""
from __future__ import annotations

import numpy as np

from . import adaptq_py  # noqa: F401  (built in-tree by adaptq_amd.build)


class Engine:
    def __init__(self, dim: int, heads: int, k_bits: int = 4, v_bits: int = 4,
                 capacity: int = 4096, seed: int = 42, v_mass: float = 0.95,
                 hybrid_thresh: int = 512):
        self.dim = dim
        self.heads = heads
        self.k_bits = k_bits
        self.v_bits = v_bits
        self.capacity = capacity
        self._ctx = adaptq_py.MHAContext(n_heads=heads, head_dim=dim, k_bits=k_bits,
                                         v_bits=v_bits, capacity=capacity, seed=seed,
                                         v_mass=v_mass, hybrid_thresh=hybrid_thresh)
        self.pos = 0

    def append(self, k: np.ndarray, v: np.ndarray) -> None:
        """Append one token's keys and values, each of shape (heads, dim)."""
        if k.shape != (self.heads, self.dim) or v.shape != (self.heads, self.dim):
            raise ValueError(f"k and v must be shape ({self.heads}, {self.dim})")
        self._ctx.append_all(np.ascontiguousarray(k, dtype=np.float32),
                             np.ascontiguousarray(v, dtype=np.float32), self.pos)
        self.pos += 1

    def compute(self, q: np.ndarray) -> np.ndarray:
        """Attention output for q of shape (heads, dim); returns (heads, dim)."""
        if q.shape != (self.heads, self.dim):
            raise ValueError(f"q must be shape ({self.heads}, {self.dim})")
        return np.asarray(self._ctx.compute_all(np.ascontiguousarray(q, dtype=np.float32)))

    def reset(self) -> None:
        self._ctx.reset()
        self.pos = 0

    @property
    def kv_bytes(self) -> int:
        return self._ctx.kv_bytes()
