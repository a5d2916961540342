"""adaptq_amd -- AdapTQ's KV-cache hot path (append + decode over packed K/V)
as hand-written gfx950 HIP kernels behind the reference's C ABI.

- ``adaptq_amd._lib``: ctypes binding of libadaptq.so (include/adaptq.h).
- ``adaptq_amd.core.Engine``: the reference's Python Engine over the
  pybind11 module ``adaptq_amd.adaptq_py``.

Build with ``python -m adaptq_amd.build``.  Importing never touches the GPU.
"""
__version__ = "0.1.0"

from ._lib import lib, last_error  # noqa: F401  (raises ImportError when unbuilt)


def __getattr__(name):
    if name == "Engine":
        from .core import Engine
        return Engine
    raise AttributeError(name)
