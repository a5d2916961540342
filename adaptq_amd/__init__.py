"""adaptq_amd -- AdapTQ's KV-cache hot path (append + decode over packed K/V)
as hand-written gfx950 HIP kernels behind the reference's C ABI.

- ``adaptq_amd._lib``: ctypes binding of libadaptq.so (include/adaptq.h).
- ``adaptq_amd.core.Engine``: the reference's Python Engine over the
  pybind11 module ``adaptq_amd.adaptq_py``.
- ``adaptq_amd.torch_adapter.AdaptQAttention``: the reference's torch module.

Build with ``python -m adaptq_amd.build``.  Importing the package loads
nothing; the first use of ``lib``, ``last_error``, ``Engine`` or
``AdaptQAttention`` loads the built library and raises ImportError when it is
missing (there is no CPU fallback).  Importing never touches the GPU.
"""
__version__ = "0.1.0"


def __getattr__(name):
    if name in ("lib", "last_error"):
        from . import _lib
        return getattr(_lib, name)
    if name == "Engine":
        from .core import Engine
        return Engine
    if name == "AdaptQAttention":
        from .torch_adapter import AdaptQAttention
        return AdaptQAttention
    raise AttributeError(name)
