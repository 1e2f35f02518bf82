"""laya_hip: the MI355X (gfx950) backend for laya-js' tensor-backend contract.

- `HipBackend` / `createHipBackend`: the `Backend` contract on
  libhipbackend.so (hand-written HIP kernels, one stream).
- `compose`, `host`, `modernbert`, `model`: host-side mirrors of the
  reference's compose helpers, host types, ModernBERT encoder and laya
  decision model, so callers run unchanged on this backend.

Importing the package does not touch the GPU; creating a backend loads the
library and fails loudly when it is missing.
"""
from .host import HostQuantized, HostTensor, QuantizedLinearOptions, QuantizedTensor, host  # noqa: F401

__all__ = ["HipBackend", "createHipBackend", "HostTensor", "HostQuantized", "QuantizedTensor", "host"]


def __getattr__(name):
    if name in ("HipBackend", "createHipBackend"):
        from . import backend
        return getattr(backend, name)
    raise AttributeError(name)
