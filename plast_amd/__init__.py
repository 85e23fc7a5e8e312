"""plast_amd — MI355X (gfx950) backend for plast's elementwise / broadcast / reduction hot path.

The product is the C-ABI library `libplast_hip.so` (include/plast_hip.h), whose entry points fill
the GPU slots of the reference's `Op` table. This package builds it (`plast_amd.build`) and wraps
it for Python callers (`plast_amd.runtime`, `plast_amd.ops`).
"""
from . import abi  # noqa: F401

__all__ = ["abi", "build", "runtime", "ops"]
