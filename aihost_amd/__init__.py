"""aihost_amd -- gfx950 (MI355X) backend for AIHost's GGUF quantized matmul path.

The product is the C-ABI shared library ``_lib/libaihost_hip.so`` (header:
``include/aihost_hip.h``).  This package builds it (``build.py``), binds it
(``_native.py``) and mirrors the reference's device/operator interface on top
of it (``compute.py``).
"""
from . import _native  # noqa: F401

__all__ = ["_native"]
