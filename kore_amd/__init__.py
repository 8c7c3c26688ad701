"""kore_amd -- MI355X (gfx950) native fused layer kernels for KORE.

The product is ``libkore_hip.so`` (C ABI in ``include/kore_hip.h``);
``kore_amd.rocm`` is the host-side mirror of KORE's ``rocm_*`` op API.
"""
from ._lib import LIB_PATH, KoreLibraryError, load as load_library  # noqa: F401

__version__ = "0.1.0"
