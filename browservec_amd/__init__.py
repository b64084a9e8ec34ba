"""browservec_amd -- BrowserVec's data-parallel search path on MI355X (gfx950).

The native library (libbrowservec_hip.so, C ABI in include/browservec_hip.h)
holds the corpus in HBM and runs every scan, top-k and re-rank on the GPU.
This package is the host side: ctypes binding, ``VectorIndex`` classes and the
``BrowserVec`` orchestration of the reference (src/index.ts).
"""

from .browservec import BrowserVec, Store, normalize_in_place  # noqa: F401
from .index import DeviceContext, FlatHit, FlatIndex, GraphSearcher, IVFIndex, IVFQuantIndex, QuantIndex  # noqa: F401

__all__ = ["BrowserVec", "Store", "normalize_in_place", "DeviceContext", "FlatHit", "FlatIndex", "GraphSearcher", "QuantIndex",
           "IVFIndex", "IVFQuantIndex"]
