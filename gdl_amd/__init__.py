"""gdl_amd — MI355X (gfx950) implementation of GeoEmbodied's point-cloud geometry kernels.

Farthest point sampling, KNN, radius graph, CSR build and segment reduce run as hand-written
HIP kernels in ``lib/libgeoembodied_hip.so`` behind the C ABI of ``include/geo_api.h``; the
Python modules mirror the reference's ``geoembodied.csrc`` dispatcher and
``geoembodied.functional`` signatures.  Import ``geoembodied`` to use the reference's module
paths.
"""

__version__ = "0.1.0"

from gdl_amd import _native  # noqa: F401


def build_info() -> str:
    """Library build string (target arch, compiler, flags)."""
    return _native.build_info()
