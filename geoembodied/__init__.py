"""Drop-in module paths of the reference package for the geometry kernels.

``geoembodied.csrc``, ``geoembodied.functional`` (with ``.fps``, ``.knn``, ``.radius_graph``,
``.segment_reduce``) and ``geoembodied.kernels`` are the ``gdl_amd`` modules themselves,
registered under the reference's names, so ``from geoembodied.functional.segment_reduce import
segment_reduce`` (nn/modules/se3_conv.py:39) and ``from geoembodied.csrc import fps_cuda``
(nn/modules/equivariant_pool.py:261) resolve to the gfx950 implementation.
"""

import importlib
import sys

_ALIASES = (
    "csrc",
    "functional",
    "functional.adaptive",
    "functional.fps",
    "functional.gather",
    "functional.knn",
    "functional.radius_graph",
    "functional.segment_reduce",
    "functional.segment_softmax",
    "kernels",
)

for _name in _ALIASES:
    _mod = importlib.import_module(f"gdl_amd.{_name}")
    sys.modules[f"{__name__}.{_name}"] = _mod
    _parent, _, _leaf = _name.rpartition(".")
    setattr(sys.modules[f"{__name__}.{_parent}"] if _parent else sys.modules[__name__], _leaf, _mod)

__version__ = importlib.import_module("gdl_amd").__version__
