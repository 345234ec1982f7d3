"""Drop-in module paths of the reference package for the geometry kernels.

``geoembodied.csrc``, ``geoembodied.functional`` (with ``.fps``, ``.knn``, ``.radius_graph``,
``.segment_reduce`` and the fused ops added here) and ``geoembodied.kernels`` (with
``.triton_sph_harm``) are the ``gdl_amd`` modules themselves, registered under the reference's
names, so ``from geoembodied.functional.segment_reduce import segment_reduce``
(nn/modules/se3_conv.py:39), ``from geoembodied.csrc import fps_cuda``
(nn/modules/equivariant_pool.py:261) and ``from geoembodied.kernels.triton_sph_harm import
spherical_harmonics`` (nn/modules/spatial_graph.py:37) resolve to the gfx950 implementation.
``geoembodied.nn.modules.spatial_graph`` is the graph container of ``gdl_amd.graph`` and
``geoembodied.nn.modules.se3_conv`` the fused convolution of ``gdl_amd.se3_conv``; the rest of
the reference's ``nn`` package (the other layers and the models) is not part of this build, so
``geoembodied.nn`` holds only those two modules.
"""

import importlib
import sys
import types

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

# module paths whose gdl_amd module has another name
_RENAMED = (
    ("kernels.triton_sph_harm", "gdl_amd.kernels.sph_harm"),
    ("nn.modules.spatial_graph", "gdl_amd.graph"),
    ("nn.modules.se3_conv", "gdl_amd.se3_conv"),
)
for _name, _target in _RENAMED:
    _parts = _name.split(".")
    for _i in range(1, len(_parts)):  # namespace packages for missing parents (geoembodied.nn ...)
        _pkg = f"{__name__}." + ".".join(_parts[:_i])
        if _pkg not in sys.modules:
            _ns = types.ModuleType(_pkg)
            _ns.__path__ = []
            sys.modules[_pkg] = _ns
            _up = _pkg.rpartition(".")[0]
            setattr(sys.modules[_up], _parts[_i - 1], _ns)
    _mod = importlib.import_module(_target)
    sys.modules[f"{__name__}.{_name}"] = _mod
    setattr(sys.modules[f"{__name__}." + ".".join(_parts[:-1])], _parts[-1], _mod)

__version__ = importlib.import_module("gdl_amd").__version__
