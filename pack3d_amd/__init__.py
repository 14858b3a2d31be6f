"""pack3d_amd: the PACK3D attention layer of amilworks/Pack3D on AMD MI355X (gfx950).

Public API mirrors ``pack3d`` (``src/pack3d/__init__.py``) with the ``hip``
backend: ``PACK3DAttention``, ``Pack3DGeometry``, ``TokenLayout``,
``build_layout``, ``prepare_geometry``, and the core ``pack3d_hip``
(the contract of ``pack3d_reference`` / ``pack3d_streamed``).
"""
from .attention import PACK3DAttention
from .core import pack3d_hip, pack3d_hip_rope
from .geometry import (Pack3DGeometry, TokenLayout, adopt_layout, build_layout, grid_coordinates, grid_tag,
                       prepare_geometry)
from .rope import balanced_pairs

__version__ = "0.1.0"
__all__ = ["PACK3DAttention", "Pack3DGeometry", "TokenLayout", "adopt_layout", "balanced_pairs", "build_layout",
           "grid_coordinates", "grid_tag", "pack3d_hip", "pack3d_hip_rope", "prepare_geometry"]
