"""CPU restatement of the amilworks/Pack3D operator -- TEST INFRASTRUCTURE ONLY.

Importable only from ``tests/``, ``__graft_entry__.smoke()`` and the
``cpu_baseline`` leg of ``bench.py``.  See ``oracle/__init__.py`` for the
pinning status of each function.
"""
from .attention import PACK3DAttention
from .compression import compress_summaries
from .core import pack3d_reference, pack3d_reference_grads, validate_inputs
from .geometry import (Pack3DGeometry, TokenLayout, build_layout, grid_coordinates,
                       morton_codes, neighbor_offsets, prepare_geometry, reverse_adjacency)
from .rope import axial_rope, balanced_pairs, frequencies

__all__ = ["PACK3DAttention", "Pack3DGeometry", "TokenLayout", "axial_rope", "balanced_pairs",
           "build_layout", "compress_summaries", "frequencies", "grid_coordinates", "morton_codes",
           "neighbor_offsets", "pack3d_reference", "pack3d_reference_grads", "prepare_geometry", "reverse_adjacency",
           "validate_inputs"]
