"""mtc.core.quadtree (mtc/core/quadtree.py): QuadtreeRD, QTAllocation, qt_dequant, qt_allocate."""

from tensorpack_amd.core.quadtree import SPLIT_FLAG_BITS, QTAllocation, QuadtreeRD, qt_allocate, qt_dequant

__all__ = ["SPLIT_FLAG_BITS", "QTAllocation", "QuadtreeRD", "qt_allocate", "qt_dequant"]
