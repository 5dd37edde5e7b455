"""mtc.core.permutation (mtc/core/permutation.py): channel-permuted quadtree allocation."""

from tensorpack_amd.core.permutation import (PermutedQTAllocation, PermutedQuadtreeRD, channel_orders, index_bits,
                                             permuted_qt_dequant, unpermute)

__all__ = ["PermutedQTAllocation", "PermutedQuadtreeRD", "channel_orders", "index_bits", "permuted_qt_dequant",
           "unpermute"]
