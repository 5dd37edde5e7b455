"""mtc.nn.layers: `LinearMTC` (a linear layer over a packed quadtree weight, in place of the
reference's cached-dequant `LinearMTCAdaptive`, mtc/nn/layers.py:115-151) and
`LinearMTCGroup` (layers that read one input, launched together)."""

from tensorpack_amd.nn import LinearMTC, LinearMTCGroup, seeded_fp32_weight

__all__ = ["LinearMTC", "LinearMTCGroup", "seeded_fp32_weight"]
