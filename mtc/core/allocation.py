"""mtc.core.allocation (mtc/core/allocation.py): code ranges, scale search and uniform-block
RD allocation. The per-block candidate search runs in the C++/OpenMP libmtc_rd.so."""

from tensorpack_amd.core.allocation import (_ALPHAS, DEFAULT_MODES, META_BITS_PER_BLOCK, QRANGE,
                                            SCALE_FORMAT_META_BITS, RDAllocation, RDCandidates, _search_mode,
                                            from_blocks, quantize_blocks, rd_allocate, rd_allocate_pair,
                                            rd_candidates, rd_dequant, rd_select, to_blocks)
from tensorpack_amd.core.allocation import round_bf16 as _round_bf16

__all__ = ["DEFAULT_MODES", "META_BITS_PER_BLOCK", "QRANGE", "SCALE_FORMAT_META_BITS", "RDAllocation",
           "RDCandidates", "from_blocks", "quantize_blocks", "rd_allocate", "rd_allocate_pair", "rd_candidates",
           "rd_dequant", "rd_select", "to_blocks"]
