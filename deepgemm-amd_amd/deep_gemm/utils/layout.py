"""Layout helpers (reference deep_gemm/utils/layout.py:1-13)."""
from .. import (  # noqa: F401
    get_tma_aligned_size,
    get_mn_major_tma_aligned_tensor,
    get_mn_major_tma_aligned_packed_ue8m0_tensor,
    set_mk_alignment_for_contiguous_layout,
    get_mk_alignment_for_contiguous_layout,
    get_theoretical_mk_alignment_for_contiguous_layout,
)

get_m_alignment_for_contiguous_layout = get_mk_alignment_for_contiguous_layout
get_k_alignment_for_contiguous_layout = get_mk_alignment_for_contiguous_layout

__all__ = ['get_tma_aligned_size', 'get_mn_major_tma_aligned_tensor',
           'get_mn_major_tma_aligned_packed_ue8m0_tensor', 'set_mk_alignment_for_contiguous_layout',
           'get_mk_alignment_for_contiguous_layout', 'get_theoretical_mk_alignment_for_contiguous_layout',
           'get_m_alignment_for_contiguous_layout', 'get_k_alignment_for_contiguous_layout']
