"""scope_amd — the SCOPE attention hot path on MI355X (gfx950).

Pointer-driven block selection, block-sparse flash attention with the
spectral bias (forward and backward) and the fused mask statistics, as
hand-written HIP kernels behind a C ABI (``include/scope_amd.h``,
``libscope_amd.so``), with the reference's Python call surface on top:

* ``SpectralBias``       – model/attn_bias.py:68-874
* ``scope_attention``    – the FlexAttention calls of scoped_medium.py:422-476
* ``ScopeBlockMask``     – the BlockMask rows (kv_num_blocks, kv_indices)
* ``ops``                – one torch wrapper per C entry point
"""
from . import ops
from ._lib import ScopeLibraryError, load as load_library
from .attention import SpectralTerms, scope_attention
from .blockmask import ScopeBlockMask, create_blockmasks
from .spectral_bias import SpectralBias

__all__ = ["ops", "ScopeLibraryError", "load_library", "SpectralTerms", "scope_attention", "ScopeBlockMask", "create_blockmasks",
           "SpectralBias"]
