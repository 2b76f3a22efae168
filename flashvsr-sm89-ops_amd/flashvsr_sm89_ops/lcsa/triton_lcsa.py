"""Import-path compatibility: the reference exposes block-sparse attention as
``flashvsr_sm89_ops.lcsa.triton_lcsa`` (lcsa/triton_lcsa.py:64-94).  This pack
has no Triton code; the names resolve to the HIP implementation."""
from .hip_lcsa import BLOCK, block_sparse_attention, build_csr  # noqa: F401
