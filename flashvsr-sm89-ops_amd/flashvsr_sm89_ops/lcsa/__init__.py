"""Block-sparse attention (LCSA) for the FlashVSR DiT: HIP kernels on gfx950."""
from .draft import draft_block_mask, draft_index, generate_draft_block_mask  # noqa: F401
from .hip_lcsa import (block_sparse_attention, block_sparse_attention_bhsd,  # noqa: F401
                       block_sparse_attention_strided, block_index, build_csr)
