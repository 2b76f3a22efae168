"""flashvsr_sm89_ops — the FlashVSR v1.1 Tiny DiT-block operator pack, MI355X
(gfx950) build.

Same package name, entry point (`enable(pipe)`) and op signatures as
aireet/flashvsr-sm89-ops; every op runs hand-written HIP kernels from
libfvsr.so through a C ABI (include/fvsr.h).  Importing the package installs
the HIP-backed ``block_sparse_attn`` module (see compat_bsa), so import it
before diffsynth, whose DiT imports block_sparse_attn at module load.

What differs from the reference package at its public surface:
- the tiling helpers (``plan_tiles``, ``render_tiled``, ``auto_tile_limits``,
  ``tile_weight``) are not part of this build: they drive the pipeline over
  spatial tiles and call none of these ops, so they stay with the reference;
  ``from flashvsr_sm89_ops import render_tiled`` raises ImportError;
- the reference's ops take bf16, fp16 or fp32 inputs and so do these
  (output in x's type; FP8Linear output bf16, a non-bf16 bias rounded to
  bf16 for its epilogue); this build's fused extensions and the ``enable()``
  block path take bf16, the dtype the FlashVSR DiT runs in;
- ``build_csr(keep)`` returns the reference's triple (host read of the
  largest count included); ``lcsa.block_index(keep)`` is the untrimmed form
  (``maxk = NK``, no host read) that the attention paths use.
"""
from .compat_bsa import active_backend, ensure_bsa_available

ensure_bsa_available()

from .fused_rms_rope import fused_rms_rope, fused_rms_rope_qk  # noqa: E402
from .fused_adaln import (fused_ln_modulate, fused_gate_add, fused_ln_modulate_quant,  # noqa: E402
                          layer_norm, layer_norm_quant)
from .fp8_quant import quantize_fp8, quantize_weight_fp8, FP8_MAX  # noqa: E402
from .fp8_linear import (FP8Linear, convert_linears_fp8, fp8_gemm,  # noqa: E402
                         load_fp8_weights, save_fp8_weights)
from .fp8_ffn import FP8FFN, convert_ffn_fp8, fused_gelu_quant_fp8  # noqa: E402
from .integrate import enable  # noqa: E402
from .lcsa import block_sparse_attention, build_csr, draft_block_mask  # noqa: E402
from .cross_attn import cross_attention, cross_attention_residual  # noqa: E402

__version__ = "0.1.0"

__all__ = [
    "enable",
    "fused_rms_rope",
    "fused_rms_rope_qk",
    "fused_ln_modulate",
    "fused_ln_modulate_quant",
    "fused_gate_add",
    "layer_norm",
    "layer_norm_quant",
    "quantize_fp8",
    "quantize_weight_fp8",
    "FP8_MAX",
    "FP8Linear",
    "convert_linears_fp8",
    "save_fp8_weights",
    "load_fp8_weights",
    "fp8_gemm",
    "FP8FFN",
    "convert_ffn_fp8",
    "fused_gelu_quant_fp8",
    "block_sparse_attention",
    "build_csr",
    "draft_block_mask",
    "cross_attention",
    "cross_attention_residual",
    "active_backend",
    "ensure_bsa_available",
]
