"""``block_sparse_attn`` stand-in backed by the gfx950 block-sparse attention.

Upstream FlashVSR does ``from block_sparse_attn import block_sparse_attn_func``
when its DiT module loads, so the pack must put a module of that name in
``sys.modules`` before diffsynth is imported (reference compat_bsa.py:1-18,
70-90).  Importing ``flashvsr_sm89_ops`` calls :func:`ensure_bsa_available`.

``FS89_LCSA`` keeps the reference's values:
  ``auto`` (default), ``hip`` or ``triton`` -> install the HIP-backed module
  (the only implementation in this pack; ``triton`` is accepted so existing
  environments keep working);
  ``bsa`` -> leave ``sys.modules`` alone (the caller supplies the module).
"""
from __future__ import annotations

import os
import sys
import types

STUB_VERSION = "flashvsr-mi355x-ops/hip-stub"


def _hip_block_sparse_attn_func(
    q, k, v,
    cu_seqlens_q, cu_seqlens_k,
    head_mask_type,
    streaming_info,
    attn_mask,
    max_seqlen_q, max_seqlen_k,
    dropout_p=0.0,
    deterministic=False,
    softmax_scale=None,
    is_causal=False,
    exact_streaming=False,
    return_attn_probs=False,
):
    """Drop-in for the one call shape FlashVSR uses (compat_bsa.py:31-67).

    q/k/v: [S, H, D] bf16 (batch 1) in window order; attn_mask:
    [1, H, Nq, Nk] bool block mask.  Returns [S, H, D]."""
    if streaming_info is not None or is_causal or dropout_p != 0.0 or return_attn_probs:
        raise NotImplementedError(
            "flashvsr_sm89_ops HIP LCSA covers the FlashVSR call shape only "
            "(dense-per-batch, no dropout, no causal, no attn-probs).")
    from .lcsa.hip_lcsa import block_sparse_attention_strided, BLOCK

    sq, heads, dim = q.shape
    keep = attn_mask[0] if attn_mask.dim() == 4 else attn_mask
    NQ, NK = keep.shape[1], keep.shape[2]
    assert sq == NQ * BLOCK and k.shape[0] == NK * BLOCK
    q2, k2, v2 = q.contiguous(), k.contiguous(), v.contiguous()
    out = q2.new_empty(q2.shape)
    return block_sparse_attention_strided(
        q2, k2, v2, keep, softmax_scale, heads=heads, head_dim=dim,
        q_strides=(heads * dim, dim), kv_strides=(heads * dim, dim), out=out)


def ensure_bsa_available():
    """Install the HIP-backed ``block_sparse_attn`` unless FS89_LCSA=bsa."""
    mode = os.environ.get("FS89_LCSA", "auto").lower()
    if mode == "bsa":
        return "bsa"
    mod = sys.modules.get("block_sparse_attn")
    if mod is not None and getattr(mod, "__version__", "") == STUB_VERSION:
        return "hip"
    stub = types.ModuleType("block_sparse_attn")
    stub.block_sparse_attn_func = _hip_block_sparse_attn_func
    stub.__version__ = STUB_VERSION
    sys.modules["block_sparse_attn"] = stub
    return "hip"


def active_backend():
    """Report which LCSA backend ``import block_sparse_attn`` resolves to
    (compat_bsa.py:93-98): ``hip``, ``bsa`` or ``unresolved``."""
    mod = sys.modules.get("block_sparse_attn")
    if mod is None:
        return "bsa" if os.environ.get("FS89_LCSA", "auto").lower() == "bsa" else "unresolved"
    return "hip" if getattr(mod, "__version__", "") == STUB_VERSION else "bsa"
