"""Block-sparse attention (LCSA) over 128-token blocks on gfx950.

Layout contract of the reference (flashvsr_sm89_ops/lcsa/triton_lcsa.py:1-11,74-94):
q/k/v arrive in window order ``[1, N_win*128, H*D]``; ``keep`` is a bool
block mask ``[H, NQ, NK]``; rows with no kept block output 0.

Differences in mechanism, not in results:
 - the block index is built on the device (``fvsr_block_index``, a ballot
   compaction) with ``MAXK = NK``, so there is no host sync
   (the reference's ``int(cnt.max())``, triton_lcsa.py:68);
 - the attention kernel reads only kept key blocks, with MFMA bf16 QK^T and
   PV and an fp32 online softmax.

``block_sparse_attention_strided`` takes any token/head strides and optional
token maps (window position -> stored token), e.g. the ``[1, H, S, D]``
layout or raster-order tensors read in window order without a copy.
"""
from __future__ import annotations

import math

import torch

from .. import _lib

BLOCK = 128


def build_csr(keep: torch.Tensor):
    """keep [H, NQ, NK] bool -> (sel [H, NQ, NK] int32, cnt [H, NQ] int32, NK).

    Kept block ids come first in ascending order (triton_lcsa.py:64-71); the
    entries after cnt are unspecified.  MAXK is NK, so nothing is read back to
    the host."""
    _lib.require_gpu(keep)
    H, NQ, NK = keep.shape
    k8 = keep.to(torch.uint8).contiguous()
    sel = torch.empty((H, NQ, max(NK, 1)), dtype=torch.int32, device=keep.device)
    cnt = torch.empty((H, NQ), dtype=torch.int32, device=keep.device)
    _lib.check(_lib.lib().fvsr_block_index(k8.data_ptr(), H, NQ, NK, sel.data_ptr(),
                                           cnt.data_ptr(), _lib.stream(keep)), "build_csr")
    return sel, cnt, max(NK, 1)


def block_sparse_attention_strided(q, k, v, keep, sm_scale=None, *, heads: int, head_dim: int,
                                   q_strides, kv_strides, out=None, o_strides=None,
                                   q_map=None, kv_map=None, index=None):
    """General entry: q/k/v/out bf16 with (token stride, head stride) in
    elements; keep [H, NQ, NK] (or a prebuilt ``index=(sel, cnt, maxk)``)."""
    _lib.require_gpu(q, k, v, out, q_map, kv_map)
    for t, n in ((q, "q"), (k, "k"), (v, "v")):
        _lib.require_dtype(t, torch.bfloat16, n)
    if index is None:
        sel, cnt, maxk = build_csr(keep)
        H, NQ, NK = keep.shape
    else:
        sel, cnt, maxk = index
        H, NQ = cnt.shape
        NK = maxk
    if H != heads:
        raise ValueError(f"block mask has {H} heads, tensors have {heads}")
    if sm_scale is None:
        sm_scale = 1.0 / math.sqrt(head_dim)
    if out is None:
        raise ValueError("out is required")
    o_strides = o_strides or q_strides
    for m in (q_map, kv_map):
        if m is not None:
            _lib.require_dtype(m, torch.int32, "token map")
    rc = _lib.lib().fvsr_bsa_fwd(
        q.data_ptr(), k.data_ptr(), v.data_ptr(), out.data_ptr(),
        q_strides[0], q_strides[1], kv_strides[0], kv_strides[1], o_strides[0], o_strides[1],
        sel.data_ptr(), cnt.data_ptr(), maxk, H, NQ, NK, head_dim, float(sm_scale),
        _lib.ptr(q_map), _lib.ptr(kv_map), _lib.stream(q))
    _lib.check(rc, "block_sparse_attention")
    return out


def block_sparse_attention(q, k, v, keep, sm_scale=None):
    """q/k/v: [1, L, H*D] bf16 in window order; keep: [H, L//128, K//128] bool.
    Returns [1, L, H*D] bf16.  Rows with no selected key blocks output 0
    (triton_lcsa.py:74-94)."""
    L, HD = q.shape[-2], q.shape[-1]
    H = keep.shape[0]
    D = HD // H
    NQ, NK = keep.shape[1], keep.shape[2]
    assert L == NQ * BLOCK and k.shape[1] == NK * BLOCK
    q2 = q.contiguous()
    k2 = k.contiguous()
    v2 = v.contiguous()
    out = torch.empty_like(q2)
    return block_sparse_attention_strided(
        q2, k2, v2, keep, sm_scale, heads=H, head_dim=D, q_strides=(HD, D),
        kv_strides=(HD, D), out=out)


def block_sparse_attention_bhsd(q, k, v, keep, sm_scale=None):
    """The same attention on [1, H, S, D] tensors (BASELINE C4 layout)."""
    _, H, S, D = q.shape
    Sk = k.shape[2]
    NQ, NK = keep.shape[1], keep.shape[2]
    assert S == NQ * BLOCK and Sk == NK * BLOCK and keep.shape[0] == H
    q2, k2, v2 = q.contiguous(), k.contiguous(), v.contiguous()
    out = torch.empty_like(q2)
    return block_sparse_attention_strided(
        q2, k2, v2, keep, sm_scale, heads=H, head_dim=D, q_strides=(D, S * D),
        kv_strides=(D, Sk * D), out=out)
