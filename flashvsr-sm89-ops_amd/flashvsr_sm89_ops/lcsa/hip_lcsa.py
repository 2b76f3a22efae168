"""Block-sparse attention (LCSA) over 128-token blocks on gfx950.

Layout contract of the reference (flashvsr_sm89_ops/lcsa/triton_lcsa.py:1-11,74-94):
q/k/v arrive in window order ``[1, N_win*128, H*D]``; ``keep`` is a bool
block mask ``[H, NQ, NK]``; rows with no kept block output 0.

Differences in mechanism, not in results:
 - the block index is built on the device (``fvsr_block_index``, a ballot
   compaction); ``build_csr`` returns the reference's triple (rows trimmed to
   ``maxk = max(cnt.max(), 1)``, which reads ``cnt`` back to the host as the
   reference does, triton_lcsa.py:68), while the attention entry points use
   ``block_index``, the same rows untrimmed (``maxk = NK``) and no host read;
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


def block_index(keep: torch.Tensor):
    """keep [H, NQ, NK] bool -> (sel [H, NQ, NK] int32, cnt [H, NQ] int32, NK):
    each row of sel holds the kept block ids ascending, then the others
    ascending (the reference's stable descending argsort, triton_lcsa.py:67),
    untrimmed, so nothing is read back to the host."""
    _lib.require_gpu(keep)
    H, NQ, NK = keep.shape
    # a bool mask is already one byte per entry: no conversion kernel
    k8 = (keep.contiguous().view(torch.uint8) if keep.dtype == torch.bool
          else keep.to(torch.uint8).contiguous())
    sel = torch.empty((H, NQ, max(NK, 1)), dtype=torch.int32, device=keep.device)
    cnt = torch.empty((H, NQ), dtype=torch.int32, device=keep.device)
    _lib.check(_lib.lib().fvsr_block_index(k8.data_ptr(), H, NQ, NK, sel.data_ptr(),
                                           cnt.data_ptr(), _lib.stream(keep)), "block_index")
    return sel, cnt, max(NK, 1)


def build_csr(keep: torch.Tensor):
    """keep [H, NQ, NK] bool -> (sel [H, NQ, MAXK] int32, cnt [H, NQ] int32,
    MAXK), the reference's build_csr (triton_lcsa.py:64-71): MAXK =
    max(cnt.max(), 1), read back to the host, and sel the first MAXK entries
    of each row of block_index's order."""
    sel, cnt, _ = block_index(keep)
    maxk = max(int(cnt.max()), 1)
    return sel[..., :min(maxk, keep.shape[-1])].contiguous(), cnt, maxk


def _check_extent(t, rows: int, tok_stride: int, head_stride: int, heads: int, head_dim: int,
                  name: str):
    """t's storage holds `rows` tokens of `heads` heads at the given strides."""
    if rows <= 0:
        return
    need = (rows - 1) * tok_stride + (heads - 1) * head_stride + head_dim
    have = t.untyped_storage().nbytes() // t.element_size() - t.storage_offset()
    if min(tok_stride, head_stride) < 0 or need > have:
        raise ValueError(f"{name}: {rows} tokens x {heads} heads at strides ({tok_stride}, "
                         f"{head_stride}) need {need} elements, its storage holds {have}")


def _check_index(sel, cnt, maxk, H, NQ):
    for t, n in ((sel, "sel"), (cnt, "cnt")):
        _lib.require_dtype(t, torch.int32, n)
        if not t.is_contiguous():
            raise ValueError(f"block index {n} must be contiguous")
    if cnt.numel() != H * NQ or sel.numel() < H * NQ * maxk or maxk < 0:
        raise ValueError(f"block index of {tuple(sel.shape)} / {tuple(cnt.shape)} entries does "
                         f"not cover {H} heads x {NQ} query blocks x {maxk} key blocks")


def block_sparse_attention_strided(q, k, v, keep, sm_scale=None, *, heads: int, head_dim: int,
                                   q_strides, kv_strides, out=None, o_strides=None,
                                   q_map=None, kv_map=None, index=None, window=None):
    """General entry: q/k/v/out bf16 with (token stride, head stride) in
    elements; keep [H, NQ, NK] (or a prebuilt ``index=(sel, cnt, maxk)``).

    ``window=(frames, height, width, kv_raster)`` (instead of maps): q/out rows
    are raster tokens of that latent grid read in the (2, 8, 8) window order of
    WindowPartition3D (integrate.py:70-94), computed in the kernel
    (fvsr_bsa_fwd_window); kv_raster says k/v are raster tokens of the same
    grid too, otherwise they are already in window order.

    Checked before the launch: the index covers H x NQ rows of maxk entries
    (contiguous int32); without maps, q/out hold NQ*128 tokens and k/v NK*128
    at their strides; maps are int32 with at least NQ*128 / NK*128 entries;
    a window grid covers exactly NQ*128 tokens.
    Not checked (a host sync would be needed): that map entries lie inside
    their tensors and that sel/cnt values lie inside [0, NK) / [0, maxk], as
    build_csr and the device draft mask produce them."""
    for t, n in ((q, "q"), (k, "k"), (v, "v")):
        _lib.require_dtype(t, torch.bfloat16, n)
    if index is None:
        H, NQ, NK = keep.shape
    else:
        # The index alone does not say how many key blocks k/v hold: raster
        # k/v of the window grid hold NQ, otherwise the rows' width (NK for
        # block_index, at most NK for build_csr's trimmed rows) is used.
        H, NQ = index[1].shape
        NK = NQ if window is not None and window[3] else index[2]
    if window is not None:
        if q_map is not None or kv_map is not None:
            raise ValueError("give either token maps or a window grid, not both")
        frames, height, width, kv_raster = window
        if frames % 2 or height % 8 or width % 8 or frames * height * width != NQ * BLOCK:
            raise ValueError(f"window grid {frames}x{height}x{width} is not NQ={NQ} windows "
                             "of 2x8x8 tokens")
        if kv_raster and NK != NQ:
            raise ValueError("raster-order k/v need as many key blocks as query blocks")
    _lib.require_gpu(q, k, v, out, q_map, kv_map)
    sel, cnt, maxk = block_index(keep) if index is None else index
    if H != heads:
        raise ValueError(f"block mask has {H} heads, tensors have {heads}")
    _lib.require_gpu(sel, cnt)
    _check_index(sel, cnt, maxk, H, NQ)
    if sm_scale is None:
        sm_scale = 1.0 / math.sqrt(head_dim)
    if out is None:
        raise ValueError("out is required")
    _lib.require_dtype(out, torch.bfloat16, "out")
    o_strides = o_strides or q_strides
    if window is not None:
        _check_extent(q, NQ * BLOCK, *q_strides, heads, head_dim, "q")
        _check_extent(out, NQ * BLOCK, *o_strides, heads, head_dim, "out")
        _check_extent(k, NK * BLOCK, *kv_strides, heads, head_dim, "k")
        _check_extent(v, NK * BLOCK, *kv_strides, heads, head_dim, "v")
        rc = _lib.lib().fvsr_bsa_fwd_window(
            q.data_ptr(), k.data_ptr(), v.data_ptr(), out.data_ptr(),
            q_strides[0], q_strides[1], kv_strides[0], kv_strides[1], o_strides[0], o_strides[1],
            sel.data_ptr(), cnt.data_ptr(), maxk, H, NQ, NK, head_dim, float(sm_scale),
            frames, height, width, int(bool(kv_raster)), _lib.stream(q))
        _lib.check(rc, "block_sparse_attention")
        return out
    if (q_map is None) != (kv_map is None):
        raise ValueError("token maps come in pairs (q_map with kv_map)")
    if q_map is None:
        _check_extent(q, NQ * BLOCK, *q_strides, heads, head_dim, "q")
        _check_extent(out, NQ * BLOCK, *o_strides, heads, head_dim, "out")
        _check_extent(k, NK * BLOCK, *kv_strides, heads, head_dim, "k")
        _check_extent(v, NK * BLOCK, *kv_strides, heads, head_dim, "v")
    else:
        for m, n, want in ((q_map, "q_map", NQ * BLOCK), (kv_map, "kv_map", NK * BLOCK)):
            _lib.require_dtype(m, torch.int32, "token map")
            if not m.is_contiguous() or m.numel() < want:
                raise ValueError(f"{n} must be contiguous with at least {want} entries, "
                                 f"got {m.numel()}")
    rc = _lib.lib().fvsr_bsa_fwd(
        q.data_ptr(), k.data_ptr(), v.data_ptr(), out.data_ptr(),
        q_strides[0], q_strides[1], kv_strides[0], kv_strides[1], o_strides[0], o_strides[1],
        sel.data_ptr(), cnt.data_ptr(), maxk, H, NQ, NK, head_dim, float(sm_scale),
        _lib.ptr(q_map), _lib.ptr(kv_map), _lib.stream(q))
    _lib.check(rc, "block_sparse_attention")
    return out


def dense_attention_strided(q, k, v, sm_scale=None, *, heads: int, head_dim: int, q_strides,
                            kv_strides, out, o_strides=None):
    """softmax(Q K^T * sm_scale) V per head over all keys (fvsr_attn_dense):
    the attention with every key block kept, for the cross-attention over
    the cached prompt (integrate.py:132-143).  q/out hold a multiple of 128
    query tokens, k/v a multiple of 128 key tokens, at the given (token,
    head) strides in elements; no block index is involved."""
    for t, n in ((q, "q"), (k, "k"), (v, "v"), (out, "out")):
        _lib.require_dtype(t, torch.bfloat16, n)
    Lq, Lk = q.shape[0], k.shape[0]
    if Lq % BLOCK or Lk % BLOCK or v.shape[0] != Lk or out.shape[0] != Lq:
        raise ValueError(f"dense attention needs multiples of {BLOCK} tokens: q {Lq}, k {Lk}, "
                         f"v {v.shape[0]}, out {out.shape[0]}")
    o_strides = o_strides or q_strides
    _check_extent(q, Lq, *q_strides, heads, head_dim, "q")
    _check_extent(out, Lq, *o_strides, heads, head_dim, "out")
    _check_extent(k, Lk, *kv_strides, heads, head_dim, "k")
    _check_extent(v, Lk, *kv_strides, heads, head_dim, "v")
    _lib.require_gpu(q, k, v, out)
    if sm_scale is None:
        sm_scale = 1.0 / math.sqrt(head_dim)
    rc = _lib.lib().fvsr_attn_dense(
        q.data_ptr(), k.data_ptr(), v.data_ptr(), out.data_ptr(), q_strides[0], q_strides[1],
        kv_strides[0], kv_strides[1], o_strides[0], o_strides[1], heads, Lq // BLOCK,
        Lk // BLOCK, head_dim, float(sm_scale), _lib.stream(q))
    _lib.check(rc, "dense_attention")
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
