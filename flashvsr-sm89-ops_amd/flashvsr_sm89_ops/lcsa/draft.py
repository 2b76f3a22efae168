"""Draft block mask of the sparse self-attention, on the device.

Reference: ``draft_block_mask`` (flashvsr_sm89_ops/lcsa/reference.py:37-64),
the selection the reference obtains from ``dit.generate_draft_block_mask`` at
integrate.py:103-104: window-mean pooled q/k per 128-token block, scaled
scores per head, -inf outside the local rule, softmax over key blocks, and a
joint top-k per (head, query time row); ``keep = attn > thr``.

For bf16 q/k every stage is rounded to bf16 as torch rounds bf16 tensors
(mean, einsum, division by sqrt(D), softmax), so ties at the threshold fall
as they do in the reference.  ``fvsr_draft_block_mask`` runs the whole chain
in three launches and can write the block index (sel, cnt) that the
attention kernel consumes directly, without the bool mask or a host sync.
"""
from __future__ import annotations

import torch

from .. import _lib

BLOCK = 128


def _rows(x: torch.Tensor, name: str):
    """[N, 128, C] or [N*128, C] bf16 -> ([N*128, C] view, token stride)."""
    _lib.require_dtype(x, torch.bfloat16, name)
    x2 = x.reshape(-1, x.shape[-1])
    if x2.stride(-1) != 1 or x2.stride(0) % 8 or x2.data_ptr() % 16:
        x2 = x2.contiguous()
    return x2, x2.stride(0)


def _local_u8(local: torch.Tensor, device) -> torch.Tensor:
    if local.dim() != 2:
        raise ValueError(f"local mask must be [sq, sk], got {tuple(local.shape)}")
    if local.dtype == torch.bool and local.device == torch.device(device):
        return local.contiguous().view(torch.uint8)  # same bytes: no conversion kernel
    return local.to(device=device, dtype=torch.uint8).contiguous()


def draft_index(q: torch.Tensor, k: torch.Tensor, *, nheads: int, q_temporal: int,
                local: torch.Tensor, topk: int, nq: int | None = None, nk: int | None = None,
                q_map: torch.Tensor | None = None, k_map: torch.Tensor | None = None,
                want_keep: bool = False, want_index: bool = True):
    """General entry.  q/k bf16 with H*D channels per token, either in window
    order (``[N, 128, H*D]`` or ``[N*128, H*D]``) or any row order with an
    int32 map from block position to row (``q_map`` [nq*128], ``k_map``
    [nk*128]).  Returns ``(sel, cnt, maxk)`` for the attention kernel and/or
    the bool keep mask [H, NQ, NK]."""
    _lib.require_gpu(q, k, q_map, k_map)
    q2, qts = _rows(q, "q")
    k2, kts = _rows(k, "k")
    HD = q2.shape[1]
    if k2.shape[1] != HD or HD % nheads:
        raise ValueError(f"q has {HD} channels, k {k2.shape[1]}, heads {nheads}")
    D = HD // nheads
    NQ = nq if nq is not None else q2.shape[0] // BLOCK
    NK = nk if nk is not None else k2.shape[0] // BLOCK
    for m, n, name in ((q_map, NQ, "q_map"), (k_map, NK, "k_map")):
        if m is not None:
            _lib.require_dtype(m, torch.int32, name)
            if m.numel() != n * BLOCK or not m.is_contiguous():
                raise ValueError(f"{name} must be contiguous with {n * BLOCK} entries")
    if q_map is None and q2.shape[0] != NQ * BLOCK:
        raise ValueError("q rows must be a whole number of 128-token blocks")
    if k_map is None and k2.shape[0] != NK * BLOCK:
        raise ValueError("k rows must be a whole number of 128-token blocks")
    loc = _local_u8(local, q.device)
    sq, sk = loc.shape
    if NQ % q_temporal or NQ % sq or NK % sk:
        raise ValueError(f"NQ={NQ}, NK={NK} must tile q_temporal={q_temporal} and the "
                         f"local mask {sq}x{sk}")
    dev = q.device
    keep = torch.empty((nheads, NQ, NK), dtype=torch.uint8, device=dev) if want_keep else None
    sel = cnt = None
    if want_index:
        sel = torch.empty((nheads, NQ, max(NK, 1)), dtype=torch.int32, device=dev)
        cnt = torch.empty((nheads, NQ), dtype=torch.int32, device=dev)
    L = _lib.lib()
    ws_n = L.fvsr_draft_workspace_floats(nheads, D, NQ, NK)
    ws = torch.empty(max(ws_n, 1), dtype=torch.float32, device=dev)
    rc = L.fvsr_draft_block_mask(q2.data_ptr(), qts, _lib.ptr(q_map), k2.data_ptr(), kts,
                                 _lib.ptr(k_map), nheads, D, NQ, NK, q_temporal, loc.data_ptr(),
                                 sq, sk, int(topk), _lib.ptr(keep), _lib.ptr(sel), _lib.ptr(cnt),
                                 ws.data_ptr(), ws_n, _lib.stream(q))
    _lib.check(rc, "draft_block_mask")
    index = (sel, cnt, max(NK, 1)) if want_index else None
    if want_keep and want_index:
        return index, keep.bool()
    return keep.bool() if want_keep else index


def draft_block_mask(q_w: torch.Tensor, k_w: torch.Tensor, nheads: int, q_temporal: int,
                     local: torch.Tensor, topk: int) -> torch.Tensor:
    """Reference signature (lcsa/reference.py:37-40): q_w [Nq, 128, h*d],
    k_w [Nk, 128, h*d] bf16, local [sq, sk] bool -> keep [h, Nq, Nk] bool."""
    return draft_index(q_w, k_w, nheads=nheads, q_temporal=q_temporal, local=local, topk=topk,
                       want_keep=True, want_index=False)


def generate_draft_block_mask(batch_size: int, nheads: int, seqlen: int, q_w: torch.Tensor,
                              k_w: torch.Tensor, topk: int = 10,
                              local_attn_mask: torch.Tensor | None = None) -> torch.Tensor:
    """Call shape of the DiT's ``generate_draft_block_mask`` (integrate.py:103-104):
    ``seqlen`` query time rows, batch 1; returns the [1, h, Nq, Nk] bool mask
    the block-sparse attention call takes."""
    if batch_size != 1:
        raise NotImplementedError("the draft block mask covers batch 1 (as the FlashVSR DiT)")
    if local_attn_mask is None:
        raise ValueError("local_attn_mask is required")
    keep = draft_block_mask(q_w, k_w, nheads, seqlen, local_attn_mask, topk)
    return keep.unsqueeze(0)
