"""Fused RMSNorm + RoPE on gfx950.

Same contract as the reference (flashvsr_sm89_ops/fused_rms_rope.py:21-83):
RMS over the full hidden dim D in fp32, ``y = bf16(x*rsqrt(ms+eps)) * w``,
then the interleaved pairs (2i, 2i+1) of every head are rotated with
cos/sin[s, i] in fp32 and stored as bf16; ``rope=False`` is plain RMSNorm.

The kernel reads (cos, sin) in the interleaved layout of
``view_as_real(freqs_cis)`` (fp32 [S, head_dim/2, 2]), so a complex64
freqs_cis is used without any copy; other dtypes are converted once and
cached per freqs tensor.

`fused_rms_rope` takes x and the weight in bf16, fp16 or fp32, each in its
own type, and returns x's type, as the reference's kernel (loads
``.to(tl.float32)``, output ``torch.empty_like(x)``); the fused q/k forms of
this module take bf16.
"""
from __future__ import annotations

import weakref

import torch

from . import _lib

_CS_CACHE: dict = {}
_CS_CACHE_MAX = 8


def _freqs_table(freqs: torch.Tensor) -> torch.Tensor:
    """complex [..., S, head_dim/2] -> fp32 [S, head_dim/2, 2] contiguous (cos, sin).

    A contiguous complex64 freqs is viewed without a copy.  Other dtypes (Wan
    builds complex128) are converted once per freqs tensor: the entry holds a
    weak reference to its source and is used only while that same tensor is
    alive and unmodified (identity and version counter), so a new tensor that
    reuses a freed one's address never gets the old table."""
    f = freqs.reshape(-1, freqs.shape[-1])
    if f.dtype == torch.complex64 and f.is_contiguous():
        return torch.view_as_real(f)
    entry = _CS_CACHE.get(id(freqs))
    if entry is not None and entry[0]() is freqs and entry[1] == freqs._version:
        return entry[2]
    t = torch.view_as_real(f.to(torch.complex64)).contiguous()
    for k in [k for k, e in _CS_CACHE.items() if e[0]() is None]:
        del _CS_CACHE[k]                      # sources already freed
    while len(_CS_CACHE) >= _CS_CACHE_MAX:
        _CS_CACHE.pop(next(iter(_CS_CACHE)))
    _CS_CACHE[id(freqs)] = (weakref.ref(freqs), freqs._version, t)
    return t


def _freqs_cos_sin(freqs: torch.Tensor):
    """[..., S, 64] complex -> (cos [S, 64] fp32, sin [S, 64] fp32), as the
    reference helper (fused_rms_rope.py:58-63)."""
    t = _freqs_table(freqs)
    return t[..., 0].contiguous(), t[..., 1].contiguous()


def _table_for(freqs, L: int, head_dim: int, device) -> torch.Tensor:
    if freqs is None:
        raise ValueError("fused_rms_rope: rope=True needs freqs_cis")
    if torch.is_tensor(freqs) and not torch.is_complex(freqs):
        # Already a (cos, sin) interleaved fp32 table.
        t = freqs.reshape(-1, head_dim // 2, 2).float().contiguous()
    else:
        t = _freqs_table(freqs)
    if t.shape[0] < L or t.shape[1] != head_dim // 2:
        raise ValueError(f"freqs table {tuple(t.shape)} does not cover L={L}, head_dim={head_dim}")
    if t.device != device:
        t = t.to(device)
    return t


def _check_weights(D: int, *weights):
    """RMSNorm weights must hold one element per channel of the D-wide rows
    (the kernels read D of them)."""
    for w in weights:
        if w.numel() != D:
            raise ValueError(f"RMSNorm weight has {w.numel()} elements, rows have D={D}")


def fused_rms_rope(x: torch.Tensor, weight: torch.Tensor, freqs_cis, eps: float = 1e-6,
                   rope: bool = True, head_dim: int = 128):
    """x [B, L, D] -> RMSNorm(weight) -> [x RoPE] (fused_rms_rope.py:66-83);
    x and weight bf16, fp16 or fp32; returns x's type."""
    B, L, D = x.shape
    _check_weights(D, weight)
    _lib.require_gpu(x, weight)
    xt, wt = _lib.dtype_code(x, "x"), _lib.dtype_code(weight, "weight")
    x2 = x.contiguous()
    w = weight.contiguous()
    out = torch.empty_like(x2)
    cs = _table_for(freqs_cis, L, head_dim, x.device) if rope else None
    _lib.check(_lib.lib().fvsr_rms_rope_dt(x2.data_ptr(), xt, w.data_ptr(), wt, _lib.ptr(cs),
                                           out.data_ptr(), B, L, D, head_dim if rope else D,
                                           float(eps), int(bool(rope)), _lib.stream(x)),
               "fused_rms_rope")
    return out


def fused_rms_rope_qk(q: torch.Tensor, k: torch.Tensor, weight_q: torch.Tensor,
                      weight_k: torch.Tensor, freqs_cis, eps: float = 1e-6, head_dim: int = 128,
                      inplace: bool = False):
    """Both self-attention RMSNorm+RoPE calls (integrate.py:59-62) in one launch.
    q, k: [B, L, D] bf16 whose rows may be strided (e.g. column slices of a
    fused QKV output, last dim contiguous).  ``inplace`` writes the results
    over q and k."""
    B, L, D = q.shape
    if k.shape != q.shape:
        raise ValueError("fused_rms_rope_qk: q and k shapes differ")
    _check_weights(D, weight_q, weight_k)
    _lib.require_gpu(q, k, weight_q, weight_k)
    if q.stride(-1) != 1 or k.stride(-1) != 1 or q.stride(1) != k.stride(1) or \
            (B > 1 and (q.stride(0) != L * q.stride(1) or k.stride(0) != L * k.stride(1))):
        q, k = q.contiguous(), k.contiguous()
        inplace = False
    wq = weight_q.to(torch.bfloat16).contiguous()
    wk = weight_k.to(torch.bfloat16).contiguous()
    cs = _table_for(freqs_cis, L, head_dim, q.device)
    if inplace:
        oq, ok = q, k
    else:
        oq = torch.empty((B, L, D), dtype=q.dtype, device=q.device)
        ok = torch.empty((B, L, D), dtype=k.dtype, device=k.device)
    _lib.check(_lib.lib().fvsr_rms_rope_qk(q.data_ptr(), k.data_ptr(), wq.data_ptr(),
                                           wk.data_ptr(), cs.data_ptr(), oq.data_ptr(),
                                           ok.data_ptr(), B, L, D, head_dim, float(eps),
                                           q.stride(1), oq.stride(1), _lib.stream(q)),
               "fused_rms_rope_qk")
    return oq, ok


def fused_rms_rope_qkv_rows(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor,
                            weight_q: torch.Tensor, weight_k: torch.Tensor, freqs_cis,
                            out_k: torch.Tensor, out_v: torch.Tensor, kv_rows: torch.Tensor,
                            eps: float = 1e-6, head_dim: int = 128) -> torch.Tensor:
    """The self-attention's RMSNorm + RoPE of q and k (integrate.py:59-62)
    with k and v written straight into a window-ordered K/V buffer
    (integrate.py:70-83 without the partition and cat copies).  q, k, v:
    [B, L, D] bf16 with unit-stride rows sharing one row stride (contiguous
    tensors or column slices of a fused qkv); q is rotated in place and returned;
    row r of k and v goes to row ``kv_rows[r]`` of ``out_k`` / ``out_v``
    ([rows, D] bf16, contiguous)."""
    for t, n in ((q, "q"), (k, "k"), (v, "v"), (out_k, "out_k"), (out_v, "out_v")):
        _lib.require_dtype(t, torch.bfloat16, n)
    _lib.require_dtype(kv_rows, torch.int32, "kv_rows")
    B, L, D = q.shape
    if k.shape != q.shape or v.shape != q.shape:
        raise ValueError("fused_rms_rope_qkv_rows: q, k, v shapes differ")
    ld = q.stride(1)
    for t in (q, k, v):
        if t.stride(-1) != 1 or t.stride(1) != ld or (B > 1 and t.stride(0) != L * ld):
            raise ValueError("fused_rms_rope_qkv_rows: q, k, v need unit-stride rows with one "
                             "common row stride (e.g. column slices of a fused qkv)")
    if out_k.shape != out_v.shape or out_k.dim() != 2 or out_k.shape[1] != D or \
            not (out_k.is_contiguous() and out_v.is_contiguous()):
        raise ValueError("fused_rms_rope_qkv_rows: out_k/out_v must be contiguous [rows, D]")
    if kv_rows.numel() != B * L or not kv_rows.is_contiguous():
        raise ValueError("fused_rms_rope_qkv_rows: kv_rows must hold B*L entries")
    _check_weights(D, weight_q, weight_k)
    _lib.require_gpu(q, k, v, weight_q, weight_k, out_k, out_v, kv_rows)
    wq = weight_q.to(torch.bfloat16).contiguous()
    wk = weight_k.to(torch.bfloat16).contiguous()
    cs = _table_for(freqs_cis, L, head_dim, q.device)
    _lib.check(_lib.lib().fvsr_rms_rope_qkv_rows(
        q.data_ptr(), k.data_ptr(), v.data_ptr(), wq.data_ptr(), wk.data_ptr(), cs.data_ptr(),
        q.data_ptr(), out_k.data_ptr(), out_v.data_ptr(), kv_rows.data_ptr(), out_k.shape[0],
        B, L, D, head_dim, float(eps), ld, ld, D, _lib.stream(q)), "fused_rms_rope_qkv_rows")
    return q
