"""Cross-attention of the DiT block on gfx950.

Reference path (flashvsr_sm89_ops/integrate.py:132-143,171):
``x + cross_attn(norm3(x), context)`` with ``norm3`` an affine LayerNorm, an
FP8 q projection, RMSNorm of q (no RoPE), dense attention of the 16896 video
tokens over the prompt K/V cached by ``init_cross_kv``, and an FP8 o
projection.  Here the dense attention runs on the attention kernel's dense
mode (fvsr_attn_dense: every 128-key block, no block index, two query blocks
per workgroup over one K/V stream), the LayerNorm emits the q projection's per-token e4m3
codes in the same pass, and the residual add is a gate-add
add with a unit gate (bf16(x + bf16(1 * y)) = bf16(x + y)), which inside a DiT
block is fused with the AdaLN that follows it.
"""
from __future__ import annotations

import math

import torch

from .fp8_linear import fp8_gemm
from .fp8_quant import quantize_fp8
from .fused_adaln import fused_gate_add, layer_norm_quant
from .fused_rms_rope import fused_rms_rope
from .lcsa.hip_lcsa import dense_attention_strided

BLOCK = 128
_ONES = {}


def supported(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor, num_heads: int) -> bool:
    """Shapes the kernel covers: batch 1, bf16 on the GPU, head_dim 128, query
    and key counts multiples of 128."""
    if not (q.is_cuda and k.is_cuda and v.is_cuda):
        return False
    if q.dtype != torch.bfloat16 or k.dtype != torch.bfloat16 or v.dtype != torch.bfloat16:
        return False
    if q.dim() != 3 or k.dim() != 3 or v.dim() != 3 or q.shape[0] != 1 or k.shape[0] != 1:
        return False
    HD = q.shape[-1]
    if HD % num_heads or HD // num_heads != 128 or k.shape[-1] != HD or v.shape != k.shape:
        return False
    return q.shape[1] % BLOCK == 0 and k.shape[1] % BLOCK == 0 and k.shape[1] > 0


def cross_attention(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor, num_heads: int,
                    sm_scale: float | None = None, out: torch.Tensor | None = None):
    """softmax(q k^T / sqrt(d)) v per head: q [1, Lq, H*128], k/v [1, Lk, H*128]
    bf16 -> [1, Lq, H*128] (the call ``self.attn(q, k, v)`` at integrate.py:141)."""
    if not supported(q, k, v, num_heads):
        raise ValueError(f"cross_attention: unsupported shapes q {tuple(q.shape)} "
                         f"k {tuple(k.shape)} heads {num_heads}")
    _, Lq, HD = q.shape
    Lk = k.shape[1]
    hd = HD // num_heads
    q2, k2, v2 = q[0], k[0], v[0]
    if q2.stride(-1) != 1 or q2.stride(0) % 8:
        q2 = q2.contiguous()
    if k2.stride(-1) != 1 or k2.stride(0) % 8:
        k2 = k2.contiguous()
    if v2.stride(-1) != 1 or v2.stride(0) % 8 or v2.stride(0) != k2.stride(0):
        v2 = v2.contiguous()
        k2 = k2.contiguous()
    if out is None:
        out = torch.empty((1, Lq, HD), dtype=torch.bfloat16, device=q.device)
    dense_attention_strided(
        q2, k2, v2, sm_scale if sm_scale is not None else 1.0 / math.sqrt(hd),
        heads=num_heads, head_dim=hd, q_strides=(q2.stride(0), hd),
        kv_strides=(k2.stride(0), hd), out=out[0], o_strides=(HD, hd))
    return out


def cross_attention_out(x: torch.Tensor, norm3_weight: torch.Tensor,
                        norm3_bias: torch.Tensor | None, q_proj: tuple,
                        norm_q_weight: torch.Tensor, cache_k: torch.Tensor,
                        cache_v: torch.Tensor, o_proj: tuple, num_heads: int,
                        eps: float = 1e-6, hook=None) -> torch.Tensor:
    """``cross_attn(norm3(x))`` for x [1, L, D] bf16 with per-token activation
    scales: q_proj / o_proj are (e4m3 weight [D, D], weight scale, bias)
    triples; cache_k / cache_v [1, Lk, D].  Returns the o projection [L, D]."""
    mark = hook or (lambda name: None)
    B, L, D = x.shape
    mark("layer_norm_quant")
    x8, xs = layer_norm_quant(x, norm3_weight, norm3_bias, eps)
    mark("gemm_cross_q")
    q = fp8_gemm(x8, xs, *q_proj).view(B, L, D)
    mark("rms_cross_q")
    q = fused_rms_rope(q, norm_q_weight, None, eps=eps, rope=False, head_dim=D // num_heads)
    mark("cross_attn")
    att = cross_attention(q, cache_k, cache_v, num_heads)
    mark("quant_cross")
    a8, as_ = quantize_fp8(att.view(L, D), per_token=True)
    mark("gemm_cross_o")
    return fp8_gemm(a8, as_, *o_proj)


def unit_gate(dim: int, device) -> torch.Tensor:
    """A [1, 1, dim] bf16 gate of ones: fused_gate_add(x, 1, y) = bf16(x + y)."""
    key = (dim, str(device))
    t = _ONES.get(key)
    if t is None:
        t = torch.ones((1, 1, dim), dtype=torch.bfloat16, device=device)
        _ONES[key] = t
    return t


def cross_attention_residual(x: torch.Tensor, norm3_weight: torch.Tensor,
                             norm3_bias: torch.Tensor | None, q_proj: tuple,
                             norm_q_weight: torch.Tensor, cache_k: torch.Tensor,
                             cache_v: torch.Tensor, o_proj: tuple, num_heads: int,
                             eps: float = 1e-6, hook=None) -> torch.Tensor:
    """``x + cross_attn(norm3(x))`` (integrate.py:171) for x [1, L, D] bf16:
    cross_attention_out followed by the residual add (a gate-add with a unit
    gate).  Inside a DiT block the add is instead fused with the AdaLN that
    follows it (fused_gate_add_ln_modulate_quant)."""
    mark = hook or (lambda name: None)
    B, L, D = x.shape
    y = cross_attention_out(x, norm3_weight, norm3_bias, q_proj, norm_q_weight, cache_k, cache_v,
                            o_proj, num_heads, eps, hook)
    mark("gate_add")
    return fused_gate_add(x, unit_gate(D, x.device), y.view(B, L, D))
