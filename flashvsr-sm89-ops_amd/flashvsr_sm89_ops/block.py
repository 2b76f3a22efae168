"""The FlashVSR-Tiny DiT block built only from this pack's HIP ops.

This is the unit the rebound ``DiTBlock.forward`` executes per streaming chunk
(reference integrate.py:151-182 with the self-attention of :47-124), laid out
for gfx950 instead of as a sequence of eager ops:

  fused_ln_modulate + per-token e4m3 quant     (1 pass, codes only; in a stack
                                                the previous block's last op)
  fused q|k|v projection                       (one FP8 GEMM, N = 3*dim)
  RMSNorm + RoPE on q and k, in place          (one launch)
  block-sparse attention                       (window order through token
                                                maps: no partition copies)
  per-token quant of the attention output
  o projection                                 (FP8 GEMM)
  gate_add + fused_ln_modulate + quant         (1 pass: x1 and the FFN's codes)
  ffn.0 + bias                                 (FP8 GEMM)
  tanh-GELU + per-token quant                  (1 pass, row in registers)
  ffn.2                                        (FP8 GEMM)
  gate_add [+ the next block's AdaLN + quant]  (1 pass)

With cross-attention weights (not part of the BASELINE C5 block stack) the
self-attention's gate_add is followed by norm3 (affine LayerNorm + quant), the
cross q projection, RMSNorm, dense attention over the cached prompt K/V, the
o projection, and the residual add fused with the FFN's AdaLN.  Weights use
per-output-channel scales, activations per-token scales.
"""
from __future__ import annotations

import math

import torch

from . import _lib
from .fp8_ffn import fused_gelu_quant_fp8
from .fp8_linear import FP8Linear, fp8_gemm
from .fp8_quant import quantize_fp8, quantize_weight_fp8
from .fused_adaln import (fused_gate_add, fused_gate_add_ln_modulate_quant,
                          fused_ln_modulate_quant)
from .fused_rms_rope import fused_rms_rope_qk
from .cross_attn import cross_attention_out, unit_gate
from .lcsa.hip_lcsa import block_sparse_attention_strided


def window_token_map(f: int, h: int, w: int, win=(2, 8, 8), device=None) -> torch.Tensor:
    """int32 [f*h*w]: position in window order -> raster token index, the
    permutation of WindowPartition3D.partition (lcsa/reference.py:15-21)."""
    wf, wh, ww = win
    t = torch.arange(f * h * w, dtype=torch.int32).reshape(f // wf, wf, h // wh, wh, w // ww, ww)
    t = t.permute(0, 2, 4, 1, 3, 5).reshape(-1)
    return t.to(device) if device is not None else t


class DiTBlockWeights:
    """FP8 weights of one DiT block: fused qkv [3*dim, dim], o [dim, dim],
    ffn0 [ffn, dim], ffn2 [dim, ffn] (e4m3 + per-channel fp32 scales, bf16
    biases), RMSNorm weights and the [6, dim] modulation; with ``cross_len``
    also the cross-attention's norm3, q/o projections, RMSNorm weight and a
    cached prompt K/V of cross_len tokens."""

    def __init__(self, dim: int, ffn_dim: int, device, generator: torch.Generator,
                 std: float = 0.02, cross_len: int = 0):
        def lin(n, k):
            w = (torch.randn(n, k, generator=generator) * std).to(torch.bfloat16).to(device)
            q, s = quantize_weight_fp8(w, per_channel=True)
            return q, s, torch.zeros(n, dtype=torch.bfloat16, device=device)

        self.qkv = lin(3 * dim, dim)
        self.o = lin(dim, dim)
        self.ffn0 = lin(ffn_dim, dim)
        self.ffn2 = lin(dim, ffn_dim)
        self.norm_q = (1 + 0.1 * torch.randn(dim, generator=generator)).to(torch.bfloat16).to(device)
        self.norm_k = (1 + 0.1 * torch.randn(dim, generator=generator)).to(torch.bfloat16).to(device)
        self.modulation = (0.1 * torch.randn(1, 6, dim, generator=generator)).to(torch.bfloat16).to(device)
        self.cross = None
        if cross_len:
            # norm3 (affine LayerNorm), cross q / o projections, RMSNorm of q and
            # the prompt K/V as cached by init_cross_kv ([1, cross_len, dim]).
            def vec(mean, std):
                return (mean + std * torch.randn(dim, generator=generator)).to(torch.bfloat16).to(device)
            kv = [(torch.randn(1, cross_len, dim, generator=generator)).to(torch.bfloat16).to(device)
                  for _ in range(2)]
            self.cross = {"norm3_w": vec(1.0, 0.1), "norm3_b": vec(0.0, 0.1), "q": lin(dim, dim),
                          "o": lin(dim, dim), "norm_q": vec(1.0, 0.1), "k": kv[0], "v": kv[1]}


def _modulation(wts: DiTBlockWeights, t_mod: torch.Tensor):
    """(shift_msa, scale_msa, gate_msa, shift_mlp, scale_mlp, gate_mlp), each
    [1, 1, dim], from modulation + t_mod (integrate.py:153-154)."""
    mod = (wts.modulation + t_mod).contiguous()
    return [mod[:, i:i + 1].contiguous() for i in range(6)]


def dit_block_forward(x: torch.Tensor, wts: DiTBlockWeights, t_mod: torch.Tensor, cs: torch.Tensor,
                      index, tok_map, heads: int = 12, eps: float = 1e-6,
                      hook=None, x8s=None, next_wts: DiTBlockWeights | None = None,
                      mods=None, next_mods=None):
    """x [1, L, dim] bf16 (raster order) -> [1, L, dim].  ``index`` is the
    device block index (sel, cnt, maxk) of the attention mask; ``tok_map``
    is the latent grid ``(f, h, w)`` whose (2, 8, 8) windows are the attention
    blocks (the kernel computes the window order), or window_token_map(f, h,
    w) itself (read as a gathered map); ``cs`` the (cos, sin) table [L, 64, 2].

    Each gated residual (integrate.py:163-182) is fused with the AdaLN that
    follows it: the self-attention's with the FFN's, the FFN's with the next
    block's (when ``next_wts`` is given; the result is then (y, the next
    block's input codes), which that block takes as ``x8s``).  ``mods`` /
    ``next_mods``, if given, are the six [1, 1, dim] modulation vectors of
    this / the next block, already added to t_mod.
    ``hook(name)``, if given, is called on the host before each launch group
    and with ``"end"`` after the last (used to place timing events)."""
    mark = hook or (lambda name: None)
    B, L, D = x.shape
    hd = D // heads
    shift_msa, scale_msa, gate_msa, shift_mlp, scale_mlp, gate_mlp = (
        mods if mods is not None else _modulation(wts, t_mod))

    if x8s is None:
        mark("ln_modulate_quant")
        x8s = fused_ln_modulate_quant(x, scale_msa, shift_msa, eps)
    x8, xs = x8s
    mark("gemm_qkv")
    qkv = fp8_gemm(x8, xs, *wts.qkv)                      # [L, 3D]
    q = qkv[:, :D].view(B, L, D)
    k = qkv[:, D:2 * D].view(B, L, D)
    mark("rms_rope_qk")
    fused_rms_rope_qk(q, k, wts.norm_q, wts.norm_k, cs, eps=eps, head_dim=hd, inplace=True)

    attn = torch.empty((L, D), dtype=torch.bfloat16, device=x.device)
    mark("bsa")
    block_sparse_attention_strided(
        qkv[:, :D], qkv[:, D:2 * D], qkv[:, 2 * D:], None, 1.0 / math.sqrt(hd), heads=heads,
        head_dim=hd, q_strides=(3 * D, hd), kv_strides=(3 * D, hd), out=attn,
        o_strides=(D, hd), index=index,
        **({"q_map": tok_map, "kv_map": tok_map} if torch.is_tensor(tok_map)
           else {"window": (*tok_map, True)}))

    mark("quant_attn")
    a8, as_ = quantize_fp8(attn, per_token=True)
    mark("gemm_o")
    yo = fp8_gemm(a8, as_, *wts.o)

    if wts.cross is None:
        mark("gate_add_ln_modulate_quant")
        x1, x8, xs = fused_gate_add_ln_modulate_quant(x, gate_msa, yo, scale_mlp, shift_mlp, eps)
    else:
        c = wts.cross
        mark("gate_add")
        x1 = fused_gate_add(x, gate_msa, yo.view(B, L, D))
        yc = cross_attention_out(x1, c["norm3_w"], c["norm3_b"], c["q"], c["norm_q"], c["k"],
                                 c["v"], c["o"], heads, eps, hook=hook)
        mark("gate_add_ln_modulate_quant")
        x1, x8, xs = fused_gate_add_ln_modulate_quant(x1, unit_gate(D, x.device), yc, scale_mlp,
                                                      shift_mlp, eps)

    mark("gemm_ffn0")
    h = fp8_gemm(x8, xs, *wts.ffn0)
    mark("gelu_quant")
    h8, hs = fused_gelu_quant_fp8(h, per_token=True)
    mark("gemm_ffn2")
    yf = fp8_gemm(h8, hs, *wts.ffn2)
    if next_wts is not None:
        n_shift, n_scale = (next_mods if next_mods is not None else _modulation(next_wts, t_mod))[:2]
        mark("gate_add_ln_modulate_quant")
        x2, x8n, xsn = fused_gate_add_ln_modulate_quant(x1, gate_mlp, yf, n_scale, n_shift, eps)
        mark("end")
        return x2, (x8n, xsn)
    mark("gate_add")
    x2 = fused_gate_add(x1, gate_mlp, yf.view(B, L, D))
    mark("end")
    return x2


class DiTStack:
    """``blocks`` DiT blocks with random-init weights (~N(0, 0.02), per-channel
    e4m3), the BASELINE C5 workload: one call = one streaming chunk."""

    def __init__(self, blocks: int = 30, dim: int = 1536, heads: int = 12, ffn_dim: int = 8960,
                 device="cuda", seed: int = 0, cross_len: int = 0):
        g = torch.Generator().manual_seed(seed)
        self.heads = heads
        self.weights = [DiTBlockWeights(dim, ffn_dim, device, g, cross_len=cross_len)
                        for _ in range(blocks)]
        self._mod_stack = None

    def __call__(self, x, t_mod, cs, index, tok_map, hook=None):
        # Every block's modulation + t_mod in one launch: [blocks, 6, dim].
        if self._mod_stack is None:
            self._mod_stack = torch.cat([w.modulation for w in self.weights]).contiguous()
        mod = self._mod_stack + t_mod
        mods = [[mod[i:i + 1, j:j + 1] for j in range(6)] for i in range(len(self.weights))]
        x8s = None
        n = len(self.weights)
        for i, w in enumerate(self.weights):
            nxt = self.weights[i + 1] if i + 1 < n else None
            r = dit_block_forward(x, w, t_mod, cs, index, tok_map, self.heads, hook=hook,
                                  x8s=x8s, next_wts=nxt, mods=mods[i],
                                  next_mods=mods[i + 1] if nxt is not None else None)
            if nxt is None:
                x = r
            else:
                x, x8s = r
        return x


__all__ = ["window_token_map", "DiTBlockWeights", "dit_block_forward", "DiTStack", "FP8Linear"]
