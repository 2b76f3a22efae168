"""PyTorch-eager restatement of the reference DiT block, on the CPU.

TEST INFRASTRUCTURE ONLY.  tests/test_oracle_block.py uses it to pin the
oracle's composition (oracle.dit_block) from an independent, operator-level
reading of the reference; bench.py's ``cpu_baseline`` leg times it as the
reference path's PyTorch eager chain on the host cores.  The product package
never imports it.

Everything is written from the reference's block (integrate.py:151-182, the
self-attention of :47-124, the cross-attention of :132-143) and the upstream
helpers it calls, with torch's own operators: F.layer_norm, the reference's
eager e4m3 quantisation expressions (fp8_quant.py:26-35,54, fp8_linear.py:20-22),
dequantised matmuls in place of torch._scaled_mm (CPU _scaled_mm has no
row-wise scales), the Wan RMSNorm and float64 complex RoPE, attention under
the block mask, and F.gelu(approximate='tanh').
"""
from __future__ import annotations

import math

import numpy as np
import torch
import torch.nn.functional as F

BF = torch.bfloat16
E4M3 = torch.float8_e4m3fn


# fl(1/448): on the GPU torch divides a tensor by a Python float as a product
# with the float reciprocal (the CPU divides), so the reference's returned
# scale `amax / FP8_MAX` (fp8_quant.py:54) is amax * fl(1/448).
_INV448 = torch.tensor(1.0 / 448.0, dtype=torch.float32)


def q_act(x, per_token):
    """Activation quantisation (fp8_quant.py:26-35,54; per row for per-token):
    s = max(amax, 1e-12)/448, e4m3(clamp(x/s, +-448)), returned scale
    amax/448 in the GPU's evaluation (amax * fl(1/448))."""
    xf = x.float()
    amax = xf.abs().amax(dim=1, keepdim=True) if per_token else xf.abs().amax().reshape(1, 1)
    s = amax.clamp(min=1e-12) / 448.0
    return (xf / s).clamp(-448.0, 448.0).to(E4M3), amax * _INV448


def q_weight(w, per_channel):
    """FP8Linear.__init__ (fp8_linear.py:20-22) as eager torch evaluates it on a
    bf16 weight; per channel the [N, 1] fp32 scale promotes w/s to fp32."""
    if per_channel:
        s = (w.abs().amax(dim=1, keepdim=True) / 448.0).clamp(min=1e-12).float()
    else:
        s = (w.abs().amax() / 448.0).clamp(min=1e-12).float()
    return (w / s).to(E4M3), s.reshape(-1)


def linear_eager(x, lin, per_token, acc=torch.float64):
    """_scaled_mm(x8, W8.t(), s_x, s_w, bias) -> bf16 as a dequantised matmul
    (``acc`` float64: exact sums; float32: the eager CPU speed path)."""
    w8, sw, b = lin
    x8, sx = q_act(x, per_token)
    y = (x8.to(acc) @ w8.to(acc).T) * sx.to(acc) * sw.to(acc).reshape(1, -1)
    return (y + b.to(acc)).float().to(BF)


def rms_norm_upstream(x, weight, eps):
    """Wan RMSNorm: (x.float() * rsqrt(mean(x^2) + eps)).to(bf16) * weight."""
    xf = x.float()
    return (xf * torch.rsqrt(xf.pow(2).mean(-1, keepdim=True) + eps)).to(BF) * weight


def rope_upstream(x, freqs, heads):
    """Wan rope_apply: float64 complex product over interleaved pairs -> bf16."""
    L, D = x.shape
    xc = torch.view_as_complex(x.double().reshape(L, heads, -1, 2))
    return torch.view_as_real(xc * freqs[:, None, :]).reshape(L, D).to(BF)


def modulate(x, shift, scale):
    return x * (1 + scale) + shift


def attention_dense(q, k, v, keep_tokens, heads):
    """Per head scaled_dot_product_attention in fp32 under a [Lq, Lk] bool mask
    (or none)."""
    hd = q.shape[1] // heads
    out = []
    for h in range(heads):
        sl = slice(h * hd, (h + 1) * hd)
        m = keep_tokens[h] if keep_tokens is not None else None
        out.append(F.scaled_dot_product_attention(q[None, :, sl].float(), k[None, :, sl].float(),
                                                  v[None, :, sl].float(), attn_mask=m)[0])
    return torch.cat(out, 1).to(BF)


def attention_blocks(q, k, v, keep, heads, block=128):
    """Per (head, query block) softmax over the kept key blocks only, in fp32
    (the reference's sparse_attention_ref loop, lcsa/reference.py:67-88);
    q/k/v [tokens, heads*hd] in window order, keep [heads, NQ, NK] bool."""
    hd = q.shape[1] // heads
    scale = 1.0 / math.sqrt(hd)
    out = torch.zeros(q.shape, dtype=torch.float32)
    keep = torch.as_tensor(keep)
    for h in range(heads):
        sl = slice(h * hd, (h + 1) * hd)
        kh = k[:, sl].float().view(-1, block, hd)
        vh = v[:, sl].float().view(-1, block, hd)
        for i in range(keep.shape[1]):
            sel = keep[h, i].nonzero(as_tuple=True)[0]
            if sel.numel() == 0:
                continue
            p = torch.softmax(q[i * block:(i + 1) * block, sl].float()
                              @ kh[sel].reshape(-1, hd).T * scale, dim=-1)
            out[i * block:(i + 1) * block, sl] = p @ vh[sel].reshape(-1, hd)
    return out.to(BF)


def closed_form_window_of(B, f, h, w):
    """(window, slot) of every token (b, t, r, c) by the closed form of a
    (2, 8, 8) window partition: windows ordered (b, t//2, r//8, c//8), slots
    (t%2, r%8, c%8)."""
    b, t, r, c = np.meshgrid(np.arange(B), np.arange(f), np.arange(h), np.arange(w), indexing="ij")
    per_b = (f // 2) * (h // 8) * (w // 8)
    win = b * per_b + ((t // 2) * (h // 8) + r // 8) * (w // 8) + c // 8
    slot = ((t % 2) * 8 + r % 8) * 8 + c % 8
    return win, slot


def window_order(f, h, w):
    """Raster token of each window position, from the closed form."""
    win, slot = closed_form_window_of(1, f, h, w)
    tok = np.empty(f * h * w, np.int64)
    tok[(win * 128 + slot).reshape(-1)] = np.arange(f * h * w)
    return torch.from_numpy(tok)


def dit_block_eager(x, mod, P, fhw, keep, freqs, heads, eps, per_token, cross=None, cache=None,
                    kv_len=None, acc=torch.float64, sparse=False):
    """The reference DiT block with its stock helpers, eager torch on bf16 CPU
    tensors.  x [L, D]; mod [6, D] = modulation + t_mod; P: q, k, v, o, ffn0,
    ffn2 as (e4m3 codes, fp32 scales, bf16 bias) and norm_q / norm_k; keep
    [heads, NQ, NK]; freqs complex128 [L, hd/2]; cache (k_w, v_w) as
    [tokens, D] window-ordered.  ``sparse`` runs the per-block attention
    instead of dense SDPA under the expanded mask.  Returns (x, k_w, v_w)."""
    f, h, w = fhw
    L, D = x.shape
    sh_a, sc_a, g_a, sh_f, sc_f, g_f = mod.chunk(6, dim=0)
    xin = modulate(F.layer_norm(x, (D,), eps=eps), sh_a, sc_a)
    q = rope_upstream(rms_norm_upstream(linear_eager(xin, P["q"], per_token, acc), P["norm_q"], eps),
                      freqs, heads)
    k = rope_upstream(rms_norm_upstream(linear_eager(xin, P["k"], per_token, acc), P["norm_k"], eps),
                      freqs, heads)
    v = linear_eager(xin, P["v"], per_token, acc)
    tok = window_order(f, h, w)
    q_w, k_w, v_w = q[tok], k[tok], v[tok]
    per_step = (L // 128) // (f // 2)
    if cache is not None:
        k_w = torch.cat([cache[0], k_w])
        v_w = torch.cat([cache[1], v_w])
    if sparse:
        att_w = attention_blocks(q_w, k_w, v_w, keep, heads)
    else:
        km = torch.from_numpy(np.asarray(keep)).repeat_interleave(128, 1).repeat_interleave(128, 2)
        att_w = attention_dense(q_w, k_w, v_w, km, heads)
    att = torch.empty_like(att_w)
    att[tok] = att_w
    x = x + g_a * linear_eager(att, P["o"], per_token, acc)
    if kv_len is not None and k_w.shape[0] // 128 // per_step > kv_len:
        k_w, v_w = k_w[per_step * 128:], v_w[per_step * 128:]
    if cross is not None:
        n3 = F.layer_norm(x, (D,), cross["norm3_w"], cross["norm3_b"], eps)
        cq = rms_norm_upstream(linear_eager(n3, cross["q"], per_token, acc), cross["norm_q"], eps)
        x = x + linear_eager(attention_dense(cq, cross["k"], cross["v"], None, heads), cross["o"],
                             per_token, acc)
    hmid = linear_eager(modulate(F.layer_norm(x, (D,), eps=eps), sh_f, sc_f), P["ffn0"], per_token,
                        acc)
    y = linear_eager(F.gelu(hmid, approximate="tanh"), P["ffn2"], per_token, acc)
    return x + g_f * y, k_w, v_w
