"""Wiring of the operator pack into a FlashVSR v1.1 Tiny pipeline.

``enable(pipe)`` honours the reference contract (flashvsr_sm89_ops/integrate.py:229-292):
one call after ``pipe.to('cuda')`` / ``pipe.enable_vram_management(...)`` and
before ``pipe.init_cross_kv()``, returning a dict of what it switched on, under
the same ``FS89_*`` flags.  What it does, in order:

* decoder memory layout: the TCDecoder goes channels_last (``FS89_TCDEC_CL``);
  ``FS89_TCDEC_COMPILE`` is accepted and reported but not applied (a
  decoder-side inductor compile is not part of this pack and would bring
  Triton back);
* FP8 weights: the DiT block Linears become ``FP8Linear`` and the FFNs
  ``FP8FFN`` (``FS89_FP8`` parts, ``FS89_FP8_FFNFUSED``), per tensor as the
  reference or, with ``FS89_FP8_SCALE=row``, per output channel / per token;
  ``FS89_FP8_WEIGHTS`` names a file of stored codes loaded instead of
  quantising;
* forwards: ``SelfAttention`` / ``CrossAttention`` / ``DiTBlock`` of the
  upstream DiT module get forwards that run the HIP kernels.  The upstream
  forwards are kept (captured before rebinding) and serve every call whose
  fused flag is off (``FS89_FUSED_ROPE``, ``FS89_FUSED_ADALN``), so a flag
  set to 0 gives the stock upstream computation;
* attention: ``block_sparse_attn`` resolves to the HIP block-sparse kernel.

Beyond the reference: the self-attention runs without its layout copies when
the shapes allow (``FS89_WINDOW``, default on), ``FS89_DRAFT=1`` computes the
draft block mask on the device, and ``FS89_CROSS_ATTN`` (default on) runs the
cross-attention's dense attention on the same HIP kernel.

Calling ``enable`` again on a patched module refreshes the flags only.
"""
from __future__ import annotations

import collections
import inspect
import os
import warnings
import weakref

import torch

from .block import window_token_map
from .compat_bsa import active_backend, ensure_bsa_available
from .cross_attn import cross_attention, unit_gate
from .cross_attn import supported as cross_supported
from .fp8_ffn import FP8FFN, convert_ffn_fp8, gemm_gelu_quant_fp8
from .fp8_linear import (FP8Linear, FP8WeightsFormatError, convert_linears_fp8, fp8_gemm,
                         load_fp8_weights, save_fp8_weights)
from .fp8_quant import quantize_fp8
from .fused_adaln import (fused_gate_add, fused_gate_add_layer_norm,
                          fused_gate_add_ln_modulate_quant, fused_ln_modulate,
                          fused_ln_modulate_quant, layer_norm)
from .fused_rms_rope import fused_rms_rope, fused_rms_rope_qkv_rows
from .lcsa.draft import draft_index
from .lcsa.hip_lcsa import block_index, block_sparse_attention_strided

WINDOW = (2, 8, 8)              # frames x rows x columns of one attention window (128 tokens)
_TOKENS_PER_WINDOW = WINDOW[0] * WINDOW[1] * WINDOW[2]
_STOCK_ATTR = "_FS89_STOCK"     # the upstream forwards, captured before rebinding

# Arguments the rebound forwards pass on by name; an upstream class lacking one
# of them is a revision this pack was not written against.
_EXPECTED_SIGS = {
    "SelfAttention": ("x", "freqs", "f", "h", "w", "local_num", "topk", "train_img",
                      "block_id", "kv_len", "is_full_block", "is_stream",
                      "pre_cache_k", "pre_cache_v", "local_range"),
    "CrossAttention": ("x", "y", "is_stream"),
    "DiTBlock": ("x", "context", "t_mod", "freqs", "f", "h", "w", "local_num", "topk",
                 "train_img", "block_id", "kv_len", "is_full_block", "is_stream",
                 "pre_cache_k", "pre_cache_v", "local_range"),
}
_UPSTREAM_HELPERS = ("WindowPartition3D", "generate_draft_block_mask")

# The six modulation vectors, in the order the upstream DiT block splits
# (modulation + t_mod) into (reference integrate.py:154-155).
Modulation = collections.namedtuple(
    "Modulation", "shift_msa scale_msa gate_msa shift_mlp scale_mlp gate_mlp")


def _on(name: str, default: str = "1") -> bool:
    return os.environ.get(name, default) == "1"


def _inner(m):
    """The module behind an enable_vram_management wrapper (or m itself)."""
    return getattr(m, "module", m)


def _eps(m, default=1e-6):
    return getattr(_inner(m), "eps", default)


# ----------------------------------------------------------------------------- geometry

def _window_path_on() -> bool:
    return _on("FS89_WINDOW") and active_backend() == "hip"


def _window_path_ok(x, f, h, w, head_dim) -> bool:
    """Shapes the copy-free self-attention serves: batch 1, bf16 on the GPU,
    whole windows, head_dim 128, a hidden size the fused kernels take."""
    B, L, D = x.shape
    whole = f % WINDOW[0] == 0 and h % WINDOW[1] == 0 and w % WINDOW[2] == 0
    return (B == 1 and x.dtype == torch.bfloat16 and x.is_cuda and head_dim == 128 and whole
            and L == f * h * w and D % head_dim == 0 and D <= 1536)


def _check_stream_geometry(x, f, h, w, is_stream, pre_k, pre_v):
    """The upstream self-attention's preconditions: a streaming run starts with
    6 latent frames and continues 2 at a time; L is f*h*w."""
    cached = pre_k is not None and pre_v is not None
    if is_stream:
        want = 2 if cached else 6
        if f != want:
            raise AssertionError(f"streaming self-attention expects f == {want} "
                                 f"({'with' if cached else 'without'} a KV cache), got {f}")
    if x.shape[1] != f * h * w:
        raise AssertionError(f"sequence length {x.shape[1]} != f*h*w = {f}*{h}*{w}")


_MAPS: dict = {}


def _window_maps(f, h, w, n_cache_rows, device):
    """(tok, kv_rows) for one geometry: tok[i] = raster token at window
    position i (the draft mask reads q through it); kv_rows[t] = row of raster
    token t in the K/V buffer (after the cached rows).  The attention itself
    computes the window order (fvsr_bsa_fwd_window)."""
    key = (f, h, w, n_cache_rows, str(device))
    hit = _MAPS.get(key)
    if hit is not None:
        return hit
    tok = window_token_map(f, h, w, device=device)
    pos = torch.empty_like(tok)
    pos[tok.long()] = torch.arange(tok.numel(), dtype=torch.int32, device=device)
    val = (tok, (pos + n_cache_rows).contiguous())
    while len(_MAPS) >= 32:          # a handful of geometries per run
        _MAPS.pop(next(iter(_MAPS)))
    _MAPS[key] = val
    return val


def _refresh_local_mask(dit, mod, h, w, local_range, device):
    """The module's local window rule, rebuilt by the upstream builder when the
    window grid or the range changes (state kept on the module as upstream does)."""
    bh, bw = h // WINDOW[1], w // WINDOW[2]
    stale = (mod.local_attn_mask is None or mod.local_attn_mask_h != bh
             or mod.local_attn_mask_w != bw or mod.local_range != local_range)
    if stale:
        mod.local_attn_mask = dit.build_local_block_mask_shifted_vec_normal_slide(
            bh, bw, local_range, local_range, include_self=True, device=device)
        mod.local_attn_mask_h, mod.local_attn_mask_w = bh, bw
        mod.local_range = local_range
    return mod.local_attn_mask


def _trim_cache(k_w, v_w, windows_per_step, kv_len):
    """Drop the oldest step's windows once the cache holds more than kv_len steps."""
    if k_w.shape[0] // windows_per_step > kv_len:
        return k_w[windows_per_step:], v_w[windows_per_step:]
    return k_w, v_w


# ----------------------------------------------------------------------------- K/V store

def _appendable(t, store, frontier):
    """t is a contiguous row range of `store` ending at row `frontier`."""
    D = store.shape[1]
    return (t.is_contiguous() and t.device == store.device and t.dtype == store.dtype
            and t.untyped_storage().data_ptr() == store.untyped_storage().data_ptr()
            and t.storage_offset() % D == 0 and t.storage_offset() + t.numel() == frontier * D)


def _kv_buffers(mod, pre_k, pre_v, cache_rows, L, D, like, grow):
    """K/V buffers [cache_rows + L, D] whose first rows hold the cached windows.

    The caches handed back are views into a per-module store with spare rows
    behind them.  When the caller passes them back unchanged (the streaming
    loop does) the next chunk lands behind them in place; any other cache, or
    a full store, is copied once into a fresh store."""
    store = getattr(mod, "_fs89_kv", None)
    if store is not None and cache_rows and pre_k is not None and pre_v is not None:
        sk, sv, end = store
        if end + L <= sk.shape[0] and _appendable(pre_k, sk, end) and _appendable(pre_v, sv, end):
            mod._fs89_kv = (sk, sv, end + L)
            first = end - cache_rows
            return sk[first:end + L], sv[first:end + L]
    rows = cache_rows + L
    cap = rows + 4 * L if grow else rows   # room for a few appended chunks
    sk = torch.empty((cap, D), dtype=like.dtype, device=like.device)
    sv = torch.empty((cap, D), dtype=like.dtype, device=like.device)
    if cache_rows:
        sk[:cache_rows].copy_(pre_k.reshape(-1, D))
        sv[:cache_rows].copy_(pre_v.reshape(-1, D))
    mod._fs89_kv = (sk, sv, rows) if grow else None
    return sk[:rows], sv[:rows]


# ----------------------------------------------------------------------------- fused q/k/v weight

def _same_tensor(ref, t) -> bool:
    if ref is None:
        return t is None
    obj, version = ref
    return t is not None and obj() is t and version == t._version


def _track(t):
    return None if t is None else (weakref.ref(t), t._version)


def _qkv_fused(mod):
    """(w3, s3, b3, per_token): one [3D, D] e4m3 weight for the module's q, k
    and v FP8Linears, so the three projections of the same activations are one
    GEMM over one quantisation of them.  Per-tensor weight scales become
    per-column vectors of the same value (the epilogue arithmetic is the same).
    Built once per module and rebuilt when any of the nine source tensors is
    replaced or changed in place (tracked by identity and version counter, so
    a new tensor at a freed one's address is not mistaken for it).  None when
    the three cannot share one GEMM."""
    lins = [getattr(mod, n, None) for n in ("q", "k", "v")]
    if not all(isinstance(l, FP8Linear) for l in lins):
        return None
    if len({(l.per_token, l.in_features, l.bias is None) for l in lins}) != 1:
        return None
    srcs = [t for l in lins for t in (l.weight, l.w_scale, l.bias)]
    cached = getattr(mod, "_fs89_qkv", None)
    if cached is not None and all(_same_tensor(r, t) for r, t in zip(cached[0], srcs)):
        return cached[1]
    w3 = torch.cat([l.weight for l in lins]).contiguous()
    s3 = torch.cat([l.w_scale.float().reshape(-1).expand(l.out_features) for l in lins])
    b3 = None if lins[0].bias is None else torch.cat([l.bias for l in lins]).contiguous()
    val = (w3, s3.contiguous(), b3, lins[0].per_token)
    mod._fs89_qkv = ([_track(t) for t in srcs], val)
    return val


# ----------------------------------------------------------------------------- self-attention

def _window_self_attention(dit, self, x, freqs, f, h, w, topk, kv_len, is_stream, pre_cache_k,
                           pre_cache_v, local_range, x8s=None):
    """Self-attention (reference integrate.py:47-124) without its layout
    copies: q stays in raster order and is read through the window map; k and
    v leave the RMSNorm/RoPE pass directly in window order behind the cached
    windows of the K/V store; the attention writes its output rows back in
    raster order.  The draft mask is the device one through the map
    (FS89_DRAFT=1) or the DiT's own on a gathered window-ordered q.
    ``x8s`` = (codes, scales) of x when the caller already quantised it.
    Returns what the upstream forward returns, window-ordered caches
    ([windows, 128, D] views of the store) included."""
    B, L, D = x.shape
    fused = _qkv_fused(self)
    if fused is not None:
        w3, s3, b3, per_token = fused
        if x8s is None:
            x8s = quantize_fp8(x.reshape(-1, D), per_token=per_token)
        qkv = fp8_gemm(x8s[0], x8s[1], w3, s3, b3)      # [L, 3D]: q | k | v columns
        q, k, v = (qkv[:, i * D:(i + 1) * D].view(B, L, D) for i in range(3))
    elif x8s is not None:
        raise ValueError("activation codes given but q/k/v are not FP8 linears")
    else:
        q, k, v = (proj(x).contiguous() for proj in (self.q, self.k, self.v))
    steps = f // WINDOW[0]
    windows_per_step = L // _TOKENS_PER_WINDOW // steps
    n_cached = 0 if pre_cache_k is None or pre_cache_v is None else pre_cache_k.shape[0]
    cache_rows = n_cached * _TOKENS_PER_WINDOW
    kbuf, vbuf = _kv_buffers(self, pre_cache_k, pre_cache_v, cache_rows, L, D, q, is_stream)
    if _eps(self.norm_k) != _eps(self.norm_q):
        raise NotImplementedError("q and k RMSNorm eps differ")
    tok, kv_rows = _window_maps(f, h, w, cache_rows, q.device)
    fused_rms_rope_qkv_rows(q, k, v, _inner(self.norm_q).weight, _inner(self.norm_k).weight,
                            freqs, kbuf, vbuf, kv_rows, eps=_eps(self.norm_q),
                            head_dim=self.head_dim)
    k_w = kbuf.view(-1, _TOKENS_PER_WINDOW, D)
    v_w = vbuf.view(-1, _TOKENS_PER_WINDOW, D)
    local = _refresh_local_mask(dit, self, h, w, local_range, k_w.device)
    q2 = q.reshape(L, D)            # rows may be strided (a column slice of qkv)
    if _on("FS89_DRAFT", "0"):
        index = draft_index(q2, k_w, nheads=self.num_heads, q_temporal=steps, local=local,
                            topk=topk, nq=L // _TOKENS_PER_WINDOW, q_map=tok)
    else:
        q_w = q2.index_select(0, tok.long()).view(-1, _TOKENS_PER_WINDOW, D)
        mask = dit.generate_draft_block_mask(B, self.num_heads, steps, q_w, k_w, topk=topk,
                                             local_attn_mask=local)
        index = block_index(mask[0] if mask.dim() == 4 else mask)
    out = torch.empty((L, D), dtype=q.dtype, device=q.device)
    hd = self.head_dim
    block_sparse_attention_strided(
        q2, kbuf, vbuf, None, None, heads=self.num_heads, head_dim=hd,
        q_strides=(q2.stride(0), hd), kv_strides=(D, hd), out=out, o_strides=(D, hd),
        window=(f, h, w, False), index=index)
    cache_k, cache_v = _trim_cache(k_w, v_w, windows_per_step, kv_len)
    y = self.o(out.view(B, L, D))
    return (y, cache_k, cache_v) if is_stream else y


def _partitioned_self_attention(dit, self, x, freqs, f, h, w, topk, kv_len, is_stream,
                                pre_cache_k, pre_cache_v, local_range):
    """Self-attention with the fused RMSNorm+RoPE on materialised window
    tensors, for shapes the copy-free path does not take: the upstream
    partition / cache concatenation / reverse, the module's own attention."""
    B, L, D = x.shape
    rope = dit.FUSED_ROPE_FN
    q = rope(self.q(x), _inner(self.norm_q).weight, freqs, eps=_eps(self.norm_q), rope=True,
             head_dim=self.head_dim)
    k = rope(self.k(x), _inner(self.norm_k).weight, freqs, eps=_eps(self.norm_k), rope=True,
             head_dim=self.head_dim)
    v = self.v(x)
    grid = (B, f, h, w, D)
    q_w, k_w, v_w = (dit.WindowPartition3D.partition(t.view(grid), WINDOW) for t in (q, k, v))
    steps = f // WINDOW[0]
    windows_per_step = k_w.shape[0] // B // steps
    if pre_cache_k is not None and pre_cache_v is not None:
        k_w = torch.cat([pre_cache_k, k_w], dim=0)
        v_w = torch.cat([pre_cache_v, v_w], dim=0)
    local = _refresh_local_mask(dit, self, h, w, local_range, k_w.device)
    draft = dit.generate_draft_block_mask
    if _on("FS89_DRAFT", "0"):
        from .lcsa.draft import generate_draft_block_mask as draft
    mask = draft(B, self.num_heads, steps, q_w, k_w, topk=topk, local_attn_mask=local)
    # window-major token sequences per batch element, as the attention takes them
    seq = [t.reshape(B, -1, D) for t in (q_w, k_w, v_w)]
    out = self.attn(*seq, mask)
    cache_k, cache_v = _trim_cache(k_w, v_w, windows_per_step, kv_len)
    out = dit.WindowPartition3D.reverse(out.reshape(-1, q_w.shape[1], D), WINDOW, (f, h, w))
    y = self.o(out.reshape(B, L, D))
    return (y, cache_k, cache_v) if is_stream else y


def _make_self_attn_forward(dit, stock):
    def forward(self, x, freqs, f=None, h=None, w=None, local_num=None, topk=None,
                train_img=False, block_id=None, kv_len=None, is_full_block=False,
                is_stream=False, pre_cache_k=None, pre_cache_v=None, local_range=9):
        if getattr(dit, "FUSED_ROPE_FN", None) is None:
            return stock(self, x, freqs, f=f, h=h, w=w, local_num=local_num, topk=topk,
                         train_img=train_img, block_id=block_id, kv_len=kv_len,
                         is_full_block=is_full_block, is_stream=is_stream,
                         pre_cache_k=pre_cache_k, pre_cache_v=pre_cache_v,
                         local_range=local_range)
        _check_stream_geometry(x, f, h, w, is_stream, pre_cache_k, pre_cache_v)
        path = (_window_self_attention
                if _window_path_ok(x, f, h, w, self.head_dim) and _window_path_on()
                else _partitioned_self_attention)
        return path(dit, self, x, freqs, f, h, w, topk, kv_len, is_stream, pre_cache_k,
                    pre_cache_v, local_range)

    forward.__doc__ = ("SelfAttention.forward with fused RMSNorm+RoPE and the HIP attention "
                       "(reference integrate.py:47-124); the upstream forward when "
                       "FS89_FUSED_ROPE is off.")
    return forward


# ----------------------------------------------------------------------------- cross-attention

def _make_cross_attn_forward(dit, stock):
    @torch.no_grad()
    def forward(self, x, y, is_stream=False):
        rope = getattr(dit, "FUSED_ROPE_FN", None)
        if rope is None:
            return stock(self, x, y, is_stream=is_stream)
        q = rope(self.q(x), _inner(self.norm_q).weight, None, eps=_eps(self.norm_q), rope=False)
        k, v = self.cache_k, self.cache_v
        if k is None or v is None:
            raise AssertionError("cross-attention needs the prompt K/V cached by init_cross_kv()")
        if _on("FS89_CROSS_ATTN") and cross_supported(q, k, v, self.num_heads):
            att = cross_attention(q, k, v, self.num_heads)
        else:
            att = self.attn(q, k, v)
        return self.o(att)

    forward.__doc__ = ("CrossAttention.forward with the fused RMSNorm of q and dense attention "
                       "over the cached prompt K/V on the HIP kernel (reference "
                       "integrate.py:132-143); the upstream forward when FS89_FUSED_ROPE is off.")
    return forward


# ----------------------------------------------------------------------------- DiT block

def _norm3_affine(m):
    """(weight, bias, eps) when m is an affine LayerNorm over bf16 on the GPU, else None."""
    m = _inner(m)
    if not isinstance(m, torch.nn.LayerNorm) or not m.elementwise_affine:
        return None
    if m.weight is None or m.weight.dtype != torch.bfloat16 or not m.weight.is_cuda:
        return None
    return m.weight, m.bias, m.eps


def _codes_dataflow(dit, blk, x, f, h, w) -> bool:
    """Whether the block runs the per-token FP8 dataflow: the AdaLN writes the
    q/k/v GEMM's codes, q/k/v are one GEMM, the self-attention is copy-free and
    the cross residual is fused with the FFN's AdaLN.  Needs the fused AdaLN
    and RoPE, the HIP attention, per-token q/k/v FP8 linears and a batch-1
    bf16 input in whole windows."""
    sa = getattr(blk, "self_attn", None)
    if sa is None or getattr(dit, "FUSED_ADALN", None) is None \
            or getattr(dit, "FUSED_ROPE_FN", None) is None:
        return False
    if not (_window_path_on() and _window_path_ok(x, f, h, w, getattr(sa, "head_dim", 0))):
        return False
    fused = _qkv_fused(sa)
    return fused is not None and fused[3]


def _gated_residual_norm3(blk, x, gate, attn_out, gate_add):
    """x + gate * attn_out and norm3 of the sum: one pass over the rows when
    norm3 is an affine bf16 LayerNorm on the GPU, else the two steps."""
    ln3 = _norm3_affine(blk.norm3)
    bf16_gpu = x.dtype == torch.bfloat16 and x.is_cuda
    if ln3 is not None and bf16_gpu and attn_out.is_contiguous() and gate.is_contiguous():
        return fused_gate_add_layer_norm(x, gate, attn_out, ln3[0], ln3[1], eps=ln3[2])
    x = gate_add(x, gate, attn_out)
    normed = layer_norm(x, ln3[0], ln3[1], eps=ln3[2]) if ln3 is not None and bf16_gpu \
        else blk.norm3(x)
    return x, normed


def _per_token_ffn(ffn) -> bool:
    """True for an FP8FFN whose two linears both quantise activations per
    token: the only FFN the per-token codes dataflow may feed directly."""
    return (isinstance(ffn, FP8FFN) and getattr(ffn.lin0, "per_token", False)
            and getattr(ffn.lin2, "per_token", False))


def _make_dit_block_forward(dit, stock):
    def forward(self, x, context, t_mod, freqs, f, h, w, local_num=None, topk=None,
                train_img=False, block_id=None, kv_len=None, is_full_block=False,
                is_stream=False, pre_cache_k=None, pre_cache_v=None, local_range=9):
        adaln = getattr(dit, "FUSED_ADALN", None)
        if adaln is None:
            return stock(self, x, context, t_mod, freqs, f, h, w, local_num=local_num,
                         topk=topk, train_img=train_img, block_id=block_id, kv_len=kv_len,
                         is_full_block=is_full_block, is_stream=is_stream,
                         pre_cache_k=pre_cache_k, pre_cache_v=pre_cache_v,
                         local_range=local_range)
        ln_mod, gate_add = adaln
        m = Modulation(*(self.modulation.to(dtype=t_mod.dtype, device=t_mod.device)
                         + t_mod).chunk(6, dim=1))
        codes = _codes_dataflow(dit, self, x, f, h, w)

        # 1) self-attention on the modulated LayerNorm of x
        if codes:
            x8s = fused_ln_modulate_quant(x, m.scale_msa, m.shift_msa, eps=_eps(self.norm1))
            r = _window_self_attention(dit, self.self_attn, x, freqs, f, h, w, topk, kv_len,
                                       is_stream, pre_cache_k, pre_cache_v, local_range,
                                       x8s=x8s)
        else:
            r = self.self_attn(ln_mod(x, m.scale_msa, m.shift_msa, eps=_eps(self.norm1)),
                               freqs, f, h, w, local_num, topk, train_img, block_id,
                               kv_len=kv_len, is_full_block=is_full_block,
                               is_stream=is_stream, pre_cache_k=pre_cache_k,
                               pre_cache_v=pre_cache_v, local_range=local_range)
        attn_out, cache_k, cache_v = r if is_stream else (r, None, None)

        # 2) gated residual, then the cross-attention on norm3 of it
        x, normed = _gated_residual_norm3(self, x, m.gate_msa, attn_out, gate_add)
        yc = self.cross_attn(normed, context, is_stream=is_stream)

        # 3) FFN on the modulated LayerNorm of x + yc, gated residual
        if codes and _per_token_ffn(self.ffn) and yc.shape == x.shape and yc.is_contiguous():
            # x + yc (a unit gate) and the FFN's AdaLN in one pass; its
            # per-token codes go straight into the FFN GEMMs (an FFN
            # converted with per-tensor activation scales keeps its own
            # forward, so its quantisation never changes)
            B, L, D = x.shape
            x, h8, hs = fused_gate_add_ln_modulate_quant(
                x, unit_gate(D, x.device), yc, m.scale_mlp, m.shift_mlp, eps=_eps(self.norm2))
            g8, gs = gemm_gelu_quant_fp8(h8, hs, self.ffn.lin0, True)
            y = self.ffn.lin2._mm(g8, gs).view(B, L, -1)
        else:
            x = x + yc
            y = self.ffn(ln_mod(x, m.scale_mlp, m.shift_mlp, eps=_eps(self.norm2)))
        x = gate_add(x, m.gate_mlp, y)
        return (x, cache_k, cache_v) if is_stream else x

    forward.__doc__ = ("DiTBlock.forward on the fused AdaLN / gated residual kernels "
                       "(reference integrate.py:151-182); the upstream forward when "
                       "FS89_FUSED_ADALN is off.")
    return forward


# ----------------------------------------------------------------------------- patching

def _check_dit_structure(dit):
    """Refuse an upstream DiT module this pack was not written against
    (FlashVSR cf910c6; the reference guards the same, integrate.py:197-214):
    each rebound class must exist with the argument names its forward is
    called with, and the layout helpers the self-attention uses must exist."""
    where = getattr(dit, "__name__", repr(dit))
    for cls_name, wanted in _EXPECTED_SIGS.items():
        cls = getattr(dit, cls_name, None)
        if cls is None:
            raise RuntimeError(f"{where} has no {cls_name}; the MI355X operator pack targets "
                               "FlashVSR v1.1 (wan_video_dit at cf910c6)")
        have = set(inspect.signature(cls.forward).parameters)
        absent = [a for a in wanted if a not in have]
        if absent:
            raise RuntimeError(f"{where}.{cls_name}.forward lacks args {absent}: not the "
                               "upstream revision (cf910c6) the rebound forwards follow")
    absent = [n for n in _UPSTREAM_HELPERS if not hasattr(dit, n)]
    if absent:
        raise RuntimeError(f"{where} lacks {' / '.join(absent)}: unsupported upstream revision")


def _patch_dit(dit, fused_rope: bool, fused_adaln: bool):
    _check_dit_structure(dit)
    dit.FUSED_ROPE_FN = fused_rms_rope if fused_rope else None
    dit.FUSED_ADALN = (fused_ln_modulate, fused_gate_add) if fused_adaln else None
    if getattr(dit, "_FS89_PATCHED", False):
        return                      # forwards already rebound; the flags above are refreshed
    stock = {n: getattr(dit, n).forward for n in _EXPECTED_SIGS}
    setattr(dit, _STOCK_ATTR, stock)
    dit.SelfAttention.forward = _make_self_attn_forward(dit, stock["SelfAttention"])
    dit.CrossAttention.forward = _make_cross_attn_forward(dit, stock["CrossAttention"])
    dit.DiTBlock.forward = _make_dit_block_forward(dit, stock["DiTBlock"])
    dit._FS89_PATCHED = True


def _import_upstream_dit():
    try:
        import diffsynth.models.wan_video_dit as dit
    except ImportError as e:
        raise ImportError("enable() could not import diffsynth.models.wan_video_dit: run from a "
                          "FlashVSR checkout, or pass dit_module=") from e
    return dit


def _setup_decoder(pipe, compile_memblocks: bool) -> dict:
    done = {}
    dec = getattr(pipe, "TCDecoder", None)
    if dec is None:
        return done
    if _on("FS89_TCDEC_CL"):
        dec.to(memory_format=torch.channels_last)
        done["tcdec_channels_last"] = True
    if compile_memblocks:
        warnings.warn("FS89_TCDEC_COMPILE / compile_memblocks is not applied by the MI355X "
                      "operator pack (decoder-side torch.compile is outside the pack).")
        done["tcdec_compiled_memblocks"] = 0
    return done


def _setup_fp8(model, parts, per_row: bool, weights_file) -> dict:
    done = {}
    if not parts:
        return done
    stored = None
    if weights_file and os.path.exists(weights_file):
        try:
            stored = load_fp8_weights(weights_file)
            done["fp8_weights"] = "loaded"
        except FP8WeightsFormatError as e:
            # a file from an earlier version: quantise again and overwrite it
            warnings.warn(f"{e}; quantising again and rewriting it", stacklevel=3)
    done["fp8_linears"] = convert_linears_fp8(model, parts=parts, per_channel=per_row,
                                              per_token=per_row, stored=stored)
    if weights_file and stored is None and done["fp8_linears"]:
        save_fp8_weights(model, weights_file)
        done["fp8_weights"] = "saved"
    if "ffn" in parts and _on("FS89_FP8_FFNFUSED"):
        done["fp8_ffn_blocks"] = convert_ffn_fp8(model)
    return done


def enable(pipe, dit_module=None, parts=None, compile_memblocks=None, verbose=True,
           scale_granularity=None, fp8_weights=None):
    """Apply the operator pack to a FlashVSRTinyPipeline; returns a dict of
    what was enabled, with the reference's keys (integrate.py:229-292).

    Extensions: ``scale_granularity`` ('tensor', the reference's default, or
    'row'; env ``FS89_FP8_SCALE``) and ``fp8_weights`` (env
    ``FS89_FP8_WEIGHTS``): a file of quantised weights, loaded instead of
    quantising when it exists and written after the conversion when it does
    not (``applied["fp8_weights"]`` says which)."""
    if parts is None:
        parts = [p for p in os.environ.get("FS89_FP8", "ffn,self,cross").split(",") if p]
    if compile_memblocks is None:
        compile_memblocks = _on("FS89_TCDEC_COMPILE", "0")
    granularity = (scale_granularity or os.environ.get("FS89_FP8_SCALE", "tensor")).lower()
    if granularity not in ("tensor", "row"):
        raise ValueError(f"scale_granularity must be 'tensor' or 'row', got {granularity!r}")
    if fp8_weights is None:
        fp8_weights = os.environ.get("FS89_FP8_WEIGHTS") or None
    dit = dit_module if dit_module is not None else _import_upstream_dit()

    applied = _setup_decoder(pipe, compile_memblocks)
    applied.update(_setup_fp8(pipe.denoising_model(), parts, granularity == "row", fp8_weights))
    rope_on, adaln_on = _on("FS89_FUSED_ROPE"), _on("FS89_FUSED_ADALN")
    _patch_dit(dit, fused_rope=rope_on, fused_adaln=adaln_on)
    applied["fused_rope"] = rope_on
    applied["fused_adaln"] = adaln_on
    ensure_bsa_available()
    applied["lcsa_backend"] = active_backend()
    if verbose:
        print("[flashvsr-mi355x-ops] enabled: " + ", ".join(f"{k}={v}" for k, v in applied.items()))
    return applied
