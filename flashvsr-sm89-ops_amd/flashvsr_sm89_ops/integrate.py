"""One-call wiring of the operator pack into a FlashVSR v1.1 Tiny pipeline.

``enable(pipe)`` keeps the reference's contract (flashvsr_sm89_ops/integrate.py:229-292):
call it once after ``pipe.to('cuda')`` / ``pipe.enable_vram_management(...)``
and before ``pipe.init_cross_kv()``.  In dependency order it

1. sets the TCDecoder to channels_last (``FS89_TCDEC_CL``, default on);
2. converts the DiT Linears to ``FP8Linear`` and the FFNs to ``FP8FFN``
   (``FS89_FP8`` parts, ``FS89_FP8_FFNFUSED``), scale granularity from
   ``FS89_FP8_SCALE`` = ``tensor`` (default, as the reference) or ``row``
   (per-output-channel weights, per-token activations);
3. rebinds upstream ``SelfAttention.forward`` / ``CrossAttention.forward`` /
   ``DiTBlock.forward`` with fused-aware copies whose stock branches are the
   upstream math, so each flag can be switched off (``FS89_FUSED_ROPE``,
   ``FS89_FUSED_ADALN``);
4. resolves ``block_sparse_attn`` to the HIP block-sparse attention;
   ``FS89_DRAFT=1`` also computes the draft block mask on the device
   (``lcsa/draft.py``, the bf16 reading of lcsa/reference.py:37-64) in place
   of the DiT's ``generate_draft_block_mask`` (default off: the DiT's own
   function is the one the reference calls);
5. runs the cross-attention's dense attention over the cached prompt K/V on
   the same HIP attention kernel with every block kept (``FS89_CROSS_ATTN``,
   default on, shapes it covers: batch 1, head_dim 128, token counts in
   multiples of 128; others keep the DiT's attention), and with
   ``FS89_FUSED_ADALN`` the affine ``norm3`` LayerNorm before it.

Re-running ``enable`` on a patched pipeline is safe.  ``FS89_TCDEC_COMPILE``
(torch.compile of the decoder MemBlocks) is accepted but not applied: it is a
decoder-side inductor compile outside this operator pack, and inductor would
bring Triton kernels back in.
"""
from __future__ import annotations

import os
import warnings

import torch

from .compat_bsa import active_backend, ensure_bsa_available
from .fp8_ffn import convert_ffn_fp8
from .fp8_linear import FP8Linear, convert_linears_fp8, fp8_gemm, load_fp8_weights, save_fp8_weights
from .fp8_quant import quantize_fp8
from .cross_attn import cross_attention
from .cross_attn import supported as cross_supported
from .fused_adaln import (fused_gate_add, fused_gate_add_layer_norm,
                          fused_gate_add_ln_modulate_quant, fused_ln_modulate,
                          fused_ln_modulate_quant, layer_norm)
from .cross_attn import unit_gate
from .fp8_ffn import FP8FFN, gemm_gelu_quant_fp8
from .block import window_token_map
from .fused_rms_rope import fused_rms_rope, fused_rms_rope_qkv_rows
from .lcsa.draft import draft_index
from .lcsa.hip_lcsa import block_sparse_attention_strided, build_csr


def _FLAG(name, default):
    return os.environ.get(name, default) == "1"


def _unwrap(m):
    """enable_vram_management wraps norms/linears in AutoWrappedModule."""
    return getattr(m, "module", m)


def _module_eps(m, default=1e-6):
    return getattr(_unwrap(m), "eps", default)


def _window_path_on() -> bool:
    return _FLAG("FS89_WINDOW", "1") and active_backend() == "hip"


def _window_path_ok(x, f, h, w, head_dim) -> bool:
    """Shapes the copy-free path serves: batch 1, bf16 on the GPU, whole
    2x8x8 windows, head_dim 128, a hidden size the fused kernels take."""
    B, L, D = x.shape
    return (B == 1 and x.dtype == torch.bfloat16 and x.is_cuda and head_dim == 128
            and f % 2 == 0 and h % 8 == 0 and w % 8 == 0 and L == f * h * w
            and D % head_dim == 0 and D <= 1536)


_MAPS = {}


def _window_maps(f, h, w, n_cache_rows, device):
    """(tok_map, kv_rows, kv_map) for one (f, h, w, cache) geometry: window
    position -> raster token; raster token -> row of the K/V buffer (after the
    cached rows); identity over the whole K/V buffer."""
    key = (f, h, w, n_cache_rows, str(device))
    m = _MAPS.get(key)
    if m is None:
        tok = window_token_map(f, h, w, device=device)
        inv = torch.empty_like(tok)
        inv[tok.long()] = torch.arange(tok.numel(), dtype=torch.int32, device=device)
        kv_rows = (inv + n_cache_rows).contiguous()
        kv_map = torch.arange(n_cache_rows + tok.numel(), dtype=torch.int32, device=device)
        if len(_MAPS) >= 32:  # a few geometries per run; keep the cache bounded
            _MAPS.pop(next(iter(_MAPS)))
        m = _MAPS[key] = (tok, kv_rows, kv_map)
    return m


def _appendable(t, store, frontier):
    """t is a contiguous row range of `store` that ends at row `frontier`."""
    D = store.shape[1]
    return (t.is_contiguous() and t.device == store.device and t.dtype == store.dtype
            and t.untyped_storage().data_ptr() == store.untyped_storage().data_ptr()
            and t.storage_offset() % D == 0 and t.storage_offset() + t.numel() == frontier * D)


def _kv_buffers(mod, pre_k, pre_v, cache_rows, L, D, like, grow):
    """K/V buffers [cache_rows + L, D] whose first rows hold the cached windows.
    The caches this path returns are views of a per-module store with room
    after them; when the caller passes them back unchanged (the streaming
    loop does), the new chunk is appended behind them in place and the cache
    is not copied (the reference concatenates).  Otherwise, or when the store
    is full, a new store is made and the cache copied into it once."""
    st = getattr(mod, "_fs89_kv", None)
    if st is not None and cache_rows and pre_k is not None and pre_v is not None:
        sk, sv, fr = st
        if fr + L <= sk.shape[0] and _appendable(pre_k, sk, fr) and _appendable(pre_v, sv, fr):
            start = fr - cache_rows
            mod._fs89_kv = (sk, sv, fr + L)
            return sk[start:fr + L], sv[start:fr + L]
    rows = cache_rows + L
    cap = rows + (4 * L if grow else 0)  # room for a few appended chunks
    sk = torch.empty((cap, D), dtype=like.dtype, device=like.device)
    sv = torch.empty((cap, D), dtype=like.dtype, device=like.device)
    if cache_rows:
        sk[:cache_rows].copy_(pre_k.reshape(-1, D))
        sv[:cache_rows].copy_(pre_v.reshape(-1, D))
    mod._fs89_kv = (sk, sv, rows) if grow else None
    return sk[:rows], sv[:rows]


def _qkv_fused(mod):
    """One [3D, D] e4m3 weight for the q, k and v FP8Linears (built once per
    module, rebuilt if any of them changes): the three projections of the
    same activations become one GEMM on one quantisation of them (the
    reference quantises the input three times).  Per-tensor weight scales
    become per-column vectors of the same value, which the GEMM epilogue
    applies with the same arithmetic.  None when the three cannot share."""
    lins = [getattr(mod, n, None) for n in ("q", "k", "v")]
    if not all(isinstance(l, FP8Linear) for l in lins):
        return None
    if len({l.per_token for l in lins}) != 1 or len({l.in_features for l in lins}) != 1:
        return None
    if len({l.bias is None for l in lins}) != 1:
        return None
    key = tuple((l.weight.data_ptr(), l.weight._version, l.w_scale.data_ptr(), l.w_scale._version,
                 None if l.bias is None else (l.bias.data_ptr(), l.bias._version)) for l in lins)
    c = getattr(mod, "_fs89_qkv", None)
    if c is not None and c[0] == key:
        return c[1]
    w3 = torch.cat([l.weight for l in lins]).contiguous()
    s3 = torch.cat([l.w_scale.float().reshape(-1).expand(l.out_features) for l in lins]).contiguous()
    b3 = None if lins[0].bias is None else torch.cat([l.bias for l in lins]).contiguous()
    val = (w3, s3, b3, lins[0].per_token)
    mod._fs89_qkv = (key, val)
    return val


def _window_self_attention(dit, self, x, freqs, f, h, w, topk, kv_len, is_stream, pre_cache_k,
                           pre_cache_v, local_range, x8s=None):
    """The self-attention of integrate.py:42-126 without its layout copies (F2):
    q stays in raster order and is read through the window map; k and v leave
    the RMSNorm/RoPE pass directly in window order, behind the cached windows,
    in the K/V buffer (no partition, no torch.cat; see _kv_buffers); the
    attention writes its output in raster order (no reverse).  The draft mask
    is the device one reading q through the map (FS89_DRAFT=1), or the DiT's
    own on a gathered window-ordered q.  Returns what the reference
    returns, the caches included (window-ordered [windows, 128, D] views)."""
    B, L, D = x.shape
    fq = _qkv_fused(self)
    if fq is not None:
        w3, s3, b3, per_token = fq
        if x8s is None:
            x8s = quantize_fp8(x.reshape(-1, D), per_token=per_token)
        qkv = fp8_gemm(x8s[0], x8s[1], w3, s3, b3)  # [L, 3D]: q, k, v column slices
        q, k, v = (qkv[:, i * D:(i + 1) * D].view(B, L, D) for i in range(3))
    else:
        if x8s is not None:
            raise ValueError("activation codes given but q/k/v are not FP8 linears")
        q = self.q(x).contiguous()
        k = self.k(x).contiguous()
        v = self.v(x).contiguous()
    win = (2, 8, 8)
    seqlen = f // win[0]
    block_s = win[0] * win[1] * win[2]
    one_len = L // block_s // seqlen
    n_cache = 0 if pre_cache_k is None or pre_cache_v is None else pre_cache_k.shape[0]
    kbuf, vbuf = _kv_buffers(self, pre_cache_k, pre_cache_v, n_cache * block_s, L, D, q,
                             is_stream)
    if _module_eps(self.norm_k) != _module_eps(self.norm_q):
        raise NotImplementedError("q and k RMSNorm eps differ")
    tok, kv_rows, kv_map = _window_maps(f, h, w, n_cache * block_s, q.device)
    fused_rms_rope_qkv_rows(q, k, v, _unwrap(self.norm_q).weight, _unwrap(self.norm_k).weight,
                            freqs, kbuf, vbuf, kv_rows, eps=_module_eps(self.norm_q),
                            head_dim=self.head_dim)
    k_w = kbuf.view(-1, block_s, D)
    v_w = vbuf.view(-1, block_s, D)

    if self.local_attn_mask is None or self.local_attn_mask_h != h // 8 \
            or self.local_attn_mask_w != w // 8 or self.local_range != local_range:
        self.local_attn_mask = dit.build_local_block_mask_shifted_vec_normal_slide(
            h // 8, w // 8, local_range, local_range, include_self=True, device=k_w.device)
        self.local_attn_mask_h = h // 8
        self.local_attn_mask_w = w // 8
        self.local_range = local_range
    nq = L // block_s
    q2 = q.reshape(L, D)  # a view (rows may be strided: column slice of the fused qkv)
    if _FLAG("FS89_DRAFT", "0"):
        index = draft_index(q2, k_w, nheads=self.num_heads, q_temporal=seqlen,
                            local=self.local_attn_mask, topk=topk, nq=nq, q_map=tok)
    else:
        # The DiT's own draft mask (the reference's call, integrate.py:103-104)
        # on window-ordered q (one gather) and the window-ordered K buffer.
        q_w = q2.index_select(0, tok.long()).view(-1, block_s, D)
        mask = dit.generate_draft_block_mask(B, self.num_heads, seqlen, q_w, k_w, topk=topk,
                                             local_attn_mask=self.local_attn_mask)
        index = build_csr(mask[0] if mask.dim() == 4 else mask)
    out = torch.empty((L, D), dtype=q.dtype, device=q.device)
    hd = self.head_dim
    block_sparse_attention_strided(
        q2, kbuf, vbuf, None, None, heads=self.num_heads, head_dim=hd,
        q_strides=(q2.stride(0), hd), kv_strides=(D, hd), out=out, o_strides=(D, hd), q_map=tok,
        kv_map=kv_map, index=index)

    cache_num = k_w.shape[0] // one_len
    if cache_num > kv_len:
        cache_k, cache_v = k_w[one_len:], v_w[one_len:]
    else:
        cache_k, cache_v = k_w, v_w
    y = self.o(out.view(B, L, D))
    if is_stream:
        return y, cache_k, cache_v
    return y


def _make_self_attn_forward(dit):
    """Fused-aware copy of upstream SelfAttention.forward (integrate.py:42-126);
    with FUSED_ROPE_FN=None the stock branch reproduces upstream exactly."""
    from einops import rearrange

    def forward(self, x, freqs, f=None, h=None, w=None, local_num=None, topk=None,
                train_img=False, block_id=None, kv_len=None, is_full_block=False,
                is_stream=False, pre_cache_k=None, pre_cache_v=None, local_range=9):
        B, L, D = x.shape
        if is_stream and pre_cache_k is not None and pre_cache_v is not None:
            assert f == 2, "f must be 2"
        if is_stream and (pre_cache_k is None or pre_cache_v is None):
            assert f == 6, " start f must be 6"
        assert L == f * h * w, "Sequence length mismatch with provided (f,h,w)."

        rope_fn = getattr(dit, "FUSED_ROPE_FN", None)
        if rope_fn is not None and _window_path_ok(x, f, h, w, self.head_dim) and _window_path_on():
            return _window_self_attention(dit, self, x, freqs, f, h, w, topk, kv_len, is_stream,
                                          pre_cache_k, pre_cache_v, local_range)
        if rope_fn is not None:
            q = rope_fn(self.q(x), _unwrap(self.norm_q).weight, freqs,
                        eps=_module_eps(self.norm_q), rope=True, head_dim=self.head_dim)
            k = rope_fn(self.k(x), _unwrap(self.norm_k).weight, freqs,
                        eps=_module_eps(self.norm_k), rope=True, head_dim=self.head_dim)
        else:
            q = self.norm_q(self.q(x))
            k = self.norm_k(self.k(x))
            q = dit.rope_apply(q, freqs, self.num_heads)
            k = dit.rope_apply(k, freqs, self.num_heads)
        v = self.v(x)

        win = (2, 8, 8)
        q = q.view(B, f, h, w, D)
        k = k.view(B, f, h, w, D)
        v = v.view(B, f, h, w, D)

        q_w = dit.WindowPartition3D.partition(q, win)
        k_w = dit.WindowPartition3D.partition(k, win)
        v_w = dit.WindowPartition3D.partition(v, win)

        seqlen = f // win[0]
        one_len = k_w.shape[0] // B // seqlen
        if pre_cache_k is not None and pre_cache_v is not None:
            k_w = torch.cat([pre_cache_k, k_w], dim=0)
            v_w = torch.cat([pre_cache_v, v_w], dim=0)

        block_n = q_w.shape[0] // B
        block_s = q_w.shape[1]
        block_n_kv = k_w.shape[0] // B

        reorder_q = rearrange(q_w, '(b block_n) (block_s) d -> b (block_n block_s) d',
                              block_n=block_n, block_s=block_s)
        reorder_k = rearrange(k_w, '(b block_n) (block_s) d -> b (block_n block_s) d',
                              block_n=block_n_kv, block_s=block_s)
        reorder_v = rearrange(v_w, '(b block_n) (block_s) d -> b (block_n block_s) d',
                              block_n=block_n_kv, block_s=block_s)

        if self.local_attn_mask is None or self.local_attn_mask_h != h // 8 \
                or self.local_attn_mask_w != w // 8 or self.local_range != local_range:
            self.local_attn_mask = dit.build_local_block_mask_shifted_vec_normal_slide(
                h // 8, w // 8, local_range, local_range, include_self=True, device=k_w.device)
            self.local_attn_mask_h = h // 8
            self.local_attn_mask_w = w // 8
            self.local_range = local_range
        draft = dit.generate_draft_block_mask
        if _FLAG("FS89_DRAFT", "0"):
            from .lcsa.draft import generate_draft_block_mask as draft
        attention_mask = draft(
            B, self.num_heads, seqlen, q_w, k_w, topk=topk, local_attn_mask=self.local_attn_mask)

        x = self.attn(reorder_q, reorder_k, reorder_v, attention_mask)

        cur_block_n, cur_block_s, _ = k_w.shape
        cache_num = cur_block_n // one_len
        if cache_num > kv_len:
            cache_k = k_w[one_len:, :, :]
            cache_v = v_w[one_len:, :, :]
        else:
            cache_k = k_w
            cache_v = v_w

        x = rearrange(x, 'b (block_n block_s) d -> (b block_n) (block_s) d',
                      block_n=block_n, block_s=block_s)
        x = dit.WindowPartition3D.reverse(x, win, (f, h, w))
        x = x.view(B, f * h * w, D)

        if is_stream:
            return self.o(x), cache_k, cache_v
        return self.o(x)

    return forward


def _make_cross_attn_forward(dit):
    """Fused-aware copy of upstream CrossAttention.forward (integrate.py:129-145)."""

    def forward(self, x, y, is_stream=False):
        rope_fn = getattr(dit, "FUSED_ROPE_FN", None)
        if rope_fn is not None:
            q = rope_fn(self.q(x), _unwrap(self.norm_q).weight, None,
                        eps=_module_eps(self.norm_q), rope=False)
        else:
            q = self.norm_q(self.q(x))
        assert self.cache_k is not None and self.cache_v is not None
        k = self.cache_k
        v = self.cache_v
        if _FLAG("FS89_CROSS_ATTN", "1") and cross_supported(q, k, v, self.num_heads):
            x = cross_attention(q, k, v, self.num_heads)
        else:
            x = self.attn(q, k, v)
        return self.o(x)

    return torch.no_grad()(forward)


def _affine_layer_norm(m):
    """(weight, bias, eps) when m is an affine nn.LayerNorm over bf16, else None."""
    m = _unwrap(m)
    if not isinstance(m, torch.nn.LayerNorm) or not m.elementwise_affine:
        return None
    w, b = m.weight, m.bias
    if w is None or w.dtype != torch.bfloat16 or not w.is_cuda:
        return None
    return w, b, m.eps


def _row_codes_block(dit, blk, x, f, h, w) -> bool:
    """The DiT block runs the per-token FP8 dataflow of the C5 block (AdaLN
    writing codes, one q/k/v GEMM, the copy-free self-attention): fused AdaLN
    and RoPE on, the HIP attention, per-token q/k/v FP8 linears, batch-1 bf16
    input in whole windows."""
    sa = getattr(blk, "self_attn", None)
    if sa is None or getattr(dit, "FUSED_ADALN", None) is None or \
            getattr(dit, "FUSED_ROPE_FN", None) is None:
        return False
    if not (_window_path_on() and _window_path_ok(x, f, h, w, getattr(sa, "head_dim", 0))):
        return False
    fq = _qkv_fused(sa)
    return fq is not None and fq[3]


def _make_dit_block_forward(dit):
    """Fused-aware copy of upstream DiTBlock.forward (integrate.py:148-184)."""

    def forward(self, x, context, t_mod, freqs, f, h, w, local_num=None, topk=None,
                train_img=False, block_id=None, kv_len=None, is_full_block=False,
                is_stream=False, pre_cache_k=None, pre_cache_v=None, local_range=9):
        shift_msa, scale_msa, gate_msa, shift_mlp, scale_mlp, gate_mlp = (
            self.modulation.to(dtype=t_mod.dtype, device=t_mod.device) + t_mod).chunk(6, dim=1)
        fa = getattr(dit, "FUSED_ADALN", None)
        if fa is not None:
            ln_mod, gate_add = fa
        rows = _row_codes_block(dit, self, x, f, h, w)
        if rows:
            # Per-token FP8 throughout: the AdaLN writes the codes the fused
            # q/k/v GEMM takes (no bf16 round trip, one quantisation).
            x8s = fused_ln_modulate_quant(x, scale_msa, shift_msa, eps=_module_eps(self.norm1))
            r = _window_self_attention(dit, self.self_attn, x, freqs, f, h, w, topk, kv_len,
                                       is_stream, pre_cache_k, pre_cache_v, local_range, x8s=x8s)
            self_attn_output, self_attn_cache_k, self_attn_cache_v = (
                r if is_stream else (r, None, None))
        else:
            if fa is not None:
                input_x = ln_mod(x, scale_msa, shift_msa, eps=_module_eps(self.norm1))
            else:
                input_x = dit.modulate(self.norm1(x), shift_msa, scale_msa)
            self_attn_output, self_attn_cache_k, self_attn_cache_v = self.self_attn(
                input_x, freqs, f, h, w, local_num, topk, train_img, block_id,
                kv_len=kv_len, is_full_block=is_full_block, is_stream=is_stream,
                pre_cache_k=pre_cache_k, pre_cache_v=pre_cache_v, local_range=local_range)

        ln3 = _affine_layer_norm(self.norm3) if fa is not None else None
        if ln3 is not None and x.dtype == torch.bfloat16 and x.is_cuda and \
                self_attn_output.is_contiguous() and gate_msa.is_contiguous():
            # the gated residual and norm3 in one pass over the rows
            x, normed = fused_gate_add_layer_norm(x, gate_msa, self_attn_output, ln3[0], ln3[1],
                                                  eps=ln3[2])
        else:
            if fa is not None:
                x = gate_add(x, gate_msa, self_attn_output)
            else:
                x = self.gate(x, gate_msa, self_attn_output)
            if ln3 is not None and x.dtype == torch.bfloat16 and x.is_cuda:
                normed = layer_norm(x, ln3[0], ln3[1], eps=ln3[2])
            else:
                normed = self.norm3(x)
        yc = self.cross_attn(normed, context, is_stream=is_stream)
        if rows and isinstance(self.ffn, FP8FFN) and yc.shape == x.shape and yc.is_contiguous():
            # x + cross-attention output and the FFN's AdaLN in one pass (a
            # unit gate), its per-token codes straight into the FFN's GEMMs.
            B, L, D = x.shape
            x, h8, hs = fused_gate_add_ln_modulate_quant(
                x, unit_gate(D, x.device), yc, scale_mlp, shift_mlp, eps=_module_eps(self.norm2))
            g8, gs = gemm_gelu_quant_fp8(h8, hs, self.ffn.lin0, True)
            yf = self.ffn.lin2._mm(g8, gs)
            x = gate_add(x, gate_mlp, yf.view(B, L, -1))
            if is_stream:
                return x, self_attn_cache_k, self_attn_cache_v
            return x
        x = x + yc
        if fa is not None:
            input_x = ln_mod(x, scale_mlp, shift_mlp, eps=_module_eps(self.norm2))
        else:
            input_x = dit.modulate(self.norm2(x), shift_mlp, scale_mlp)
        if fa is not None:
            x = gate_add(x, gate_mlp, self.ffn(input_x))
        else:
            x = self.gate(x, gate_mlp, self.ffn(input_x))
        if is_stream:
            return x, self_attn_cache_k, self_attn_cache_v
        return x

    return forward


_EXPECTED_SIGS = {
    "SelfAttention": ("x", "freqs", "f", "h", "w", "local_num", "topk", "train_img",
                      "block_id", "kv_len", "is_full_block", "is_stream",
                      "pre_cache_k", "pre_cache_v", "local_range"),
    "DiTBlock": ("x", "context", "t_mod", "freqs", "f", "h", "w", "local_num", "topk",
                 "train_img", "block_id", "kv_len", "is_full_block", "is_stream",
                 "pre_cache_k", "pre_cache_v", "local_range"),
}


def _check_dit_structure(dit):
    """Guard against upstream drift (integrate.py:197-214): the rebound classes
    must exist and keep the argument names the forwards pass positionally."""
    import inspect
    for cls, expected in _EXPECTED_SIGS.items():
        c = getattr(dit, cls, None)
        if c is None:
            raise RuntimeError(f"upstream wan_video_dit has no {cls}; this pack "
                               f"targets FlashVSR v1.1 — got {dit}")
        params = tuple(inspect.signature(c.forward).parameters)
        missing = [p for p in expected if p not in params]
        if missing:
            raise RuntimeError(
                f"upstream {cls}.forward lacks args {missing} — upstream signature "
                f"changed since the tested revision (cf910c6).")
    if not hasattr(dit, "WindowPartition3D") or not hasattr(dit, "generate_draft_block_mask"):
        raise RuntimeError("upstream wan_video_dit lacks WindowPartition3D / "
                           "generate_draft_block_mask — unsupported revision.")


def _patch_dit(dit, fused_rope, fused_adaln):
    _check_dit_structure(dit)
    dit.FUSED_ROPE_FN = fused_rms_rope if fused_rope else None
    dit.FUSED_ADALN = (fused_ln_modulate, fused_gate_add) if fused_adaln else None
    if getattr(dit, "_FS89_PATCHED", False):
        return  # forwards already rebound; flags above refreshed
    dit.SelfAttention.forward = _make_self_attn_forward(dit)
    dit.CrossAttention.forward = _make_cross_attn_forward(dit)
    dit.DiTBlock.forward = _make_dit_block_forward(dit)
    dit._FS89_PATCHED = True


def enable(pipe, dit_module=None, parts=None, compile_memblocks=None, verbose=True,
           scale_granularity=None, fp8_weights=None):
    """Apply the operator pack to a FlashVSRTinyPipeline; returns a dict of
    what was enabled (same keys as the reference).  ``fp8_weights`` (or
    ``FS89_FP8_WEIGHTS``) names a file of quantised weights: loaded instead of
    quantising when it exists, written after the conversion when it does not
    (then ``applied["fp8_weights"]`` says which)."""
    if parts is None:
        parts = [p for p in os.environ.get("FS89_FP8", "ffn,self,cross").split(",") if p]
    if compile_memblocks is None:
        compile_memblocks = _FLAG("FS89_TCDEC_COMPILE", "0")
    if scale_granularity is None:
        scale_granularity = os.environ.get("FS89_FP8_SCALE", "tensor").lower()
    if scale_granularity not in ("tensor", "row"):
        raise ValueError(f"scale_granularity must be 'tensor' or 'row', got {scale_granularity!r}")
    row = scale_granularity == "row"

    applied = {}

    if dit_module is None:
        try:
            import diffsynth.models.wan_video_dit as dit_module
        except ImportError as e:
            raise ImportError(
                "enable() could not import diffsynth.models.wan_video_dit. Run from a "
                "FlashVSR checkout (or pass dit_module=).") from e

    if hasattr(pipe, "TCDecoder") and _FLAG("FS89_TCDEC_CL", "1"):
        pipe.TCDecoder.to(memory_format=torch.channels_last)
        applied["tcdec_channels_last"] = True

    if compile_memblocks and hasattr(pipe, "TCDecoder"):
        warnings.warn("FS89_TCDEC_COMPILE / compile_memblocks is not applied by the MI355X "
                      "operator pack (decoder-side torch.compile is outside the pack).")
        applied["tcdec_compiled_memblocks"] = 0

    if fp8_weights is None:
        fp8_weights = os.environ.get("FS89_FP8_WEIGHTS") or None
    if parts:
        stored = None
        if fp8_weights and os.path.exists(fp8_weights):
            stored = load_fp8_weights(fp8_weights)
            applied["fp8_weights"] = "loaded"
        n = convert_linears_fp8(pipe.denoising_model(), parts=parts, per_channel=row,
                                per_token=row, stored=stored)
        applied["fp8_linears"] = n
        if fp8_weights and stored is None and n:
            save_fp8_weights(pipe.denoising_model(), fp8_weights)
            applied["fp8_weights"] = "saved"
        if "ffn" in parts and _FLAG("FS89_FP8_FFNFUSED", "1"):
            applied["fp8_ffn_blocks"] = convert_ffn_fp8(pipe.denoising_model())

    _patch_dit(dit_module,
               fused_rope=_FLAG("FS89_FUSED_ROPE", "1"),
               fused_adaln=_FLAG("FS89_FUSED_ADALN", "1"))
    applied["fused_rope"] = _FLAG("FS89_FUSED_ROPE", "1")
    applied["fused_adaln"] = _FLAG("FS89_FUSED_ADALN", "1")

    ensure_bsa_available()
    applied["lcsa_backend"] = active_backend()

    if verbose:
        bits = [f"{k}={v}" for k, v in applied.items()]
        print(f"[flashvsr-mi355x-ops] enabled: {', '.join(bits)}")
    return applied
