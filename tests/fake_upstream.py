"""A stand-in for FlashVSR's ``diffsynth.models.wan_video_dit`` for GPU tests
of ``enable()``: the three classes it rebinds with the upstream module
structure (q/k/v/o Linears, RMSNorm q/k norms, the block's three LayerNorms,
the FFN ``Sequential(Linear, GELU(tanh), Linear)``, the [1, 6, dim]
modulation) and the helpers the self-attention calls.  The stock forwards
are not modelled: they raise, so a test fails if a fused path falls back to
them.  ``attn`` of the self-attention goes through the installed
``block_sparse_attn`` module, as the upstream one does."""
import types

import torch
import torch.nn as nn

BF = torch.bfloat16


def partition(x, win):
    """[B, f, h, w, C] -> [B * windows, wf*wh*ww, C], windows ordered
    (b, f//wf, h//wh, w//ww), tokens inside (f%wf, h%wh, w%ww)."""
    B, f, h, w, C = x.shape
    wf, wh, ww = win
    t = x.view(B, f // wf, wf, h // wh, wh, w // ww, ww, C).permute(0, 1, 3, 5, 2, 4, 6, 7)
    return t.reshape(-1, wf * wh * ww, C)


def reverse(x, win, fhw):
    f, h, w = fhw
    wf, wh, ww = win
    C = x.shape[-1]
    B = x.shape[0] // ((f // wf) * (h // wh) * (w // ww))
    t = x.view(B, f // wf, h // wh, w // ww, wf, wh, ww, C).permute(0, 1, 4, 2, 5, 3, 6, 7)
    return t.reshape(B, f, h, w, C)


def local_mask(bh, bw, rh, rw, include_self=True, device=None):
    """Windows of one time row within rh//2 rows and rw//2 columns of each other."""
    i = torch.arange(bh * bw, device=device)
    r, c = i // bw, i % bw
    m = ((r[:, None] - r[None, :]).abs() <= rh // 2) & ((c[:, None] - c[None, :]).abs() <= rw // 2)
    return m if include_self else m & ~torch.eye(bh * bw, dtype=torch.bool, device=device)


class RMSNorm(nn.Module):
    """Wan's RMSNorm: (x.float() * rsqrt(mean(x^2) + eps)).to(x.dtype) * weight."""

    def __init__(self, dim, eps, weight):
        super().__init__()
        self.eps = eps
        self.weight = nn.Parameter(weight)

    def forward(self, x):
        xf = x.float()
        return (xf * torch.rsqrt(xf.pow(2).mean(-1, keepdim=True) + self.eps)).to(x.dtype) \
            * self.weight


def make(dim, heads, ffn, g, device="cuda", cross_len=256, std=0.05):
    """(module, model): the fake upstream module and a model with one DiT
    block (``model.blocks[0]``) of bf16 weights drawn from generator g."""
    from flashvsr_sm89_ops.lcsa.draft import generate_draft_block_mask

    dit = types.ModuleType("fake_upstream_wan_video_dit")

    def linear(n, k):
        lin = nn.Linear(k, n, dtype=BF)
        with torch.no_grad():
            lin.weight.copy_(torch.randn(n, k, generator=g) * std)
            lin.bias.copy_(torch.randn(n, generator=g) * 0.02)
        return lin

    def vec(mean, s):
        return (mean + s * torch.randn(dim, generator=g)).to(BF)

    class SelfAttention(nn.Module):
        def __init__(self):
            super().__init__()
            self.num_heads, self.head_dim = heads, dim // heads
            self.q, self.k, self.v, self.o = (linear(dim, dim) for _ in range(4))
            self.norm_q, self.norm_k = RMSNorm(dim, 1e-6, vec(1, 0.1)), RMSNorm(dim, 1e-6, vec(1, 0.1))
            self.local_attn_mask = None
            self.local_attn_mask_h = self.local_attn_mask_w = self.local_range = None

        def attn(self, q, k, v, mask):
            import block_sparse_attn
            H, hd = self.num_heads, self.head_dim
            out = block_sparse_attn.block_sparse_attn_func(
                q[0].view(-1, H, hd), k[0].view(-1, H, hd), v[0].view(-1, H, hd), None, None,
                None, None, mask, q.shape[1], k.shape[1])
            return out.reshape(1, -1, H * hd)

        def forward(self, x, freqs, f=None, h=None, w=None, local_num=None, topk=None,
                    train_img=False, block_id=None, kv_len=None, is_full_block=False,
                    is_stream=False, pre_cache_k=None, pre_cache_v=None, local_range=9):
            raise AssertionError("stock self-attention called")

    class CrossAttention(nn.Module):
        def __init__(self):
            super().__init__()
            self.num_heads, self.head_dim = heads, dim // heads
            self.q, self.k, self.v, self.o = (linear(dim, dim) for _ in range(4))
            self.norm_q = RMSNorm(dim, 1e-6, vec(1, 0.1))
            self.cache_k = (torch.randn(1, cross_len, dim, generator=g)).to(BF)
            self.cache_v = (torch.randn(1, cross_len, dim, generator=g)).to(BF)

        def attn(self, q, k, v):
            raise AssertionError("the DiT's dense attention called: the HIP path was expected")

        def forward(self, x, y, is_stream=False):
            raise AssertionError("stock cross-attention called")

    class DiTBlock(nn.Module):
        def __init__(self):
            super().__init__()
            self.self_attn = SelfAttention()
            self.cross_attn = CrossAttention()
            self.norm1 = nn.LayerNorm(dim, eps=1e-6, elementwise_affine=False)
            self.norm2 = nn.LayerNorm(dim, eps=1e-6, elementwise_affine=False)
            self.norm3 = nn.LayerNorm(dim, eps=1e-6, dtype=BF)
            with torch.no_grad():
                self.norm3.weight.copy_(vec(1, 0.1))
                self.norm3.bias.copy_(vec(0, 0.1))
            self.ffn = nn.Sequential(linear(ffn, dim), nn.GELU(approximate="tanh"),
                                     linear(dim, ffn))
            self.modulation = nn.Parameter((torch.randn(1, 6, dim, generator=g) * 0.1).to(BF))

        def gate(self, x, gate, residual):
            return x + gate * residual

        def forward(self, x, context, t_mod, freqs, f, h, w, local_num=None, topk=None,
                    train_img=False, block_id=None, kv_len=None, is_full_block=False,
                    is_stream=False, pre_cache_k=None, pre_cache_v=None, local_range=9):
            raise AssertionError("stock DiT block called")

    dit.SelfAttention, dit.CrossAttention, dit.DiTBlock = SelfAttention, CrossAttention, DiTBlock
    dit.WindowPartition3D = types.SimpleNamespace(partition=partition, reverse=reverse)
    dit.build_local_block_mask_shifted_vec_normal_slide = local_mask
    dit.generate_draft_block_mask = generate_draft_block_mask
    dit.modulate = lambda x, shift, scale: x * (1 + scale) + shift

    model = nn.Module()
    model.blocks = nn.ModuleList([DiTBlock()])
    model.to(device)
    blk = model.blocks[0]
    blk.cross_attn.cache_k = blk.cross_attn.cache_k.to(device)
    blk.cross_attn.cache_v = blk.cross_attn.cache_v.to(device)
    return dit, model


class Pipe:
    def __init__(self, model):
        self.model = model

    def denoising_model(self):
        return self.model
