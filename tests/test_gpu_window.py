"""F2: the self-attention without its layout copies (integrate.py:42-126 with
the window-order layout folded into the RMSNorm/RoPE pass and the attention's
token maps) against the reference sequence of the same forward: partition of
q/k/v, torch.cat with the KV cache, rearrange, attention on window-ordered
tensors, reverse.  Both run the same kernels (projections, RMSNorm+RoPE,
device draft mask, block-sparse attention), so outputs and caches must agree
bit for bit over a streaming pair of chunks (6 latent frames, then 2 with the
cache)."""
import types

import pytest
import torch

pytestmark = pytest.mark.gpu

D, HD = 256, 128
WIN = (2, 8, 8)


def _partition(x, win):
    """WindowPartition3D.partition for [B, f, h, w, C] -> [B*nwin, 128, C]
    (the order lcsa/reference.py:15-21 describes)."""
    B, f, h, w, C = x.shape
    wf, wh, ww = win
    t = x.view(B, f // wf, wf, h // wh, wh, w // ww, ww, C).permute(0, 1, 3, 5, 2, 4, 6, 7)
    return t.reshape(-1, wf * wh * ww, C)


def _reverse(x, win, fhw):
    f, h, w = fhw
    wf, wh, ww = win
    C = x.shape[-1]
    B = x.shape[0] // ((f // wf) * (h // wh) * (w // ww))
    t = x.view(B, f // wf, h // wh, w // ww, wf, wh, ww, C).permute(0, 1, 4, 2, 5, 3, 6, 7)
    return t.reshape(B, f, h, w, C)


def _local_mask(bh, bw, rh, rw, include_self=True, device=None):
    """A neighbourhood rule over the bh x bw windows of one time row."""
    i = torch.arange(bh * bw, device=device)
    r, c = i // bw, i % bw
    m = ((r[:, None] - r[None, :]).abs() <= rh // 2) & ((c[:, None] - c[None, :]).abs() <= rw // 2)
    return m if include_self else m & ~torch.eye(bh * bw, dtype=torch.bool, device=device)


class _Norm(torch.nn.Module):
    def __init__(self, g):
        super().__init__()
        self.weight = torch.nn.Parameter((1 + 0.1 * torch.randn(D, generator=g)).to(torch.bfloat16))
        self.eps = 1e-6


def _fake_dit():
    from flashvsr_sm89_ops.compat_bsa import _hip_block_sparse_attn_func
    from flashvsr_sm89_ops.lcsa.draft import generate_draft_block_mask

    dit = types.ModuleType("fake_dit_for_window_path")

    class SelfAttention(torch.nn.Module):
        def __init__(self, g):
            super().__init__()
            self.num_heads, self.head_dim = D // HD, HD
            for n in ("q", "k", "v", "o"):
                lin = torch.nn.Linear(D, D, dtype=torch.bfloat16)
                with torch.no_grad():
                    lin.weight.copy_(torch.randn(D, D, generator=g) * 0.05)
                    lin.bias.copy_(torch.randn(D, generator=g) * 0.02)
                setattr(self, n, lin)
            self.norm_q, self.norm_k = _Norm(g), _Norm(g)
            self.local_attn_mask = None
            self.local_attn_mask_h = self.local_attn_mask_w = self.local_range = None

        def attn(self, q, k, v, mask):
            H = self.num_heads
            out = _hip_block_sparse_attn_func(
                q[0].view(-1, H, HD), k[0].view(-1, H, HD), v[0].view(-1, H, HD), None, None,
                None, None, mask, q.shape[1], k.shape[1])
            return out.reshape(1, -1, D)

        def forward(self, x, freqs, f=None, h=None, w=None, local_num=None, topk=None,
                    train_img=False, block_id=None, kv_len=None, is_full_block=False,
                    is_stream=False, pre_cache_k=None, pre_cache_v=None, local_range=9):
            raise AssertionError("rebound by enable()")

    class CrossAttention(torch.nn.Module):
        def forward(self, x, y, is_stream=False):
            raise AssertionError

    class DiTBlock(torch.nn.Module):
        def forward(self, x, context, t_mod, freqs, f, h, w, local_num=None, topk=None,
                    train_img=False, block_id=None, kv_len=None, is_full_block=False,
                    is_stream=False, pre_cache_k=None, pre_cache_v=None, local_range=9):
            raise AssertionError

    dit.SelfAttention, dit.CrossAttention, dit.DiTBlock = SelfAttention, CrossAttention, DiTBlock
    dit.WindowPartition3D = types.SimpleNamespace(partition=_partition, reverse=_reverse)
    dit.build_local_block_mask_shifted_vec_normal_slide = _local_mask
    dit.generate_draft_block_mask = generate_draft_block_mask
    dit.modulate = lambda x, shift, scale: x * (1 + scale) + shift
    return dit


class _Pipe:
    def __init__(self):
        self.model = torch.nn.Module()

    def denoising_model(self):
        return self.model


def _freqs(L, device):
    ang = torch.rand(L, 1, HD // 2, dtype=torch.float64) * 6.28
    return torch.polar(torch.ones_like(ang), ang).to(torch.complex64).to(device)


@pytest.mark.parametrize("hw,draft", [((16, 16), "1"), ((16, 24), "1"), ((16, 24), "0")])
def test_window_path_equals_copy_path(monkeypatch, hw, draft):
    import flashvsr_sm89_ops as fv
    from flashvsr_sm89_ops import integrate
    h, w = hw
    taken = []
    real = integrate._window_self_attention

    def spy(*a, **k):
        taken.append(1)
        return real(*a, **k)
    monkeypatch.setattr(integrate, "_window_self_attention", spy)
    dev = "cuda"
    dit = _fake_dit()
    monkeypatch.setenv("FS89_FP8", "")
    # "0": the DiT's own draft function (here the same restatement, called on
    # window-ordered q and k) instead of the device draft through the map
    monkeypatch.setenv("FS89_DRAFT", draft)
    fv.enable(_Pipe(), dit_module=dit, verbose=False)
    g = torch.Generator().manual_seed(5)
    attn = dit.SelfAttention(g).to(dev)
    kv_len, topk = 2, 3
    # 6 latent frames, then 2-frame steps with the cache; step 3 passes a copy
    # of the cache (not the store's view), which must take the copying route.
    chunks = [(6, torch.randn(1, 6 * h * w, D, generator=g))] + [
        (2, torch.randn(1, 2 * h * w, D, generator=g)) for _ in range(4)]
    res, stores = {}, []
    for mode in ("0", "1"):
        monkeypatch.setenv("FS89_WINDOW", mode)
        attn.local_attn_mask = None
        attn._fs89_kv = None
        ck = cv = None
        outs = []
        for i, (f, x) in enumerate(chunks):
            x = x.to(torch.bfloat16).to(dev)
            fr = _freqs(f * h * w, dev) if ("fr", i) not in res else res[("fr", i)]
            res[("fr", i)] = fr
            if i == 3:
                ck, cv = ck.clone(), cv.clone()
            with torch.no_grad():
                y, ck, cv = attn(x, fr, f, h, w, None, topk, kv_len=kv_len, is_stream=True,
                                 pre_cache_k=ck, pre_cache_v=cv)
            if mode == "1":
                stores.append(ck.untyped_storage().data_ptr())
            outs.append((y.clone(), ck.clone(), cv.clone()))
        res[mode] = outs
    torch.cuda.synchronize()
    assert len(taken) == len(chunks)  # the window path served mode "1" only
    # appended in place at steps 1, 2 and 4; a new store at step 3 (foreign cache)
    assert stores[1] == stores[0] and stores[2] == stores[0]
    assert stores[3] != stores[0] and stores[4] == stores[3]
    for (y0, k0, v0), (y1, k1, v1) in zip(res["0"], res["1"]):
        assert k0.shape == k1.shape and v0.shape == v1.shape
        assert torch.equal(k0, k1) and torch.equal(v0, v1)
        assert torch.isfinite(y0.float()).all()
        assert torch.equal(y0, y1)


def test_qkv_rows_kernel_matches_partition():
    """fused_rms_rope_qkv_rows == fused_rms_rope_qk followed by the
    partition copy (k, v) into the rows behind a cache, bit for bit; rows
    mapped outside the buffer are skipped."""
    from flashvsr_sm89_ops.block import window_token_map
    from flashvsr_sm89_ops.fused_rms_rope import fused_rms_rope_qk, fused_rms_rope_qkv_rows
    dev = "cuda"
    f, h, w, ncache = 2, 16, 24, 256
    L = f * h * w
    g = torch.Generator().manual_seed(11)
    q, k, v = (torch.randn(1, L, D, generator=g).to(torch.bfloat16).to(dev) for _ in range(3))
    wq, wk = ((1 + 0.1 * torch.randn(D, generator=g)).to(torch.bfloat16).to(dev) for _ in range(2))
    fr = _freqs(L, dev)
    rq, rk = fused_rms_rope_qk(q, k, wq, wk, fr, eps=1e-6, head_dim=HD)
    tok = window_token_map(f, h, w, device=dev)
    inv = torch.empty_like(tok)
    inv[tok.long()] = torch.arange(L, dtype=torch.int32, device=dev)
    kbuf = torch.full((ncache + L, D), 7.0, dtype=torch.bfloat16, device=dev)
    vbuf = kbuf.clone()
    rows = inv + ncache
    rows[0] = -1                      # skipped
    rows[1] = ncache + L              # outside the buffer: skipped
    q2 = q.clone()
    out_q = fused_rms_rope_qkv_rows(q2, k, v, wq, wk, fr, kbuf, vbuf, rows.contiguous(), eps=1e-6,
                                    head_dim=HD)
    torch.cuda.synchronize()
    assert torch.equal(out_q, rq)
    want_k = rk[0][tok.long()]
    want_v = v[0][tok.long()]
    skip = torch.zeros(L, dtype=torch.bool, device=dev)
    skip[inv[:2].long()] = True
    assert torch.equal(kbuf[ncache:][~skip], want_k[~skip])
    assert torch.equal(vbuf[ncache:][~skip], want_v[~skip])
    assert (kbuf[:ncache] == 7).all() and (kbuf[ncache:][skip] == 7).all()


def _fake_block_dit(per_token, g, ffn_dim=512):
    """The window test's DiT plus a DiTBlock whose q/k/v/o and FFN are the FP8
    modules enable() installs (per-channel weights; per-token or per-tensor
    activations), a stand-in cross-attention and the upstream norms."""
    from flashvsr_sm89_ops.fp8_ffn import FP8FFN
    from flashvsr_sm89_ops.fp8_linear import FP8Linear
    dit = _fake_dit()
    SA = dit.SelfAttention

    def fp8(n, k):
        lin = torch.nn.Linear(k, n, dtype=torch.bfloat16)
        with torch.no_grad():
            lin.weight.copy_(torch.randn(n, k, generator=g) * 0.05)
            lin.bias.copy_(torch.randn(n, generator=g) * 0.02)
        return FP8Linear(lin.cuda(), per_channel=True, per_token=per_token)

    class DiTBlock(torch.nn.Module):
        def __init__(self):
            super().__init__()
            self.self_attn = SA(g)
            for n in ("q", "k", "v", "o"):
                setattr(self.self_attn, n, fp8(D, D))
            self.modulation = torch.nn.Parameter(
                (torch.randn(1, 6, D, generator=g) * 0.1).to(torch.bfloat16))
            self.norm1 = torch.nn.LayerNorm(D, eps=1e-6, elementwise_affine=False)
            self.norm2 = torch.nn.LayerNorm(D, eps=1e-6, elementwise_affine=False)
            self.norm3 = torch.nn.LayerNorm(D, eps=1e-6, dtype=torch.bfloat16)
            with torch.no_grad():
                self.norm3.weight.copy_(1 + 0.1 * torch.randn(D, generator=g))
                self.norm3.bias.copy_(0.1 * torch.randn(D, generator=g))
            self.ffn = FP8FFN(fp8(ffn_dim, D), fp8(D, ffn_dim))

        def cross_attn(self, x, ctx, is_stream=False):
            return (x * 0.5 + 0.25).contiguous()

        def gate(self, x, gate, residual):
            return x + gate * residual

        def forward(self, x, context, t_mod, freqs, f, h, w, local_num=None, topk=None,
                    train_img=False, block_id=None, kv_len=None, is_full_block=False,
                    is_stream=False, pre_cache_k=None, pre_cache_v=None, local_range=9):
            raise AssertionError("rebound by enable()")

    dit.DiTBlock = DiTBlock
    return dit


@pytest.mark.parametrize("per_token", [True, False])
def test_fused_block_equals_reference_dataflow(monkeypatch, per_token):
    """The rebound DiTBlock with the copy-free self-attention, one q/k/v GEMM
    on one quantisation (and, per token, the AdaLN writing the codes and the
    cross residual fused with the FFN's AdaLN) equals the reference's dataflow
    (FS89_WINDOW=0: three quantisations, three GEMMs, bf16 AdaLN outputs,
    partition/cat/reverse) bit for bit over a streaming run."""
    import flashvsr_sm89_ops as fv
    from flashvsr_sm89_ops import integrate
    h, w = 16, 24
    g = torch.Generator().manual_seed(9)
    dit = _fake_block_dit(per_token, g)
    monkeypatch.setenv("FS89_FP8", "")
    monkeypatch.setenv("FS89_DRAFT", "1")
    fv.enable(_Pipe(), dit_module=dit, verbose=False)
    blk = dit.DiTBlock().cuda()
    calls = []
    real = integrate.fused_ln_modulate_quant

    def spy(*a, **k):
        calls.append(1)
        return real(*a, **k)
    monkeypatch.setattr(integrate, "fused_ln_modulate_quant", spy)
    t_mod = (torch.randn(1, 6, D, generator=g) * 0.1).to(torch.bfloat16).cuda()
    chunks = [(6, torch.randn(1, 6 * h * w, D, generator=g))] + [
        (2, torch.randn(1, 2 * h * w, D, generator=g)) for _ in range(2)]
    frs = [_freqs(f * h * w, "cuda") for f, _ in chunks]
    res = {}
    for mode in ("0", "1"):
        monkeypatch.setenv("FS89_WINDOW", mode)
        blk.self_attn.local_attn_mask = None
        blk.self_attn._fs89_kv = None
        ck = cv = None
        outs = []
        for (f, x), fr in zip(chunks, frs):
            x = x.to(torch.bfloat16).cuda()
            with torch.no_grad():
                y, ck, cv = blk(x, None, t_mod, fr, f, h, w, None, 3, kv_len=2, is_stream=True,
                                pre_cache_k=ck, pre_cache_v=cv)
            outs.append((y.clone(), ck.clone(), cv.clone()))
        res[mode] = outs
    torch.cuda.synchronize()
    assert len(calls) == (3 if per_token else 0)  # the fused AdaLN served the per-token run only
    for (y0, k0, v0), (y1, k1, v1) in zip(res["0"], res["1"]):
        assert torch.isfinite(y0.float()).all()
        assert torch.equal(k0, k1) and torch.equal(v0, v1)
        assert torch.equal(y0, y1)


def test_qkv_rows_kernel_batch2_strided():
    """Two batch elements and q/k/v as column slices of one [B, L, 3D] tensor
    (the fused projection's output): RoPE position is the row within its
    batch element, k and v rows land where kv_rows sends them."""
    from flashvsr_sm89_ops.fused_rms_rope import fused_rms_rope_qk, fused_rms_rope_qkv_rows
    dev = "cuda"
    B, L = 2, 384
    g = torch.Generator().manual_seed(21)
    qkv = torch.randn(B, L, 3 * D, generator=g).to(torch.bfloat16).to(dev)
    q, k, v = (qkv[..., i * D:(i + 1) * D] for i in range(3))
    wq, wk = ((1 + 0.1 * torch.randn(D, generator=g)).to(torch.bfloat16).to(dev) for _ in range(2))
    fr = _freqs(L, dev)
    rq, rk = fused_rms_rope_qk(q.contiguous(), k.contiguous(), wq, wk, fr, eps=1e-6, head_dim=HD)
    perm = torch.randperm(B * L, generator=g).to(torch.int32).to(dev)
    kbuf = torch.zeros((B * L, D), dtype=torch.bfloat16, device=dev)
    vbuf = torch.zeros_like(kbuf)
    vref = v.contiguous().reshape(B * L, D)
    fused_rms_rope_qkv_rows(q, k, v, wq, wk, fr, kbuf, vbuf, perm, eps=1e-6, head_dim=HD)
    torch.cuda.synchronize()
    assert torch.equal(q, rq)  # rotated in place inside the fused tensor
    assert torch.equal(kbuf[perm.long()], rk.reshape(B * L, D))
    assert torch.equal(vbuf[perm.long()], vref)
