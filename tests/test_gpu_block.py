"""GPU parity of the DiT block's cross-attention path (norm3 LayerNorm, dense
attention over the cached prompt K/V, the residual through the o projection's
epilogue) and of whole DiT blocks with and without it, against the CPU oracle.

Bars: bf16 outputs within rtol 2e-2 / atol 2e-2 (with a mismatch-fraction
check), attention max-abs-err <= 1e-2, e4m3 codes bit-exact for the same
bf16 input.
"""
import numpy as np
import pytest
import torch

from oracle import oracle as O

pytestmark = pytest.mark.gpu

DEV = "cuda"


def dev_bf16(vals):
    return torch.from_numpy(np.ascontiguousarray(O.bf16_bits(vals)).view(np.int16)) \
        .view(torch.bfloat16).to(DEV)


def host_f(t):
    return t.detach().float().cpu().numpy()


def host_bits(t):
    return t.detach().contiguous().view(torch.int16).cpu().numpy().view(np.uint16)


def _close(out, ref, frac=1e-3):
    err = np.abs(out - ref)
    bad = err > 2e-2 + 2e-2 * np.abs(ref)
    assert bad.mean() <= frac, f"{bad.mean():.2e} beyond rtol/atol 2e-2, max {err.max():.3g}"


@pytest.mark.parametrize("rows,D", [(4224, 1536), (33, 1536), (7, 1000), (0, 1536)])
def test_layer_norm_affine(rows, D):
    from flashvsr_sm89_ops import layer_norm, layer_norm_quant
    rng = np.random.default_rng(rows + D)
    x = O.bf16(rng.standard_normal((rows, D)).astype(np.float32) * 2 + 0.3)
    w = O.bf16((1 + 0.1 * rng.standard_normal(D)).astype(np.float32))
    b = O.bf16((0.1 * rng.standard_normal(D)).astype(np.float32))
    xd, wd, bd = dev_bf16(x), dev_bf16(w), dev_bf16(b)
    y = layer_norm(xd, wd, bd, eps=1e-6)
    if rows == 0:
        assert y.shape == (0, D)
        return
    ref = O.layer_norm_affine(x, w, b, 1e-6)
    ulp = np.abs(host_bits(y).astype(np.int32) - O.bf16_bits(ref).astype(np.int32))
    # fp32 statistics and one bf16 rounding against the float64 oracle: almost
    # all equal, the rest one bf16 step apart, except where w * x_hat and b
    # nearly cancel (small y, large ulp distance, tiny absolute error).
    err = np.abs(host_f(y) - ref)
    i = np.unravel_index(np.argmax(err), err.shape)
    msg = f"worst {tuple(int(a) for a in i)}: got {host_f(y)[i]} ref {ref[i]} ulp {ulp[i]}"
    assert (ulp == 0).mean() > 0.99, msg
    assert (ulp <= 1).mean() > 0.999, msg
    _close(host_f(y), ref, frac=0.0)
    q, s, y2 = layer_norm_quant(xd, wd, bd, eps=1e-6, write_bf16=True)
    assert np.array_equal(host_bits(y2), host_bits(y))
    # the codes are those of the device's own bf16 rows, bit for bit
    rq, rs = O.quantize_fp8(host_bits(y), per_row=True)
    assert np.array_equal(q.view(torch.uint8).cpu().numpy(), rq)
    assert np.array_equal(s.cpu().numpy().reshape(-1), rs.reshape(-1))


@pytest.mark.parametrize("Lq,Lk,heads", [(1024, 512, 12), (256, 128, 2), (384, 1024, 4)])
def test_cross_attention_dense(Lq, Lk, heads):
    from flashvsr_sm89_ops import cross_attention
    rng = np.random.default_rng(Lq + Lk)
    D = heads * 128
    q = O.bf16(rng.standard_normal((Lq, D)).astype(np.float32))
    k = O.bf16(rng.standard_normal((Lk, D)).astype(np.float32))
    v = O.bf16(rng.standard_normal((Lk, D)).astype(np.float32))
    out = cross_attention(dev_bf16(q)[None], dev_bf16(k)[None], dev_bf16(v)[None], heads)
    ref = O.dense_attention(q.reshape(Lq, heads, 128), k.reshape(Lk, heads, 128),
                            v.reshape(Lk, heads, 128)).reshape(Lq, D)
    err = np.abs(host_f(out)[0] - ref).max()
    assert err <= 1e-2, f"max abs err {err}"


def test_cross_attention_supported_shapes():
    from flashvsr_sm89_ops.cross_attn import supported
    q = torch.empty(1, 256, 1536, dtype=torch.bfloat16, device=DEV)
    k = torch.empty(1, 512, 1536, dtype=torch.bfloat16, device=DEV)
    assert supported(q, k, k, 12)
    assert not supported(q, k[:, :500], k[:, :500], 12)     # keys not a multiple of 128
    assert not supported(q[:, :200], k, k, 12)              # queries not a multiple of 128
    assert not supported(q, k, k, 24)                       # head_dim 64
    assert not supported(q.float(), k, k, 12)


def _lin_host(p):
    return (p[0].view(torch.uint8).cpu().numpy(), p[1].cpu().numpy(), p[2].float().cpu().numpy())


def _block_case(L_f_h_w, cross_len, seed):
    from flashvsr_sm89_ops.block import DiTBlockWeights
    f, h, w = L_f_h_w
    dim, heads, ffn = 1536, 12, 8960
    g = torch.Generator().manual_seed(seed)
    wts = DiTBlockWeights(dim, ffn, DEV, g, cross_len=cross_len)
    L = f * h * w
    x = torch.randn(1, L, dim, generator=g).to(torch.bfloat16)
    t_mod = (0.1 * torch.randn(1, 6, dim, generator=g)).to(torch.bfloat16)
    return wts, x, t_mod


def test_cross_attention_residual_vs_oracle():
    from flashvsr_sm89_ops import cross_attention_residual
    wts, x, _ = _block_case((2, 16, 16), 256, 5)
    c = wts.cross
    L = x.shape[1]
    out = cross_attention_residual(x.to(DEV), c["norm3_w"], c["norm3_b"], c["q"], c["norm_q"],
                                   c["k"], c["v"], c["o"], 12)
    xf = x.float().numpy()[0]
    ref = O.cross_attention_block(xf, host_f(c["norm3_w"]), host_f(c["norm3_b"]), _lin_host(c["q"]),
                                  host_f(c["norm_q"]), host_f(c["k"])[0], host_f(c["v"])[0],
                                  _lin_host(c["o"]), 12)
    assert out.shape == (1, L, 1536)
    _close(host_f(out)[0], ref)


@pytest.mark.parametrize("cross_len", [0, 512])
def test_dit_block_vs_oracle(cross_len):
    """One DiT block (C5 unit) with and without the cross-attention residual."""
    from flashvsr_sm89_ops.block import dit_block_forward, window_token_map
    from flashvsr_sm89_ops.lcsa import build_csr
    f, h, w = 2, 16, 24
    wts, x, t_mod = _block_case((f, h, w), cross_len, 6)
    heads, dim = 12, 1536
    L = f * h * w
    cos, sin = O.wan_rope_cos_sin(f, h, w)
    cs = torch.from_numpy(np.stack([cos, sin], -1)).to(DEV)
    nb = L // 128
    keep = O.random_block_mask(heads, nb, nb, 0.5, seed=2)
    index = build_csr(torch.from_numpy(keep).to(DEV))
    y = dit_block_forward(x.to(DEV), wts, t_mod.to(DEV), cs, index,
                          window_token_map(f, h, w, device=DEV), heads)
    qkv = _lin_host(wts.qkv)
    params = {"q": tuple(a[:dim] for a in qkv), "k": tuple(a[dim:2 * dim] for a in qkv),
              "v": tuple(a[2 * dim:] for a in qkv), "o": _lin_host(wts.o),
              "ffn0": _lin_host(wts.ffn0), "ffn2": _lin_host(wts.ffn2),
              "norm_q": host_f(wts.norm_q), "norm_k": host_f(wts.norm_k)}
    cross = None
    if wts.cross is not None:
        c = wts.cross
        cross = {"norm3_w": host_f(c["norm3_w"]), "norm3_b": host_f(c["norm3_b"]),
                 "q": _lin_host(c["q"]), "o": _lin_host(c["o"]), "norm_q": host_f(c["norm_q"]),
                 "k": host_f(c["k"])[0], "v": host_f(c["v"])[0]}
    mod = (wts.modulation.cpu().float() + t_mod.float()).to(torch.bfloat16).float().numpy()[0]
    ref = O.dit_block(x.float().numpy()[0], mod, params, (f, h, w), keep, cos, sin, heads,
                      cross=cross)
    _close(host_f(y)[0], ref)


@pytest.mark.parametrize("B,L,D", [(1, 4224, 1536), (2, 33, 1536), (1, 7, 512), (3, 5, 768)])
def test_gate_add_layer_norm_fused_equals_separate(B, L, D):
    """The self-attention's gated residual + norm3 in one pass is
    bit-identical to fused_gate_add followed by the affine layer_norm; odd
    row counts put a batch boundary inside a wavefront's row pair."""
    import flashvsr_sm89_ops as fv
    from flashvsr_sm89_ops.fused_adaln import fused_gate_add_layer_norm, layer_norm
    g = torch.Generator().manual_seed(3 * B * L + D)
    x, r = (torch.randn(B, L, D, generator=g).bfloat16().to(DEV) for _ in range(2))
    gate = (0.3 * torch.randn(B, 1, D, generator=g)).bfloat16().to(DEV)
    w = (1 + 0.1 * torch.randn(D, generator=g)).bfloat16().to(DEV)
    b = (0.1 * torch.randn(D, generator=g)).bfloat16().to(DEV)
    x1, y = fused_gate_add_layer_norm(x, gate, r, w, b, eps=1e-6)
    x1r = fv.fused_gate_add(x, gate, r)
    yr = layer_norm(x1r, w, b, eps=1e-6)
    assert torch.equal(x1, x1r) and torch.equal(y, yr)


@pytest.mark.parametrize("B,L,D", [(1, 4224, 1536), (2, 33, 1536), (1, 7, 512)])
def test_gate_add_ln_modulate_fused_equals_separate(B, L, D):
    """The fused pass is bit-identical to fused_gate_add followed by
    fused_ln_modulate_quant (same arithmetic on the same bf16 row)."""
    import flashvsr_sm89_ops as fv
    from flashvsr_sm89_ops.fused_adaln import fused_gate_add_ln_modulate_quant
    g = torch.Generator().manual_seed(B * L + D)
    x, r = (torch.randn(B, L, D, generator=g).bfloat16().to(DEV) for _ in range(2))
    gate, sc, sh = ((0.3 * torch.randn(B, 1, D, generator=g)).bfloat16().to(DEV) for _ in range(3))
    x1, q, s, y = fused_gate_add_ln_modulate_quant(x, gate, r, sc, sh, write_bf16=True)
    x1r = fv.fused_gate_add(x, gate, r)
    qr, sr, yr = fv.fused_ln_modulate_quant(x1r, sc, sh, write_bf16=True)
    assert torch.equal(x1, x1r) and torch.equal(y, yr)
    assert torch.equal(q.view(torch.uint8), qr.view(torch.uint8)) and torch.equal(s, sr)


def test_dit_stack_two_blocks_vs_oracle():
    """Two blocks through DiTStack: the first block's last gated residual is
    fused with the second block's AdaLN."""
    from flashvsr_sm89_ops.block import DiTStack, window_token_map
    from flashvsr_sm89_ops.lcsa import build_csr
    f, h, w = 2, 16, 24
    heads, dim = 12, 1536
    L = f * h * w
    stack = DiTStack(2, dim, heads, 8960, device=DEV, seed=7)
    g = torch.Generator().manual_seed(8)
    x = torch.randn(1, L, dim, generator=g).to(torch.bfloat16)
    t_mod = (0.1 * torch.randn(1, 6, dim, generator=g)).to(torch.bfloat16)
    cos, sin = O.wan_rope_cos_sin(f, h, w)
    cs = torch.from_numpy(np.stack([cos, sin], -1)).to(DEV)
    nb = L // 128
    keep = O.random_block_mask(heads, nb, nb, 0.5, seed=3)
    y = stack(x.to(DEV), t_mod.to(DEV), cs, build_csr(torch.from_numpy(keep).to(DEV)),
              window_token_map(f, h, w, device=DEV))
    ref = x.float().numpy()[0]
    for wts in stack.weights:
        qkv = _lin_host(wts.qkv)
        params = {"q": tuple(a[:dim] for a in qkv), "k": tuple(a[dim:2 * dim] for a in qkv),
                  "v": tuple(a[2 * dim:] for a in qkv), "o": _lin_host(wts.o),
                  "ffn0": _lin_host(wts.ffn0), "ffn2": _lin_host(wts.ffn2),
                  "norm_q": host_f(wts.norm_q), "norm_k": host_f(wts.norm_k)}
        mod = (wts.modulation.cpu().float() + t_mod.float()).to(torch.bfloat16).float().numpy()[0]
        ref = O.dit_block(ref, mod, params, (f, h, w), keep, cos, sin, heads)
    _close(host_f(y)[0], ref)


@pytest.mark.parametrize("per_channel", [False, True])
def test_fp8_weights_persist_bit_identical(tmp_path, per_channel):
    """Weights quantised on the device, saved, and loaded into a fresh model
    give the same codes, scales and forward outputs bit for bit."""
    import copy
    from flashvsr_sm89_ops.fp8_linear import (convert_linears_fp8, load_fp8_weights,
                                              save_fp8_weights)
    g = torch.Generator().manual_seed(11)
    model = torch.nn.Module()
    model.blocks = torch.nn.ModuleList([torch.nn.Module()])
    model.blocks[0].cross_attn = torch.nn.Module()
    for n in "qo":
        lin = torch.nn.Linear(1536, 1536)
        with torch.no_grad():
            lin.weight.copy_(torch.randn(1536, 1536, generator=g) * 0.02)
            lin.bias.copy_(torch.randn(1536, generator=g) * 0.1)
        setattr(model.blocks[0].cross_attn, n, lin)
    model = model.to(DEV).to(torch.bfloat16)
    fresh = copy.deepcopy(model)
    assert convert_linears_fp8(model, parts=("cross",), per_channel=per_channel,
                               per_token=per_channel) == 2
    path = str(tmp_path / "w.safetensors")
    save_fp8_weights(model, path)
    assert convert_linears_fp8(fresh, parts=("cross",), per_channel=per_channel,
                               per_token=per_channel, stored=load_fp8_weights(path)) == 2
    x = torch.randn(1, 256, 1536, generator=g).to(torch.bfloat16).to(DEV)
    for n in "qo":
        a, b = getattr(model.blocks[0].cross_attn, n), getattr(fresh.blocks[0].cross_attn, n)
        assert torch.equal(a.weight.view(torch.uint8), b.weight.view(torch.uint8))
        assert torch.equal(a.w_scale, b.w_scale) and torch.equal(a.bias, b.bias)
        assert torch.equal(a(x), b(x))
