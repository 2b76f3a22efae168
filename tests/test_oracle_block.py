"""Independent pins of the oracle's composition: the window permutation by its
closed form, and one DiT block (oracle.dit_block with oracle.self_attention,
oracle.cross_attention_block and oracle.ffn_fp8) against a torch-eager block
written from the reference's block (integrate.py:151-182, with the
self-attention of :47-124 and the cross-attention of :132-143) out of torch's
own operators (oracle/eager.py): F.layer_norm, the reference's eager e4m3
quantisation expressions, dequantised matmuls, the upstream RMSNorm and
float64 complex RoPE, scaled_dot_product_attention under the expanded block
mask, F.gelu(approximate='tanh').  A slip in the oracle's composition (modulation
chunk order, (scale, shift) swapped, a residual dropped, the cache trimmed
from the wrong end, a transposed window) fails these tests by far more than
the tolerance, which only absorbs FP8 codes flipped by last-bit differences.
"""
import numpy as np
import pytest
import torch
import torch.nn.functional as F

from oracle import oracle as O
from oracle.eager import (attention_blocks, attention_dense, closed_form_window_of,
                          dit_block_eager, modulate, q_weight)

BF = torch.bfloat16
E4M3 = torch.float8_e4m3fn


# ----------------------------------------------------------------------------- window permutation

@pytest.mark.parametrize("B,f,h,w", [(1, 2, 8, 8), (1, 4, 16, 24), (2, 6, 8, 16)])
def test_window_partition_closed_form(B, f, h, w):
    win, slot = closed_form_window_of(B, f, h, w)
    raster = np.arange(f * h * w)[None].repeat(B, 0).reshape(B, f, h, w)
    x = np.stack([np.broadcast_to(np.arange(B)[:, None, None, None], raster.shape), raster],
                 -1).astype(np.float32)
    xw = O.window_partition(x)
    assert xw.shape == (B * (f // 2) * (h // 8) * (w // 8), 128, 2)
    assert np.array_equal(xw[win, slot, 0], x[..., 0])
    assert np.array_equal(xw[win, slot, 1], x[..., 1])
    back = O.window_reverse(xw, (f, h, w), batch=B)
    assert np.array_equal(back, x.reshape(B, f * h * w, 2))
    # a window of columns-before-rows (a transposed slot order) is told apart
    bad = ((np.arange(f)[:, None, None] % 2) * 8 + np.arange(w)[None, None, :] % 8) * 8 \
        + np.arange(h)[None, :, None] % 8
    assert not np.array_equal(bad[None].repeat(B, 0), slot)


# ----------------------------------------------------------------------------- torch-eager block

def _np_lin(lin):
    w8, s, b = lin
    return (w8.view(torch.uint8).numpy(), s.numpy(), b.float().numpy())


def _bar(got, ref, what, frac=1e-3):
    err = np.abs(got - ref)
    bad = err > 2e-2 + 2e-2 * np.abs(ref)
    assert bad.mean() <= frac, f"{what}: {bad.mean():.2e} beyond rtol/atol 2e-2, max {err.max():.3g}"


@pytest.mark.parametrize("per_token", [True, False])
@pytest.mark.parametrize("with_cross", [False, True])
def test_dit_block_oracle_vs_torch_eager(per_token, with_cross):
    """oracle.dit_block == the torch-eager reference block over a streaming
    pair (6 latent frames, then 2 with the KV cache, kv_len 2), per token and
    per tensor, with and without the cross-attention residual."""
    g = torch.Generator().manual_seed(31 + 2 * per_token + with_cross)
    D, heads, ffn, h, w, eps = 256, 2, 512, 16, 16, 1e-6

    def bf(*shape, std=1.0, mean=0.0):
        return (mean + std * torch.randn(*shape, generator=g)).to(BF)

    def lin(n, k):
        w8, s = q_weight(bf(n, k, std=0.05), per_channel=per_token)
        return w8, s, bf(n, std=0.02)

    P = {n: lin(D, D) for n in ("q", "k", "v", "o")}
    P["ffn0"], P["ffn2"] = lin(ffn, D), lin(D, ffn)
    P["norm_q"], P["norm_k"] = bf(D, mean=1, std=0.1), bf(D, mean=1, std=0.1)
    mod = bf(6, D, std=0.1) + bf(6, D, std=0.1)              # modulation + t_mod in bf16
    cross = None
    if with_cross:
        cross = {"norm3_w": bf(D, mean=1, std=0.1), "norm3_b": bf(D, std=0.1), "q": lin(D, D),
                 "o": lin(D, D), "norm_q": bf(D, mean=1, std=0.1), "k": bf(256, D), "v": bf(256, D)}
    Pn = {n: _np_lin(P[n]) for n in ("q", "k", "v", "o", "ffn0", "ffn2")}
    Pn["norm_q"], Pn["norm_k"] = P["norm_q"].float().numpy(), P["norm_k"].float().numpy()
    crossn = None
    if cross is not None:
        crossn = {"norm3_w": cross["norm3_w"].float().numpy(),
                  "norm3_b": cross["norm3_b"].float().numpy(),
                  "q": _np_lin(cross["q"]), "o": _np_lin(cross["o"]),
                  "norm_q": cross["norm_q"].float().numpy(),
                  "k": cross["k"].float().numpy(), "v": cross["v"].float().numpy()}
    cache_t = cache_o = None
    for step, f in enumerate((6, 2)):
        L = f * h * w
        x = bf(L, D)
        ang = torch.rand(L, 64, generator=g, dtype=torch.float64) * 6.28
        freqs = torch.polar(torch.ones_like(ang), ang)              # complex128, like Wan's
        nq = L // 128
        nk = nq + (0 if cache_t is None else cache_t[0].shape[0] // 128)
        keep = O.random_block_mask(heads, nq, nk, 0.4, seed=step, keep_diag=False)
        keep[:, np.arange(nq), nk - nq + np.arange(nq)] = True      # each query block sees itself
        yt, kt, vt = dit_block_eager(x, mod, P, (f, h, w), keep, freqs, heads, eps, per_token,
                                     cross, cache_t, kv_len=2)
        cs = torch.view_as_real(freqs.to(torch.complex64)).numpy()
        yo, ko, vo = O.dit_block(x.float().numpy(), mod.float().numpy(), Pn, (f, h, w), keep,
                                 cs[..., 0], cs[..., 1], heads, eps, cross=crossn,
                                 per_token=per_token, cache=cache_o, kv_len=2, return_cache=True)
        _bar(yo, yt.float().numpy(), f"step {step} output")
        _bar(ko.reshape(-1, D), kt.float().numpy(), f"step {step} k cache")
        _bar(vo.reshape(-1, D), vt.float().numpy(), f"step {step} v cache")
        cache_t, cache_o = (kt, vt), (ko, vo)
    # the streaming cache keeps kv_len steps: 2 steps of 4 windows after the second chunk
    assert cache_o[0].shape == (8, 128, D)


def test_dit_block_oracle_detects_modulation_swap():
    """The comparison above is sharp enough to see a (scale, shift) swap in the
    attention AdaLN, the bug class the reference's integration notes name."""
    g = torch.Generator().manual_seed(5)
    D, heads = 256, 2
    x = torch.randn(512, D, generator=g).to(BF)
    mod = (0.3 * torch.randn(6, D, generator=g)).to(BF)
    a = O.ln_modulate(x.float().numpy()[None], mod[1].float().numpy(), mod[0].float().numpy())[0]
    b = modulate(F.layer_norm(x, (D,), eps=1e-6), mod[1], mod[0]).float().numpy()  # swapped
    err = np.abs(a - b)
    assert (err > 2e-2 + 2e-2 * np.abs(b)).mean() > 0.1


@pytest.mark.parametrize("zero", [False, True])
def test_quantize_input_eager_branch_vs_torch(zero):
    """oracle.quantize_input for a non-contiguous activation equals the
    reference's eager expression evaluated by torch on a strided bf16 tensor
    (fp8_linear.py:38-40): codes and the 0-dim scale, bit for bit."""
    g = torch.Generator().manual_seed(2)
    base = (torch.randn(64, 96, generator=g) * 3).to(BF)
    if zero:
        base.zero_()
    x2 = base[:, 16:80]                        # a column slice: rows 96 apart
    assert not x2.is_contiguous()
    s = (x2.abs().amax() / 448.0).clamp(min=1e-12).float()
    x8 = (x2 / s).to(E4M3)
    bits = x2.contiguous().view(torch.int16).numpy().view(np.uint16)
    q, so = O.quantize_input(bits, per_token=False, contiguous=False)
    assert np.array_equal(q, x8.view(torch.uint8).numpy())
    assert so.reshape(()) == s.numpy()
    # the contiguous path quantises differently (fp32 quotient, clamp on amax)
    q2, s2 = O.quantize_input(bits, per_token=False, contiguous=True)
    if not zero:
        assert s2[0] != so[0] or not np.array_equal(q2, q)


@pytest.mark.parametrize("with_cross", [False, True])
def test_dit_block_window_subset_equals_full(with_cross):
    """dit_block(windows=...) (used at full size, where the whole oracle
    block is too slow) gives exactly the full block's rows of those windows'
    tokens, and window_tokens lists them in window order."""
    rng = np.random.default_rng(4)
    D, heads, ffn, fhw = 256, 2, 512, (2, 16, 24)
    L = 2 * 16 * 24

    def lin(n, k):
        q, s = O.quantize_weight(O.bf16_bits(rng.standard_normal((n, k)).astype(np.float32) * .05),
                                 per_channel=True)
        return q, s, O.bf16(rng.standard_normal(n).astype(np.float32) * .02)

    P = {n: lin(D, D) for n in "qkvo"}
    P["ffn0"], P["ffn2"] = lin(ffn, D), lin(D, ffn)
    P["norm_q"] = P["norm_k"] = O.bf16(1 + 0.1 * rng.standard_normal(D).astype(np.float32))
    cross = None
    if with_cross:
        cross = {"norm3_w": O.bf16(np.ones(D, np.float32)), "norm3_b": O.bf16(np.zeros(D, np.float32)),
                 "q": lin(D, D), "o": lin(D, D), "norm_q": P["norm_q"],
                 "k": O.bf16(rng.standard_normal((256, D)).astype(np.float32)),
                 "v": O.bf16(rng.standard_normal((256, D)).astype(np.float32))}
    x = O.bf16(rng.standard_normal((L, D)).astype(np.float32))
    mod = O.bf16(0.1 * rng.standard_normal((6, D)).astype(np.float32))
    cos, sin = O.wan_rope_cos_sin(*fhw)
    keep = O.random_block_mask(heads, L // 128, L // 128, 0.5, seed=1)
    full = O.dit_block(x, mod, P, fhw, keep, cos, sin, heads, cross=cross)
    wins = np.array([4, 1])
    tok = O.window_tokens(fhw, wins)
    # 3 windows per row of the 16 x 24 grid: window 4 is (row 1, column 1)
    want = np.arange(L).reshape(2, 16, 24)[:, 8:16, 8:16]
    assert np.array_equal(tok[:128], want.reshape(-1))
    sub = O.dit_block(x, mod, P, fhw, keep, cos, sin, heads, cross=cross, windows=wins)
    assert np.array_equal(sub, full[tok])


def test_eager_block_attention_matches_dense_sdpa():
    """oracle.eager.attention_blocks (the per-block loop bench.py's CPU
    baseline runs at full size) equals SDPA under the expanded mask."""
    g = torch.Generator().manual_seed(9)
    heads, NQ, NK = 2, 3, 5
    q = torch.randn(NQ * 128, heads * 128, generator=g).to(torch.bfloat16)
    k = torch.randn(NK * 128, heads * 128, generator=g).to(torch.bfloat16)
    v = torch.randn(NK * 128, heads * 128, generator=g).to(torch.bfloat16)
    keep = O.random_block_mask(heads, NQ, NK, 0.5, seed=3)
    km = torch.from_numpy(keep).repeat_interleave(128, 1).repeat_interleave(128, 2)
    a = attention_blocks(q, k, v, keep, heads).float()
    b = attention_dense(q, k, v, km, heads).float()
    assert (a - b).abs().max() <= 1.6e-2          # both rounded to bf16 once
    assert (a == b).float().mean() > 0.95
