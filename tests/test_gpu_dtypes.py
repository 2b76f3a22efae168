"""GPU parity of the fp16 / fp32 inputs of the reference's op API.

The reference's kernels load every floating input with .to(tl.float32) and
store into torch.empty_like(x) (fp8_quant.py:20,33; fused_adaln.py:29,37-38,
53-55; fused_rms_rope.py:33,36,44), and FP8Linear quantises a weight with
eager expressions in the weight's own type (fp8_linear.py:19-22).  Here the
same ops run through libfvsr.so's *_dt entry points on fp16, fp32 and mixed
inputs, checked against the CPU oracle and, where the reference's expression
is plain torch, against torch evaluating it on this GPU.

Bars: FP8 codes and scales bit-exact (a NaN code may carry either sign);
gate_add bitwise; LayerNorm / RMSNorm outputs within the bf16 ops' tolerance
(rtol/atol 2e-2, max abs 1/32) after the oracle's bf16 result is cast to x's
type as the kernels cast theirs; bf16 values in fp32 tensors give the bf16
path's results bit for bit where the kernels share the arithmetic.
"""
import numpy as np
import pytest
import torch

from oracle import oracle as O

pytestmark = pytest.mark.gpu

DEV = "cuda"
DT = {torch.bfloat16: O.DT_BF16, torch.float16: O.DT_F16, torch.float32: O.DT_F32}
F16_F32 = [torch.float16, torch.float32]


@pytest.fixture(scope="module")
def ops():
    import flashvsr_sm89_ops as f
    return f


def rnd(shape, seed, dtype, scale=1.0):
    g = torch.Generator().manual_seed(seed)
    return (torch.randn(shape, generator=g) * scale).to(dtype)


def codes(t):
    return t.detach().contiguous().view(torch.uint8).cpu().numpy()


def host_f(t):
    return t.detach().float().cpu().numpy()


def as_type(ref, dtype):
    """The oracle's (bf16-valued) float32 result stored in dtype, as the kernels store."""
    return torch.from_numpy(np.ascontiguousarray(ref, np.float32)).to(dtype).float().numpy()


def codes_equal_nan(got, ref):
    nan = (ref & 0x7F) == 0x7F
    assert np.array_equal(got[~nan], ref[~nan])
    assert ((got[nan] & 0x7F) == 0x7F).all()


def close(out, ref, max_abs=0.03125, frac=0.05):
    np.testing.assert_allclose(out, ref, rtol=2e-2, atol=2e-2)
    assert np.abs(out - ref).max() <= max_abs
    assert (out != ref).mean() < frac


# ----------------------------------------------------------------------------- quantisation

QSHAPES = [(4224, 1536), (33, 8960), (7, 1000), (5, 1003), (1, 8)]


@pytest.mark.parametrize("dtype", F16_F32)
@pytest.mark.parametrize("shape", QSHAPES)
@pytest.mark.parametrize("per_token", [True, False])
def test_quantize_fp8_dtypes(ops, dtype, shape, per_token):
    print(f"case quantize_fp8 {dtype} {shape} per_token={per_token}", flush=True)
    x = rnd(shape, shape[0] + shape[1], dtype, 4.0)
    if shape[0] > 2:
        x[1] = 0                                   # all-zero row
        x[2, 0] = 1e4                              # outlier
    xd = x.to(DEV)
    q, s = ops.quantize_fp8(xd, per_token=per_token)
    torch.cuda.synchronize()
    rq, rs = O.quantize_fp8_values(x.float().numpy(), per_row=per_token)
    assert np.array_equal(codes(q), rq)
    assert np.array_equal(host_f(s).reshape(-1), rs)
    xf = xd.float().abs()
    amax = xf.amax(dim=1, keepdim=True) if per_token else xf.amax()
    assert torch.equal(s.reshape(-1), (amax / 448.0).reshape(-1))  # fp8_quant.py:54 on this GPU


@pytest.mark.parametrize("dtype", F16_F32)
def test_quantize_fp8_dtypes_strided_rows(ops, dtype):
    wide = rnd((64, 2048), 11, dtype)
    xd = wide.to(DEV)[:, 256:256 + 1536]
    for per_token in (True, False):
        q, s = ops.quantize_fp8(xd, per_token=per_token)
        rq, rs = O.quantize_fp8_values(wide[:, 256:256 + 1536].float().numpy(), per_row=per_token)
        assert np.array_equal(codes(q), rq) and np.array_equal(host_f(s).reshape(-1), rs)


@pytest.mark.parametrize("shape", [(4224, 1536), (33, 8960), (5, 1003)])
def test_quantize_fp32_holding_bf16_values_equals_bf16_path(ops, shape):
    """The fp32 kernels (IEEE quotient) and the bf16 vector kernels (fma
    quotient) give the same codes and scales on the same values."""
    x = rnd(shape, 3, torch.bfloat16, 3.0).to(DEV)
    for per_token in (True, False):
        for gelu in (False, True):
            f = ops.fused_gelu_quant_fp8 if gelu else ops.quantize_fp8
            q1, s1 = f(x, per_token=per_token)
            q2, s2 = f(x.float(), per_token=per_token)
            assert torch.equal(q1.view(torch.uint8), q2.view(torch.uint8))
            assert torch.equal(s1, s2)


@pytest.mark.parametrize("dtype", F16_F32)
@pytest.mark.parametrize("per_token", [True, False])
def test_gelu_quant_dtypes(ops, dtype, per_token):
    y = rnd((33, 8960), 5, dtype, 2.0)
    q, s = ops.fused_gelu_quant_fp8(y.to(DEV), per_token=per_token)
    rq, rs = O.quantize_fp8_values(y.float().numpy(), per_row=per_token, gelu=True)
    assert np.array_equal(codes(q), rq)
    assert np.array_equal(host_f(s).reshape(-1), rs)


@pytest.mark.parametrize("dtype", F16_F32)
@pytest.mark.parametrize("per_channel", [False, True])
def test_weight_quant_dtypes(ops, dtype, per_channel):
    """Against the oracle, and per tensor against the reference's own
    expressions (fp8_linear.py:20-22) evaluated by torch on this GPU; the
    weight scales span fp16's subnormal range (std 0.002) and a zero weight."""
    print(f"case weight quant {dtype} per_channel={per_channel}", flush=True)
    for i, std in enumerate((0.02, 0.002, 30.0, 0.0)):
        w = rnd((96, 1536), 20 + i, dtype, std)
        wd = w.to(DEV)
        q, s = ops.quantize_weight_fp8(wd, per_channel=per_channel)
        torch.cuda.synchronize()
        rq, rs = O.quantize_weight_values(w.float().numpy(), DT[dtype], per_channel=per_channel)
        codes_equal_nan(codes(q), rq)
        assert np.array_equal(host_f(s).reshape(-1), rs)
        if not per_channel:
            st = (wd.abs().amax() / 448.0).clamp(min=1e-12).float()
            qt = (wd / st).to(torch.float8_e4m3fn)
            assert torch.equal(s, st)
            codes_equal_nan(codes(q), codes(qt))


@pytest.mark.parametrize("dtype", F16_F32)
@pytest.mark.parametrize("strided", [False, True])
def test_fp8_linear_dtypes(ops, dtype, strided):
    """FP8Linear over an fp16 / fp32 nn.Linear: weight codes and scale, the
    activation codes its GEMM receives (a column slice takes the reference's
    eager expression in x's type, fp8_linear.py:38-40), and the bf16 output
    against the oracle's GEMM of those codes with the bias rounded to bf16."""
    from flashvsr_sm89_ops import FP8Linear
    g = torch.Generator().manual_seed(7)
    N, K = 640, 1536
    lin = torch.nn.Linear(K, N, dtype=dtype)
    with torch.no_grad():
        lin.weight.copy_(torch.randn(N, K, generator=g) * 0.02)
        lin.bias.copy_(torch.randn(N, generator=g) * 0.1)
    lin = lin.to(DEV)
    m = FP8Linear(lin)
    wq, ws = O.quantize_weight_values(host_f(lin.weight), DT[dtype])
    assert np.array_equal(codes(m.weight), wq) and host_f(m.w_scale).reshape(-1)[0] == ws[0]
    wide = (torch.randn(2, 300, K + 96, generator=g) * 2).to(dtype).to(DEV)
    x = wide[..., 48:48 + K] if strided else wide[..., :K].contiguous()
    seen = []
    real = m._mm
    m._mm = lambda x8, s, out=None: (seen.append((codes(x8), host_f(s).reshape(-1))),
                                     real(x8, s, out=out))[1]
    y = m(x)
    torch.cuda.synchronize()
    assert y.shape == (2, 300, N) and y.dtype == torch.bfloat16
    x2 = host_f(x.reshape(-1, K))
    if strided:
        rq, rs = O.quantize_weight_values(x2, DT[dtype])
    else:
        rq, rs = O.quantize_fp8_values(x2)
    assert np.array_equal(seen[0][0], rq) and np.array_equal(seen[0][1], rs)
    ref = O.fp8_gemm(rq, rs, wq, ws, O.bf16(host_f(lin.bias)))
    out = host_f(y).reshape(-1, N)
    assert (np.abs(out - ref) <= 2e-2 + 2e-2 * np.abs(ref)).all()
    assert (out == ref).mean() >= 0.97


# ----------------------------------------------------------------------------- AdaLN

LN_TYPES = [(torch.float16, torch.float16), (torch.float32, torch.float32),
            (torch.bfloat16, torch.float32), (torch.float32, torch.bfloat16),
            (torch.float16, torch.float32)]


@pytest.mark.parametrize("xdt,pdt", LN_TYPES)
@pytest.mark.parametrize("BLD", [(2, 37, 1536), (1, 9, 100)])
def test_ln_modulate_dtypes(ops, xdt, pdt, BLD):
    B, L, D = BLD
    x = rnd(BLD, L, xdt)
    sc = rnd((B, 1, D), L + 1, pdt, 0.1)
    sh = rnd((B, 1, D), L + 2, pdt, 0.1)
    out = ops.fused_ln_modulate(x.to(DEV), sc.to(DEV), sh.to(DEV), eps=1e-6)
    assert out.dtype == xdt and out.shape == x.shape
    ref = O.ln_modulate(x.float().numpy(), sc.float().numpy(), sh.float().numpy(), 1e-6)
    close(host_f(out), as_type(ref, xdt))


@pytest.mark.parametrize("xdt,gdt,rdt", [(torch.float16,) * 3, (torch.float32,) * 3,
                                         (torch.float32, torch.float32, torch.bfloat16),
                                         (torch.bfloat16, torch.float32, torch.float16)])
@pytest.mark.parametrize("BLD", [(1, 4224, 1536), (2, 7, 100)])
def test_gate_add_dtypes(ops, xdt, gdt, rdt, BLD):
    B, L, D = BLD
    x, r = rnd(BLD, 1, xdt), rnd(BLD, 2, rdt)
    g = rnd((B, 1, D), 3, gdt, 0.5)
    out = ops.fused_gate_add(x.to(DEV), g.to(DEV), r.to(DEV))
    assert out.dtype == xdt
    ref = O.gate_add(x.float().numpy(), g.float().numpy(), r.float().numpy())
    assert np.array_equal(host_f(out), as_type(ref, xdt))


# ----------------------------------------------------------------------------- RMSNorm + RoPE

@pytest.mark.parametrize("xdt,wdt", [(torch.float16, torch.float32), (torch.float32, torch.float32),
                                     (torch.bfloat16, torch.float32),
                                     (torch.float32, torch.bfloat16)])
@pytest.mark.parametrize("fhw", [(2, 4, 6), (2, 48, 88)])
def test_rms_rope_dtypes(ops, xdt, wdt, fhw):
    L, D = fhw[0] * fhw[1] * fhw[2], 1536
    x = rnd((1, L, D), fhw[1], xdt)
    w = (1 + 0.1 * rnd(D, fhw[1] + 1, torch.float32)).to(wdt)
    c, s = O.wan_rope_cos_sin(*fhw)
    freqs = torch.view_as_complex(torch.from_numpy(np.stack([c, s], -1)).to(DEV))
    for rope in (True, False):
        out = ops.fused_rms_rope(x.to(DEV), w.to(DEV), freqs if rope else None, eps=1e-6,
                                 rope=rope)
        assert out.dtype == xdt
        ref = O.rms_rope(x.float().numpy(), w.float().numpy(), c, s, 1e-6, rope=rope)
        close(host_f(out), as_type(ref, xdt))


@pytest.mark.parametrize("fhw", [(2, 4, 6), (2, 48, 88)])
def test_rms_rope_fp32_holding_bf16_values_equals_bf16_path(ops, fhw):
    """The element-load kernel sums squares in the vector kernel's order, so
    bf16 values in an fp32 tensor give the bf16 results bit for bit."""
    L, D = fhw[0] * fhw[1] * fhw[2], 1536
    x = rnd((1, L, D), 9, torch.bfloat16).to(DEV)
    w = (1 + 0.1 * rnd(D, 10, torch.float32)).to(torch.bfloat16).to(DEV)
    c, s = O.wan_rope_cos_sin(*fhw)
    freqs = torch.view_as_complex(torch.from_numpy(np.stack([c, s], -1)).to(DEV))
    for rope in (True, False):
        f = freqs if rope else None
        ob = ops.fused_rms_rope(x, w, f, rope=rope)
        of = ops.fused_rms_rope(x.float(), w, f, rope=rope)
        assert of.dtype == torch.float32
        assert torch.equal(ob.float(), of)


@pytest.mark.parametrize("dtype", F16_F32)
def test_fp8_ffn_dtypes(ops, dtype):
    """FP8FFN over fp16 / fp32 Linears (fp8_ffn.py:84-96), per tensor (the
    reference's default): mm2 against the oracle's GEMM of the codes the
    device fed it, and the whole chain (input codes in x's type, mm0, GELU
    requantisation, mm2) against the oracle's at the chain bar (at most 0.1%
    of elements beyond rtol/atol 2e-2)."""
    from flashvsr_sm89_ops import FP8FFN, FP8Linear
    g = torch.Generator().manual_seed(11)
    D, F = 512, 1024

    def lin(n, k):
        m = torch.nn.Linear(k, n, dtype=dtype)
        with torch.no_grad():
            m.weight.copy_(torch.randn(n, k, generator=g) * 0.03)
            m.bias.copy_(torch.randn(n, generator=g) * 0.1)
        return m.to(DEV)
    l0, l2 = lin(F, D), lin(D, F)
    ffn = FP8FFN(FP8Linear(l0), FP8Linear(l2))
    x = (torch.randn(2, 300, D, generator=g) * 2).to(dtype).to(DEV)
    seen = []
    for m in (ffn.lin2,):
        real = m._mm
        m._mm = lambda x8, s, out=None, real=real: (seen.append((codes(x8), host_f(s).reshape(-1))),
                                                    real(x8, s, out=out))[1]
    y = ffn(x)
    torch.cuda.synchronize()
    assert y.shape == (2, 300, D) and y.dtype == torch.bfloat16
    w0q, w0s = O.quantize_weight_values(host_f(l0.weight), DT[dtype])
    w2q, w2s = O.quantize_weight_values(host_f(l2.weight), DT[dtype])
    xq, xs = O.quantize_fp8_values(host_f(x).reshape(-1, D))
    h_ref = O.fp8_gemm(xq, xs, w0q, w0s, O.bf16(host_f(l0.bias)))
    h8, hs = seen[0]                      # the codes the device fed mm2
    out = host_f(y).reshape(-1, D)
    assert (np.abs(out - O.fp8_gemm(h8, hs, w2q, w2s, O.bf16(host_f(l2.bias))))
            <= 2e-2 + 2e-2 * np.abs(out)).all()
    ref = O.fp8_gemm(*O.quantize_fp8(O.bf16_bits(h_ref), per_row=False, gelu=True), w2q, w2s,
                     O.bf16(host_f(l2.bias)))
    bad = np.abs(out - ref) > 2e-2 + 2e-2 * np.abs(ref)
    assert bad.mean() <= 1e-3, f"chain {bad.mean():.2e}"


@pytest.mark.parametrize("dtype", F16_F32)
def test_dtype_paths_edge_shapes(ops, dtype):
    """Empty inputs, D not a multiple of 8 (RMSNorm without RoPE, LN,
    gate_add) and an odd row count, against the oracle."""
    q, s = ops.quantize_fp8(torch.zeros(0, 24, dtype=dtype, device=DEV))
    assert q.shape == (0, 24) and s.shape == (1,) and float(s) == 0.0
    q, s = ops.quantize_fp8(torch.zeros(0, 24, dtype=dtype, device=DEV), per_token=True)
    assert q.shape == (0, 24) and s.shape == (0, 1)
    x = rnd((1, 7, 100), 31, dtype)
    w = (1 + 0.1 * rnd(100, 32, torch.float32)).to(dtype)
    out = ops.fused_rms_rope(x.to(DEV), w.to(DEV), None, rope=False)
    ref = O.rms_rope(x.float().numpy(), w.float().numpy(), rope=False)
    close(host_f(out), as_type(ref, dtype))
    sc, sh = rnd((1, 1, 100), 33, dtype, 0.1), rnd((1, 1, 100), 34, dtype, 0.1)
    out = ops.fused_ln_modulate(x.to(DEV), sc.to(DEV), sh.to(DEV))
    close(host_f(out), as_type(O.ln_modulate(x.float().numpy(), sc.float().numpy(),
                                             sh.float().numpy()), dtype))
    r = rnd((1, 7, 100), 35, dtype)
    out = ops.fused_gate_add(x.to(DEV), sc.to(DEV), r.to(DEV))
    assert np.array_equal(host_f(out), as_type(O.gate_add(x.float().numpy(), sc.float().numpy(),
                                                          r.float().numpy()), dtype))
    q, s = ops.quantize_fp8(x.reshape(7, 100).to(DEV), per_token=True)
    rq, rs = O.quantize_fp8_values(x.reshape(7, 100).float().numpy(), per_row=True)
    assert np.array_equal(codes(q), rq) and np.array_equal(host_f(s).reshape(-1), rs)
