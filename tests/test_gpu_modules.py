"""GPU parity of the module layer against the oracle: ``FP8Linear.forward``
(reference fp8_linear.py:32-42) and ``FP8FFN.forward`` (fp8_ffn.py:84-96),
per tensor (the reference's default) and per token, on contiguous inputs and
on strided ones (a column slice, for which the reference quantises with its
eager expression, fp8_linear.py:38-40).

Bars: weight codes and scales bit-exact; the activation codes the module
fed its GEMM bit-exact (read back through ``_mm``); outputs within rtol/atol
2e-2 everywhere and bit-equal to the float64 oracle for >= 99% of elements
(the GEMM's fp32 sums change the last bf16 bit now and then).
"""
import numpy as np
import pytest
import torch

from oracle import oracle as O

pytestmark = pytest.mark.gpu

DEV = "cuda"


def bits(t):
    return t.detach().contiguous().view(torch.int16).cpu().numpy().view(np.uint16)


def host_f(t):
    return t.detach().float().cpu().numpy()


def _close(out, ref, what):
    err = np.abs(out - ref)
    assert (err <= 2e-2 + 2e-2 * np.abs(ref)).all(), f"{what}: max err {err.max():.3g}"
    assert (out == ref).mean() >= 0.97, f"{what}: only {(out == ref).mean():.4f} bit-equal"


def _linear(n, k, g, std=0.02):
    lin = torch.nn.Linear(k, n, dtype=torch.bfloat16)
    with torch.no_grad():
        lin.weight.copy_(torch.randn(n, k, generator=g) * std)
        lin.bias.copy_(torch.randn(n, generator=g) * 0.1)
    return lin.to(DEV)


def _input(shape, g, strided):
    """bf16 [2, T, K] ~N(0, 1): contiguous, or a column slice of a wider tensor."""
    B, T, K = shape
    if not strided:
        return torch.randn(B, T, K, generator=g).to(torch.bfloat16).to(DEV)
    wide = torch.randn(B, T, K + 96, generator=g).to(torch.bfloat16).to(DEV)
    x = wide[..., 48:48 + K]
    assert not x.reshape(-1, K).is_contiguous()
    return x


def _spy_mm(module):
    """Record the (codes, scale) each _mm call receives."""
    seen = []
    real = module._mm

    def mm(x8, s, out=None):
        seen.append((x8.view(torch.uint8).cpu().numpy(), s.float().cpu().numpy().reshape(-1)))
        return real(x8, s, out=out)
    module._mm = mm
    return seen


@pytest.mark.parametrize("per_token", [False, True])
@pytest.mark.parametrize("strided", [False, True])
def test_fp8_linear_forward_vs_oracle(per_token, strided):
    from flashvsr_sm89_ops import FP8Linear
    g = torch.Generator().manual_seed(3 + 2 * per_token + strided)
    N, K = 1536, 1536
    lin = _linear(N, K, g)
    m = FP8Linear(lin, per_channel=per_token, per_token=per_token)
    wq, ws = O.quantize_weight(bits(lin.weight), per_channel=per_token)
    assert np.array_equal(m.weight.view(torch.uint8).cpu().numpy(), wq)
    assert np.array_equal(host_f(m.w_scale).reshape(-1), ws)
    assert (m.w_scale.dim() == 0) != per_token          # 0-dim per tensor, as the reference
    x = _input((2, 300, K), g, strided)
    seen = _spy_mm(m)
    y = m(x)
    torch.cuda.synchronize()
    assert y.shape == (2, 300, N) and y.dtype == torch.bfloat16
    xb = bits(x.reshape(-1, K))
    rq, rs = O.quantize_input(xb, per_token=per_token, contiguous=not strided)
    assert np.array_equal(seen[0][0], rq), "activation codes"
    assert np.array_equal(seen[0][1], rs.reshape(-1)), "activation scales"
    ref = O.linear_fp8(O.from_bf16_bits(xb), wq, ws, host_f(lin.bias), per_token=per_token,
                       contiguous=not strided)
    _close(host_f(y).reshape(-1, N), ref, "FP8Linear")


@pytest.mark.parametrize("per_token", [False, True])
@pytest.mark.parametrize("strided", [False, True])
def test_fp8_ffn_forward_vs_oracle(monkeypatch, per_token, strided):
    """Stage by stage: the input codes; mm0's bf16 output h against the
    oracle's GEMM of those codes; the GELU requantisation codes bit-exact
    against the oracle's requantisation of the device's own h; mm2 against
    the oracle's GEMM of those codes; and the whole chain against the oracle's
    chain from the input."""
    from flashvsr_sm89_ops import FP8FFN, FP8Linear, fp8_ffn
    g = torch.Generator().manual_seed(11 + 2 * per_token + strided)
    D, FF = 1536, 8960
    l0, l2 = _linear(FF, D, g), _linear(D, FF, g)
    m = FP8FFN(FP8Linear(l0, per_channel=per_token, per_token=per_token),
               FP8Linear(l2, per_channel=per_token, per_token=per_token))
    w1q, w1s = O.quantize_weight(bits(l0.weight), per_channel=per_token)
    w2q, w2s = O.quantize_weight(bits(l2.weight), per_channel=per_token)
    x = _input((1, 520, D), g, strided)
    hs_seen = []
    real_gemm = fp8_ffn.fp8_gemm

    def spy_gemm(x8, s, *a, **k):
        hs_seen.append((x8.view(torch.uint8).cpu().numpy(), s.float().cpu().numpy().reshape(-1)))
        out = real_gemm(x8, s, *a, **k)
        hs_seen.append(out.clone())
        return out
    monkeypatch.setattr(fp8_ffn, "fp8_gemm", spy_gemm)
    seen = _spy_mm(m.lin2)
    y = m(x)
    torch.cuda.synchronize()
    (x8, xs), h_dev = hs_seen
    xb = bits(x.reshape(-1, D))
    q, s = O.quantize_input(xb, per_token=per_token, contiguous=not strided)
    assert np.array_equal(x8, q) and np.array_equal(xs, s.reshape(-1)), "input codes"
    b1, b2 = host_f(l0.bias), host_f(l2.bias)
    _close(host_f(h_dev), O.fp8_gemm(q, s, w1q, w1s, b1), "mm0")
    hq, hsc = O.quantize_fp8(bits(h_dev), per_row=per_token, gelu=True)
    assert np.array_equal(seen[0][0], hq), "GELU requant codes"
    assert np.array_equal(seen[0][1], hsc.reshape(-1)), "GELU requant scales"
    _close(host_f(y).reshape(-1, D), O.fp8_gemm(hq, hsc, w2q, w2s, b2), "mm2")
    ref = O.ffn_fp8(O.from_bf16_bits(xb), w1q, w1s, b1, w2q, w2s, b2, per_token=per_token,
                    contiguous=not strided)
    err = np.abs(host_f(y).reshape(-1, D) - ref)
    bad = err > 2e-2 + 2e-2 * np.abs(ref)
    assert bad.mean() <= 1e-3, f"FP8FFN chain: {bad.mean():.2e} beyond 2e-2, max {err.max():.3g}"


def test_fp8_linear_weight_types():
    """fp32 and fp16 Linears convert (their weights are quantised in their own
    type, covered in test_gpu_dtypes.py); any other type is refused."""
    from flashvsr_sm89_ops import FP8Linear
    for dt in (torch.float32, torch.float16):
        m = FP8Linear(torch.nn.Linear(16, 16).to(dt).to(DEV))
        assert m.weight.dtype == torch.float8_e4m3fn and m.w_scale.dtype == torch.float32
    with pytest.raises(TypeError, match="bfloat16, float16 or float32"):
        FP8Linear(torch.nn.Linear(16, 16).double().to(DEV))
