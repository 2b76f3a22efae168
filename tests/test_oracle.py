"""Pins for the CPU oracle (oracle/oracle.py + oracle/fvsr_oracle.c).

Each oracle function is checked against something independent of it: torch
CPU eager arithmetic (the golden fixtures of tests/golden/make_golden.py and
direct torch calls), closed forms, brute force on tiny inputs, or invariants,
chosen so that a plausible slip (a dropped term, a swapped operand, a wrong
rounding step) fails at least one of them.
"""
import math
import os

import numpy as np
import pytest
import torch
import torch.nn.functional as F

from oracle import oracle as O

GOLD = np.load(os.path.join(os.path.dirname(__file__), "golden", "golden.npz"))


def t_bf16(bits):
    return torch.from_numpy(np.ascontiguousarray(bits).view(np.int16)).view(torch.bfloat16)


def torch_e4m3(x):
    return torch.from_numpy(np.ascontiguousarray(x, np.float32)).to(torch.float8_e4m3fn) \
        .view(torch.uint8).numpy()


# ----------------------------------------------------------------------------- e4m3 / bf16

def test_e4m3_encode_all_bf16_patterns():
    x = (np.arange(65536, dtype=np.uint32) << 16).view(np.float32)
    x = np.where(np.isnan(x), 0, x).astype(np.float32)
    assert (O.e4m3_encode(x) == torch_e4m3(x)).all()


def test_e4m3_encode_midpoints_and_random():
    grid = O.e4m3_decode(np.arange(0x7F, dtype=np.uint8))  # 0 .. 448, no NaN
    mids = ((grid[:-1].astype(np.float64) + grid[1:]) / 2).astype(np.float32)
    u = mids.view(np.uint32)[1:].astype(np.int64)  # skip the 0/2^-10 midpoint's -ulp underflow
    probe = np.concatenate([(u + d).astype(np.uint32).view(np.float32) for d in (-2, -1, 0, 1, 2)])
    probe = np.concatenate([probe, -probe, np.float32([464, 463.99, 464.01, 479.9, 480, 1e30])])
    assert (O.e4m3_encode(probe) == torch_e4m3(probe)).all()
    rng = np.random.default_rng(0)
    r = (rng.integers(0, 2**32, 1 << 20, dtype=np.uint64).astype(np.uint32) & 0xC3FFFFFF) \
        .view(np.float32)
    r = np.where(np.isnan(r), 0, r).astype(np.float32)
    assert (O.e4m3_encode(r) == torch_e4m3(r)).all()


def test_e4m3_decode_roundtrip():
    c = np.arange(256, dtype=np.uint8)
    v = O.e4m3_decode(c)
    ok = ~np.isnan(v)
    assert ((c & 0x7F) == 0x7F).sum() == (~ok).sum() == 2
    assert (O.e4m3_encode(v[ok]) == c[ok]).all()
    tv = torch.from_numpy(c).view(torch.float8_e4m3fn).float().numpy()
    assert np.array_equal(v[ok], tv[ok])


def test_bf16_round_matches_torch():
    rng = np.random.default_rng(1)
    x = rng.standard_normal(1 << 16).astype(np.float32) * np.float32(1e3)
    x[:4] = [0.5 + 2**-9, 1.0 + 2**-8, 1.0 + 3 * 2**-8, -(1.0 + 2**-8)]  # ties
    assert np.array_equal(O.bf16(x), torch.from_numpy(x).to(torch.bfloat16).float().numpy())


# ----------------------------------------------------------------------------- exp / GELU

def test_shared_expf_accuracy():
    """Cody-Waite exp on its domain [-40, 40]: within 5 ulp of float64 exp
    (measured 3.7); clamped outside."""
    xs = np.concatenate([np.linspace(-40, 40, 40001), np.linspace(-1, 1, 2001)]).astype(np.float32)
    e = np.array([O.expf(float(v)) for v in xs], np.float64)
    ref = np.exp(xs.astype(np.float64))
    rel = np.abs(e - ref) / ref
    assert rel.max() < 5 * 2.0**-24
    assert O.expf(0.0) == 1.0
    assert O.expf(1000.0) == O.expf(40.0) and O.expf(-1000.0) == O.expf(-40.0)


def test_gelu_rowmax_shortcut_preconditions():
    """What the per-tensor GELU requantisation relies on, checked over every
    finite bf16 input: GELU is non-decreasing for x >= -0.75 and |GELU(x)| < 0.17
    for x < 0."""
    x = O.from_bf16_bits(np.arange(65536, dtype=np.uint32).astype(np.uint16))
    x = x[np.isfinite(x)]
    pos = np.sort(x[x >= -0.75])
    g = O.from_bf16_bits(O.gelu_bf16(O.bf16_bits(pos)))
    assert np.all(np.diff(g) >= 0)
    neg = x[x < 0]
    assert np.abs(O.from_bf16_bits(O.gelu_bf16(O.bf16_bits(neg)))).max() < 0.17


def test_gelu_against_torch_all_bf16():
    """Bitwise equal to torch's bf16 tanh-GELU except where the reference's
    1-2/(exp(2u)+1) identity cancels (x in [-5.1, -3.4], |GELU| < 7e-4);
    there the absolute difference is below 5e-6."""
    gin = GOLD["gelu_in"]
    ours = O.from_bf16_bits(O.gelu_bf16(gin))
    ref = O.from_bf16_bits(GOLD["gelu_out"])
    x = O.from_bf16_bits(gin)
    diff = ours != ref
    assert diff.sum() <= 64
    assert np.all((x[diff] >= -5.1) & (x[diff] <= -3.4))
    assert np.abs(ours[diff] - ref[diff]).max() < 5e-6


def test_gelu_formula_restatement_independent():
    """The C GELU equals the same operation sequence evaluated with numpy
    float32 arithmetic and a float64 exp rounded to float32, except where the
    two exps differ by an ulp (rare)."""
    xs = O.from_bf16_bits(GOLD["gelu_in"])
    xs = xs[np.abs(xs) < 20]
    f = np.float32
    u = f(0.7978845608028654) * (xs + ((f(0.044715) * xs) * xs) * xs)
    with np.errstate(over="ignore"):
        e = np.exp((f(2.0) * u).astype(np.float64)).astype(np.float32)
    t = f(1.0) - f(2.0) / (e + f(1.0))
    g = O.bf16((f(0.5) * xs) * (f(1.0) + t))
    ours = O.from_bf16_bits(O.gelu_bf16(O.bf16_bits(xs)))
    assert (ours != g).mean() < 1e-3


# ----------------------------------------------------------------------------- quantisation

def test_quant_tensor_and_row_golden():
    x = GOLD["quant_x"].reshape(48, 1536)
    q, s = O.quantize_fp8(x, per_row=False)
    assert np.array_equal(q, GOLD["quant_tensor_q"].reshape(q.shape))
    assert np.array_equal(s, GOLD["quant_tensor_s"])
    q, s = O.quantize_fp8(x, per_row=True)
    assert np.array_equal(q, GOLD["quant_row_q"].reshape(q.shape))
    assert np.array_equal(s, GOLD["quant_row_s"])
    assert s[5] == 0 and (q[5] == 0).all()  # all-zero row: scale 0, codes 0


def test_quant_invariants():
    rng = np.random.default_rng(2)
    x = O.bf16_bits(rng.standard_normal((32, 200)).astype(np.float32) * 5)
    q, s = O.quantize_fp8(x, per_row=True)
    xf = O.from_bf16_bits(x)
    am = np.abs(xf).argmax(1)
    assert ((q[np.arange(32), am] & 0x7F) == 0x7E).all()  # the amax element hits 448
    qn, sn = O.quantize_fp8((x ^ 0x8000).astype(np.uint16), per_row=True)  # negate
    assert np.array_equal(sn, s)
    assert np.array_equal(qn ^ 0x80, q) or np.array_equal((qn ^ 0x80)[q != 0], q[q != 0])


def test_weight_quant_golden():
    w = GOLD["wq_w"].reshape(96, 256)
    q, s = O.quantize_weight(w, per_channel=False)
    assert np.array_equal(q, GOLD["wq_tensor_q"].reshape(q.shape))
    assert np.array_equal(s, GOLD["wq_tensor_s"])
    q, s = O.quantize_weight(w, per_channel=True)
    assert np.array_equal(q, GOLD["wq_channel_q"].reshape(q.shape))
    assert np.array_equal(s, GOLD["wq_channel_s"])


def test_f16_round_matches_numpy():
    """O.f16 (binary16 round-to-nearest-even) against numpy's float16 cast:
    every fp16 value, the fp32 values one ulp either side of every midpoint
    between neighbours (the ties themselves included), the overflow boundary
    and random fp32 bit patterns (subnormals, NaN, inf)."""
    h = np.arange(0x7C00, dtype=np.uint16).view(np.float16).astype(np.float32)  # finite, >= 0
    mid = ((h[:-1].astype(np.float64) + h[1:]) / 2).astype(np.float32)
    up = np.nextafter(mid, np.float32(np.inf))
    dn = np.nextafter(mid, np.float32(-np.inf))
    edge = np.float32([65504, 65519.99, 65520, 65536, 1e9, 2.0 ** -25, 2.0 ** -24 * 1.5,
                       np.inf, np.nan])
    rnd = np.random.default_rng(7).integers(0, 2 ** 32, 200000, dtype=np.uint64) \
        .astype(np.uint32).view(np.float32)
    x = np.concatenate([h, mid, up, dn, edge, rnd])
    x = np.concatenate([x, -x])
    with np.errstate(over="ignore"):
        ref = x.astype(np.float16).astype(np.float32)
    got = O.f16(x)
    assert np.array_equal(got, ref, equal_nan=True)


def test_scale_over_448_reciprocal_rounds_like_division():
    """amax / 448 in bf16 or fp16 (FP8Linear's weight scale): torch on the GPU
    multiplies by fl(1/448) in fp32 and rounds to the 16-bit type.  For every
    finite bf16 amax, and every fp16 amax whose quotient is a normal fp16, that
    equals rounding the IEEE quotient (1/7 is periodic in binary, so neither
    form lands near a tie).  Below fp16's normal range the quotient can sit
    exactly on a tie of the subnormal grid, where the product's one-ulp error
    decides the rounding; the oracle and the kernels form the product, as the
    GPU does.  In fp32 the two forms differ for about half of all inputs."""
    inv = np.float32(1.0) / np.float32(448.0)
    b = (np.arange(0x7F80, dtype=np.uint32) << 16).view(np.float32)
    assert np.array_equal(O.bf16(b * inv), O.bf16(b / np.float32(448.0)))
    h = np.arange(0x7C00, dtype=np.uint16).view(np.float16).astype(np.float32)
    diff = O.f16(h * inv) != O.f16(h / np.float32(448.0))
    q = h[diff].astype(np.float64) / 448
    assert (q < 2.0 ** -14).all()                        # subnormal results only
    assert np.array_equal(q * 2.0 ** 24 % 1, np.full(q.size, 0.5))  # exact grid ties
    assert 0 < diff.sum() < 64
    assert (b * inv != b / np.float32(448.0)).mean() > 0.4


@pytest.mark.parametrize("per_channel", [False, True])
def test_weight_quant_fp16_vs_torch_eager(per_channel):
    """fp16 weights: the oracle against FP8Linear.__init__'s expressions
    (fp8_linear.py:20-22) run by torch on fp16 tensors (CPU and GPU round the
    16-bit scale the same way, checked above), including an all-zero weight,
    whose scale is 0 in fp16 (1e-12 rounds to 0) and whose codes are NaN."""
    g = torch.Generator().manual_seed(4)
    for scale in (0.02, 30.0, 0.0):
        w = (torch.randn(40, 96, generator=g) * scale).to(torch.float16)
        w[3, 5] = 1e-7 if scale else 0.0                  # an fp16 subnormal
        if per_channel:
            s = (w.abs().amax(dim=1, keepdim=True) / 448.0).clamp(min=1e-12).float()
        else:
            s = (w.abs().amax() / 448.0).clamp(min=1e-12).float()
        ref = (w / s).to(torch.float8_e4m3fn).view(torch.uint8).numpy()
        q, so = O.quantize_weight_values(w.float().numpy(), O.DT_F16, per_channel=per_channel)
        assert np.array_equal(so, s.reshape(-1).numpy())
        nan = (ref & 0x7F) == 0x7F
        assert np.array_equal(q[~nan], ref[~nan]) and ((q[nan] & 0x7F) == 0x7F).all()
        assert nan.all() == (scale == 0.0)


def test_weight_quant_fp32_and_bf16_forms():
    """fp32 weights: the per-tensor expression with the GPU's reciprocal
    multiply written out (torch CPU would divide), codes from torch's cast of
    the fp32 quotient; bf16-valued weights given as floats reproduce the bf16
    oracle (whose scale divides: equal by the check above)."""
    g = torch.Generator().manual_seed(5)
    w = torch.randn(64, 80, generator=g) * 0.05
    s = (w.abs().amax() * torch.tensor(1.0 / 448.0)).clamp(min=1e-12)
    ref = (w / s).to(torch.float8_e4m3fn).view(torch.uint8).numpy()
    q, so = O.quantize_weight_values(w.numpy(), O.DT_F32)
    assert so[0] == s.item() and np.array_equal(q, ref)
    wb = O.bf16_bits(w.numpy())
    for pc in (False, True):
        q1, s1 = O.quantize_weight(wb, per_channel=pc)
        q2, s2 = O.quantize_weight_values(O.from_bf16_bits(wb), O.DT_BF16, per_channel=pc)
        assert np.array_equal(q1, q2) and np.array_equal(s1, s2)


@pytest.mark.parametrize("per_row", [False, True])
def test_quant_values_vs_torch_eager(per_row):
    """Activation quantisation of fp32 and fp16 inputs against the reference's
    formula in torch (fp8_quant.py:26-35,54: IEEE quotient, clamp, e4m3 cast;
    returned scale amax * fl(1/448)), and bf16 values given as floats against
    the bf16 oracle."""
    g = torch.Generator().manual_seed(6)
    for dt in (torch.float32, torch.float16):
        x = (torch.randn(24, 520, generator=g) * 7).to(dt).float()
        x[2] = 0
        amax = x.abs().amax(dim=1, keepdim=True) if per_row else x.abs().amax()
        s = amax.clamp(min=1e-12) / 448.0
        ref = (x / s).clamp(-448, 448).to(torch.float8_e4m3fn).view(torch.uint8).numpy()
        q, so = O.quantize_fp8_values(x.numpy(), per_row=per_row)
        assert np.array_equal(q, ref)
        assert np.array_equal(so, (amax * torch.tensor(1.0 / 448.0)).reshape(-1).numpy())
    xb = O.bf16_bits(np.random.default_rng(3).standard_normal((9, 77)).astype(np.float32))
    for gelu in (False, True):
        q1, s1 = O.quantize_fp8(xb, per_row=per_row, gelu=gelu)
        q2, s2 = O.quantize_fp8_values(O.from_bf16_bits(xb), per_row=per_row, gelu=gelu)
        assert np.array_equal(q1, q2) and np.array_equal(s1, s2)


def test_gelu_on_fp32_inputs_vs_torch():
    """The GELU of the requantisation on fp32 inputs (the reference's kernel
    rounds it to bf16 whatever the input type, fp8_ffn.py:24-30): equal to the
    reference's 1 - 2/(exp(2u)+1) form evaluated in numpy float32 with a
    float64 exp (the formula pin), and to torch's fp32 tanh-GELU rounded to
    bf16 outside the band where that identity cancels (x in [-5.2, -3.3]),
    but for one-step moves next to a bf16 rounding boundary."""
    x = np.random.default_rng(8).standard_normal(100000).astype(np.float32) * 4
    x[:4] = [1e30, -1e30, 0.0, -0.0]
    got = O.gelu_values(x)
    f = np.float32
    with np.errstate(over="ignore", invalid="ignore"):
        u = f(0.7978845608028654) * (x + ((f(0.044715) * x) * x) * x)
        e = np.exp((f(2.0) * u).astype(np.float64)).astype(np.float32)
        g = O.bf16((f(0.5) * x) * (f(1.0) + (f(1.0) - f(2.0) / (e + f(1.0)))))
    fin = np.isfinite(g)
    assert (got[fin] == g[fin]).mean() > 0.999
    assert got[0] == O.bf16(np.float32([1e30]))[0] and got[1] == 0 and got[2] == 0
    ref = F.gelu(torch.from_numpy(x), approximate="tanh").to(torch.bfloat16).float().numpy()
    out = (x < -5.2) | (x > -3.3)
    same = got[out] == ref[out]
    assert same.mean() > 0.999
    a, b = got[out][~same], ref[out][~same]
    assert (np.abs(a - b) <= np.abs(b) * 2.0 ** -7).all()
    assert np.abs(got - ref).max() < 1e-3


def test_gelu_quant_vs_unfused_torch_chain():
    """Codes equal the torch chain quantize(F.gelu(h)) except at elements
    whose GELU value differs (the cancellation band), which move by <= 1 code."""
    h = GOLD["gq_h"].reshape(16, 1024)
    q, s = O.quantize_fp8(h, per_row=True, gelu=True)
    ref = GOLD["gq_row_q"].reshape(q.shape)
    g_ours = O.from_bf16_bits(O.gelu_bf16(h))
    g_torch = F.gelu(t_bf16(h), approximate="tanh").float().numpy()
    same_g = g_ours == g_torch
    assert np.array_equal(s, GOLD["gq_row_s"])  # amax never falls in the band
    assert np.array_equal(q[same_g], ref[same_g])
    d = np.abs(q[~same_g].astype(int) - ref[~same_g].astype(int))
    assert d.size == 0 or d.max() <= 1


# ----------------------------------------------------------------------------- GEMM

def test_gemm_golden():
    a = GOLD["gemm_a"].reshape(64, 256)
    b = GOLD["gemm_b"].reshape(96, 256)
    y = O.fp8_gemm(a, GOLD["gemm_sa"], b, GOLD["gemm_sb"], O.from_bf16_bits(GOLD["gemm_bias"]))
    assert np.array_equal(O.bf16_bits(y), GOLD["gemm_out"].reshape(64, 96))


def test_gemm_brute_force_and_identity():
    rng = np.random.default_rng(3)
    a = O.e4m3_encode(rng.standard_normal((5, 64)).astype(np.float32) * 30)
    b = O.e4m3_encode(rng.standard_normal((7, 64)).astype(np.float32) * 30)
    sa, sb = np.float32([0.5]), rng.random(7).astype(np.float32)
    y = O.fp8_gemm(a, sa, b, sb)
    A, B = O.e4m3_decode(a).astype(np.float64), O.e4m3_decode(b).astype(np.float64)
    for m in range(5):
        for n in range(7):
            ref = sum(A[m, k] * B[n, k] for k in range(64)) * 0.5 * float(sb[n])
            assert y[m, n] == O.bf16(np.float32(ref))
    # identity weight with code(1.0) returns the dequantised activations
    eye = np.where(np.eye(64, dtype=bool), np.uint8(0x38), np.uint8(0))
    y = O.fp8_gemm(a, sa, eye, np.float32([1.0]))
    assert np.array_equal(y, O.bf16(O.e4m3_decode(a) * 0.5))


# ----------------------------------------------------------------------------- AdaLN

def test_ln_modulate_golden():
    x = O.from_bf16_bits(GOLD["ln_x"]).reshape(2, 16, 1536)
    sc = O.from_bf16_bits(GOLD["ln_scale"]).reshape(2, 1, 1536)
    sh = O.from_bf16_bits(GOLD["ln_shift"]).reshape(2, 1, 1536)
    ours = O.ln_modulate(x, sc, sh, 1e-6)
    ref = O.from_bf16_bits(GOLD["ln_out"]).reshape(ours.shape)
    assert (ours != ref).mean() < 0.02  # layer_norm's own reduction order differs by an ulp
    np.testing.assert_allclose(ours, ref, atol=2e-2, rtol=2e-2)
    # scale = shift = 0 is plain LayerNorm
    z = np.zeros_like(sc)
    ln = F.layer_norm(torch.from_numpy(x).to(torch.bfloat16), (1536,), eps=1e-6).float().numpy()
    np.testing.assert_allclose(O.ln_modulate(x, z, z), ln, atol=1.6e-2, rtol=0)


def test_gate_add_golden_bitwise():
    x = O.from_bf16_bits(GOLD["ln_x"]).reshape(2, 16, 1536)
    g = O.from_bf16_bits(GOLD["ga_gate"]).reshape(2, 1, 1536)
    r = O.from_bf16_bits(GOLD["ga_res"]).reshape(2, 16, 1536)
    assert np.array_equal(O.bf16_bits(O.gate_add(x, g, r)), GOLD["ga_out"].reshape(2, 16, 1536))


# ----------------------------------------------------------------------------- RMSNorm + RoPE

def test_rms_rope_golden_and_invariants():
    L, D = 48, 1536
    x = O.from_bf16_bits(GOLD["rope_x"]).reshape(1, L, D)
    w = O.from_bf16_bits(GOLD["rope_w"])
    fr = GOLD["rope_freqs"]
    cos, sin = fr[..., 0].astype(np.float32), fr[..., 1].astype(np.float32)
    out = O.rms_rope(x, w, cos, sin, 1e-6)
    ref = O.from_bf16_bits(GOLD["rope_out"]).reshape(out.shape)
    np.testing.assert_allclose(out, ref, atol=2e-2, rtol=2e-2)
    # the fused form drops eager's bf16 round trip after the weight multiply:
    # 1-ulp differences, max 0.03125 as recorded in benchmarks/fused_rope_bench.json:4
    d = np.abs(out - ref)
    assert d.max() <= 0.03125 and (d > 1e-2).mean() < 1e-2
    norm = O.rms_rope(x, w, rope=False)
    np.testing.assert_allclose(norm, O.from_bf16_bits(GOLD["rope_norm_only"]).reshape(norm.shape),
                               atol=2e-2, rtol=2e-2)
    # position 0 has cos=1, sin=0: RoPE is the identity there
    assert np.array_equal(out[0, 0], norm[0, 0])
    # the oracle's own table equals the fixture's float64 table rounded to fp32
    c2, s2 = O.wan_rope_cos_sin(2, 4, 6)
    assert np.array_equal(c2, cos) and np.array_equal(s2, sin)


def test_rope_preserves_pair_norms():
    rng = np.random.default_rng(4)
    x = O.bf16(rng.standard_normal((1, 8, 256)).astype(np.float32))
    c, s = O.wan_rope_cos_sin(2, 2, 2, head_dim=128)
    y0 = O.rms_rope(x, np.ones(256, np.float32), rope=False).reshape(8, -1, 2)
    y1 = O.rms_rope(x, np.ones(256, np.float32), c, s).reshape(8, -1, 2)
    np.testing.assert_allclose(np.hypot(y1[..., 0], y1[..., 1]),
                               np.hypot(y0[..., 0], y0[..., 1]), rtol=1e-2, atol=1e-2)


def test_wan_rope_closed_form():
    c, s = O.wan_rope_cos_sin(3, 5, 7, head_dim=128)
    assert c.shape == (105, 64)
    # token (f=1, h=2, w=3): pair 0 rotates by f, pair 22 by h, pair 43 by w (44/42/42 dims)
    t = (1 * 5 + 2) * 7 + 3
    assert np.isclose(c[t, 0], math.cos(1.0)) and np.isclose(s[t, 22], math.sin(2.0))
    assert np.isclose(c[t, 43], math.cos(3.0))
    assert np.isclose(s[t, 1], math.sin(1.0 * 10000 ** (-2 / 44)))


# ----------------------------------------------------------------------------- attention

def test_sparse_attention_golden_dense_sdpa():
    q = O.from_bf16_bits(GOLD["attn_q"]).reshape(256, 2, 128)
    k = O.from_bf16_bits(GOLD["attn_k"]).reshape(384, 2, 128)
    v = O.from_bf16_bits(GOLD["attn_v"]).reshape(384, 2, 128)
    keep = GOLD["attn_keep"]
    np.testing.assert_allclose(O.sparse_attention(q, k, v, keep), GOLD["attn_out"], atol=1e-5)
    np.testing.assert_allclose(O.dense_masked_attention(q, k, v, keep), GOLD["attn_out"], atol=1e-6)


def test_sparse_attention_invariants():
    rng = np.random.default_rng(5)
    q = O.bf16(rng.standard_normal((256, 1, 128)).astype(np.float32))
    k = O.bf16(rng.standard_normal((384, 1, 128)).astype(np.float32))
    v = O.bf16(rng.standard_normal((384, 1, 128)).astype(np.float32))
    full = np.ones((1, 2, 3), bool)
    sd = F.scaled_dot_product_attention(torch.from_numpy(q).transpose(0, 1),
                                        torch.from_numpy(k).transpose(0, 1),
                                        torch.from_numpy(v).transpose(0, 1)).transpose(0, 1)
    np.testing.assert_allclose(O.sparse_attention(q, k, v, full), sd.numpy(), atol=1e-5)
    keep = np.array([[[False, False, False], [False, True, False]]])
    out = O.sparse_attention(q, k, v, keep)
    assert (out[:128] == 0).all()  # empty row -> zeros
    # a single kept block is plain softmax attention against that block
    s = q[128:, 0] @ k[128:256, 0].T / math.sqrt(128)
    p = np.exp(s - s.max(1, keepdims=True))
    np.testing.assert_allclose(out[128:, 0], (p / p.sum(1, keepdims=True)) @ v[128:256, 0], atol=1e-5)


def test_build_csr_brute_force():
    keep = O.random_block_mask(3, 5, 7, 0.4, seed=1)
    sel, cnt, maxk = O.build_csr(keep)
    for h in range(3):
        for i in range(5):
            ids = [j for j in range(7) if keep[h, i, j]]
            rest = [j for j in range(7) if not keep[h, i, j]]
            assert cnt[h, i] == len(ids)
            assert list(sel[h, i]) == (ids + rest)[:maxk]
    assert maxk == cnt.max()


def test_build_csr_vs_reference_torch_expression():
    """The reference's own expressions (lcsa/triton_lcsa.py:66-69) run by
    torch: cnt, maxk = max(cnt.max(), 1) and the stable descending argsort of
    keep as int8, trimmed to maxk; an all-empty mask gives maxk 1."""
    for seed, dens in enumerate((0.3, 0.02, 0.0)):
        keep = O.random_block_mask(4, 11, 33, dens, seed=10 + seed)
        t = torch.from_numpy(keep)
        tc = t.sum(-1)
        tm = max(int(tc.max()), 1)
        ts = torch.argsort(t.to(torch.int8), dim=-1, descending=True, stable=True)[..., :tm]
        sel, cnt, maxk = O.build_csr(keep)
        assert maxk == tm and np.array_equal(cnt, tc.numpy())
        assert np.array_equal(sel, ts.to(torch.int32).numpy())


def test_c4_mask_density_and_diagonal():
    keep = O.c4_block_mask()
    assert keep.shape == (12, 132, 132)
    assert abs(keep.mean() - 0.30) < 0.01
    assert all(keep[:, i, i].all() for i in range(132))
    local = O.build_local_block_mask(6, 11, 7)  # within one latent time row
    assert abs(local.mean() / 2 - 0.2238) < 0.002  # 22.4% of the 132x132 grid


def test_local_and_draft_masks():
    local = O.build_local_block_mask(6, 11, 11)
    assert local.all(axis=None) is False or local.mean() > 0.7
    assert np.array_equal(local, local.T)
    rng = np.random.default_rng(6)
    qw = rng.standard_normal((66 * 2, 128, 256)).astype(np.float32)
    kw = rng.standard_normal((66 * 2, 128, 256)).astype(np.float32)
    lm = O.build_local_block_mask(6, 11, 9)
    keep = O.draft_block_mask(qw, kw, 2, 2, lm, topk=500)
    assert keep.shape == (2, 132, 132)
    # kept blocks lie inside the tiled local mask; joint top-k per (head, time row)
    tiled = np.tile(lm, (2, 2))
    assert not (keep & ~tiled[None]).any()
    per_group = keep.reshape(2, 2, 66, 132).sum((2, 3))
    assert (per_group <= 500).all()


def test_draft_topk_threshold_brute_force():
    """keep_i = v_i > (k+1)-th largest  <=>  v_i is a number and at most k values
    (NaN counted as largest, torch.topk's order) are >= v_i."""
    rng = np.random.default_rng(11)
    for trial in range(200):
        n = int(rng.integers(1, 30))
        v = rng.integers(0, 6, (1, n)).astype(np.float32) / 8
        v[rng.random((1, n)) < 0.1] = np.nan
        topk = int(rng.integers(0, n + 3))
        got = O._topk_threshold_keep(v, topk)[0]
        k = min(n - 1, topk)
        ge = lambda a, b: np.isnan(a) or (not np.isnan(b) and a >= b)
        want = [not np.isnan(v[0, i]) and sum(ge(v[0, j], v[0, i]) for j in range(n)) <= k
                for i in range(n)]
        assert list(got) == want, (v, topk)


def _torch_bf16_draft(qb, kb, nheads, q_temporal, local, topk):
    """lcsa/reference.py:41-63 run by torch itself on bf16 CPU tensors."""
    import torch
    from einops import rearrange
    tq = torch.from_numpy(O.from_bf16_bits(qb)).bfloat16()
    tk = torch.from_numpy(O.from_bf16_bits(kb)).bfloat16()
    aq = rearrange(torch.mean(tq, dim=1), "s (h d) -> h s d", h=nheads)
    ak = rearrange(torch.mean(tk, dim=1), "s (h d) -> h s d", h=nheads)
    scores = torch.einsum("hld,hmd->hlm", aq, ak) / math.sqrt(aq.shape[-1])
    sq, sk = local.shape
    lm = torch.from_numpy(local).unsqueeze(1).unsqueeze(0).repeat(
        scores.shape[1] // sq, 1, scores.shape[2] // sk, 1)
    lm = rearrange(lm, "x a y b -> (x a) (y b)")
    scores = scores + torch.zeros_like(scores).masked_fill(~lm.unsqueeze(0), float("-inf"))
    attn = torch.softmax(scores, dim=-1)
    flat = rearrange(attn, "h (t s) m -> (h t) (s m)", t=q_temporal)
    k = min(flat.shape[1] - 1, topk)
    thr = torch.topk(flat, k=k + 1, dim=1, largest=True).values[:, -1].unsqueeze(1)
    keep = rearrange(flat > thr, "(h t) (s m) -> h (t s) m", t=q_temporal,
                     s=scores.shape[1] // q_temporal)
    return keep.numpy(), attn.float().numpy()


@pytest.mark.parametrize("seed,scale,empty_row", [(3, 2.0, False), (4, 0.05, False),
                                                  (5, 1.0, True)])
def test_draft_mask_bf16_matches_torch_bf16_run(seed, scale, empty_row):
    """The oracle's bf16 run against torch's own bf16 kernels on the CPU
    (mean, einsum, scalar division, softmax, topk): every stage's rounding,
    the NaN rows of an empty local row, and the threshold ties.  The float32
    reading of the same lines differs, so the staging is what is pinned."""
    rng = np.random.default_rng(seed)
    H, D, Nq, Nk = 4, 128, 24, 36
    qb = O.bf16_bits(rng.standard_normal((Nq, 128, H * D)).astype(np.float32) * scale)
    kb = O.bf16_bits(rng.standard_normal((Nk, 128, H * D)).astype(np.float32) * scale)
    local = O.build_local_block_mask(3, 4, 3)
    if empty_row:
        local[7, :] = False
    for topk in (5, 60, 400):
        keep, attn = O.draft_block_mask(qb, kb, H, 2, local, topk, return_attn=True)
        tkeep, tattn = _torch_bf16_draft(qb, kb, H, 2, local, topk)
        assert np.array_equal(np.isnan(attn), np.isnan(tattn))
        assert np.array_equal(np.nan_to_num(attn), np.nan_to_num(tattn))
        assert np.array_equal(keep, tkeep)
    k32 = O.draft_block_mask(O.from_bf16_bits(qb), O.from_bf16_bits(kb), H, 2, local, 60)
    if not empty_row and scale > 1:
        assert not np.array_equal(k32, _torch_bf16_draft(qb, kb, H, 2, local, 60)[0])


@pytest.mark.parametrize("seed,scale", [(12, 1.0), (13, 30.0)])
def test_layer_norm_affine_vs_torch_bf16(seed, scale):
    """norm3: torch's own LayerNorm(elementwise_affine=True) on bf16 CPU tensors
    against the oracle; equal except where the float64 value sits within an
    fp32 rounding of a bf16 boundary."""
    rng = np.random.default_rng(seed)
    x = O.bf16(rng.standard_normal((64, 1536)).astype(np.float32) * scale + 0.5)
    w = O.bf16((1 + 0.1 * rng.standard_normal(1536)).astype(np.float32))
    b = O.bf16((0.1 * rng.standard_normal(1536)).astype(np.float32))
    ref = F.layer_norm(torch.from_numpy(x).bfloat16(), (1536,), torch.from_numpy(w).bfloat16(),
                       torch.from_numpy(b).bfloat16(), eps=1e-6).float().numpy()
    got = O.layer_norm_affine(x, w, b, 1e-6)
    ulp = np.abs(O.bf16_bits(got).astype(np.int32) - O.bf16_bits(ref).astype(np.int32))
    assert ulp.max() <= 1 and (ulp == 0).mean() > 0.99
    # without affine parameters it is the LayerNorm inside ln_modulate
    plain = O.layer_norm_affine(x, np.ones(1536, np.float32), np.zeros(1536, np.float32))
    ref0 = F.layer_norm(torch.from_numpy(x).bfloat16(), (1536,), eps=1e-6).float().numpy()
    assert np.abs(O.bf16_bits(plain).astype(np.int32) - O.bf16_bits(ref0).astype(np.int32)).max() <= 1


def test_dense_attention_vs_masked_and_sdpa():
    rng = np.random.default_rng(14)
    q = rng.standard_normal((256, 2, 64))
    k = rng.standard_normal((384, 2, 64))
    v = rng.standard_normal((384, 2, 64))
    got = O.dense_attention(q, k, v)
    keep = np.ones((2, 2, 3), bool)
    assert np.allclose(got, O.dense_masked_attention(q, k, v, keep), atol=1e-12)
    t = [torch.from_numpy(a).permute(1, 0, 2)[None] for a in (q, k, v)]
    ref = F.scaled_dot_product_attention(*t)[0].permute(1, 0, 2).numpy()
    assert np.allclose(got, ref, atol=1e-10)


def test_window_partition_roundtrip_and_token_map():
    rng = np.random.default_rng(7)
    x = rng.standard_normal((1, 4, 16, 24, 3)).astype(np.float32)
    xw = O.window_partition(x)
    assert xw.shape == (4 // 2 * 2 * 3, 128, 3)
    back = O.window_reverse(xw, (4, 16, 24))
    assert np.array_equal(back.reshape(x.shape), x)
