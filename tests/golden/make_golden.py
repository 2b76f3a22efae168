"""Writes tests/golden/golden.npz: known-answer vectors from torch CPU eager.

The reference publishes no golden vectors (its tests seed a CUDA RNG).  These
fixtures pin the oracle and the HIP path to torch's own eager CPU arithmetic
for each op's stock math, i.e. what the reference kernels replace:
  quant_*      fp32 eager chain of the quantisation contract
               (flashvsr_sm89_ops/fp8_quant.py:26-35,54: amax, clamp(1e-12)/448,
               x/s, clamp +-448, cast to float8_e4m3fn); the returned scale
               `amax / FP8_MAX` as torch evaluates it on the GPU (gpu_over_448)
  wq_*         weight quantisation eager expressions (fp8_linear.py:20-22) and
               their per-output-channel form
  gelu_*       F.gelu(approximate='tanh') in bf16 over every bf16 bit pattern
  gq_*         quantisation of that GELU (the unfused chain fp8_ffn.py:7-10 compares to)
  ln_*         nn.LayerNorm(no affine) then x*(1+scale)+shift in bf16 eager
  ga_*         x + gate*res in bf16 eager
  rope_*       Wan-style RMSNorm (float, type_as, *weight) then float64 complex RoPE
  attn_*       float64 SDPA with the block mask expanded to tokens
  gemm_*       float64 dequantised matmul + bias, rounded to bf16
Inputs come from a seeded CPU torch.Generator.  Run: python tests/golden/make_golden.py
"""
import math
import os

import numpy as np
import torch
import torch.nn.functional as F

OUT = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden.npz")


def bits(t: torch.Tensor) -> np.ndarray:
    assert t.dtype == torch.bfloat16
    return t.contiguous().view(torch.int16).numpy().view(np.uint16).copy()


def codes(t: torch.Tensor) -> np.ndarray:
    return t.contiguous().view(torch.uint8).numpy().copy()


def gpu_over_448(t: torch.Tensor) -> torch.Tensor:
    """`t / 448.0` for an fp32 tensor as torch computes it on the GPU: a
    tensor divided by a Python float is multiplied by the float reciprocal
    there (fl(1/448)), whereas the CPU divides.  The reference's returned
    scales (fp8_quant.py:54, fp8_ffn.py:72) are such a division of a device
    tensor."""
    return t * torch.tensor(1.0 / 448.0, dtype=torch.float32)


def main():
    g = torch.Generator().manual_seed(20261201)
    out = {}

    # --- activation quantisation (tensor and row) ---
    x = torch.randn(48, 1536, generator=g).mul(3.0).to(torch.bfloat16)
    x[5] = 0  # an all-zero row
    x[7, 3] = 300.0  # an outlier
    xf = x.float()
    amax = xf.abs().amax()
    s = torch.clamp(amax, min=1e-12) / 448.0
    out["quant_x"] = bits(x)
    out["quant_tensor_q"] = codes((xf / s).clamp(-448.0, 448.0).to(torch.float8_e4m3fn))
    out["quant_tensor_s"] = gpu_over_448(amax).reshape(1).numpy()
    amax_r = xf.abs().amax(dim=1, keepdim=True)
    s_r = torch.clamp(amax_r, min=1e-12) / 448.0
    out["quant_row_q"] = codes((xf / s_r).clamp(-448.0, 448.0).to(torch.float8_e4m3fn))
    out["quant_row_s"] = gpu_over_448(amax_r).reshape(-1).numpy()

    # --- weight quantisation ---
    w = (torch.randn(96, 256, generator=g) * 0.02).to(torch.bfloat16)
    ws = (w.abs().amax() / 448.0).clamp(min=1e-12).float()
    out["wq_w"] = bits(w)
    out["wq_tensor_q"] = codes((w / ws).to(torch.float8_e4m3fn))
    out["wq_tensor_s"] = ws.reshape(1).numpy()
    wsc = (w.abs().amax(dim=1, keepdim=True) / 448.0).clamp(min=1e-12).float()
    out["wq_channel_q"] = codes((w / wsc).to(torch.float8_e4m3fn))
    out["wq_channel_s"] = wsc.reshape(-1).numpy()

    # --- tanh-GELU over all finite bf16 patterns, and its quantisation ---
    allb = torch.arange(65536, dtype=torch.int32).to(torch.int16).view(torch.bfloat16)
    fin = torch.isfinite(allb.float())
    hb = allb[fin]
    out["gelu_in"] = bits(hb)
    out["gelu_out"] = bits(F.gelu(hb, approximate="tanh"))
    h = torch.randn(16, 1024, generator=g).mul(2.0).to(torch.bfloat16)
    gq = F.gelu(h, approximate="tanh").float()
    ga = gq.abs().amax(dim=1, keepdim=True)
    out["gq_h"] = bits(h)
    out["gq_row_q"] = codes((gq / (torch.clamp(ga, min=1e-12) / 448.0)).clamp(-448, 448)
                           .to(torch.float8_e4m3fn))
    out["gq_row_s"] = gpu_over_448(ga).reshape(-1).numpy()

    # --- LayerNorm + modulate, gate_add ---
    B, L, D = 2, 16, 1536
    lx = torch.randn(B, L, D, generator=g).to(torch.bfloat16)
    sc = (torch.randn(B, 1, D, generator=g) * 0.1).to(torch.bfloat16)
    sh = (torch.randn(B, 1, D, generator=g) * 0.1).to(torch.bfloat16)
    xn = F.layer_norm(lx, (D,), eps=1e-6)
    out["ln_x"], out["ln_scale"], out["ln_shift"] = bits(lx), bits(sc), bits(sh)
    out["ln_out"] = bits(xn * (1 + sc) + sh)
    gate = (torch.randn(B, 1, D, generator=g) * 0.5).to(torch.bfloat16)
    res = torch.randn(B, L, D, generator=g).to(torch.bfloat16)
    out["ga_gate"], out["ga_res"] = bits(gate), bits(res)
    out["ga_out"] = bits(lx + gate * res)

    # --- RMSNorm + RoPE (Wan stock chain) ---
    f, hh, ww, heads, hd = 2, 4, 6, 12, 128
    Lr = f * hh * ww
    rx = torch.randn(1, Lr, heads * hd, generator=g).to(torch.bfloat16)
    rw = (1 + 0.1 * torch.randn(heads * hd, generator=g)).to(torch.bfloat16)
    d6 = hd // 6
    dims = (hd - 4 * d6, 2 * d6, 2 * d6)

    def rope_params(n, dim, theta=10000.0):
        fr = torch.outer(torch.arange(n, dtype=torch.float64),
                         1.0 / torch.pow(theta, torch.arange(0, dim, 2).to(torch.float64).div(dim)))
        return torch.polar(torch.ones_like(fr), fr)

    fq = torch.cat([
        rope_params(f, dims[0]).view(f, 1, 1, -1).expand(f, hh, ww, -1),
        rope_params(hh, dims[1]).view(1, hh, 1, -1).expand(f, hh, ww, -1),
        rope_params(ww, dims[2]).view(1, 1, ww, -1).expand(f, hh, ww, -1),
    ], dim=-1).reshape(Lr, 1, -1)
    xnorm = rx.float()
    xnorm = (xnorm * torch.rsqrt(xnorm.pow(2).mean(dim=-1, keepdim=True) + 1e-6)).type_as(rx) * rw
    xc = torch.view_as_complex(xnorm.to(torch.float64).reshape(Lr, heads, -1, 2))
    ro = torch.view_as_real(xc * fq).flatten(2).to(torch.bfloat16).reshape(1, Lr, heads * hd)
    out["rope_x"], out["rope_w"] = bits(rx), bits(rw)
    out["rope_freqs"] = torch.view_as_real(fq.reshape(Lr, -1)).numpy()  # float64 [L,64,2]
    out["rope_out"] = bits(ro)
    out["rope_norm_only"] = bits(xnorm)  # rope=False reference (RMSNorm * weight)

    # --- block-sparse attention: dense SDPA with the expanded block mask ---
    Hh, NQ, NK = 2, 2, 3
    aq = torch.randn(NQ * 128, Hh, 128, generator=g).to(torch.bfloat16)
    ak = torch.randn(NK * 128, Hh, 128, generator=g).to(torch.bfloat16)
    av = torch.randn(NK * 128, Hh, 128, generator=g).to(torch.bfloat16)
    keep = torch.tensor([[[1, 0, 1], [0, 1, 1]], [[1, 1, 1], [1, 0, 0]]], dtype=torch.bool)
    mask = keep.repeat_interleave(128, 1).repeat_interleave(128, 2)  # [H, Lq, Lk]
    o = F.scaled_dot_product_attention(aq.double().transpose(0, 1), ak.double().transpose(0, 1),
                                       av.double().transpose(0, 1), attn_mask=mask,
                                       scale=1.0 / math.sqrt(128)).transpose(0, 1)
    out["attn_q"], out["attn_k"], out["attn_v"] = bits(aq), bits(ak), bits(av)
    out["attn_keep"] = keep.numpy()
    out["attn_out"] = o.float().numpy()

    # --- FP8 GEMM: float64 dequantised matmul + bias ---
    M, N, K = 64, 96, 256
    a8 = (torch.randn(M, K, generator=g) * 60).clamp(-448, 448).to(torch.float8_e4m3fn)
    b8 = (torch.randn(N, K, generator=g) * 60).clamp(-448, 448).to(torch.float8_e4m3fn)
    sa = torch.rand(M, 1, generator=g) * 0.01 + 1e-4
    sb = torch.rand(N, generator=g) * 0.01 + 1e-4
    bias = torch.randn(N, generator=g).to(torch.bfloat16)
    y = (a8.double() * sa.double()) @ (b8.double() * sb.double()[:, None]).T + bias.double()
    out["gemm_a"], out["gemm_b"] = codes(a8), codes(b8)
    out["gemm_sa"], out["gemm_sb"] = sa.reshape(-1).numpy(), sb.numpy()
    out["gemm_bias"] = bits(bias)
    out["gemm_out"] = bits(y.float().to(torch.bfloat16))

    np.savez_compressed(OUT, **out)
    print(OUT, os.path.getsize(OUT), "bytes")


if __name__ == "__main__":
    main()
