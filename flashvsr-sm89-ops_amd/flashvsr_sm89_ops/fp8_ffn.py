"""FFN with the GELU(tanh) -> FP8 mid-section fused into one pass.

The reference (flashvsr_sm89_ops/fp8_ffn.py:75-96) runs
quantize -> mm0 -> [gelu+absmax] -> [gelu+quantize] -> mm2, evaluating GELU
twice per element.  Here GELU runs once per element:
  per-token scales  one kernel keeps each bf16 row of h = mm0's output in
                    registers, applies GELU, reduces the row amax and writes
                    the e4m3 codes;
  per-tensor scale  mm0's epilogue also writes the maximum of h per
                    (row, 128-column slab); GELU is non-decreasing above -0.75
                    and below 0.17 in magnitude for negative inputs, so the
                    tensor's max|gelu(h)| is gelu(max h) (one scan of the
                    tensor otherwise), and the quantisation pass applies GELU
                    once.
Codes and scales are exactly those of ``quantize_fp8(gelu(h))`` for the bf16 h
mm0 produced.  GELU is the reference form 1 - 2/(exp(2u)+1) (fp8_ffn.py:24-30)
with a Cody-Waite exp that the CPU oracle evaluates identically.
"""
from __future__ import annotations

import torch
import torch.nn as nn

from . import _lib
from .fp8_linear import FP8Linear, fp8_gemm, quantize_input_fp8
from .fp8_quant import FP8_MAX, quantize_fp8, quantize_rows_fp8  # noqa: F401


def fused_gelu_quant_fp8(y2: torch.Tensor, per_token: bool = False):
    """y2: [M, K] bf16, fp16 or fp32 -> (e4m3 codes of bf16(gelu_tanh(y2)),
    scale), the GELU never materialised (fp8_ffn.py:34-72: loaded as fp32,
    GELU rounded to bf16, quantised as quantize_fp8)."""
    return quantize_rows_fp8(y2, per_token, gelu=True, what="fused_gelu_quant_fp8")


def gemm_gelu_quant_fp8(x8: torch.Tensor, s: torch.Tensor, lin, per_token: bool):
    """mm0 then the GELU requantisation of its bf16 output: returns
    (codes, scale) of quantize_fp8(gelu(bf16(x8 @ W.T * s * w_scale + b)))."""
    if per_token:
        h = fp8_gemm(x8, s, lin.weight, lin.w_scale, lin.bias)
        return fused_gelu_quant_fp8(h, per_token=True)
    M = x8.shape[0]
    N = lin.weight.shape[0]
    nparts = int(_lib.lib().fvsr_gemm_amax_parts(N))
    hmax = torch.empty((M, nparts), dtype=torch.float32, device=x8.device)
    h = fp8_gemm(x8, s, lin.weight, lin.w_scale, lin.bias, epilogue=_lib.EPI_ROWMAX,
                 amax_part=hmax)
    h8 = torch.empty((M, N), dtype=torch.float8_e4m3fn, device=x8.device)
    hs = (torch.zeros if M == 0 or N == 0 else torch.empty)(1, dtype=torch.float32,
                                                             device=x8.device)
    ws = torch.empty(2 * int(_lib.lib().fvsr_quant_workspace_floats(M, N, 0)), dtype=torch.float32,
                     device=x8.device)
    _lib.check(_lib.lib().fvsr_gelu_quant_fp8_tensor(h.data_ptr(), M, N, hmax.data_ptr(), nparts,
                                                     h8.data_ptr(), hs.data_ptr(), ws.data_ptr(),
                                                     ws.numel(), _lib.stream(h)),
               "gelu requantisation")
    return h8, hs


class FP8FFN(nn.Module):
    """Drop-in for a DiT FFN `Sequential(Linear, GELU(tanh), Linear)` whose two
    Linears are already FP8Linear (fp8_ffn.py:75-96)."""

    def __init__(self, lin0, lin2):
        super().__init__()
        self.lin0 = lin0
        self.lin2 = lin2

    def forward(self, x):
        shape = x.shape
        per_token = getattr(self.lin0, "per_token", False)
        x8, s = quantize_input_fp8(x.reshape(-1, shape[-1]), per_token)
        h8, hs = gemm_gelu_quant_fp8(x8, s, self.lin0, per_token)
        out = self.lin2._mm(h8, hs)
        return out.reshape(*shape[:-1], out.shape[-1])


def _is_block_ffn(name: str) -> bool:
    parts = name.split(".")
    return len(parts) == 3 and parts[0] == "blocks" and parts[1].isdigit() and parts[2] == "ffn"


def convert_ffn_fp8(model: nn.Module) -> int:
    """Replace each DiT block's ``blocks.<i>.ffn`` = Sequential(Linear,
    GELU(tanh), Linear) by FP8FFN over its two Linears; returns how many were
    replaced (reference fp8_ffn.py:99-115).  The Linears must already be
    FP8Linear (convert_linears_fp8 with the "ffn" part): otherwise
    AssertionError, as in the reference.  FFNs already converted are left
    alone, so a second call replaces nothing."""
    found = [(name, mod) for name, mod in model.named_modules()
             if _is_block_ffn(name) and not isinstance(mod, FP8FFN)]
    for name, seq in found:
        up, down = seq[0], seq[2]
        assert isinstance(up, FP8Linear) and isinstance(down, FP8Linear), \
            f"{name}: its Linears are not FP8 yet; run convert_linears_fp8(parts=['ffn']) first"
        model.get_submodule(name.rpartition(".")[0]).ffn = FP8FFN(up, down)
    return len(found)
