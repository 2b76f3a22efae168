"""Fused AdaLN elementwise chains on gfx950.

`fused_ln_modulate(x, scale, shift)`: LayerNorm (no affine) then
``x*(1+scale)+shift`` with eager's per-op bf16 roundings
(flashvsr_sm89_ops/fused_adaln.py:22-42,60-71).  Note the argument order:
(scale, shift), the reverse of upstream ``modulate(x, shift, scale)``.
`fused_gate_add(x, gate, residual)`: ``bf16(x + bf16(gate*residual))``,
bitwise equal to eager (fused_adaln.py:45-57,74-85).
`fused_ln_modulate_quant` additionally returns the per-row e4m3 codes of the
modulated rows from the same pass (the activation quantisation of the FP8
linear that consumes them).

The two reference ops take x and the [B, 1, D] parameters in bf16, fp16 or
fp32, each in its own type, and return x's type, as the reference's kernels
(loads ``.to(tl.float32)``, output ``torch.empty_like(x)``); the fused
extensions of this module take bf16.
"""
from __future__ import annotations

import torch

from . import _lib


def _check_param_sizes(x, *ps):
    """Every [B, 1, D] parameter holds B*D elements (the kernels read them all)."""
    B, L, D = x.shape
    for p in ps:
        if p.numel() != B * D:
            raise ValueError(f"modulation parameter shape {tuple(p.shape)} does not match "
                             f"[B, 1, D] = [{B}, 1, {D}]")


def _check_params(x, *ps):
    """The fused extensions' operands: bf16 x and bf16 [B, 1, D] parameters."""
    _lib.require_dtype(x, torch.bfloat16, "x")
    for p in ps:
        _lib.require_dtype(p, torch.bfloat16, "modulation parameter")
    _check_param_sizes(x, *ps)


def fused_ln_modulate(x: torch.Tensor, scale: torch.Tensor, shift: torch.Tensor,
                      eps: float = 1e-6):
    """LayerNorm(affine=False) + modulate. x [B, L, D] contiguous; scale/shift
    [B, 1, D]; each bf16, fp16 or fp32.  Returns x's type."""
    B, L, D = x.shape
    assert x.is_contiguous() and scale.is_contiguous() and shift.is_contiguous()
    _lib.require_gpu(x, scale, shift)
    dts = (_lib.dtype_code(x, "x"), _lib.dtype_code(scale, "scale"),
           _lib.dtype_code(shift, "shift"))
    _check_param_sizes(x, scale, shift)
    out = torch.empty_like(x)
    _lib.check(_lib.lib().fvsr_ln_modulate_dt(x.data_ptr(), dts[0], scale.data_ptr(), dts[1],
                                              shift.data_ptr(), dts[2], out.data_ptr(), B, L, D,
                                              float(eps), _lib.stream(x)), "fused_ln_modulate")
    return out


def fused_ln_modulate_quant(x: torch.Tensor, scale: torch.Tensor, shift: torch.Tensor,
                            eps: float = 1e-6, write_bf16: bool = False):
    """fused_ln_modulate + per-row e4m3 quantisation of its output in one pass.
    Returns (codes [B*L, D] e4m3, row scales [B*L, 1] fp32[, bf16 out])."""
    B, L, D = x.shape
    assert x.is_contiguous() and scale.is_contiguous() and shift.is_contiguous()
    _lib.require_gpu(x, scale, shift)
    _check_params(x, scale, shift)
    q = torch.empty((B * L, D), dtype=torch.float8_e4m3fn, device=x.device)
    s = torch.empty((B * L, 1), dtype=torch.float32, device=x.device)
    out = torch.empty_like(x) if write_bf16 else None
    _lib.check(_lib.lib().fvsr_ln_modulate(x.data_ptr(), scale.data_ptr(), shift.data_ptr(),
                                           _lib.ptr(out), B, L, D, float(eps), q.data_ptr(),
                                           s.data_ptr(), _lib.stream(x)),
               "fused_ln_modulate_quant")
    return (q, s, out) if write_bf16 else (q, s)


def fused_gate_add(x: torch.Tensor, gate: torch.Tensor, residual: torch.Tensor):
    """x + gate * residual. x/residual [B, L, D] contiguous; gate [B, 1, D];
    each bf16, fp16 or fp32.  Returns x's type."""
    B, L, D = x.shape
    assert x.is_contiguous() and residual.is_contiguous() and gate.is_contiguous()
    if residual.shape != x.shape:
        raise ValueError(f"fused_gate_add: residual {tuple(residual.shape)} does not match x "
                         f"{tuple(x.shape)}")
    _lib.require_gpu(x, gate, residual)
    dts = (_lib.dtype_code(x, "x"), _lib.dtype_code(gate, "gate"),
           _lib.dtype_code(residual, "residual"))
    _check_param_sizes(x, gate)
    out = torch.empty_like(x)
    _lib.check(_lib.lib().fvsr_gate_add_dt(x.data_ptr(), dts[0], gate.data_ptr(), dts[1],
                                           residual.data_ptr(), dts[2], out.data_ptr(), B, L, D,
                                           _lib.stream(x)), "fused_gate_add")
    return out


def _ln_affine_args(x, weight, bias):
    _lib.require_gpu(x, weight, bias)
    _lib.require_dtype(x, torch.bfloat16, "x")
    D = x.shape[-1]
    w = weight.to(torch.bfloat16).contiguous()
    b = bias.to(torch.bfloat16).contiguous() if bias is not None else torch.zeros_like(w)
    if w.numel() != D or b.numel() != D:
        raise ValueError(f"LayerNorm weight/bias must have {D} elements")
    return x.contiguous(), w, b


def layer_norm(x: torch.Tensor, weight: torch.Tensor, bias: torch.Tensor | None,
               eps: float = 1e-6) -> torch.Tensor:
    """nn.LayerNorm(elementwise_affine=True) over the last dim of a bf16
    tensor: the DiT block's norm3 before the cross-attention
    (flashvsr_sm89_ops/integrate.py:171), torch's fp32 arithmetic, one rounding."""
    x2, w, b = _ln_affine_args(x, weight, bias)
    out = torch.empty_like(x2)
    D = x2.shape[-1]
    _lib.check(_lib.lib().fvsr_layer_norm(x2.data_ptr(), w.data_ptr(), b.data_ptr(),
                                          out.data_ptr(), x2.numel() // D, D, float(eps), None,
                                          None, _lib.stream(x2)), "layer_norm")
    return out


def fused_gate_add_layer_norm(x: torch.Tensor, gate: torch.Tensor, residual: torch.Tensor,
                              weight: torch.Tensor, bias: torch.Tensor | None,
                              eps: float = 1e-6):
    """x1 = fused_gate_add(x, gate, residual) and layer_norm(x1, weight, bias)
    in one pass over the rows: the self-attention's gated residual and the
    norm3 before the cross-attention (integrate.py:151-171).  x, residual
    [B, L, D] bf16 (residual may be a [B*L, D] view), gate [B, 1, D].
    Returns (x1, normed), each [B, L, D] bf16, equal to the two-step results."""
    B, L, D = x.shape
    res = residual.reshape(B, L, D)
    for t in (x, res, gate):
        if not t.is_contiguous():
            raise ValueError("fused_gate_add_layer_norm: tensors must be contiguous")
    _lib.require_gpu(x, res, gate)
    _lib.require_dtype(res, torch.bfloat16, "residual")
    _lib.require_dtype(gate, torch.bfloat16, "gate")
    if tuple(gate.shape) != (B, 1, D):
        raise ValueError(f"gate must be [{B}, 1, {D}], got {tuple(gate.shape)}")
    x2, w, b = _ln_affine_args(x, weight, bias)
    x1 = torch.empty_like(x2)
    out = torch.empty_like(x2)
    _lib.check(_lib.lib().fvsr_gate_add_layer_norm(
        x2.data_ptr(), gate.data_ptr(), res.data_ptr(), x1.data_ptr(), w.data_ptr(), b.data_ptr(),
        out.data_ptr(), B, L, D, float(eps), None, None, _lib.stream(x2)),
        "fused_gate_add_layer_norm")
    return x1, out


def layer_norm_quant(x: torch.Tensor, weight: torch.Tensor, bias: torch.Tensor | None,
                     eps: float = 1e-6, write_bf16: bool = False):
    """layer_norm + per-row e4m3 quantisation of its output in one pass.
    Returns (codes [rows, D] e4m3, row scales [rows, 1] fp32[, bf16 out])."""
    x2, w, b = _ln_affine_args(x, weight, bias)
    D = x2.shape[-1]
    rows = x2.numel() // D
    q = torch.empty((rows, D), dtype=torch.float8_e4m3fn, device=x2.device)
    s = torch.empty((rows, 1), dtype=torch.float32, device=x2.device)
    out = torch.empty_like(x2) if write_bf16 else None
    _lib.check(_lib.lib().fvsr_layer_norm(x2.data_ptr(), w.data_ptr(), b.data_ptr(),
                                          _lib.ptr(out), rows, D, float(eps), q.data_ptr(),
                                          s.data_ptr(), _lib.stream(x2)), "layer_norm_quant")
    return (q, s, out) if write_bf16 else (q, s)


def fused_gate_add_ln_modulate_quant(x: torch.Tensor, gate: torch.Tensor, residual: torch.Tensor,
                                     scale: torch.Tensor, shift: torch.Tensor, eps: float = 1e-6,
                                     write_bf16: bool = False):
    """x1 = fused_gate_add(x, gate, residual), then fused_ln_modulate_quant(x1,
    scale, shift), in one pass over the rows: the gated residual that ends a
    DiT sub-block and the AdaLN that starts the next (integrate.py:151-182).
    x, residual [B, L, D] bf16 (residual may be a [B*L, D] view); gate,
    scale, shift [B, 1, D].  Returns (x1, codes [B*L, D] e4m3, row scales
    [B*L, 1] fp32[, LN-modulated bf16])."""
    B, L, D = x.shape
    res = residual.reshape(B, L, D)
    for t in (x, res, gate, scale, shift):
        if not t.is_contiguous():
            raise ValueError("fused_gate_add_ln_modulate_quant: tensors must be contiguous")
    _lib.require_gpu(x, res, gate, scale, shift)
    _check_params(x, gate, scale, shift)
    _lib.require_dtype(res, torch.bfloat16, "residual")
    x1 = torch.empty_like(x)
    q = torch.empty((B * L, D), dtype=torch.float8_e4m3fn, device=x.device)
    s = torch.empty((B * L, 1), dtype=torch.float32, device=x.device)
    out = torch.empty_like(x) if write_bf16 else None
    _lib.check(_lib.lib().fvsr_gate_add_ln_modulate(
        x.data_ptr(), gate.data_ptr(), res.data_ptr(), x1.data_ptr(), scale.data_ptr(),
        shift.data_ptr(), _lib.ptr(out), B, L, D, float(eps), q.data_ptr(), s.data_ptr(),
        _lib.stream(x)), "fused_gate_add_ln_modulate_quant")
    return (x1, q, s, out) if write_bf16 else (x1, q, s)
