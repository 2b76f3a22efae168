"""Dynamic FP8 (OCP e4m3fn) quantisation on gfx950.

`quantize_fp8(x2)` keeps the reference contract (flashvsr_sm89_ops/fp8_quant.py:42-55):
``s = max(amax,1e-12)/448; q = e4m3(clamp(x/s, +-448))`` with a true fp32
divide, returning ``(q, amax/448)`` with the scale left on the device (no host
sync); the returned scale is ``amax * fl(1/448)``, the value torch gives the
reference's ``amax / FP8_MAX`` on the GPU.  ``per_token=True`` gives one scale
per row (``[M, 1]``), the layout torch._scaled_mm takes for row-wise scales;
per-token quantisation is a single HBM pass (one wavefront per row, the row
stays in registers).  Inputs may be bf16, fp16 or fp32 (the reference's
kernels load any of them as fp32); bf16 runs the vector kernels.
"""
from __future__ import annotations

import torch

from . import _lib

FP8_MAX = 448.0


def _workspace(x: torch.Tensor, rows: int, cols: int, mode: int):
    """Per-tensor partial maxima (None for per-row scales, which need none)."""
    n = int(_lib.lib().fvsr_quant_workspace_floats(rows, cols, mode))
    return torch.empty(n, dtype=torch.float32, device=x.device) if n else None


def quantize_fp8(x2: torch.Tensor, per_token: bool = False):
    """x2: [M, K] bf16, fp16 or fp32 (rows may be strided, last dim contiguous)
    -> (float8_e4m3fn [M, K], fp32 scale: [1] per tensor, [M, 1] per token)."""
    return quantize_rows_fp8(x2, per_token, gelu=False, what="quantize_fp8")


def quantize_rows_fp8(x2: torch.Tensor, per_token: bool, gelu: bool, what: str):
    """Activation quantisation of x2 (or of tanh-GELU(x2) rounded to bf16) through
    fvsr_quant_fp8_dt."""
    _lib.require_gpu(x2)
    dt = _lib.dtype_code(x2, "x2")
    if x2.dim() != 2:
        raise ValueError(f"{what} expects a 2-D tensor, got shape {tuple(x2.shape)}")
    M, K = x2.shape
    if x2.numel() and x2.stride(1) != 1:
        x2 = x2.contiguous()
    q = torch.empty((M, K), dtype=torch.float8_e4m3fn, device=x2.device)
    # The kernels write every scale; only an empty input keeps amax = 0.
    alloc = torch.zeros if x2.numel() == 0 else torch.empty
    s = alloc((M, 1) if per_token else (1,), dtype=torch.float32, device=x2.device)
    if x2.numel() == 0:
        return q, s
    mode = _lib.SCALE_ROW if per_token else _lib.SCALE_TENSOR
    ws = None if per_token else _workspace(x2, M, K, mode)  # per-row scales need none
    _lib.check(_lib.lib().fvsr_quant_fp8_dt(x2.data_ptr(), dt, M, K, x2.stride(0), mode,
                                            int(gelu), q.data_ptr(), s.data_ptr(), _lib.ptr(ws),
                                            0 if ws is None else ws.numel(), _lib.stream(x2)),
               what)
    return q, s


def quantize_weight_fp8(w: torch.Tensor, per_channel: bool = False):
    """Static weight quantisation of FP8Linear.__init__ (fp8_linear.py:17-22):
    per tensor -> (q [N,K], 0-dim fp32 scale); per channel -> (q, [N] scales).
    w is bf16, fp16 or fp32; the scale and the quotient are evaluated in w's
    type, as eager torch evaluates the reference's expressions."""
    _lib.require_gpu(w)
    dt = _lib.dtype_code(w, "weight")
    w = w.contiguous()
    N, K = w.shape
    q = torch.empty((N, K), dtype=torch.float8_e4m3fn, device=w.device)
    s = torch.empty(N if per_channel else 1, dtype=torch.float32, device=w.device)
    if w.numel():
        mode = _lib.SCALE_ROW if per_channel else _lib.SCALE_TENSOR
        ws = _workspace(w, N, K, mode)
        _lib.check(_lib.lib().fvsr_quant_weight_fp8_dt(w.data_ptr(), dt, N, K, mode,
                                                       q.data_ptr(), s.data_ptr(), _lib.ptr(ws),
                                                       0 if ws is None else ws.numel(),
                                                       _lib.stream(w)), "quantize_weight_fp8")
    return q, (s if per_channel else s.reshape(()))
