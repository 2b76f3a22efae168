"""FP8 (e4m3fn) Linear on CDNA4 FP8 matrix cores.

`FP8Linear` mirrors the reference module (flashvsr_sm89_ops/fp8_linear.py:16-42):
the weight is quantised once at conversion (``.weight`` float8_e4m3fn [N, K],
``.w_scale`` fp32, ``.bias`` bf16 kept), activations are quantised on every
forward, and ``_mm(x8, s)`` is the scaled GEMM with bias and bf16 output.
The GEMM is the hand-written gfx950 kernel behind ``fvsr_fp8_gemm``.

Scale granularity is per tensor by default, as in the reference.
``per_channel=True`` quantises the weight per output channel and
``per_token=True`` the activations per row (the BASELINE configurations).

Weights and activations may be bf16, fp16 or fp32: the weight is quantised
with eager's arithmetic in its own type (reference fp8_linear.py:19-22) and
activations as the reference's quantisation kernel loads them (as fp32).  The
output is bf16 (``out_dtype=torch.bfloat16`` there); a bias of another type
is rounded to bf16 for the epilogue (torch._scaled_mm itself refuses a
non-bf16 bias with a bf16 output).
"""
from __future__ import annotations

import hashlib
import json
import re

import torch
import torch.nn as nn

from . import _lib
from .fp8_quant import FP8_MAX, quantize_fp8, quantize_weight_fp8  # noqa: F401


def _check_gemm_args(x8, s, w8, w_scale, bias, out, epilogue, amax_part, res, gate):
    """Operand checks of fp8_gemm: everything the kernel indexes must exist
    at the size it assumes."""
    _lib.require_dtype(x8, torch.float8_e4m3fn, "x8")
    _lib.require_dtype(w8, torch.float8_e4m3fn, "weight")
    if x8.dim() != 2 or w8.dim() != 2:
        raise ValueError(f"fp8_gemm: x8 and weight must be 2-D, got {tuple(x8.shape)} and "
                         f"{tuple(w8.shape)}")
    M, K = x8.shape
    N, K2 = w8.shape
    if K != K2:
        raise ValueError(f"fp8_gemm: K mismatch {K} vs {K2}")
    if s.numel() not in (1, M) or w_scale.numel() not in (1, N):
        raise ValueError("fp8_gemm: scale shapes must be per-tensor or per-row/column")
    if bias is not None and (bias.dim() != 1 or bias.numel() != N):
        raise ValueError(f"fp8_gemm: bias must be 1-D with N={N} elements, got "
                         f"{tuple(bias.shape)}")
    if epilogue not in (_lib.EPI_BIAS, _lib.EPI_ROWMAX, _lib.EPI_GATE_ADD):
        raise ValueError(f"fp8_gemm: unknown epilogue {epilogue}")
    if out is not None:
        _lib.require_dtype(out, torch.bfloat16, "out")
        if tuple(out.shape) != (M, N) or out.stride(1) != 1 or out.stride(0) < N:
            raise ValueError(f"fp8_gemm: out must be [{M}, {N}] with unit column stride, got "
                             f"shape {tuple(out.shape)} strides {out.stride()}")
    ldc = out.stride(0) if out is not None else N
    if epilogue == _lib.EPI_ROWMAX:
        need = M * int(_lib.lib().fvsr_gemm_amax_parts(N))
        if amax_part is None:
            raise ValueError("fp8_gemm: the row-max epilogue needs amax_part")
        _lib.require_dtype(amax_part, torch.float32, "amax_part")
        if not amax_part.is_contiguous() or amax_part.numel() < need:
            raise ValueError(f"fp8_gemm: amax_part needs {need} contiguous fp32 elements "
                             f"(M * ceil(N/128)), got {amax_part.numel()}")
    if epilogue == _lib.EPI_GATE_ADD:
        if res is None or gate is None:
            raise ValueError("fp8_gemm: the gate-add epilogue needs res and gate")
        _lib.require_dtype(res, torch.bfloat16, "res")
        _lib.require_dtype(gate, torch.bfloat16, "gate")
        if tuple(res.shape) != (M, N) or res.stride(1) != 1 or res.stride(0) != ldc:
            raise ValueError(f"fp8_gemm: res must be [{M}, {N}] with out's row stride {ldc}, "
                             f"got shape {tuple(res.shape)} strides {res.stride()}")
        if gate.numel() != N or not gate.is_contiguous():
            raise ValueError(f"fp8_gemm: gate must hold N={N} contiguous elements, got "
                             f"{tuple(gate.shape)}")


def fp8_gemm(x8: torch.Tensor, s: torch.Tensor, w8: torch.Tensor, w_scale: torch.Tensor,
             bias: torch.Tensor | None = None, out: torch.Tensor | None = None,
             epilogue: int = _lib.EPI_BIAS, amax_part: torch.Tensor | None = None,
             res: torch.Tensor | None = None, gate: torch.Tensor | None = None) -> torch.Tensor:
    """bf16(x8 @ w8.T * s * w_scale + bias): x8 [M,K] e4m3, w8 [N,K] e4m3,
    s [1]/[M]/[M,1] fp32, w_scale 0-dim/[1]/[N] fp32, bias [N] bf16 or None.

    ``out`` (optional) is [M, N] bf16 with unit column stride; epilogue
    EPI_ROWMAX needs ``amax_part`` fp32 with M * ceil(N/128) contiguous
    elements, EPI_GATE_ADD needs ``res`` [M, N] bf16 laid out like ``out``
    (same row stride) and ``gate`` [N] bf16.  Every size is checked here,
    before the launch, as torch._scaled_mm checks its operands (reference
    fp8_linear.py:28-30); a mismatch raises ValueError / TypeError."""
    _check_gemm_args(x8, s, w8, w_scale, bias, out, epilogue, amax_part, res, gate)
    _lib.require_gpu(x8, s, w8, w_scale, bias, out, amax_part, res, gate)
    M, K = x8.shape
    N = w8.shape[0]
    if x8.stride(1) != 1:
        x8 = x8.contiguous()
    if w8.stride(1) != 1:
        w8 = w8.contiguous()
    sa_mode = _lib.SCALE_ROW if s.numel() == M and M != 1 else _lib.SCALE_TENSOR
    sb_mode = _lib.SCALE_ROW if w_scale.numel() == N and N != 1 else _lib.SCALE_TENSOR
    s = s.float().contiguous()
    w_scale = w_scale.float().contiguous()
    if bias is not None:
        bias = bias.to(torch.bfloat16).contiguous()
    if out is None:
        out = torch.empty((M, N), dtype=torch.bfloat16, device=x8.device)
    rc = _lib.lib().fvsr_fp8_gemm(
        x8.data_ptr(), x8.stride(0), s.data_ptr(), sa_mode,
        w8.data_ptr(), w8.stride(0), w_scale.data_ptr(), sb_mode,
        _lib.ptr(bias), out.data_ptr(), out.stride(0), M, N, K, epilogue,
        _lib.ptr(amax_part), _lib.ptr(res), _lib.ptr(gate), _lib.stream(x8))
    _lib.check(rc, "fp8_gemm")
    return out


def quantize_input_fp8(x2: torch.Tensor, per_token: bool = False):
    """Activation quantisation as FP8Linear.forward / FP8FFN.forward do it
    (reference fp8_linear.py:35-40, fp8_ffn.py:88-92).  A contiguous [M, K]
    goes through quantize_fp8.  For any other layout the reference evaluates
    ``s = (x2.abs().amax() / 448).clamp(min=1e-12).float()`` and
    ``(x2 / s).to(e4m3)`` eagerly in x2's type, so the scale and x/s are each
    rounded to that type before the cast.  That is the expression of its
    per-tensor weight quantisation, so those codes come from the same kernel
    (on a contiguous copy).  Per-token scales (this build's extension) read
    strided rows directly."""
    if per_token or x2.is_contiguous():
        return quantize_fp8(x2, per_token=per_token)
    _lib.require_gpu(x2)
    return quantize_weight_fp8(x2.contiguous(), per_channel=False)


def source_fingerprint(weight: torch.Tensor, bias: torch.Tensor | None) -> str:
    """Checksum of the weights an FP8Linear is quantised from (shape, dtype and
    two wrapping int64 sums of the bit patterns, one position-weighted, for
    the weight and the bias), computed where the tensors live.  A stored FP8
    weight file records it per module so that codes are never applied to a
    model whose source weights differ."""
    parts = []
    for t in (weight, bias):
        if t is None:
            parts.append(None)
            continue
        t = t.detach().contiguous().reshape(-1)
        as_int = {1: torch.uint8, 2: torch.int16, 4: torch.int32, 8: torch.int64}[t.element_size()]
        v = t.view(as_int).to(torch.int64)
        pos = torch.arange(v.numel(), device=v.device, dtype=torch.int64)
        mix = (pos * 0x9E3779B1 + 0x7F4A7C15) & 0xFFFFFFFF
        parts.append((tuple(t.shape), str(t.dtype), int(v.sum()), int((v * mix).sum())))
    parts.insert(0, tuple(weight.shape))
    return hashlib.sha256(repr(parts).encode()).hexdigest()[:32]


class StoredFP8Weights(dict):
    """{module name: (codes uint8 [N, K], scales fp32, bias or None)} plus
    ``fingerprints`` {module name: source_fingerprint of the weights the codes
    were quantised from}."""

    def __init__(self, *a, fingerprints=None, **k):
        super().__init__(*a, **k)
        self.fingerprints = dict(fingerprints or {})


class FP8Linear(nn.Module):
    """Drop-in for the reference FP8Linear (fp8_linear.py:16-42)."""

    def __init__(self, linear: nn.Linear | None, per_channel: bool = False,
                 per_token: bool = False):
        super().__init__()
        self.per_channel = per_channel
        self.per_token = per_token
        if linear is None:  # filled by from_quantized
            return
        w = linear.weight.detach()
        q, s = quantize_weight_fp8(w, per_channel=per_channel)
        bias = linear.bias.detach().clone() if linear.bias is not None else None
        self._set(q, s, bias)

    def _set(self, weight8: torch.Tensor, w_scale: torch.Tensor, bias: torch.Tensor | None):
        self.w_scale = w_scale
        self.weight = nn.Parameter(weight8, requires_grad=False)
        self.bias = nn.Parameter(bias, requires_grad=False) if bias is not None else None
        self.out_features, self.in_features = weight8.shape

    @classmethod
    def from_quantized(cls, weight8: torch.Tensor, w_scale: torch.Tensor,
                       bias: torch.Tensor | None = None, per_token: bool = False) -> "FP8Linear":
        """An FP8Linear from stored codes (float8_e4m3fn, or their uint8 bit
        patterns) [N, K] and scales (0-dim / [1] per tensor, [N] per channel),
        without quantising again."""
        if weight8.dtype == torch.uint8:
            weight8 = weight8.view(torch.float8_e4m3fn)
        if weight8.dtype != torch.float8_e4m3fn or weight8.dim() != 2:
            raise ValueError("from_quantized: weight must be e4m3 codes [N, K]")
        N = weight8.shape[0]
        w_scale = w_scale.float()
        if w_scale.numel() not in (1, N):
            raise ValueError(f"from_quantized: {w_scale.numel()} scales for {N} output channels")
        if bias is not None and (bias.dim() != 1 or bias.numel() != N):
            raise ValueError(f"from_quantized: bias must be 1-D with {N} elements, got "
                             f"{tuple(bias.shape)}")
        if w_scale.numel() == 1:
            w_scale = w_scale.reshape(())  # the reference keeps a 0-dim per-tensor scale
        m = cls(None, per_channel=w_scale.numel() == N and N != 1, per_token=per_token)
        m._set(weight8.contiguous(), w_scale, bias)
        return m

    def _mm(self, x8, s, out=None):
        return fp8_gemm(x8, s, self.weight, self.w_scale, self.bias, out=out)

    def forward(self, x):
        shape = x.shape
        x8, s = quantize_input_fp8(x.reshape(-1, shape[-1]), self.per_token)
        y = self._mm(x8, s)
        return y.reshape(*shape[:-1], y.shape[-1])

    def extra_repr(self):
        g = "channel" if self.per_channel else "tensor"
        a = "token" if self.per_token else "tensor"
        return (f"in_features={self.in_features}, out_features={self.out_features}, "
                f"weight_scale=per-{g}, act_scale=per-{a}, bias={self.bias is not None}")


def convert_linears_fp8(model: nn.Module, parts=("ffn", "self", "cross"), per_channel: bool = False,
                        per_token: bool = False, stored: dict | None = None) -> int:
    """Convert DiT-block Linears whose module names match `parts`
    ("ffn" / "self" / "cross"); returns the number converted
    (fp8_linear.py:45-67).  Idempotent: FP8Linear is not an nn.Linear.
    ``stored`` (from load_fp8_weights) supplies saved codes and scales by
    module name; those modules are not quantised again, and when ``stored``
    carries fingerprints each must match the module's current weights."""
    allowed = []
    if "self" in parts:
        allowed.append(r"^blocks\.\d+\.self_attn\.[qkvo]$")
    if "cross" in parts:
        allowed.append(r"^blocks\.\d+\.cross_attn\.[qkvo]$")
    if "ffn" in parts:
        allowed.append(r"^blocks\.\d+\.ffn\.[02]$")
    pats = [re.compile(p) for p in allowed]
    n = 0
    for name, mod in list(model.named_modules()):
        if not isinstance(mod, nn.Linear) or not any(p.match(name) for p in pats):
            continue
        parent_name, _, leaf = name.rpartition(".")
        parent = model.get_submodule(parent_name) if parent_name else model
        fp = source_fingerprint(mod.weight, mod.bias)
        if stored is not None and name in stored:
            w8, ws, b = stored[name]
            if tuple(w8.shape) != tuple(mod.weight.shape):
                raise ValueError(f"stored FP8 weight for {name} has shape {tuple(w8.shape)}, "
                                 f"the module {tuple(mod.weight.shape)}")
            if (ws.numel() == w8.shape[0] and w8.shape[0] != 1) != per_channel:
                raise ValueError(f"stored FP8 weight for {name} has the other scale granularity")
            want = getattr(stored, "fingerprints", {}).get(name)
            if want is not None and want != fp:
                raise ValueError(f"stored FP8 weight for {name} was quantised from different "
                                 "weights than the module holds (source fingerprint mismatch); "
                                 "delete the file to quantise again")
            dev = mod.weight.device
            new = FP8Linear.from_quantized(w8.to(dev), ws.to(dev),
                                           b.to(dev) if b is not None else None, per_token)
        else:
            new = FP8Linear(mod, per_channel=per_channel, per_token=per_token)
        new.source_fingerprint = fp
        setattr(parent, leaf, new)
        n += 1
    return n


FP8_WEIGHTS_FORMAT = "flashvsr-fp8-weights/2"


class FP8WeightsFormatError(ValueError):
    """A weight file written by an earlier version of save_fp8_weights (an
    older ``flashvsr-fp8-weights/<n>`` format): its codes cannot be used
    as they are, but quantising again and overwriting it is safe."""


def save_fp8_weights(model: nn.Module, path: str) -> int:
    """Persist every FP8Linear of ``model`` (codes as uint8 bit patterns, fp32
    scales, bf16 biases, and in the metadata the fingerprint of the weights
    each was quantised from) to a safetensors file; returns the number saved.
    Reloading gives bit-identical modules without quantising again."""
    from safetensors.torch import save_file
    tensors, prints = {}, {}
    for name, mod in model.named_modules():
        if not isinstance(mod, FP8Linear):
            continue
        fp = getattr(mod, "source_fingerprint", None)
        if fp is None:
            raise ValueError(f"{name}: FP8Linear without a source fingerprint (made outside "
                             "convert_linears_fp8); cannot be saved as a weight file")
        prints[name] = fp
        tensors[f"{name}.weight"] = mod.weight.detach().view(torch.uint8).contiguous().cpu()
        tensors[f"{name}.w_scale"] = mod.w_scale.detach().float().reshape(-1).contiguous().cpu()
        if mod.bias is not None:
            tensors[f"{name}.bias"] = mod.bias.detach().contiguous().cpu()
    save_file(tensors, path, metadata={"format": FP8_WEIGHTS_FORMAT,
                                       "fingerprints": json.dumps(prints, sort_keys=True)})
    return len(prints)


def load_fp8_weights(path: str) -> StoredFP8Weights:
    """The contents of a file written by save_fp8_weights (CPU tensors;
    nothing is executed from the file), with the source fingerprints that
    convert_linears_fp8 checks against the model."""
    from safetensors import safe_open
    with safe_open(path, framework="pt", device="cpu") as f:
        meta = f.metadata() or {}
        fmt = meta.get("format") or ""
        if fmt != FP8_WEIGHTS_FORMAT:
            if fmt.startswith(FP8_WEIGHTS_FORMAT.split("/")[0] + "/"):
                raise FP8WeightsFormatError(f"{path}: {fmt} file, this version reads "
                                            f"{FP8_WEIGHTS_FORMAT}; delete it to quantise again")
            raise ValueError(f"{path}: not a {FP8_WEIGHTS_FORMAT} file")
        out = StoredFP8Weights(fingerprints=json.loads(meta.get("fingerprints", "{}")))
        keys = set(f.keys())
        for k in sorted(keys):
            if not k.endswith(".weight"):
                continue
            name = k[:-len(".weight")]
            if name not in out.fingerprints:
                raise ValueError(f"{path}: no source fingerprint for {name}")
            b = f.get_tensor(f"{name}.bias") if f"{name}.bias" in keys else None
            out[name] = (f.get_tensor(k), f.get_tensor(f"{name}.w_scale"), b)
    return out
