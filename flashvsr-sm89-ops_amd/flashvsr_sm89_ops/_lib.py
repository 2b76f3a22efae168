"""ctypes binding of libfvsr.so, the gfx950 kernels behind a C ABI.

The library is loaded on first use.  There is no fallback: if the shared
library is missing, or a tensor is not on a HIP device, the op raises.  All
launches go on torch's current stream of the tensor's device; the C side never
allocates and never synchronises.
"""
from __future__ import annotations

import ctypes
import os
import threading

import torch

_HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.environ.get("FVSR_LIB", os.path.join(_HERE, "libfvsr.so"))

FVSR_OK, FVSR_EINVAL, FVSR_EHIP, FVSR_EUNSUPPORTED, FVSR_EWORKSPACE = 0, -1, -2, -3, -4
SCALE_TENSOR, SCALE_ROW = 0, 1
EPI_BIAS, EPI_ROWMAX, EPI_GATE_ADD = 0, 1, 2
DT_BF16, DT_F16, DT_F32 = 0, 1, 2
_DT = {torch.bfloat16: DT_BF16, torch.float16: DT_F16, torch.float32: DT_F32}

_ERR = {
    FVSR_EINVAL: "invalid argument",
    FVSR_EHIP: "HIP launch error",
    FVSR_EUNSUPPORTED: "unsupported shape/stride/alignment",
    FVSR_EWORKSPACE: "workspace too small",
}

_P = ctypes.c_void_p
_I64 = ctypes.c_int64
_I = ctypes.c_int
_F = ctypes.c_float

_SIGS = {
    "fvsr_version": ([], ctypes.c_char_p),
    "fvsr_quant_workspace_floats": ([_I64, _I64, _I], _I64),
    "fvsr_quant_fp8": ([_P, _I64, _I64, _I64, _I, _I, _P, _P, _P, _I64, _P], _I),
    "fvsr_quant_fp8_noalloc": ([_P, _I64, _I64, _I64, _I, _I, _P, _P, _P], _I),
    "fvsr_gelu_quant_fp8_tensor": ([_P, _I64, _I64, _P, _I64, _P, _P, _P, _I64, _P], _I),
    "fvsr_quant_weight_fp8": ([_P, _I64, _I64, _I, _P, _P, _P, _I64, _P], _I),
    "fvsr_quant_fp8_dt": ([_P, _I, _I64, _I64, _I64, _I, _I, _P, _P, _P, _I64, _P], _I),
    "fvsr_quant_weight_fp8_dt": ([_P, _I, _I64, _I64, _I, _P, _P, _P, _I64, _P], _I),
    "fvsr_ln_modulate_dt": ([_P, _I, _P, _I, _P, _I, _P, _I64, _I64, _I64, _F, _P], _I),
    "fvsr_gate_add_dt": ([_P, _I, _P, _I, _P, _I, _P, _I64, _I64, _I64, _P], _I),
    "fvsr_rms_rope_dt": ([_P, _I, _P, _I, _P, _P, _I64, _I64, _I64, _I64, _F, _I, _P], _I),
    "fvsr_fp8_gemm": ([_P, _I64, _P, _I, _P, _I64, _P, _I, _P, _P, _I64, _I64, _I64, _I64, _I,
                       _P, _P, _P, _P], _I),
    "fvsr_gemm_amax_parts": ([_I64], _I64),
    "fvsr_ln_modulate": ([_P, _P, _P, _P, _I64, _I64, _I64, _F, _P, _P, _P], _I),
    "fvsr_gate_add": ([_P, _P, _P, _P, _I64, _I64, _I64, _P], _I),
    "fvsr_layer_norm": ([_P, _P, _P, _P, _I64, _I64, _F, _P, _P, _P], _I),
    "fvsr_gate_add_ln_modulate": ([_P, _P, _P, _P, _P, _P, _P, _I64, _I64, _I64, _F, _P, _P, _P],
                                  _I),
    "fvsr_gate_add_layer_norm": ([_P, _P, _P, _P, _P, _P, _P, _I64, _I64, _I64, _F, _P, _P, _P],
                                 _I),
    "fvsr_rms_rope": ([_P, _P, _P, _P, _I64, _I64, _I64, _I64, _F, _I, _P], _I),
    "fvsr_rms_rope_qk": ([_P, _P, _P, _P, _P, _P, _P, _I64, _I64, _I64, _I64, _F, _I64, _I64,
                          _P], _I),
    "fvsr_rms_rope_qkv_rows": ([_P, _P, _P, _P, _P, _P, _P, _P, _P, _P, _I64, _I64, _I64, _I64,
                                _I64, _F, _I64, _I64, _I64, _P], _I),
    "fvsr_block_index": ([_P, _I64, _I64, _I64, _P, _P, _P], _I),
    "fvsr_draft_workspace_floats": ([_I64, _I64, _I64, _I64], _I64),
    "fvsr_draft_block_mask": ([_P, _I64, _P, _P, _I64, _P, _I64, _I64, _I64, _I64, _I64, _P,
                               _I64, _I64, _I64, _P, _P, _P, _P, _I64, _P], _I),
    "fvsr_bsa_fwd": ([_P, _P, _P, _P, _I64, _I64, _I64, _I64, _I64, _I64, _P, _P, _I64, _I64,
                      _I64, _I64, _I64, _F, _P, _P, _P], _I),
    "fvsr_attn_dense": ([_P, _P, _P, _P, _I64, _I64, _I64, _I64, _I64, _I64, _I64, _I64, _I64,
                         _I64, _F, _P], _I),
    "fvsr_bsa_fwd_window": ([_P, _P, _P, _P, _I64, _I64, _I64, _I64, _I64, _I64, _P, _P, _I64,
                             _I64, _I64, _I64, _I64, _F, _I64, _I64, _I64, _I, _P], _I),
}

_lib = None
_lock = threading.Lock()


def exported_symbols():
    """Names the C ABI exports (declared in include/fvsr.h)."""
    return tuple(_SIGS)


def lib():
    """Load libfvsr.so once; raise if it is missing (no fallback path exists)."""
    global _lib
    if _lib is None:
        with _lock:
            if _lib is None:
                if not os.path.exists(LIB_PATH):
                    raise RuntimeError(
                        f"flashvsr_sm89_ops: {LIB_PATH} is not built. Build it with "
                        "`python flashvsr-sm89-ops_amd/build.py` (hipcc, gfx950).")
                L = ctypes.CDLL(LIB_PATH)
                for name, (args, res) in _SIGS.items():
                    fn = getattr(L, name)
                    fn.argtypes = args
                    fn.restype = res
                _lib = L
    return _lib


def check(rc: int, what: str):
    if rc != FVSR_OK:
        raise RuntimeError(f"{what} failed: {_ERR.get(rc, rc)} (status {rc})")


def ptr(t) -> int | None:
    return None if t is None else t.data_ptr()


_raw_stream = getattr(torch._C, "_cuda_getCurrentRawStream", None)


def stream(t: torch.Tensor) -> int:
    """torch's current stream of t's device, as the raw handle the C ABI takes
    (without building a torch.cuda.Stream object per call)."""
    if _raw_stream is not None:
        return _raw_stream(t.device.index)
    return torch.cuda.current_stream(t.device).cuda_stream


def require_gpu(*ts):
    for t in ts:
        if t is not None and not t.is_cuda:
            raise RuntimeError(
                "flashvsr_sm89_ops kernels run on the GPU only (HIP/gfx950); got a tensor on "
                f"{t.device}")


def require_dtype(t: torch.Tensor, dtype, name: str):
    if t.dtype != dtype:
        raise TypeError(f"{name} must be {dtype}, got {t.dtype}")


def dtype_code(t: torch.Tensor, name: str) -> int:
    """FVSR_DT_* code of a floating tensor of the *_dt entry points: bf16,
    fp16 or fp32, the input types the reference's kernels load."""
    code = _DT.get(t.dtype)
    if code is None:
        raise TypeError(f"{name} must be bfloat16, float16 or float32, got {t.dtype}")
    return code


def version() -> str:
    return lib().fvsr_version().decode()
