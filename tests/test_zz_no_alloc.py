"""fvsr_quant_fp8_noalloc (the allocation-free entry point, library-owned
scratch) against fvsr_quant_fp8 (caller workspace), both through the C ABI:
codes and scales bit-identical, on two calls in a row (the second with a
smaller input, so stale partial maxima of the first would show), per tensor
with and without GELU, and per row."""
import numpy as np
import pytest
import torch

pytestmark = pytest.mark.gpu

DEV = "cuda"


def _both(L, x, mode, gelu):
    from flashvsr_sm89_ops import _lib
    M, K = x.shape
    st = torch.cuda.current_stream().cuda_stream
    out = []
    for entry in ("with_workspace", "noalloc"):
        q = torch.full((M, K), 0x55, dtype=torch.uint8, device=DEV)
        s = torch.full((M if mode else 1,), -1.0, dtype=torch.float32, device=DEV)
        if entry == "noalloc":
            rc = L.fvsr_quant_fp8_noalloc(x.data_ptr(), M, K, x.stride(0), mode, gelu,
                                          q.data_ptr(), s.data_ptr(), st)
        else:
            n = int(L.fvsr_quant_workspace_floats(M, K, mode))
            ws = torch.empty(max(n, 1), dtype=torch.float32, device=DEV)
            rc = L.fvsr_quant_fp8(x.data_ptr(), M, K, x.stride(0), mode, gelu, q.data_ptr(),
                                  s.data_ptr(), ws.data_ptr(), ws.numel(), st)
        assert rc == _lib.FVSR_OK, (entry, rc)
        out.append((q, s))
    torch.cuda.synchronize()
    return out


@pytest.mark.parametrize("mode,gelu", [(0, 0), (0, 1), (1, 0), (1, 1)])
def test_noalloc_matches_workspace_entry(mode, gelu):
    from flashvsr_sm89_ops import _lib
    L = _lib.lib()
    g = torch.Generator().manual_seed(40 + 2 * mode + gelu)
    # a large input (many partial maxima, a big amax), then a smaller one whose
    # amax is far below the first's: a partial left over from call 1 would
    # raise call 2's scale and change its codes
    big = (torch.randn(9000, 1536, generator=g) * 8).to(torch.bfloat16).to(DEV)
    small = (torch.randn(300, 1536, generator=g) * 0.5).to(torch.bfloat16).to(DEV)
    for x in (big, small):
        (q0, s0), (q1, s1) = _both(L, x, mode, gelu)
        assert torch.equal(q0, q1), f"codes differ for {tuple(x.shape)}"
        assert torch.equal(s0, s1), f"scales differ for {tuple(x.shape)}"
    # a strided input (a column slice, rows 2048 apart)
    wide = torch.randn(257, 2048, generator=g).to(torch.bfloat16).to(DEV)
    (q0, s0), (q1, s1) = _both(L, wide[:, 256:1792], mode, gelu)
    assert torch.equal(q0, q1) and torch.equal(s0, s1)


def test_noalloc_argument_checks():
    from flashvsr_sm89_ops import _lib
    L = _lib.lib()
    p = 16
    assert L.fvsr_quant_fp8_noalloc(p, 4, 8, 4, 0, 0, p, p, None) == _lib.FVSR_EINVAL  # ld < cols
    assert L.fvsr_quant_fp8_noalloc(p, 4, 8, 8, 7, 0, p, p, None) == _lib.FVSR_EINVAL  # mode
    assert L.fvsr_quant_fp8_noalloc(None, 0, 8, 8, 0, 0, None, None, None) == _lib.FVSR_OK
