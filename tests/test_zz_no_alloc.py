"""fvsr_quant_fp8_noalloc (the allocation-free entry point, library-owned
scratch) against fvsr_quant_fp8 (caller workspace), both through the C ABI:
codes and scales bit-identical, on two calls in a row (the second with a
smaller input, so stale partial maxima of the first would show), per tensor
with and without GELU, and per row; and captured in a HIP graph, replayed."""
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


def test_noalloc_in_graph_capture():
    """Captured in a HIP graph (torch.cuda.graph) and replayed: per tensor
    with and without GELU, and per row, each replay bit-identical to the
    workspace entry run eagerly on the same input, with eager work and a new
    input between replays.  This test comes first in the file so that, in a
    fresh process, the captured call is also the one that first resolves the
    library's device scratch address (no other test calls the entry point
    before it)."""
    from flashvsr_sm89_ops import _lib
    L = _lib.lib()
    g = torch.Generator().manual_seed(77)
    M, K = 3000, 1536
    inputs = [(torch.randn(M, K, generator=g) * sc).to(torch.bfloat16) for sc in (4.0, 0.25, 9.0)]
    x = inputs[0].to(DEV)
    cases = [(0, 0), (0, 1), (1, 0)]
    outs = [(torch.empty((M, K), dtype=torch.uint8, device=DEV),
             torch.empty((M if mode else 1,), dtype=torch.float32, device=DEV))
            for mode, _ in cases]
    graph = torch.cuda.CUDAGraph()
    rcs = []
    with torch.cuda.graph(graph):
        st = torch.cuda.current_stream().cuda_stream
        for (mode, gelu), (q, s) in zip(cases, outs):
            rcs.append(L.fvsr_quant_fp8_noalloc(x.data_ptr(), M, K, K, mode, gelu,
                                                q.data_ptr(), s.data_ptr(), st))
    assert rcs == [_lib.FVSR_OK] * len(cases), rcs
    for rep, host in enumerate(inputs + inputs[:1]):
        x.copy_(host.to(DEV))
        torch.cuda.synchronize()
        graph.replay()
        torch.cuda.synchronize()
        got = [(q.clone(), s.clone()) for q, s in outs]
        _ = (x.float() * 2).sum()          # eager work between replays
        for (mode, gelu), (q, s) in zip(cases, got):
            (q0, s0), _unused = _both(L, x, mode, gelu)
            assert torch.equal(q0, q), f"replay {rep}: codes differ (mode {mode}, gelu {gelu})"
            assert torch.equal(s0, s), f"replay {rep}: scales differ (mode {mode}, gelu {gelu})"


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
