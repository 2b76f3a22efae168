"""HIP-graph capture of the operator pack.

The C ABI allocates nothing, never synchronises and records no memset, so a
whole DiT block -- AdaLN, the fused q/k/v GEMM, RMSNorm + RoPE, block-sparse
attention through the window token map, the O and FFN GEMMs with the GELU
requantisation and both gated residuals, with and without the cross-attention
residual -- can be captured into one graph (torch.cuda.CUDAGraph drives HIP
graph capture) and replayed.  Every replay is compared bitwise with the eager
result, with the program's own eager work and synchronisations between the
replays (a fill or memset node that misbehaved after its first replay, or a
kernel reading state left by an earlier launch, would show here).
"""
import numpy as np
import pytest
import torch

from oracle import oracle as O

pytestmark = pytest.mark.gpu

DEV = "cuda"


def _case(f, h, w, cross_len, seed):
    from flashvsr_sm89_ops.block import DiTBlockWeights, window_token_map
    from flashvsr_sm89_ops.lcsa import build_csr
    dim, heads, ffn = 1536, 12, 8960
    g = torch.Generator().manual_seed(seed)
    wts = DiTBlockWeights(dim, ffn, DEV, g, cross_len=cross_len)
    L = f * h * w
    x = torch.randn(1, L, dim, generator=g).to(torch.bfloat16).to(DEV)
    t_mod = (0.1 * torch.randn(1, 6, dim, generator=g)).to(torch.bfloat16).to(DEV)
    cos, sin = O.wan_rope_cos_sin(f, h, w)
    cs = torch.from_numpy(np.stack([cos, sin], -1)).to(DEV)
    nb = L // 128
    keep = O.random_block_mask(heads, nb, nb, 0.5, seed=seed + 1)
    index = build_csr(torch.from_numpy(keep).to(DEV))
    return wts, x, t_mod, cs, index, window_token_map(f, h, w, device=DEV), heads


def _capture(fn):
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        fn()  # warm-up on a side stream, as torch asks before a capture
    torch.cuda.current_stream().wait_stream(side)
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        out = fn()
    return graph, out


@pytest.mark.parametrize("cross_len", [0, 256])
def test_dit_block_graph_replays_match_eager(cross_len):
    from flashvsr_sm89_ops.block import dit_block_forward
    wts, x, t_mod, cs, index, tmap, heads = _case(2, 16, 24, cross_len, 11 + cross_len)
    xs = x.clone()  # the graph's static input
    eager = dit_block_forward(x, wts, t_mod, cs, index, tmap, heads)
    torch.cuda.synchronize()
    print(f"[graph] block cross_len={cross_len}: capture", flush=True)
    graph, out = _capture(lambda: dit_block_forward(xs, wts, t_mod, cs, index, tmap, heads))
    for r in range(3):
        out.fill_(0)  # eager work between the replays
        torch.cuda.synchronize()
        graph.replay()
        torch.cuda.synchronize()
        assert torch.equal(out, eager), f"replay {r} differs from the eager block"
    # a new input copied into the static buffer is picked up by the replay
    x2 = (x.float() * 0.5).to(torch.bfloat16)
    eager2 = dit_block_forward(x2, wts, t_mod, cs, index, tmap, heads)
    xs.copy_(x2)
    graph.replay()
    torch.cuda.synchronize()
    assert torch.equal(out, eager2)
    del graph


def test_dit_stack_graph_replays_match_eager():
    """Two fused blocks (the second's AdaLN fused with the first's last gated
    residual) captured as one graph."""
    from flashvsr_sm89_ops.block import DiTStack
    _, x, t_mod, cs, index, tmap, heads = _case(2, 16, 16, 0, 23)
    stack = DiTStack(2, 1536, heads, 8960, device=DEV, seed=5)
    xs = x.clone()
    eager = stack(x, t_mod, cs, index, tmap)
    torch.cuda.synchronize()
    print("[graph] 2-block stack: capture", flush=True)
    graph, out = _capture(lambda: stack(xs, t_mod, cs, index, tmap))
    for r in range(3):
        torch.cuda.synchronize()
        graph.replay()
        torch.cuda.synchronize()
        assert torch.equal(out, eager), f"replay {r} differs from the eager stack"
        eager_again = stack(x, t_mod, cs, index, tmap)  # eager run between replays
        torch.cuda.synchronize()
        assert torch.equal(eager_again, eager)
    del graph
