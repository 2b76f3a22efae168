"""Benchmark of the MI355X FlashVSR DiT-block operator pack.

    python bench.py [--gpus 1] [--steps K] [--warmup W] [--no-cpu-baseline]

Workload (one "step"): BASELINE C5, one streaming chunk at the 1408x768
FlashVSR-Tiny shape through the 30-block DiT stack: 16896 tokens
(4 latent frames x 48 x 88), dim 1536, 12 heads x 128, FFN 8960,
random-init weights ~N(0, 0.02) quantised to e4m3 per output channel,
per-token activation scales, block-sparse attention with the C4 mask
(~30% of the 132x132 block grid).  Inputs are resident in HBM before the
timed region.  ``value`` is ms per DiT layer (block); lower is better.

Alongside it the JSON line carries
  roofline      the dominant kernel of the step, timed with HIP events on the
                stream it runs on during the timed steps, against MI355X peak;
  graph_ms_per_step  the same chunk captured once as a HIP graph and
                replayed (checked bitwise against the eager output first);
  components    op-level measurements at the other BASELINE configs
                (C1 FP8 linear, C2 RMSNorm+RoPE, C3 AdaLN + FP8 FFN, C4 BSA),
                inputs rotated over > 512 MB so the 256 MB MALL cannot serve them;
  cpu_baseline  the reference path's PyTorch eager chain (oracle/eager.py)
                running one DiT block of the same workload on this machine's
                host cores.

    python bench.py --blaslt          torch._scaled_mm (hipBLASLt) at the same
                                      GEMM shapes, for comparison
    python bench.py --mfma-from CSV   MFMA utilisation from a rocprofv3 --pmc
                                      run over the MFMA counters
"""
from __future__ import annotations

import argparse
import json
import math
import os
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path[:0] = [ROOT, os.path.join(ROOT, "flashvsr-sm89-ops_amd")]

METRIC = "FP8 GEMM TFLOP/s, fused-op HBM GB/s, BSA ms/layer @1408×768; % roofline"
PEAK = {"fp8": 5.0e15, "bf16": 2.5e15, "hbm": 8.0e12}
F, H, W = 4, 48, 88            # latent frames x height x width at 1408x768
L = F * H * W                  # 16896 tokens
DIM, HEADS, HD, FFN = 1536, 12, 128, 8960


def log(msg):
    print(f"[bench] {msg}", file=sys.stderr, flush=True)


class EventTimer:
    """Events recorded on the current stream at hook points; durations by name."""

    def __init__(self, torch, only=None):
        self.torch, self.only = torch, only
        self.marks = []

    def __call__(self, name):
        if self.only is not None and name != self.only and not (
                self.marks and self.marks[-1][0] == self.only and self.marks[-1][2]):
            return
        ev = self.torch.cuda.Event(enable_timing=True)
        ev.record()
        self.marks.append((name, ev, name == self.only))

    def durations(self):
        out = {}
        for (n0, e0, _), (n1, e1, _) in zip(self.marks, self.marks[1:]):
            if self.only is not None and n0 != self.only:
                continue
            out.setdefault(n0, []).append(e0.elapsed_time(e1))
        return out


def block_costs():
    """Algorithmic work per DiT block (per launch of each op)."""
    gem = {
        "gemm_qkv": 2 * L * DIM * 3 * DIM,
        "gemm_o": 2 * L * DIM * DIM,
        "gemm_ffn0": 2 * L * DIM * FFN,
        "gemm_ffn2": 2 * L * FFN * DIM,
    }
    return gem


def run_stack(args, torch, fv):
    from flashvsr_sm89_ops.block import DiTStack
    from flashvsr_sm89_ops.lcsa import block_index
    from flashvsr_sm89_ops.lcsa.masks import window_plus_random_mask
    from flashvsr_sm89_ops.rope import wan_freqs_cis

    dev = "cuda"
    log(f"building {args.blocks}-block stack (random weights, e4m3 per channel)")
    stack = DiTStack(args.blocks, DIM, HEADS, FFN, device=dev, seed=0)
    g = torch.Generator().manual_seed(1)
    x = torch.randn(1, L, DIM, generator=g).to(torch.bfloat16).to(dev)
    t_mod = (0.1 * torch.randn(1, 6, DIM, generator=g)).to(torch.bfloat16).to(dev)
    cs = torch.view_as_real(wan_freqs_cis(F, H, W, HD).reshape(L, HD // 2)).to(dev)
    keep = window_plus_random_mask(HEADS, 2, 6, 11, 7, 10, seed=7, device=dev)
    kept = int(keep.sum().item())
    index = block_index(keep)
    tmap = (F, H, W)     # the attention computes the (2, 8, 8) window order of this grid
    torch.cuda.synchronize()

    # Per-op breakdown (untimed pass) to find the dominant kernel.
    for _ in range(args.warmup):
        y = stack(x, t_mod, cs, index, tmap)
    # One hooked pass first: the first pass that records events has a one-off
    # host stall (~15 ms) that would be charged to whichever op it falls in.
    stack(x, t_mod, cs, index, tmap, hook=EventTimer(torch))
    torch.cuda.synchronize()
    prof = EventTimer(torch)
    stack(x, t_mod, cs, index, tmap, hook=prof)
    torch.cuda.synchronize()
    per_op = {k: sum(v) for k, v in prof.durations().items()}
    dominant = max(per_op, key=per_op.get)
    log("per-op ms per chunk: " + ", ".join(f"{k}={v:.3f}" for k, v in per_op.items()))

    # Timed region: K steps; events only around the dominant kernel.
    dom = EventTimer(torch, only=dominant)
    torch.cuda.synchronize()
    t0 = torch.cuda.Event(enable_timing=True)
    t1 = torch.cuda.Event(enable_timing=True)
    wall0 = time.perf_counter()
    t0.record()
    for _ in range(args.steps):
        y = stack(x, t_mod, cs, index, tmap, hook=dom)
    t1.record()
    torch.cuda.synchronize()
    wall = time.perf_counter() - wall0
    ms_step = t0.elapsed_time(t1) / args.steps
    assert torch.isfinite(y.float()).all()
    dom_ms = dom.durations()[dominant]
    dom_avg = sum(dom_ms) / len(dom_ms)
    log(f"timed {args.steps} steps: {ms_step:.3f} ms/step (wall {wall:.2f}s); "
        f"dominant {dominant}: {dom_avg:.4f} ms avg over {len(dom_ms)} launches")
    # The same chunk captured once as a HIP graph and replayed (the kernels
    # are identical; what goes is the host work and launch gaps between them).
    # Reported beside the eager figure, not as the line's value.
    graph_ms = None
    try:
        xs = x.clone()
        side = torch.cuda.Stream()
        side.wait_stream(torch.cuda.current_stream())
        with torch.cuda.stream(side):
            stack(xs, t_mod, cs, index, tmap)
        torch.cuda.current_stream().wait_stream(side)
        torch.cuda.synchronize()
        graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(graph):
            yg = stack(xs, t_mod, cs, index, tmap)
        graph.replay()
        torch.cuda.synchronize()
        if not torch.equal(yg, y):
            raise RuntimeError("graph replay differs from the eager chunk")
        g0, g1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        g0.record()
        for _ in range(args.steps):
            graph.replay()
        g1.record()
        torch.cuda.synchronize()
        graph_ms = g0.elapsed_time(g1) / args.steps
        log(f"graph replay: {graph_ms:.3f} ms/step")
        del graph, yg, xs
    except Exception as exc:  # the eager figure stands on its own
        log(f"graph replay unavailable: {exc}")
    return dict(ms_step=ms_step, per_op=per_op, dominant=dominant, dom_avg=dom_avg,
                kept=kept, density=kept / (HEADS * 132 * 132), graph_ms=graph_ms)


def roofline_for(name, avg_ms, kept):
    costs = block_costs()
    if name in costs:
        ach = costs[name] / (avg_ms * 1e-3)
        return {"kernel": name, "bound": "mfma", "achieved": ach / 1e12, "peak": PEAK["fp8"] / 1e12,
                "unit": "TFLOP/s", "frac": ach / PEAK["fp8"],
                "work_per_launch": f"{costs[name] / 1e9:.1f} GFLOP (2*M*N*K)"}
    if name == "bsa":
        fl = 4 * 128 ** 3 * kept
        ach = fl / (avg_ms * 1e-3)
        return {"kernel": name, "bound": "mfma", "achieved": ach / 1e12, "peak": PEAK["bf16"] / 1e12,
                "unit": "TFLOP/s", "frac": ach / PEAK["bf16"],
                "work_per_launch": f"{fl / 1e9:.1f} GFLOP (4*128^3 per kept block, {kept} blocks)"}
    return {"kernel": name, "bound": "hbm", "achieved": None, "peak": PEAK["hbm"] / 1e9,
            "unit": "GB/s", "frac": None}


def timeit(torch, fn, n_sets, iters=20, warmup=3):
    """Average ms per call, cycling through n_sets input sets."""
    for i in range(warmup):
        fn(i % n_sets)
    torch.cuda.synchronize()
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    e0.record()
    for i in range(iters):
        fn(i % n_sets)
    e1.record()
    torch.cuda.synchronize()
    return e0.elapsed_time(e1) / iters


def gtime(torch, fn, n_sets, iters=20, replays=3):
    """Device-only ms per call: `iters` calls (cycling through the input sets)
    captured in one HIP graph and replayed, so no host work sits between the
    kernels (the ops used here allocate nothing outside torch's graph pool and
    issue no memsets).  None if the capture fails."""
    try:
        side = torch.cuda.Stream()
        side.wait_stream(torch.cuda.current_stream())
        with torch.cuda.stream(side):
            for i in range(3):
                fn(i % n_sets)
        torch.cuda.current_stream().wait_stream(side)
        torch.cuda.synchronize()
        graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(graph):
            for i in range(iters):
                fn(i % n_sets)
        graph.replay()
        torch.cuda.synchronize()
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        e0.record()
        for _ in range(replays):
            graph.replay()
        e1.record()
        torch.cuda.synchronize()
        del graph
        return e0.elapsed_time(e1) / (replays * iters)
    except Exception as exc:  # a capture problem must not end the bench
        print(f"[bench] graph timing unavailable: {exc}", file=sys.stderr, flush=True)
        return None


def n_sets_for(bytes_per_set, target=640e6):
    return max(2, int(math.ceil(target / bytes_per_set)))


def components(torch, fv):
    from flashvsr_sm89_ops.fp8_ffn import gemm_gelu_quant_fp8
    from flashvsr_sm89_ops.lcsa.hip_lcsa import block_sparse_attention_bhsd
    from flashvsr_sm89_ops.lcsa.masks import window_plus_random_mask
    from flashvsr_sm89_ops.rope import wan_freqs_cis
    from flashvsr_sm89_ops import _lib
    from types import SimpleNamespace

    dev = "cuda"
    g = torch.Generator(device=dev).manual_seed(0)
    out = {}

    def randn(*s, std=1.0):
        return (torch.randn(*s, generator=g, device=dev) * std).to(torch.bfloat16)

    def gbs(nbytes, ms):
        return nbytes / (ms * 1e-3) / 1e9

    # C1: FP8 linear [4224,1536] x [1536,1536]^T, per-token x, per-channel W.
    M, K, N = 4224, 1536, 1536
    ns = n_sets_for(M * K * 2)
    xs = [randn(M, K) for _ in range(ns)]
    w8, ws = fv.quantize_weight_fp8(randn(N, K, std=0.02), per_channel=True)
    bias = torch.zeros(N, dtype=torch.bfloat16, device=dev)
    q = [fv.quantize_fp8(x, per_token=True) for x in xs]
    t_q = timeit(torch, lambda i: fv.quantize_fp8(xs[i], per_token=True), ns)
    t_g = timeit(torch, lambda i: fv.fp8_gemm(q[i][0], q[i][1], w8, ws, bias), ns)
    k_q = gtime(torch, lambda i: fv.quantize_fp8(xs[i], per_token=True), ns)
    k_g = gtime(torch, lambda i: fv.fp8_gemm(q[i][0], q[i][1], w8, ws, bias), ns)
    qbytes = M * K * 3 + M * 4
    out["C1_fp8_linear"] = {
        "quant_ms": t_q, "quant_GBps": gbs(qbytes, t_q), "quant_frac_hbm": gbs(qbytes, t_q) * 1e9 / PEAK["hbm"],
        "quant_kernel_ms": k_q,
        "quant_kernel_frac_hbm": gbs(qbytes, k_q) * 1e9 / PEAK["hbm"] if k_q else None,
        "gemm_kernel_ms": k_g,
        "gemm_ms": t_g, "gemm_TFLOPs": 2 * M * N * K / (t_g * 1e-3) / 1e12,
        "gemm_frac_fp8": 2 * M * N * K / (t_g * 1e-3) / PEAK["fp8"]}
    del xs, q

    # C2: RMSNorm + RoPE on q and k [1, 8448, 1536], Wan 3-D freqs (2, 48, 88).
    L2 = 2 * 48 * 88
    nbytes = 4 * L2 * DIM * 2 + 2 * DIM * 2 + L2 * 64 * 8
    ns = n_sets_for(nbytes)
    qs = [randn(1, L2, DIM) for _ in range(ns)]
    ks = [randn(1, L2, DIM) for _ in range(ns)]
    wq, wk = (1 + 0.1 * torch.randn(DIM, device=dev, generator=g)).to(torch.bfloat16), \
        (1 + 0.1 * torch.randn(DIM, device=dev, generator=g)).to(torch.bfloat16)
    fc = wan_freqs_cis(2, 48, 88, device=dev)
    t = timeit(torch, lambda i: fv.fused_rms_rope_qk(qs[i], ks[i], wq, wk, fc), ns)
    kt = gtime(torch, lambda i: fv.fused_rms_rope_qk(qs[i], ks[i], wq, wk, fc), ns)
    out["C2_rms_rope_qk"] = {"ms": t, "GBps": gbs(nbytes, t), "frac_hbm": gbs(nbytes, t) * 1e9 / PEAK["hbm"],
                             "kernel_ms": kt,
                             "kernel_frac_hbm": gbs(nbytes, kt) * 1e9 / PEAK["hbm"] if kt else None,
                             "algorithmic_MB": nbytes / 1e6}
    del qs, ks

    # C3: AdaLN + FP8 FFN at M = 16896.
    M3 = L
    mod = (0.1 * torch.randn(1, 6, DIM, generator=g, device=dev)).to(torch.bfloat16)
    sh, sc, gt = mod[:, 3:4].contiguous(), mod[:, 4:5].contiguous(), mod[:, 5:6].contiguous()
    ns = n_sets_for(M3 * DIM * 2)
    xs = [randn(1, M3, DIM) for _ in range(ns)]
    t_ln = timeit(torch, lambda i: fv.fused_ln_modulate_quant(xs[i], sc, sh), ns)
    ln_bytes = M3 * DIM * 3 + M3 * 4 + 2 * DIM * 2
    t_lnb = timeit(torch, lambda i: fv.fused_ln_modulate(xs[i], sc, sh), ns)
    lnb_bytes = M3 * DIM * 4 + 2 * DIM * 2
    w1, s1 = fv.quantize_weight_fp8(randn(FFN, DIM, std=0.02), per_channel=True)
    w2, s2 = fv.quantize_weight_fp8(randn(DIM, FFN, std=0.02), per_channel=True)
    b1 = torch.zeros(FFN, dtype=torch.bfloat16, device=dev)
    b2 = torch.zeros(DIM, dtype=torch.bfloat16, device=dev)
    lin1 = SimpleNamespace(weight=w1, w_scale=s1, bias=b1)
    # GEMM inputs rotated past the MALL: ffn0 reads 26 MB of codes per call
    # (its 303 MB output alone exceeds the MALL), ffn2 151 MB.
    x8s = [fv.fused_ln_modulate_quant(xs[i % ns], sc, sh) for i in range(n_sets_for(M3 * DIM))]
    nx = len(x8s)
    hb = torch.empty((M3, FFN), dtype=torch.bfloat16, device=dev)
    t_g1 = timeit(torch, lambda i: fv.fp8_gemm(x8s[i % nx][0], x8s[i % nx][1], w1, s1, b1, out=hb), nx)
    nh = n_sets_for(M3 * FFN * 2)
    hs_ = [fv.fp8_gemm(x8s[i % nx][0], x8s[i % nx][1], w1, s1, b1) for i in range(nh)]
    t_rq = timeit(torch, lambda i: fv.fused_gelu_quant_fp8(hs_[i % nh], per_token=True), nh)
    rq_bytes = M3 * FFN * 3 + M3 * 4
    hqs = [fv.fused_gelu_quant_fp8(hs_[i], per_token=True) for i in range(min(nh, 5))]
    hqs_src = hs_[:3]
    del hs_
    nq = len(hqs)
    res = xs[0].view(M3, DIM)
    o2 = torch.empty((M3, DIM), dtype=torch.bfloat16, device=dev)
    t_g2 = timeit(torch, lambda i: fv.fp8_gemm(hqs[i % nq][0], hqs[i % nq][1], w2, s2, b2, out=o2), nq)
    t_g2g = timeit(torch, lambda i: fv.fp8_gemm(hqs[i % nq][0], hqs[i % nq][1], w2, s2, b2, out=o2,
                                                epilogue=_lib.EPI_GATE_ADD, res=res,
                                                gate=gt.view(DIM)), nq)
    t_ga = timeit(torch, lambda i: fv.fused_gate_add(xs[i], gt, xs[(i + 1) % ns]), ns)
    ga_bytes = M3 * DIM * 6 + DIM * 2
    from flashvsr_sm89_ops.fused_adaln import fused_gate_add_ln_modulate_quant
    t_gal = timeit(torch, lambda i: fused_gate_add_ln_modulate_quant(
        xs[i], gt, xs[(i + 1) % ns], sc, sh), ns)
    gal_bytes = M3 * DIM * (2 + 2 + 2 + 1) + M3 * 4 + 4 * DIM * 2
    t_ffn = timeit(torch, lambda i: (lambda h8: fv.fp8_gemm(h8[0], h8[1], w2, s2, b2))(
        gemm_gelu_quant_fp8(x8s[i % nx][0], x8s[i % nx][1], lin1, True)), nx)
    fl = 2 * M3 * DIM * FFN
    # device-only times of the row kernels (graph replays, no host work)
    k3 = {"ln_modulate_quant": (gtime(torch, lambda i: fv.fused_ln_modulate_quant(xs[i], sc, sh), ns),
                                ln_bytes),
          "gelu_quant": (gtime(torch, lambda i: fv.fused_gelu_quant_fp8(hqs_src[i % len(hqs_src)],
                                                                        per_token=True),
                               len(hqs_src)), rq_bytes),
          "gate_add": (gtime(torch, lambda i: fv.fused_gate_add(xs[i], gt, xs[(i + 1) % ns]), ns),
                       ga_bytes),
          "gate_add_ln_modulate_quant": (gtime(torch, lambda i: fused_gate_add_ln_modulate_quant(
              xs[i], gt, xs[(i + 1) % ns], sc, sh), ns), gal_bytes)}
    out["C3_adaln_fp8_ffn"] = {
        "ln_modulate_quant_ms": t_ln, "ln_modulate_quant_GBps": gbs(ln_bytes, t_ln),
        "ln_modulate_quant_frac_hbm": gbs(ln_bytes, t_ln) * 1e9 / PEAK["hbm"],
        "ln_modulate_bf16_ms": t_lnb, "ln_modulate_bf16_GBps": gbs(lnb_bytes, t_lnb),
        "gemm_ffn0_ms": t_g1, "gemm_ffn0_TFLOPs": fl / (t_g1 * 1e-3) / 1e12,
        "gemm_ffn0_frac_fp8": fl / (t_g1 * 1e-3) / PEAK["fp8"],
        "gelu_quant_ms": t_rq, "gelu_quant_GBps": gbs(rq_bytes, t_rq),
        "gemm_ffn2_ms": t_g2, "gemm_ffn2_TFLOPs": fl / (t_g2 * 1e-3) / 1e12,
        "gemm_ffn2_frac_fp8": fl / (t_g2 * 1e-3) / PEAK["fp8"],
        "gemm_ffn2_gate_epilogue_ms": t_g2g,
        "gemm_ffn0_kernel_ms": gtime(torch, lambda i: fv.fp8_gemm(
            x8s[i % nx][0], x8s[i % nx][1], w1, s1, b1, out=hb), nx),
        "gemm_ffn2_kernel_ms": gtime(torch, lambda i: fv.fp8_gemm(
            hqs[i % nq][0], hqs[i % nq][1], w2, s2, b2, out=o2), nq),
        "gate_add_ms": t_ga, "gate_add_GBps": gbs(ga_bytes, t_ga),
        "gate_add_frac_hbm": gbs(ga_bytes, t_ga) * 1e9 / PEAK["hbm"],
        "gate_add_ln_modulate_quant_ms": t_gal,
        "gate_add_ln_modulate_quant_GBps": gbs(gal_bytes, t_gal),
        "gate_add_ln_modulate_quant_frac_hbm": gbs(gal_bytes, t_gal) * 1e9 / PEAK["hbm"],
        "ffn_chain_ms": t_ffn}
    for name, (kt, nb) in k3.items():
        out["C3_adaln_fp8_ffn"][name + "_kernel_ms"] = kt
        out["C3_adaln_fp8_ffn"][name + "_kernel_frac_hbm"] = (gbs(nb, kt) * 1e9 / PEAK["hbm"]
                                                              if kt else None)
    del xs, x8s, hqs, hb, hqs_src

    # C4: block-sparse attention [1,12,16896,128], C4 mask, plus a density sweep;
    # q/k/v rotated over 4 sets (623 MB > the 256 MB MALL).
    ns4 = n_sets_for(3 * HEADS * L * HD * 2)
    qkvs = [[randn(1, HEADS, L, HD) for _ in range(3)] for _ in range(ns4)]
    qkv = qkvs[0]
    keep = window_plus_random_mask(device=dev)
    kept = int(keep.sum().item())
    t4 = timeit(torch, lambda i: block_sparse_attention_bhsd(*qkvs[i], keep), ns4, iters=12)
    k4 = gtime(torch, lambda i: block_sparse_attention_bhsd(*qkvs[i], keep), ns4, iters=12)
    fl4 = 4 * 128 ** 3 * kept
    sweep = []
    from flashvsr_sm89_ops.lcsa.masks import density_mask
    for d in (0.1, 0.2, 0.3, 0.5, 0.75, 1.0):
        km = density_mask(HEADS, 132, 132, d, seed=11, device=dev)
        kk = int(km.sum().item())
        td = timeit(torch, lambda i: block_sparse_attention_bhsd(*qkvs[i], km), ns4, iters=8)
        sweep.append({"density": kk / (HEADS * 132 * 132), "ms": td,
                      "TFLOPs": 4 * 128 ** 3 * kk / (td * 1e-3) / 1e12})
    out["C4_bsa"] = {"ms_per_layer": t4, "density": kept / (HEADS * 132 * 132), "input_sets": ns4,
                     "TFLOPs": fl4 / (t4 * 1e-3) / 1e12, "frac_bf16": fl4 / (t4 * 1e-3) / PEAK["bf16"],
                     "kernel_ms": k4,
                     "kernel_frac_bf16": fl4 / (k4 * 1e-3) / PEAK["bf16"] if k4 else None,
                     "density_sweep": sweep}
    del qkv, qkvs

    # Draft block mask + block index at the C5 geometry: q, k raster [16896, 1536]
    # read through the window token map, local range 7 on the 6x11 block grid,
    # 2 time rows, top-k 30% of a time row's 66 x 132 scores.
    from flashvsr_sm89_ops.block import window_token_map
    from flashvsr_sm89_ops.lcsa.masks import local_block_mask
    NB = L // 128
    ns = n_sets_for(2 * L * DIM * 2)
    qd = [randn(L, DIM) for _ in range(ns)]
    kd = [randn(L, DIM) for _ in range(ns)]
    tm = window_token_map(4, 48, 88, device=dev)
    loc = torch.from_numpy(local_block_mask(6, 11, 7)).to(dev, torch.uint8)
    topk = int(0.3 * 66 * NB)
    sel = torch.empty((HEADS, NB, NB), dtype=torch.int32, device=dev)
    cnt = torch.empty((HEADS, NB), dtype=torch.int32, device=dev)
    Ld = _lib.lib()
    wn = Ld.fvsr_draft_workspace_floats(HEADS, HD, NB, NB)
    wsd = torch.empty(wn, dtype=torch.float32, device=dev)

    def draft(i):
        st = _lib.stream(wsd)  # the current stream at call time (graph capture uses its own)
        _lib.check(Ld.fvsr_draft_block_mask(
            qd[i].data_ptr(), DIM, tm.data_ptr(), kd[i].data_ptr(), DIM, tm.data_ptr(), HEADS, HD,
            NB, NB, 2, loc.data_ptr(), 66, 66, topk, None, sel.data_ptr(), cnt.data_ptr(),
            wsd.data_ptr(), wn, st), "draft")
    t_d = timeit(torch, draft, ns, iters=50)
    k_d = gtime(torch, draft, ns, iters=50)
    pool_bytes = 2 * L * DIM * 2
    out["F1_draft_index"] = {"ms": t_d, "kernel_ms": k_d, "pool_MB": pool_bytes / 1e6,
                             "GBps_pool_bytes": gbs(pool_bytes, t_d),
                             "kept_frac": float(cnt.sum().item()) / (HEADS * NB * NB)}
    del qd, kd

    # F2: the self-attention's layout work at the C5 geometry for one streaming
    # step with a KV cache of 2 time rows (132 windows): the reference's
    # sequence (RMSNorm+RoPE of q and of k, WindowPartition3D of q/k/v,
    # torch.cat with the cache, reverse of the attention output) against the
    # fused pass (cache copied into the K/V buffer, fvsr_rms_rope_qkv_rows).
    from flashvsr_sm89_ops.fused_rms_rope import fused_rms_rope, fused_rms_rope_qkv_rows
    f2, h2, w2 = 4, 48, 88
    ncw = NB
    ns = n_sets_for(4 * L * DIM * 2)
    sets = [[randn(1, L, DIM) for _ in range(4)] for _ in range(ns)]
    ck, cv = randn(ncw, 128, DIM), randn(ncw, 128, DIM)
    wq2, wk2 = randn(DIM, std=0.1) + 1, randn(DIM, std=0.1) + 1
    fr2 = wan_freqs_cis(f2, h2, w2, HD).to(dev)
    inv = torch.empty_like(tm)
    inv[tm.long()] = torch.arange(L, dtype=torch.int32, device=dev)
    kvr = (inv + ncw * 128).contiguous()

    def part(t):
        return t.view(1, f2 // 2, 2, h2 // 8, 8, w2 // 8, 8, DIM).permute(
            0, 1, 3, 5, 2, 4, 6, 7).reshape(-1, 128, DIM)

    def rev(t):
        return t.view(1, f2 // 2, h2 // 8, w2 // 8, 2, 8, 8, DIM).permute(
            0, 1, 4, 2, 5, 3, 6, 7).reshape(1, L, DIM)

    def layout_ref(i):
        q, k, v, o = sets[i]
        qq = fused_rms_rope(q, wq2, fr2, head_dim=HD)
        kk = fused_rms_rope(k, wk2, fr2, head_dim=HD)
        qw, kw, vw = part(qq), part(kk), part(v)
        kw = torch.cat([ck, kw], dim=0)
        vw = torch.cat([cv, vw], dim=0)
        return rev(o.view(-1, 128, DIM)), qw, kw, vw

    def layout_f2(i):
        q, k, v, _ = sets[i]
        kb = torch.empty((ncw * 128 + L, DIM), dtype=torch.bfloat16, device=dev)
        vb = torch.empty_like(kb)
        kb[:ncw * 128].copy_(ck.view(-1, DIM))
        vb[:ncw * 128].copy_(cv.view(-1, DIM))
        fused_rms_rope_qkv_rows(q, k, v, wq2, wk2, fr2, kb, vb, kvr, head_dim=HD)
        return kb, vb
    # Steady streaming state: the cache is the store's own view, so the new
    # chunk is appended behind it in place (no copy of the cache).
    kst = torch.empty((ncw * 128 + L, DIM), dtype=torch.bfloat16, device=dev)
    vst = torch.empty_like(kst)

    def layout_f2_append(i):
        q, k, v, _ = sets[i]
        fused_rms_rope_qkv_rows(q, k, v, wq2, wk2, fr2, kst, vst, kvr, head_dim=HD)
    t_lr = timeit(torch, layout_ref, ns)
    t_lf = timeit(torch, layout_f2, ns)
    t_la = timeit(torch, layout_f2_append, ns)
    out["F2_window_layout"] = {"reference_sequence_ms": t_lr, "fused_with_cache_copy_ms": t_lf,
                               "fused_appended_ms": t_la,
                               "saved_ms_per_block": t_lr - t_la,
                               "saved_ms_per_chunk_30_blocks": 30 * (t_lr - t_la),
                               "cache_windows": ncw}
    del sets, ck, cv

    # F3: x + cross_attn(norm3(x)) at the C5 shape, prompt K/V of 512 tokens
    # (LayerNorm+quant, FP8 q, RMSNorm, dense attention, quant, FP8 o + residual).
    from flashvsr_sm89_ops.block import DiTBlockWeights
    from flashvsr_sm89_ops.cross_attn import cross_attention, cross_attention_residual
    LK = 512
    c = DiTBlockWeights(DIM, FFN, dev, torch.Generator().manual_seed(1), cross_len=LK).cross
    ns = n_sets_for(L * DIM * 2)
    xs = [randn(1, L, DIM) for _ in range(ns)]
    t_x = timeit(torch, lambda i: cross_attention_residual(
        xs[i], c["norm3_w"], c["norm3_b"], c["q"], c["norm_q"], c["k"], c["v"], c["o"], HEADS), ns)
    t_a = timeit(torch, lambda i: cross_attention(xs[i], c["k"], c["v"], HEADS), ns)
    att_out = torch.empty((1, L, DIM), dtype=torch.bfloat16, device=dev)
    k_a = gtime(torch, lambda i: cross_attention(xs[i], c["k"], c["v"], HEADS, out=att_out), ns)
    fl_a = 4 * L * LK * DIM
    fl_g = 2 * 2 * L * DIM * DIM
    out["F3_cross_attn"] = {"ms": t_x, "prompt_tokens": LK, "attn_ms": t_a,
                            "attn_TFLOPs": fl_a / (t_a * 1e-3) / 1e12,
                            "attn_frac_bf16": fl_a / (t_a * 1e-3) / PEAK["bf16"],
                            "attn_kernel_ms": k_a,
                            "attn_kernel_frac_bf16":
                                fl_a / (k_a * 1e-3) / PEAK["bf16"] if k_a else None,
                            "gemm_GFLOP": fl_g / 1e9, "attn_GFLOP": fl_a / 1e9}
    del xs
    out["enable_block_step"] = enable_block_step(torch, fv, dev, per_token=True)
    out["enable_block_step_per_tensor"] = enable_block_step(torch, fv, dev, per_token=False)
    return out


def enable_block_step(torch, fv, dev, per_token=True):
    """One DiT block through the forwards enable() installs, one streaming step
    at the C5 geometry (f=2, 48x88 latent, cache of 2 time rows), FP8 q/k/v/o
    and FFN per token x per channel (or per tensor, the reference's default),
    draft top-k 30%: the fused dataflow
    (FS89_WINDOW=1) against the reference's (FS89_WINDOW=0).  The
    cross-attention is a stand-in returning a fixed tensor (F3 is timed above)."""
    import types
    from flashvsr_sm89_ops import integrate
    from flashvsr_sm89_ops.fp8_ffn import FP8FFN
    from flashvsr_sm89_ops.fp8_linear import FP8Linear
    from flashvsr_sm89_ops.lcsa.draft import generate_draft_block_mask
    from flashvsr_sm89_ops.lcsa.masks import local_block_mask
    from flashvsr_sm89_ops.rope import wan_freqs_cis
    from flashvsr_sm89_ops.compat_bsa import _hip_block_sparse_attn_func
    g = torch.Generator().manual_seed(3)
    f2, h2, w2 = 2, 48, 88
    Ls = f2 * h2 * w2

    def lin(n, k):
        m = torch.nn.Linear(k, n, dtype=torch.bfloat16)
        with torch.no_grad():
            m.weight.copy_(torch.randn(n, k, generator=g) * 0.02)
            m.bias.zero_()
        return FP8Linear(m.to(dev), per_channel=per_token, per_token=per_token)

    def part(x, win):
        B, f, h, w, C = x.shape
        return x.view(B, f // 2, 2, h // 8, 8, w // 8, 8, C).permute(
            0, 1, 3, 5, 2, 4, 6, 7).reshape(-1, 128, C)

    def rev(x, win, fhw):
        f, h, w = fhw
        C = x.shape[-1]
        return x.view(1, f // 2, h // 8, w // 8, 2, 8, 8, C).permute(
            0, 1, 4, 2, 5, 3, 6, 7).reshape(1, f, h, w, C)

    loc = torch.from_numpy(local_block_mask(6, 11, 7)).to(dev)

    class SelfAttention(torch.nn.Module):
        def forward(self, x, freqs, f=None, h=None, w=None, local_num=None, topk=None,
                    train_img=False, block_id=None, kv_len=None, is_full_block=False,
                    is_stream=False, pre_cache_k=None, pre_cache_v=None, local_range=9):
            raise AssertionError

        def attn(self, q, k, v, mask):
            return _hip_block_sparse_attn_func(
                q[0].view(-1, HEADS, HD), k[0].view(-1, HEADS, HD), v[0].view(-1, HEADS, HD),
                None, None, None, None, mask, q.shape[1], k.shape[1]).reshape(1, -1, DIM)

    class CrossAttention(torch.nn.Module):
        def forward(self, x, y, is_stream=False):
            raise AssertionError

    class DiTBlock(torch.nn.Module):
        def forward(self, x, context, t_mod, freqs, f, h, w, local_num=None, topk=None,
                    train_img=False, block_id=None, kv_len=None, is_full_block=False,
                    is_stream=False, pre_cache_k=None, pre_cache_v=None, local_range=9):
            raise AssertionError

    dit = types.SimpleNamespace(
        SelfAttention=SelfAttention, CrossAttention=CrossAttention, DiTBlock=DiTBlock,
        WindowPartition3D=types.SimpleNamespace(partition=part, reverse=rev),
        build_local_block_mask_shifted_vec_normal_slide=lambda *a, **k: loc,
        generate_draft_block_mask=generate_draft_block_mask, modulate=None)

    class Pipe:
        model = torch.nn.Module()

        def denoising_model(self):
            return self.model
    env0 = {k: os.environ.get(k) for k in ("FS89_FP8", "FS89_DRAFT", "FS89_WINDOW")}
    os.environ["FS89_FP8"], os.environ["FS89_DRAFT"] = "", "1"
    fv.enable(Pipe(), dit_module=dit, verbose=False)
    blk = DiTBlock()
    sa = blk.self_attn = SelfAttention()
    sa.num_heads, sa.head_dim = HEADS, HD
    for n in ("q", "k", "v", "o"):
        setattr(sa, n, lin(DIM, DIM))
    nw = torch.nn.Module()
    nw.weight = torch.nn.Parameter((1 + 0.1 * torch.randn(DIM, generator=g)).to(torch.bfloat16).to(dev))
    nw.eps = 1e-6
    sa.norm_q = sa.norm_k = nw
    sa.local_attn_mask = None
    sa.local_attn_mask_h = sa.local_attn_mask_w = sa.local_range = None
    blk.modulation = (0.1 * torch.randn(1, 6, DIM, generator=g)).to(torch.bfloat16).to(dev)
    blk.norm1 = torch.nn.LayerNorm(DIM, eps=1e-6, elementwise_affine=False)
    blk.norm2 = torch.nn.LayerNorm(DIM, eps=1e-6, elementwise_affine=False)
    blk.norm3 = torch.nn.LayerNorm(DIM, eps=1e-6, dtype=torch.bfloat16).to(dev)
    blk.ffn = FP8FFN(lin(FFN, DIM), lin(DIM, FFN))
    yc = (0.1 * torch.randn(1, Ls, DIM, generator=g)).to(torch.bfloat16).to(dev)
    blk.cross_attn = lambda x, ctx, is_stream=False: yc
    t_mod = (0.1 * torch.randn(1, 6, DIM, generator=g)).to(torch.bfloat16).to(dev)
    fr = wan_freqs_cis(f2, h2, w2, HD).to(dev)
    topk = int(0.3 * 66 * 3 * 66)
    xs = [(torch.randn(1, Ls, DIM, generator=g)).to(torch.bfloat16).to(dev) for _ in range(2)]
    res = {}
    for mode in ("0", "1"):
        os.environ["FS89_WINDOW"] = mode
        sa._fs89_kv = None
        ck = (torch.randn(2 * 66, 128, DIM, generator=g)).to(torch.bfloat16).to(dev)
        cv = ck.clone()
        state = {"ck": ck, "cv": cv}

        def step(i):
            with torch.no_grad():
                _, state["ck"], state["cv"] = blk(
                    xs[i], None, t_mod, fr, f2, h2, w2, None, topk, kv_len=2, is_stream=True,
                    pre_cache_k=state["ck"], pre_cache_v=state["cv"])
        res[mode] = timeit(torch, step, 2, iters=10)
    for k, v in env0.items():
        if v is None:
            os.environ.pop(k, None)
        else:
            os.environ[k] = v
    return {"reference_dataflow_ms": res["0"], "fused_ms": res["1"],
            "saved_ms_per_chunk_30_blocks": 30 * (res["0"] - res["1"]),
            "geometry": "f=2, 48x88 latent, 132-window cache, top-k 30% of 3 time rows"}


def cpu_model() -> str:
    try:
        with open("/proc/cpuinfo") as fh:
            for line in fh:
                if line.startswith("model name"):
                    return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return "unknown"


def cpu_baseline(args):
    """One DiT block of the C5 workload as the reference's PyTorch eager chain
    on the host cores (oracle/eager.py: F.layer_norm, eager e4m3 quantisation,
    fp32 dequant matmuls, upstream RMSNorm + complex RoPE, the per-block
    sparse attention loop, F.gelu) with the same weights' codes and the C4
    block mask."""
    import numpy as np
    import torch
    from oracle import oracle as O
    from oracle.eager import dit_block_eager, q_weight

    threads = int(os.environ.get("OMP_NUM_THREADS", os.cpu_count() or 1))
    torch.set_num_threads(threads)
    g = torch.Generator().manual_seed(0)

    def lin(n, k):
        w8, s = q_weight((torch.randn(n, k, generator=g) * 0.02).to(torch.bfloat16), True)
        return w8, s, torch.zeros(n, dtype=torch.bfloat16)

    P = {n: lin(DIM, DIM) for n in "qkvo"}
    P["ffn0"], P["ffn2"] = lin(FFN, DIM), lin(DIM, FFN)
    P["norm_q"] = P["norm_k"] = (1 + 0.1 * torch.randn(DIM, generator=g)).to(torch.bfloat16)
    x = torch.randn(L, DIM, generator=g).to(torch.bfloat16)
    mod = (0.1 * torch.randn(6, DIM, generator=g)).to(torch.bfloat16)
    cos, sin = O.wan_rope_cos_sin(F, H, W)
    freqs = torch.complex(torch.from_numpy(cos), torch.from_numpy(sin)).to(torch.complex128)
    keep = O.c4_block_mask()
    times = []
    for _ in range(4):  # one warm-up, then the median of 3
        t0 = time.perf_counter()
        y, _, _ = dit_block_eager(x, mod, P, (F, H, W), keep, freqs, HEADS, 1e-6, True,
                                  acc=torch.float32, sparse=True)
        times.append(time.perf_counter() - t0)
        assert torch.isfinite(y.float()).all()
    dt = sorted(times[1:])[1]
    return {"value": dt * 1e3, "unit": "ms/layer", "cores": threads, "kind": "port",
            "cpu": cpu_model(),
            "sample": "1 of the 30 DiT blocks of the C5 chunk (16896 tokens, C4 mask ~30%): the "
                      "reference path's PyTorch eager chain (oracle/eager.py, fp32 dequant "
                      "matmuls, per-block sparse attention); one warm-up, median of 3 wall "
                      "times on the host cores"}


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=10)
    ap.add_argument("--warmup", type=int, default=3)
    ap.add_argument("--blocks", type=int, default=30)
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--no-components", action="store_true")
    ap.add_argument("--copy-probe-mib", type=int, default=0,
                    help="first run a float32 negation over this many MiB (read + write), the "
                         "known-size kernel that calibrates FETCH_SIZE / WRITE_SIZE counters")
    ap.add_argument("--traffic-from", nargs=2, metavar=("FETCH_CSV", "WRITE_CSV"),
                    help="summarise two rocprofv3 --pmc counter_collection.csv files "
                         "(FETCH_SIZE, WRITE_SIZE) of a --copy-probe-mib run into JSON and exit")
    ap.add_argument("--mfma-from", metavar="CSV",
                    help="summarise a rocprofv3 --pmc counter_collection.csv of the MFMA "
                         "counters (" + " ".join(MFMA_COUNTERS) + ") into JSON and exit")
    ap.add_argument("--blaslt", action="store_true",
                    help="time torch._scaled_mm (hipBLASLt) at the BASELINE GEMM shapes and exit")
    ap.add_argument("--ktrace-from", metavar="CSV",
                    help="summarise a rocprofv3 --kernel-trace kernel_trace.csv per kernel and "
                         "grid size (the GEMM shapes share one kernel name) as a markdown table "
                         "and exit")
    args = ap.parse_args()
    if args.ktrace_from:
        print(summarize_ktrace(args.ktrace_from))
        return
    if args.traffic_from:
        print(json.dumps(summarize_traffic(*args.traffic_from, args.copy_probe_mib), indent=1))
        return
    if args.mfma_from:
        print(json.dumps(summarize_mfma(args.mfma_from), indent=1))
        return
    if args.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) != 1:
        print("bench.py: this operator pack runs on one GPU; multi-GPU runs are not part of "
              "this build (the row-local ops shard by tokens, attention by heads).", file=sys.stderr)
        sys.exit(2)

    import torch
    import flashvsr_sm89_ops as fv
    from flashvsr_sm89_ops import _lib

    log(f"{_lib.version()} on {torch.cuda.get_device_name(0)}")
    if args.blaslt:
        for r in blaslt_same_box(torch):
            print(json.dumps(r), flush=True)
        return
    if args.copy_probe_mib:
        n = args.copy_probe_mib * (1 << 20) // 4
        src = torch.ones(n, dtype=torch.float32, device="cuda")
        dst = torch.empty_like(src)
        for _ in range(3):
            torch.neg(src, out=dst)
        torch.cuda.synchronize()
        del src, dst
    r = run_stack(args, torch, fv)
    roof = roofline_for(r["dominant"], r["dom_avg"], r["kept"])
    roof["traffic"] = load_traffic(r["dominant"])
    comps = {} if args.no_components else components(torch, fv)
    comps["C5_per_op_ms_per_chunk"] = r["per_op"]
    cpu = None if args.no_cpu_baseline else cpu_baseline(args)
    ms_layer = r["ms_step"] / args.blocks
    line = {
        "metric": METRIC, "value": ms_layer, "unit": "ms/layer", "n_gpus": 1,
        "steps": args.steps, "warmup": args.warmup, "ms_per_step": r["ms_step"],
        "higher_is_better": False, "scaling": "weak", "vs_baseline": None,
        "dtype": "e4m3+bf16", "data": "synthetic",
        "config": {"workload": f"C5: {args.blocks}-block FlashVSR-Tiny DiT stack, one chunk @1408x768",
                   "tokens": L, "dim": DIM, "heads": HEADS, "head_dim": HD, "ffn": FFN,
                   "blocks": args.blocks, "bsa_density": r["density"], "scales": "per-token x per-channel"},
        "roofline": roof, "cpu_baseline": cpu,
        "graph_ms_per_step": r["graph_ms"],
        "components": comps,
    }
    print(json.dumps(line), flush=True)


# op -> (kernel name fragment, grid size in threads or None) for each op of the
# C5 stack whose dispatches can be told apart in a counter file.  qkv, o and
# ffn0 share one GEMM kernel and differ by persistent grid (qkv 240 workgroups,
# o 200, ffn0 232); ffn2 (K = 8960) runs the variant with the L2 prefetch.
OP_KERNELS = {
    "ln_modulate_quant": ("ln_modulate_row<false, true, false>", None),
    "gemm_qkv": ("gemm_fp8_ring<0, true, 4, false>", 240 * 256),
    "rms_rope_qk": ("rms_rope_qk_vec", None),
    "bsa": ("bsa_fwd_kernel<2, 2, false>", None),
    "quant_attn": ("quant_rows_vec<3, false>", None),
    "gemm_o": ("gemm_fp8_ring<0, true, 4, false>", 200 * 256),
    "gate_add_ln_modulate_quant": ("ln_modulate_row<false, true, true>", None),
    "gemm_ffn0": ("gemm_fp8_ring<0, true, 4, false>", 232 * 256),
    "gelu_quant": ("quant_rows_gelu_table", None),
    "gemm_ffn2": ("gemm_fp8_ring<0, true, 4, true>", 200 * 256),
    "gate_add": ("gate_add_vec", None),
}


def summarize_traffic(fetch_csv, write_csv, copy_mib):
    """HBM bytes per dispatch from two rocprofv3 --pmc runs of
    ``bench.py --copy-probe-mib N --blocks 1 ...``: FETCH_SIZE and WRITE_SIZE
    (KiB per dispatch) averaged per kernel and scaled by the factor that makes
    the probe's negation over N MiB read and write exactly N MiB."""
    import csv

    def per_kernel(path, counter):
        acc = {}
        with open(path) as fh:
            for row in csv.DictReader(fh):
                if row["Counter_Name"] != counter:
                    continue
                key = (row["Kernel_Name"], int(row.get("Grid_Size") or 0))
                d = acc.setdefault(key, {})
                d[row["Dispatch_Id"]] = d.get(row["Dispatch_Id"], 0.0) + float(row["Counter_Value"])
        return {k: sum(v.values()) / len(v) for k, v in acc.items()}

    fetch, write = per_kernel(fetch_csv, "FETCH_SIZE"), per_kernel(write_csv, "WRITE_SIZE")
    probe = [k for k in fetch if "neg" in k[0].lower()]
    if not probe or copy_mib <= 0:
        raise SystemExit("no calibration kernel (run with --copy-probe-mib)")
    want = copy_mib * 1024.0
    f_fac = want / (sum(fetch[k] for k in probe) / len(probe))
    w_fac = want / (sum(write[k] for k in probe) / len(probe))
    out = {"calibration": {"kernel": probe[0][0][:120], "bytes": copy_mib << 20,
                           "fetch_factor": f_fac, "write_factor": w_fac}}
    for op, (frag, grid) in OP_KERNELS.items():
        keys = [k for k in fetch if frag in k[0] and (grid is None or k[1] == grid)]
        if len(keys) != 1 or keys[0] not in write:
            continue
        fb, wb = fetch[keys[0]] * 1024 * f_fac, write[keys[0]] * 1024 * w_fac
        out[op] = {"kernel": keys[0][0][:120], "fetch_bytes": fb, "write_bytes": wb,
                   "traffic": fb + wb}
    return out


MFMA_COUNTERS = ("SQ_VALU_MFMA_BUSY_CYCLES", "SQ_INSTS_VALU_MFMA_MOPS_F8",
                 "SQ_INSTS_VALU_MFMA_MOPS_BF16", "GRBM_GUI_ACTIVE")
MFMA_KERNELS = {"gemm_fp8": "gemm_fp8", "bsa": "bsa_fwd_kernel"}


def summarize_ktrace(csv_path, top=24):
    """Per (kernel, workgroups) dispatch count and duration statistics of a
    rocprofv3 kernel_trace.csv, largest total time first, as markdown."""
    import csv
    groups = {}
    with open(csv_path) as fh:
        for r in csv.DictReader(fh):
            wg = int(r["Grid_Size_X"]) // max(1, int(r["Workgroup_Size_X"]))
            name = r["Kernel_Name"].replace("(anonymous namespace)::", "")
            name = name[5:] if name.startswith("void ") else name
            key = (name.split("(")[0][:90], wg)
            groups.setdefault(key, []).append((int(r["End_Timestamp"]) - int(r["Start_Timestamp"])) / 1e3)
    total = sum(sum(v) for v in groups.values())
    rows = sorted(groups.items(), key=lambda kv: -sum(kv[1]))[:top]
    out = ["| kernel | workgroups | calls | avg us | median us | min us | max us | % time |",
           "|---|---:|---:|---:|---:|---:|---:|---:|"]
    for (name, wg), d in rows:
        d = sorted(d)
        out.append(f"| `{name}` | {wg} | {len(d)} | {sum(d) / len(d):.1f} | {d[len(d) // 2]:.1f} | "
                   f"{d[0]:.1f} | {d[-1]:.1f} | {100 * sum(d) / total:.2f} |")
    return "\n".join(out)


def summarize_mfma(csv_path, simds=1024, xcds=8):
    """MFMA utilisation per kernel from one rocprofv3 --pmc pass over
    MFMA_COUNTERS: busy = SQ_VALU_MFMA_BUSY_CYCLES summed over the SIMDs,
    divided by (GPU-active cycles x SIMDs); GRBM_GUI_ACTIVE in the file is the
    sum over the XCDs, so one XCD's active cycles are that over ``xcds``.
    MOPS x 512 = the flops the matrix cores executed, against 2MNK /
    4*128^3*blocks; the clock implied by the active cycles and the dispatch's
    duration is reported as a check of that reading."""
    import csv
    acc = {}
    with open(csv_path) as fh:
        for row in csv.DictReader(fh):
            name = row["Kernel_Name"]
            op = next((k for k, frag in MFMA_KERNELS.items() if frag in name), None)
            if op is None:
                continue
            d = acc.setdefault((op, name[:100], row["Dispatch_Id"]), {})
            d[row["Counter_Name"]] = d.get(row["Counter_Name"], 0.0) + float(row["Counter_Value"])
            d["ns"] = float(row["End_Timestamp"]) - float(row["Start_Timestamp"])
    out = {}
    for (op, name, _), d in acc.items():
        e = out.setdefault(op + " | " + name, {"dispatches": 0, "busy": 0.0, "active": 0.0,
                                                "mops_f8": 0.0, "mops_bf16": 0.0, "ns": 0.0})
        e["dispatches"] += 1
        e["busy"] += d.get("SQ_VALU_MFMA_BUSY_CYCLES", 0.0)
        e["active"] += d.get("GRBM_GUI_ACTIVE", 0.0) / xcds
        e["mops_f8"] += d.get("SQ_INSTS_VALU_MFMA_MOPS_F8", 0.0)
        e["mops_bf16"] += d.get("SQ_INSTS_VALU_MFMA_MOPS_BF16", 0.0)
        e["ns"] += d["ns"]
    res = {}
    for k, e in out.items():
        n = e["dispatches"]
        res[k] = {"dispatches": n, "mfma_busy_frac": e["busy"] / (e["active"] * simds),
                  "mfma_flop_per_dispatch": (e["mops_f8"] + e["mops_bf16"]) * 512 / n,
                  "avg_us": e["ns"] / n / 1e3, "implied_GHz": e["active"] / e["ns"]}
    return res


def blaslt_same_box(torch):
    """torch._scaled_mm (hipBLASLt) against fvsr_fp8_gemm on the same operands
    the bench's components feed the GEMMs: per-token e4m3 codes of
    LayerNorm-modulated rows (C1: of N(0,1) rows) for qkv, o, ffn0 and C1,
    GELU-requantised codes of ffn0's output for ffn2, per-channel weight codes
    of N(0, 0.02) weights, row-wise scales and a bias.  Input sets rotate past
    the 256 MB MALL and the two libraries are timed alternately, twice each
    (the better of the two runs is reported), on the same stream."""
    from flashvsr_sm89_ops import fp8_gemm, fused_gelu_quant_fp8, fused_ln_modulate_quant, \
        quantize_fp8, quantize_weight_fp8
    dev = "cuda"
    g = torch.Generator(device=dev).manual_seed(5)

    def randn(*s, std=1.0):
        return (torch.randn(*s, generator=g, device=dev) * std).to(torch.bfloat16)

    mod = (0.1 * torch.randn(1, 6, DIM, generator=g, device=dev)).to(torch.bfloat16)
    sh, sc = mod[:, 3:4].contiguous(), mod[:, 4:5].contiguous()

    def ln_codes(M, K, n):
        return [fused_ln_modulate_quant(randn(1, M, K), sc[..., :K].contiguous(),
                                        sh[..., :K].contiguous()) for _ in range(n)]

    rows = []
    shapes = [("C1", 4224, 1536, 1536), ("qkv", L, 3 * DIM, DIM), ("o", L, DIM, DIM),
              ("ffn0", L, FFN, DIM), ("ffn2", L, DIM, FFN)]
    w1 = None
    for name, M, N, K in shapes:
        w8, ws = quantize_weight_fp8(randn(N, K, std=0.02), per_channel=True)
        bias = randn(N, std=0.02)
        n = n_sets_for(M * K + M * N * 2)
        if name == "C1":
            xs = [quantize_fp8(randn(M, K), per_token=True) for _ in range(n)]
        elif name == "ffn2":
            src = ln_codes(M, DIM, 2)
            xs = []
            for i in range(n):
                h = fp8_gemm(src[i % 2][0], src[i % 2][1], w1[0], w1[1], w1[2])
                xs.append(fused_gelu_quant_fp8(h, per_token=True))
                del h
        else:
            xs = ln_codes(M, K, n)
        if name == "ffn0":
            w1 = (w8, ws, bias)
        outs = [torch.empty((M, N), dtype=torch.bfloat16, device=dev) for _ in range(2)]
        sb_row = ws.reshape(1, N).contiguous()
        sa_rows = [x[1].reshape(M, 1).contiguous() for x in xs]

        def ours(i):
            fp8_gemm(xs[i][0], xs[i][1], w8, ws, bias, out=outs[0])

        use_bias = True

        def theirs(i):
            return torch._scaled_mm(xs[i][0], w8.t(), scale_a=sa_rows[i], scale_b=sb_row,
                                    bias=bias if use_bias else None, out_dtype=torch.bfloat16)
        try:
            theirs(0)
        except RuntimeError:
            use_bias = False       # row-wise scales with a bias unsupported: time without
        t_ours, t_theirs = [], []
        for _ in range(2):
            t_ours.append(timeit(torch, ours, n, iters=20))
            t_theirs.append(timeit(torch, theirs, n, iters=20))
        ours(0)
        ref = theirs(0)
        torch.cuda.synchronize()
        diff = (outs[0].float() - ref.float()).abs()
        flop = 2 * M * N * K
        rows.append({"gemm": name, "M": M, "N": N, "K": K, "scales": "row x channel",
                     "bias_in_blaslt": use_bias,
                     "fvsr_us": min(t_ours) * 1e3, "blaslt_us": min(t_theirs) * 1e3,
                     "fvsr_TFLOPs": flop / (min(t_ours) * 1e-3) / 1e12,
                     "blaslt_TFLOPs": flop / (min(t_theirs) * 1e-3) / 1e12,
                     "max_abs_diff": float(diff.max()),
                     "frac_bitwise_equal": float((diff == 0).float().mean()) if use_bias else None,
                     "input_sets": n})
        del xs, outs, ref
    return rows


def load_traffic(op):
    """HBM bytes per launch of ``op``'s kernel from the committed rocprofv3
    counter summary (profiles/traffic.json), or None."""
    p = os.path.join(ROOT, "profiles", "traffic.json")
    try:
        with open(p) as fh:
            ent = json.load(fh).get(op)
    except (OSError, ValueError):
        return None
    return None if ent is None else ent["traffic"]


if __name__ == "__main__":
    main()
