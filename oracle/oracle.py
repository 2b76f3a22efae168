"""CPU oracle for the FlashVSR DiT-block operator pack (numpy + the C helpers).

TEST INFRASTRUCTURE ONLY.  Only tests/, ``__graft_entry__.smoke()`` and
bench.py's ``cpu_baseline`` leg import this module, always as the checker;
the product package never does.

Every function restates one piece of the reference path
(aireet/flashvsr-sm89-ops, read-only) and cites the lines it follows.  Byte
exact pieces (e4m3 encoding, activation/weight quantisation, the tanh-GELU
used before requantisation) live in ``fvsr_oracle.c``; the floating-point
pieces are numpy float32/float64 with explicit bf16 rounding where eager
rounds.  How each function is pinned (golden vectors from torch CPU eager,
closed forms, brute force, invariants) is listed in tests/test_oracle.py.
"""
from __future__ import annotations

import ctypes
import math
import os
import subprocess

import numpy as np

_HERE = os.path.dirname(os.path.abspath(__file__))
_LIB_PATH = os.path.join(_HERE, "liboracle.so")
_lib = None

FP8_MAX = 448.0


def build(force: bool = False) -> str:
    """Compile fvsr_oracle.c into oracle/liboracle.so with gcc."""
    if force or not os.path.exists(_LIB_PATH):
        subprocess.check_call(["bash", os.path.join(_HERE, "build_oracle.sh")])
    return _LIB_PATH


def lib():
    global _lib
    if _lib is None:
        build()
        L = ctypes.CDLL(_LIB_PATH)
        P, I64 = ctypes.c_void_p, ctypes.c_int64
        L.orc_e4m3_encode.argtypes = [P, P, I64]
        L.orc_e4m3_decode.argtypes = [P, P, I64]
        L.orc_bf16_round.argtypes = [P, P, I64]
        L.orc_gelu_bf16.argtypes = [P, P, I64]
        L.orc_quant_rows.argtypes = [P, I64, I64, I64, ctypes.c_int, ctypes.c_int, P, P]
        L.orc_quant_weight.argtypes = [P, I64, I64, ctypes.c_int, P, P]
        L.orc_quant_rows_f32.argtypes = [P, I64, I64, I64, ctypes.c_int, ctypes.c_int, P, P]
        L.orc_quant_weight_f32.argtypes = [P, I64, I64, ctypes.c_int, ctypes.c_int, P, P]
        L.orc_f16_round.argtypes = [P, P, I64]
        L.orc_gelu_f32.argtypes = [P, P, I64]
        L.orc_expf.argtypes = [ctypes.c_float]
        L.orc_expf.restype = ctypes.c_float
        _lib = L
    return _lib


def _p(a: np.ndarray):
    assert a.flags["C_CONTIGUOUS"]
    return a.ctypes.data_as(ctypes.c_void_p)


# ----------------------------------------------------------------------------
# bf16 / e4m3 helpers
# ----------------------------------------------------------------------------

def bf16(x) -> np.ndarray:
    """Round float32 values to bf16 (RNE), returned as float32."""
    x = np.ascontiguousarray(x, dtype=np.float32)
    u = x.view(np.uint32)
    nan = (u & 0x7FFFFFFF) > 0x7F800000
    r = (u + np.uint32(0x7FFF) + ((u >> 16) & 1)) & np.uint32(0xFFFF0000)
    r = np.where(nan, (u | 0x00400000) & 0xFFFF0000, r).astype(np.uint32)
    return r.view(np.float32)


def bf16_bits(x) -> np.ndarray:
    return (bf16(x).view(np.uint32) >> 16).astype(np.uint16)


def from_bf16_bits(b) -> np.ndarray:
    return (np.ascontiguousarray(b, dtype=np.uint16).astype(np.uint32) << 16).view(np.float32)


def e4m3_encode(x) -> np.ndarray:
    x = np.ascontiguousarray(x, dtype=np.float32)
    q = np.empty(x.shape, np.uint8)
    lib().orc_e4m3_encode(_p(x), _p(q), x.size)
    return q


def e4m3_decode(q) -> np.ndarray:
    q = np.ascontiguousarray(q, dtype=np.uint8)
    x = np.empty(q.shape, np.float32)
    lib().orc_e4m3_decode(_p(q), _p(x), q.size)
    return x


def expf(x: float) -> float:
    return float(lib().orc_expf(ctypes.c_float(x)))


# ----------------------------------------------------------------------------
# Quantisation (contracts Q-A, Q-W, G)
# ----------------------------------------------------------------------------

def quantize_fp8(x_bits: np.ndarray, per_row: bool = False, gelu: bool = False):
    """Q-A over a bf16 [M, K] matrix given as uint16 bits.

    Follows flashvsr_sm89_ops/fp8_quant.py:16-35 (amax, s = max(amax,1e-12)/448,
    e4m3(clamp(x/s, +-448))) and :54 (returned scale = amax/448, unclamped).
    ``per_row`` is the per-token generalisation (one scale per row);
    ``gelu`` quantises tanh-GELU(x) as fp8_ffn.py:43-54 does.
    Returns (codes uint8 [M,K], scale float32 [1] or [M]).
    """
    x_bits = np.ascontiguousarray(x_bits, dtype=np.uint16)
    M, K = x_bits.shape
    q = np.empty((M, K), np.uint8)
    s = np.empty(M if per_row else 1, np.float32)
    lib().orc_quant_rows(_p(x_bits), M, K, K, int(per_row), int(gelu), _p(q), _p(s))
    return q, s


def quantize_weight(w_bits: np.ndarray, per_channel: bool = False):
    """Q-W: fp8_linear.py:17-22 (per tensor) or its per-output-channel form.
    Returns (codes uint8 [N,K], scale float32 [1] or [N])."""
    w_bits = np.ascontiguousarray(w_bits, dtype=np.uint16)
    N, K = w_bits.shape
    q = np.empty((N, K), np.uint8)
    s = np.empty(N if per_channel else 1, np.float32)
    lib().orc_quant_weight(_p(w_bits), N, K, int(per_channel), _p(q), _p(s))
    return q, s


def f16(x) -> np.ndarray:
    """Round float32 values to IEEE binary16 (nearest even), returned as float32."""
    x = np.ascontiguousarray(x, dtype=np.float32)
    y = np.empty_like(x)
    lib().orc_f16_round(_p(x), _p(y), x.size)
    return y


DT_BF16, DT_F16, DT_F32 = 0, 1, 2


def quantize_fp8_values(x: np.ndarray, per_row: bool = False, gelu: bool = False):
    """Q-A as quantize_fp8 on fp16 or fp32 inputs, given as their float32
    values (the reference's kernels load any input as fp32, fp8_quant.py:20,33)."""
    x = np.ascontiguousarray(x, dtype=np.float32)
    M, K = x.shape
    q = np.empty((M, K), np.uint8)
    s = np.empty(M if per_row else 1, np.float32)
    lib().orc_quant_rows_f32(_p(x), M, K, K, int(per_row), int(gelu), _p(q), _p(s))
    return q, s


def quantize_weight_values(w: np.ndarray, dt: int, per_channel: bool = False):
    """Q-W on a weight of type dt (DT_BF16 / DT_F16 / DT_F32) given as its
    float32 values: fp8_linear.py:19-22 evaluated in that type (see
    orc_quant_weight_f32).  Returns (codes uint8 [N,K], scale float32 [1] or [N])."""
    w = np.ascontiguousarray(w, dtype=np.float32)
    N, K = w.shape
    q = np.empty((N, K), np.uint8)
    s = np.empty(N if per_channel else 1, np.float32)
    lib().orc_quant_weight_f32(_p(w), N, K, int(per_channel), int(dt), _p(q), _p(s))
    return q, s


def gelu_values(x: np.ndarray) -> np.ndarray:
    """bf16(tanh-GELU(x)) for float32 inputs, as float32 (the same sequence as
    gelu_bf16; fp8_ffn.py:24-30 rounds to bf16 whatever the input type)."""
    x = np.ascontiguousarray(x, dtype=np.float32)
    g = np.empty_like(x)
    lib().orc_gelu_f32(_p(x), _p(g), x.size)
    return g


def gelu_bf16(h_bits: np.ndarray) -> np.ndarray:
    """bf16(tanh-GELU(h)) with the shared exp (fp8_ffn.py:24-30); uint16 bits."""
    h_bits = np.ascontiguousarray(h_bits, dtype=np.uint16)
    g = np.empty_like(h_bits)
    lib().orc_gelu_bf16(_p(h_bits), _p(g), h_bits.size)
    return g


# ----------------------------------------------------------------------------
# FP8 GEMM (contract M)
# ----------------------------------------------------------------------------

def fp8_gemm(a8: np.ndarray, sa: np.ndarray, b8: np.ndarray, sb: np.ndarray,
             bias=None, acc_dtype=np.float64) -> np.ndarray:
    """bf16(sum_k a8[m,k]*b8[n,k] * sa[m] * sb[n] + bias[n]) as float32.

    Restates torch._scaled_mm(x8, W8.t(), scale_a, scale_b, bias, bf16) at
    fp8_linear.py:28-30; fp8*fp8 products are exact, so with float64
    accumulation the only freedom left is the final rounding.  ``acc_dtype``
    float32 (for the full-size checks) keeps the products exact and rounds
    the sums: the bf16 result then differs from the float64 one only where the
    exact value lies within ~1e-6 (relative) of a bf16 rounding boundary.
    ``sa`` is [1] or [M]; ``sb`` is [1] or [N]."""
    A = e4m3_decode(a8).astype(acc_dtype)
    B = e4m3_decode(b8).astype(acc_dtype)
    y = A @ B.T
    y *= np.asarray(sa, np.float32).reshape(-1, 1).astype(acc_dtype)
    y *= np.asarray(sb, np.float32).reshape(1, -1).astype(acc_dtype)
    if bias is not None:
        y += np.asarray(bias, np.float32).reshape(1, -1)
    return bf16(y.astype(np.float32))


# ----------------------------------------------------------------------------
# AdaLN (contracts LN, GA)
# ----------------------------------------------------------------------------

def ln_modulate(x: np.ndarray, scale: np.ndarray, shift: np.ndarray, eps: float = 1e-6):
    """LayerNorm(no affine) then modulate with eager's bf16 rounding chain.

    fused_adaln.py:29-41: mean/var in fp32 (biased, /D);
    xn = bf16((x-mean)/sqrt(var+eps)); y = bf16(xn * bf16(1+s)); out = bf16(y+shift).
    x [B,L,D] bf16 values (float32); scale/shift [B,1,D]."""
    x = np.asarray(x, np.float32)
    mean = x.astype(np.float64).mean(-1, keepdims=True).astype(np.float32)
    d = x - mean
    var = (d.astype(np.float64) ** 2).mean(-1, keepdims=True).astype(np.float32)
    xn = bf16(d / np.sqrt(var + np.float32(eps)))
    y = bf16(xn * bf16(np.float32(1.0) + np.asarray(scale, np.float32)))
    return bf16(y + np.asarray(shift, np.float32))


def gate_add(x: np.ndarray, gate: np.ndarray, residual: np.ndarray):
    """bf16(x + bf16(gate*residual)) (fused_adaln.py:56-57); bitwise vs eager."""
    y = bf16(np.asarray(gate, np.float32) * np.asarray(residual, np.float32))
    return bf16(np.asarray(x, np.float32) + y)


# ----------------------------------------------------------------------------
# RMSNorm + RoPE (contract R)
# ----------------------------------------------------------------------------

def rope_params(max_len: int, dim: int, theta: float = 10000.0) -> np.ndarray:
    """Angles [max_len, dim//2] float64, Wan 2.1 convention
    pos * theta^(-(2i)/dim) (upstream wan_video_dit rope_params; upstream code is
    not in the reference checkout, the formula is the public Wan 2.1 one)."""
    inv = 1.0 / np.power(theta, np.arange(0, dim, 2, dtype=np.float64) / dim)
    return np.outer(np.arange(max_len, dtype=np.float64), inv)


def wan_rope_cos_sin(f: int, h: int, w: int, head_dim: int = 128, theta: float = 10000.0,
                     f_offset: int = 0):
    """3-D rotary table for a (f,h,w) token grid: head_dim split into
    head_dim-4*(head_dim//6) / 2*(head_dim//6) / 2*(head_dim//6) dims over
    (f, h, w) (44/42/42 for 128).  Returns (cos, sin) float32 [f*h*w, head_dim//2],
    i.e. view_as_real(freqs_cis).float() as fused_rms_rope.py:58-63 builds it."""
    d6 = head_dim // 6
    dims = (head_dim - 4 * d6, 2 * d6, 2 * d6)
    af = rope_params(max(f + f_offset, 1), dims[0], theta)[f_offset:f_offset + f]
    ah = rope_params(h, dims[1], theta)
    aw = rope_params(w, dims[2], theta)
    ang = np.concatenate([
        np.broadcast_to(af[:, None, None, :], (f, h, w, af.shape[1])),
        np.broadcast_to(ah[None, :, None, :], (f, h, w, ah.shape[1])),
        np.broadcast_to(aw[None, None, :, :], (f, h, w, aw.shape[1])),
    ], axis=-1).reshape(f * h * w, head_dim // 2)
    return np.cos(ang).astype(np.float32), np.sin(ang).astype(np.float32)


def rms_rope(x: np.ndarray, weight: np.ndarray, cos=None, sin=None, eps: float = 1e-6,
             rope: bool = True, head_dim: int = 128):
    """fused_rms_rope.py:27-55: RMS over the full D in fp32, r = rsqrt(ms+eps),
    y = bf16(x*r) * w; interleaved pairs (2i, 2i+1) per head rotated with
    cos/sin[s, i] in fp32; bf16 out.  x [B,L,D]; position s = row % L."""
    x = np.asarray(x, np.float32)
    B, L, D = x.shape
    ms = (x.astype(np.float64) ** 2).sum(-1, keepdims=True) / D
    r = (1.0 / np.sqrt(ms + eps)).astype(np.float32)
    y = bf16(x * r) * np.asarray(weight, np.float32)
    if not rope:
        return bf16(y)
    yp = y.reshape(B, L, D // head_dim, head_dim // 2, 2)
    c = np.asarray(cos, np.float32)[:L][None, :, None, :]
    s = np.asarray(sin, np.float32)[:L][None, :, None, :]
    ye, yo = yp[..., 0], yp[..., 1]
    out = np.stack([ye * c - yo * s, ye * s + yo * c], axis=-1)
    return bf16(out.reshape(B, L, D))


# ----------------------------------------------------------------------------
# Block-sparse attention (contract BSA) and its masks
# ----------------------------------------------------------------------------

def window_partition(x: np.ndarray, win=(2, 8, 8)) -> np.ndarray:
    """[B,F,H,W,C] -> [Nwin, wf*wh*ww, C] (lcsa/reference.py:15-21)."""
    B, F, H, W, C = x.shape
    wf, wh, ww = win
    x = x.reshape(B, F // wf, wf, H // wh, wh, W // ww, ww, C)
    x = x.transpose(0, 1, 3, 5, 2, 4, 6, 7)
    return np.ascontiguousarray(x).reshape(-1, wf * wh * ww, C)


def window_reverse(xw: np.ndarray, fhw, win=(2, 8, 8), batch: int = 1) -> np.ndarray:
    """Inverse of window_partition: [Nwin, 128, C] -> [B, F*H*W, C]."""
    F, H, W = fhw
    wf, wh, ww = win
    C = xw.shape[-1]
    x = xw.reshape(batch, F // wf, H // wh, W // ww, wf, wh, ww, C)
    x = x.transpose(0, 1, 4, 2, 5, 3, 6, 7)
    return np.ascontiguousarray(x).reshape(batch, F * H * W, C)


def build_local_block_mask(bh: int, bw: int, rng: int) -> np.ndarray:
    """Sliding-window local block mask [bh*bw, bh*bw] bool
    (lcsa/reference.py:24-34)."""
    r_all, c_all = np.meshgrid(np.arange(bh), np.arange(bw), indexing="ij")
    r_all, c_all = r_all.reshape(-1), c_all.reshape(-1)
    sr = r_all - rng // 2
    sc = c_all - rng // 2
    in_row = (r_all[None, :] >= sr[:, None]) & (r_all[None, :] <= sr[:, None] + rng - 1)
    in_col = (c_all[None, :] >= sc[:, None]) & (c_all[None, :] <= sc[:, None] + rng - 1)
    return in_row & in_col


def _topk_threshold_keep(flat: np.ndarray, topk: int) -> np.ndarray:
    """keep = flat > the (k+1)-th largest value of each row, k = min(topk,
    n-1), in torch.topk's order (NaN above every number; lcsa/reference.py:59-62)."""
    k = min(flat.shape[1] - 1, topk)
    order = np.where(np.isnan(flat), np.inf, flat)  # attn <= 1: inf only stands for NaN
    thr = -np.sort(-order, axis=1)[:, k]
    thr = np.where(np.isinf(thr), np.nan, thr)[:, None]
    with np.errstate(invalid="ignore"):
        return flat > thr


def draft_block_mask(q_w, k_w, nheads: int, q_temporal: int, local: np.ndarray, topk: int,
                     return_attn: bool = False):
    """Window-mean pooled block scores -> local mask -> softmax -> joint top-k
    per (head, query time row) (lcsa/reference.py:37-64).  Returns [h,Nq,Nk]
    bool (and the attn map with ``return_attn``).

    q_w/k_w [N, 128, h*d] as float32 values follow torch's float32 run of those
    lines.  As uint16 bf16 bits they follow its bf16 run, where every stage is
    rounded to bf16: mean = bf16(fp32 sum * 2^-7) (reference.py:41-42),
    einsum = bf16(fp32 dot) then ``/ math.sqrt(D)`` = bf16(s * fp32(1/fp32(sqrt
    D))), the reciprocal form the GPU division by a scalar takes (:47),
    -inf outside the tiled local mask (:49-55), softmax = bf16(fp32 exp(s -
    max) / fp32 sum) (:57).  The bf16 run's sums are taken in float64 (exact
    for bf16 data of ordinary range) and rounded once."""
    local = np.asarray(local, bool)
    sq, sk = local.shape
    if np.asarray(q_w).dtype == np.uint16:
        q = from_bf16_bits(q_w).astype(np.float64)
        k = from_bf16_bits(k_w).astype(np.float64)
        avg_q = bf16(q.sum(1).astype(np.float32) * np.float32(2.0 ** -7))
        avg_k = bf16(k.sum(1).astype(np.float32) * np.float32(2.0 ** -7))
        Nq, HD = avg_q.shape
        Nk = avg_k.shape[0]
        D = HD // nheads
        aq = avg_q.reshape(Nq, nheads, D).transpose(1, 0, 2).astype(np.float64)
        ak = avg_k.reshape(Nk, nheads, D).transpose(1, 0, 2).astype(np.float64)
        raw = bf16((aq @ ak.transpose(0, 2, 1)).astype(np.float32))
        inv = np.float32(1.0) / np.float32(math.sqrt(D))
        scores = bf16(raw * inv)
        scores = np.where(np.tile(local, (Nq // sq, Nk // sk))[None], scores,
                          np.float32(-np.inf))
        with np.errstate(invalid="ignore"):
            d = scores - scores.max(-1, keepdims=True)
            e = np.exp(d.astype(np.float64)).astype(np.float32)
            tot = e.astype(np.float64).sum(-1, keepdims=True).astype(np.float32)
            attn = bf16(e / tot)
        attn = np.where(np.isnan(attn), from_bf16_bits(np.uint16(0x7FC0)), attn)
    else:
        avg_q = np.asarray(q_w, np.float32).mean(1)
        avg_k = np.asarray(k_w, np.float32).mean(1)
        Nq, HD = avg_q.shape
        Nk = avg_k.shape[0]
        D = HD // nheads
        aq = avg_q.reshape(Nq, nheads, D).transpose(1, 0, 2)
        ak = avg_k.reshape(Nk, nheads, D).transpose(1, 0, 2)
        scores = aq @ ak.transpose(0, 2, 1) / math.sqrt(D)
        scores = np.where(np.tile(local, (Nq // sq, Nk // sk))[None], scores, -np.inf)
        with np.errstate(invalid="ignore"):
            scores = scores - scores.max(-1, keepdims=True)
            e = np.exp(scores)
            attn = (e / e.sum(-1, keepdims=True)).astype(np.float32)
    flat = attn.reshape(nheads * q_temporal, (Nq // q_temporal) * Nk)
    keep = _topk_threshold_keep(flat, topk).reshape(nheads, Nq, Nk)
    return (keep, attn) if return_attn else keep


def c4_block_mask(heads: int = 12, time_rows: int = 2, bh: int = 6, bw: int = 11,
                  local_range: int = 7, extra: int = 10, seed: int = 7) -> np.ndarray:
    """The C4 benchmark mask: within each latent time row the 2-D local rule
    build_local_block_mask(bh, bw, local_range), plus ``extra`` blocks per
    (head, query block) drawn without replacement from the blocks not yet kept
    (numpy PCG64, ``seed``).  The diagonal is always kept, so no row is empty."""
    nb = bh * bw
    N = time_rows * nb
    local = build_local_block_mask(bh, bw, local_range)
    base = np.zeros((N, N), bool)
    for t in range(time_rows):
        base[t * nb:(t + 1) * nb, t * nb:(t + 1) * nb] = local
    keep = np.broadcast_to(base, (heads, N, N)).copy()
    rng = np.random.Generator(np.random.PCG64(seed))
    for h in range(heads):
        for i in range(N):
            cand = np.flatnonzero(~keep[h, i])
            if len(cand):
                pick = rng.choice(cand, size=min(extra, len(cand)), replace=False)
                keep[h, i, pick] = True
    return keep


def random_block_mask(heads: int, nq: int, nk: int, density: float, seed: int,
                      keep_diag: bool = True) -> np.ndarray:
    """Seeded Bernoulli block mask used for density sweeps and parity tests."""
    rng = np.random.Generator(np.random.PCG64(seed))
    keep = rng.random((heads, nq, nk)) < density
    if keep_diag:
        for i in range(min(nq, nk)):
            keep[:, i, i] = True
    return keep


def build_csr(keep: np.ndarray):
    """keep [H,NQ,NK] -> (sel [H,NQ,MAXK] int32, cnt [H,NQ] int32, MAXK):
    kept block ids ascending first, then the others ascending
    (lcsa/triton_lcsa.py:64-71, stable descending argsort of keep)."""
    keep = np.asarray(keep, bool)
    cnt = keep.sum(-1).astype(np.int32)
    maxk = max(int(cnt.max()) if cnt.size else 0, 1)
    order = np.argsort(~keep, axis=-1, kind="stable")
    return order[..., :maxk].astype(np.int32), cnt, maxk


def sparse_attention(q, k, v, keep, sm_scale=None, block: int = 128) -> np.ndarray:
    """Exact block-sparse attention in float32, per (head, query block)
    (lcsa/reference.py:67-88 restated on [L, H, D] tensors in window order).
    q [Lq,H,D], k/v [Lk,H,D]; keep [H, Lq/128, Lk/128].  Rows with no kept
    block are 0 (lcsa/triton_lcsa.py:59-60).  Returns float32 [Lq,H,D]."""
    q = np.asarray(q, np.float32)
    k = np.asarray(k, np.float32)
    v = np.asarray(v, np.float32)
    Lq, H, D = q.shape
    if sm_scale is None:
        sm_scale = 1.0 / math.sqrt(D)
    NQ = Lq // block
    out = np.zeros_like(q)
    for h in range(H):
        kh = k[:, h].reshape(-1, block, D)
        vh = v[:, h].reshape(-1, block, D)
        for i in range(NQ):
            sel = np.flatnonzero(keep[h, i])
            if len(sel) == 0:
                continue
            kk = kh[sel].reshape(-1, D)
            vv = vh[sel].reshape(-1, D)
            s = (q[i * block:(i + 1) * block, h] @ kk.T) * np.float32(sm_scale)
            s = s - s.max(-1, keepdims=True)
            p = np.exp(s)
            p /= p.sum(-1, keepdims=True)
            out[i * block:(i + 1) * block, h] = p @ vv
    return out


def dense_masked_attention(q, k, v, keep, sm_scale=None, block: int = 128) -> np.ndarray:
    """Textbook softmax(QK^T*scale + mask) V with the block mask expanded to
    tokens; float64.  Small sizes only (the pin for sparse_attention)."""
    q = np.asarray(q, np.float64)
    k = np.asarray(k, np.float64)
    v = np.asarray(v, np.float64)
    Lq, H, D = q.shape
    if sm_scale is None:
        sm_scale = 1.0 / math.sqrt(D)
    out = np.zeros_like(q)
    for h in range(H):
        m = np.repeat(np.repeat(keep[h], block, 0), block, 1)
        s = q[:, h] @ k[:, h].T * sm_scale
        s = np.where(m, s, -np.inf)
        s = s - s.max(-1, keepdims=True)
        p = np.exp(s)
        p /= p.sum(-1, keepdims=True)
        out[:, h] = p @ v[:, h]
    return out


def layer_norm_affine(x: np.ndarray, weight: np.ndarray, bias: np.ndarray,
                      eps: float = 1e-6) -> np.ndarray:
    """nn.LayerNorm(elementwise_affine=True) on bf16 values over the last dim,
    the DiT block's norm3 (integrate.py:171): mean and biased variance, then
    bf16(w * ((x - mean) / sqrt(var + eps)) + b) with one rounding; computed in
    float64 (torch computes it in fp32, which differs only where the float64
    value sits at a bf16 rounding boundary)."""
    x = np.asarray(x, np.float64)
    mean = x.mean(-1, keepdims=True)
    var = ((x - mean) ** 2).mean(-1, keepdims=True)
    y = (x - mean) / np.sqrt(var + eps) * np.asarray(weight, np.float64) + np.asarray(bias, np.float64)
    return bf16(y.astype(np.float32))


def dense_attention(q, k, v, sm_scale=None) -> np.ndarray:
    """softmax(q k^T * scale) v per head in float64; q [Lq, H, D], k/v [Lk, H, D]
    (the cross-attention over the cached prompt K/V, integrate.py:141-143)."""
    q = np.asarray(q, np.float64)
    k = np.asarray(k, np.float64)
    v = np.asarray(v, np.float64)
    Lq, H, D = q.shape
    if sm_scale is None:
        sm_scale = 1.0 / math.sqrt(D)
    out = np.empty_like(q)
    for h in range(H):
        s = q[:, h] @ k[:, h].T * sm_scale
        s -= s.max(-1, keepdims=True)
        p = np.exp(s)
        p /= p.sum(-1, keepdims=True)
        out[:, h] = p @ v[:, h]
    return out


def _stage(teacher, name: str, value):
    """The value a composition continues with after stage ``name``: the
    oracle's own, or what ``teacher(name, value)`` returns (a test hands back
    the device's value of that stage after comparing the two, so each stage
    is checked on exactly the device's input to it)."""
    return value if teacher is None else teacher(name, value)


def cross_attention_block(x, norm3_w, norm3_b, params_q, norm_q_w, cache_k, cache_v, params_o,
                          heads: int = 12, eps: float = 1e-6, per_token: bool = True,
                          teacher=None):
    """x + cross_attn(norm3(x)) on [L, dim] bf16 values (integrate.py:132-143,171):
    LayerNorm(affine) -> FP8 q -> RMSNorm (no RoPE) -> dense attention over the
    cached K/V [Lk, dim] -> FP8 o -> residual add in bf16.  Stages: norm3,
    cross_q, cross_q_rms, cross_attn, cross_o, cross_res."""
    L, dim = x.shape
    xin = _stage(teacher, "norm3", layer_norm_affine(x, norm3_w, norm3_b, eps))
    q = _stage(teacher, "cross_q", linear_fp8(xin, *params_q, per_token=per_token))
    q = _stage(teacher, "cross_q_rms", rms_rope(q[None], norm_q_w, eps=eps, rope=False)[0])
    hd = dim // heads
    att = bf16(dense_attention(q.reshape(L, heads, hd), np.asarray(cache_k).reshape(-1, heads, hd),
                               np.asarray(cache_v).reshape(-1, heads, hd)).astype(np.float32))
    att = _stage(teacher, "cross_attn", att.reshape(L, dim))
    o = _stage(teacher, "cross_o", linear_fp8(att, *params_o, per_token=per_token))
    return _stage(teacher, "cross_res", bf16(np.asarray(x, np.float32) + o))


# ----------------------------------------------------------------------------
# DiT block composition (the C5 unit; integrate.py:151-182 with 47-124)
# ----------------------------------------------------------------------------

def quantize_input(x_bits: np.ndarray, per_token: bool = False, contiguous: bool = True):
    """The activation quantisation of FP8Linear.forward / FP8FFN.forward
    (fp8_linear.py:35-40, fp8_ffn.py:88-92): quantize_fp8 for a contiguous
    input; for a non-contiguous one the reference's eager expression
    ``s = (x2.abs().amax() / 448).clamp(min=1e-12).float(); (x2 / s).to(e4m3)``
    on bf16 tensors, which rounds the scale and x/s to bf16 - the per-tensor
    weight formula Q-W.  Per-token scales (the BASELINE extension) have one
    form only."""
    if per_token or contiguous:
        return quantize_fp8(x_bits, per_row=per_token)
    return quantize_weight(x_bits, per_channel=False)


def linear_fp8(x: np.ndarray, wq, ws, bias, per_token: bool = True,
               contiguous: bool = True, acc=np.float64) -> np.ndarray:
    """FP8Linear.forward (fp8_linear.py:32-42) on [T, K] bf16 values."""
    q, s = quantize_input(bf16_bits(x), per_token, contiguous)
    return fp8_gemm(q, s, wq, ws, bias, acc_dtype=acc)


def ffn_fp8(x: np.ndarray, w1q, w1s, b1, w2q, w2s, b2, per_token: bool = True,
            contiguous: bool = True, acc=np.float64) -> np.ndarray:
    """FP8FFN.forward (fp8_ffn.py:84-96): quant -> mm0 -> GELU requant -> mm2."""
    q, s = quantize_input(bf16_bits(x), per_token, contiguous)
    h = fp8_gemm(q, s, w1q, w1s, b1, acc_dtype=acc)
    hq, hs = quantize_fp8(bf16_bits(h), per_row=per_token, gelu=True)
    return fp8_gemm(hq, hs, w2q, w2s, b2, acc_dtype=acc)


def self_attention(xin, params, fhw, keep, cos, sin, heads: int = 12, eps: float = 1e-6,
                   per_token: bool = True, cache=None, kv_len=None, windows=None,
                   acc=np.float64, teacher=None):
    """The DiT self-attention (integrate.py:47-124) on [L, dim] bf16 values:
    FP8 q/k/v -> RMSNorm+RoPE(q, k) -> window partition (2,8,8) -> cached
    windows in front of k and v -> block-sparse attention (kept blocks
    ``keep`` [heads, NQ, NK], NK counting the cached windows) -> reverse ->
    FP8 o.  ``cache`` = (k_w, v_w) window-ordered [windows, 128, dim]; the
    returned cache drops the oldest step's windows once it holds more than
    ``kv_len`` steps (integrate.py:81-83,108-115).
    ``windows`` (per-token scales only, where rows are independent outside
    the attention): evaluate q, the attention and o only for the tokens of
    these query windows; o then holds those tokens' rows, in window order.
    Stages (``teacher``, whole-sequence evaluation only): q_proj, k_proj,
    v_proj, q_rope, k_rope ([L, dim] raster order), attn (window order),
    o_proj.  Returns (o, cache_k, cache_v)."""
    f, h, w = fhw
    L, dim = xin.shape
    hd = dim // heads
    k, v = (_stage(teacher, n + "_proj", linear_fp8(xin, *params[n], per_token=per_token,
                                                    acc=acc)) for n in ("k", "v"))
    k = _stage(teacher, "k_rope", rms_rope(k[None], params["norm_k"], cos, sin, eps)[0])
    kw, vw = (window_partition(t.reshape(1, f, h, w, dim)) for t in (k, v))
    if windows is None:
        q = _stage(teacher, "q_proj", linear_fp8(xin, *params["q"], per_token=per_token, acc=acc))
        q = _stage(teacher, "q_rope", rms_rope(q[None], params["norm_q"], cos, sin, eps)[0])
        qw = window_partition(q.reshape(1, f, h, w, dim))
        qkeep = keep
    else:
        assert per_token, "a window subset needs row-local (per-token) quantisation"
        tok = window_tokens(fhw, windows)
        q = linear_fp8(xin[tok], *params["q"], per_token=True, acc=acc)
        qw = rms_rope(q[None], params["norm_q"], np.asarray(cos)[tok], np.asarray(sin)[tok],
                      eps)[0].reshape(-1, 128, dim)
        qkeep = np.asarray(keep)[:, windows]
    per_step = kw.shape[0] // (f // 2)
    if cache is not None:
        kw = np.concatenate([cache[0], kw])
        vw = np.concatenate([cache[1], vw])
    att = bf16(sparse_attention(qw.reshape(-1, heads, hd), kw.reshape(-1, heads, hd),
                                vw.reshape(-1, heads, hd), qkeep))
    att = _stage(teacher, "attn", att.reshape(-1, dim))
    if windows is None:
        att = window_reverse(att.reshape(-1, 128, dim), (f, h, w))[0]
    o = _stage(teacher, "o_proj", linear_fp8(att, *params["o"], per_token=per_token, acc=acc))
    if kv_len is not None and kw.shape[0] // per_step > kv_len:
        kw, vw = kw[per_step:], vw[per_step:]
    return o, kw, vw


def window_tokens(fhw, windows) -> np.ndarray:
    """Raster token indices of the given windows' tokens, in window order."""
    f, h, w = fhw
    order = window_partition(np.arange(f * h * w, dtype=np.float32).reshape(1, f, h, w, 1))
    return order[np.asarray(windows)].reshape(-1).astype(np.int64)


def dit_block(x, mod, params, fhw, keep, cos, sin, heads: int = 12, eps: float = 1e-6,
              cross=None, per_token: bool = True, cache=None, kv_len=None,
              return_cache: bool = False, windows=None, acc=np.float64, teacher=None):
    """One DiT block on [L, dim] bf16 values (batch 1), integrate.py:151-182:
    AdaLN -> self-attention (above) -> gate_add -> [x + cross-attention of
    norm3(x)] -> AdaLN -> FP8 GELU FFN -> gate_add.
    ``mod`` is [6, dim] = modulation + t_mod, split (shift, scale, gate) for
    the attention then the FFN (integrate.py:154-155).  ``params`` holds the
    quantised weights q, k, v, o, ffn0, ffn2 as (codes, scale, bias) and
    norm_q / norm_k.  ``cross`` (norm3_w, norm3_b, q, o, norm_q, k, v) adds the
    cross-attention residual (integrate.py:171).  ``per_token`` picks per-token
    activation scales (else per tensor, the reference's default).
    ``windows``: the output rows of those query windows' tokens only (in
    window order; see self_attention).  ``teacher(name, value)``, if given,
    is called with each stage's value and returns the one to continue with
    (stages ln1, the self-attention's, gate1, the cross-attention's, ln2, ffn,
    out).  With ``return_cache`` returns (out, cache_k, cache_v)."""
    shift_msa, scale_msa, gate_msa, shift_mlp, scale_mlp, gate_mlp = \
        [mod[i][None, None] for i in range(6)]
    xin = _stage(teacher, "ln1", ln_modulate(x[None], scale_msa, shift_msa, eps)[0])
    o, ck, cv = self_attention(xin, params, fhw, keep, cos, sin, heads, eps, per_token, cache,
                               kv_len, windows, acc, teacher)
    if windows is not None:
        x = np.asarray(x)[window_tokens(fhw, windows)]
    x = _stage(teacher, "gate1", gate_add(x[None], gate_msa, o[None])[0])
    if cross is not None:
        x = cross_attention_block(x, cross["norm3_w"], cross["norm3_b"], cross["q"],
                                  cross["norm_q"], cross["k"], cross["v"], cross["o"], heads, eps,
                                  per_token=per_token, teacher=teacher)
    xin = _stage(teacher, "ln2", ln_modulate(x[None], scale_mlp, shift_mlp, eps)[0])
    y = _stage(teacher, "ffn", ffn_fp8(xin, *params["ffn0"], *params["ffn2"],
                                        per_token=per_token, acc=acc))
    out = _stage(teacher, "out", gate_add(x[None], gate_mlp, y[None])[0])
    return (out, ck, cv) if return_cache else out
