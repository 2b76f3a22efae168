"""CPU tests of the host side: the C ABI library (load, exports, argument
checks that run before any launch), the no-fallback rule, the
``block_sparse_attn`` module injection and ``enable()``'s wiring logic.
Nothing here launches a kernel."""
import ctypes
import os
import re
import sys
import types

import numpy as np
import pytest
import torch

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HEADER = os.path.join(ROOT, "include", "fvsr.h")


def declared_symbols():
    text = open(HEADER).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(fvsr_\w+)\s*\(", text)))


@pytest.fixture(scope="module")
def L():
    from flashvsr_sm89_ops import _lib
    return _lib.lib()


def test_header_and_binding_agree():
    from flashvsr_sm89_ops import _lib
    assert declared_symbols() == sorted(_lib.exported_symbols())


def test_library_exports_every_declared_symbol(L):
    for name in declared_symbols():
        assert hasattr(L, name), name
    out = os.popen(f"nm -D --defined-only {L._name}").read()
    for name in declared_symbols():
        assert re.search(rf"\bT {name}$", out, re.M), name


def test_version(L):
    assert L.fvsr_version().decode().startswith("fvsr ")


def test_argument_checks_before_launch(L):
    from flashvsr_sm89_ops import _lib
    p = ctypes.c_void_p(16)  # never dereferenced: every call below fails its host checks
    # GEMM: K must be a multiple of 16
    assert L.fvsr_fp8_gemm(p, 17, p, 0, p, 17, p, 0, None, p, 8, 8, 8, 17, 0, None, None, None,
                           None) == _lib.FVSR_EUNSUPPORTED
    assert L.fvsr_fp8_gemm(p, 16, p, 0, p, 16, p, 0, None, p, 8, -1, 8, 16, 0, None, None, None,
                           None) == _lib.FVSR_EINVAL
    # GELU epilogue without its amax buffer
    assert L.fvsr_fp8_gemm(p, 16, p, 0, p, 16, p, 0, None, p, 8, 8, 8, 16, 1, None, None, None,
                           None) == _lib.FVSR_EINVAL
    assert L.fvsr_fp8_gemm(p, 16, p, 0, p, 16, p, 0, None, p, 8, 8, 8, 16, 9, None, None, None,
                           None) == _lib.FVSR_EINVAL
    # empty problems are a no-op
    assert L.fvsr_fp8_gemm(None, 16, None, 0, None, 16, None, 0, None, None, 8, 0, 8, 16, 0, None,
                           None, None, None) == _lib.FVSR_OK
    assert L.fvsr_quant_fp8(p, 4, 8, 8, 7, 0, p, p, p, 1, None) == _lib.FVSR_EINVAL
    assert L.fvsr_quant_fp8(p, 4, 8, 4, 1, 0, p, p, p, 1, None) == _lib.FVSR_EINVAL  # ld < cols
    assert L.fvsr_quant_fp8(p, 4, 8, 8, 0, 0, p, p, p, 0, None) == _lib.FVSR_EWORKSPACE
    assert L.fvsr_quant_fp8(None, 0, 8, 8, 0, 0, None, None, None, 0, None) == _lib.FVSR_OK
    assert L.fvsr_quant_workspace_floats(10_000, 1536, 0) == 1024
    assert L.fvsr_quant_workspace_floats(3, 1536, 0) == 1
    assert L.fvsr_gemm_amax_parts(8960) == 70
    assert L.fvsr_bsa_fwd(p, p, p, p, 1536, 128, 1536, 128, 1536, 128, p, p, 4, 12, 4, 4, 64, 0.1,
                          None, None, None) == _lib.FVSR_EUNSUPPORTED
    assert L.fvsr_bsa_fwd(p, p, p, p, 1537, 128, 1536, 128, 1536, 128, p, p, 4, 12, 4, 4, 128, 0.1,
                          None, None, None) == _lib.FVSR_EUNSUPPORTED
    assert L.fvsr_rms_rope_qk(p, p, p, p, p, p, p, 1, 4, 1536, 128, 1e-6, 1000, 1536,
                              None) == _lib.FVSR_EINVAL
    assert L.fvsr_rms_rope(p, p, None, p, 1, 4, 1536, 128, 1e-6, 1, None) == _lib.FVSR_EINVAL
    assert L.fvsr_ln_modulate(p, p, p, None, 1, 4, 1536, 1e-6, None, None, None) == _lib.FVSR_EINVAL
    assert L.fvsr_block_index(None, 0, 4, 4, None, None, None) == _lib.FVSR_OK


def test_dtype_entry_points_check_codes(L):
    """The *_dt entry points take FVSR_DT_* codes (bf16 0, fp16 1, fp32 2) and
    refuse any other before launching; empty calls return at once; the
    wrappers map torch dtypes to codes and refuse other types."""
    from flashvsr_sm89_ops import _lib
    p = ctypes.c_void_p(16)  # never dereferenced
    E, OK = _lib.FVSR_EINVAL, _lib.FVSR_OK
    assert L.fvsr_gate_add_dt(p, 3, p, 0, p, 0, p, 1, 4, 8, None) == E
    assert L.fvsr_gate_add_dt(p, 0, p, 0, p, -1, p, 1, 4, 8, None) == E
    assert L.fvsr_ln_modulate_dt(p, 0, p, -1, p, 0, p, 1, 4, 8, 1e-6, None) == E
    assert L.fvsr_ln_modulate_dt(p, 1, p, 2, p, 2, p, 1, 4, 0, 1e-6, None) == E   # D = 0
    assert L.fvsr_rms_rope_dt(p, 0, p, 5, None, p, 1, 4, 8, 8, 1e-6, 0, None) == E
    assert L.fvsr_rms_rope_dt(p, 2, p, 2, None, p, 1, 4, 8, 8, 1e-6, 1, None) == E  # rope, no cs
    assert L.fvsr_quant_fp8_dt(p, 9, 4, 8, 8, 1, 0, p, p, None, 0, None) == E
    assert L.fvsr_quant_fp8_dt(p, 2, 4, 8, 8, 0, 0, p, p, p, 0, None) == _lib.FVSR_EWORKSPACE
    assert L.fvsr_quant_weight_fp8_dt(p, 9, 4, 8, 1, p, p, None, 0, None) == E
    assert L.fvsr_gate_add_dt(None, 2, None, 1, None, 2, None, 0, 4, 8, None) == OK
    assert L.fvsr_quant_fp8_dt(None, 1, 0, 8, 8, 1, 0, None, None, None, 0, None) == OK
    assert L.fvsr_quant_weight_fp8_dt(None, 2, 0, 8, 0, None, None, None, 0, None) == OK
    for dt, code in ((torch.bfloat16, 0), (torch.float16, 1), (torch.float32, 2)):
        assert _lib.dtype_code(torch.zeros(1, dtype=dt), "x") == code == getattr(
            _lib, {0: "DT_BF16", 1: "DT_F16", 2: "DT_F32"}[code])
    for dt in (torch.float64, torch.int32, torch.float8_e4m3fn):
        with pytest.raises(TypeError, match="bfloat16, float16 or float32"):
            _lib.dtype_code(torch.zeros(1).to(dt), "x")


def test_no_cpu_fallback():
    import flashvsr_sm89_ops as f
    x = torch.zeros(4, 16, dtype=torch.bfloat16)
    with pytest.raises(RuntimeError, match="GPU only"):
        f.quantize_fp8(x)
    with pytest.raises(RuntimeError, match="GPU only"):
        f.fused_gate_add(x[None], x[:1][None], x[None])
    with pytest.raises(RuntimeError, match="GPU only"):
        f.fused_rms_rope(x[None], x[0], None, rope=False)


def test_missing_library_fails_loudly(tmp_path, monkeypatch):
    from flashvsr_sm89_ops import _lib
    monkeypatch.setattr(_lib, "LIB_PATH", str(tmp_path / "absent.so"))
    monkeypatch.setattr(_lib, "_lib", None)
    with pytest.raises(RuntimeError, match="not built"):
        _lib.lib()


# ----------------------------------------------------------------------------- compat_bsa

def test_bsa_stub_modes(monkeypatch):
    from flashvsr_sm89_ops import compat_bsa as cb
    monkeypatch.delitem(sys.modules, "block_sparse_attn", raising=False)
    monkeypatch.setenv("FS89_LCSA", "bsa")
    assert cb.ensure_bsa_available() == "bsa"
    assert "block_sparse_attn" not in sys.modules
    assert cb.active_backend() == "bsa"
    for mode in ("auto", "hip", "triton"):
        monkeypatch.setenv("FS89_LCSA", mode)
        monkeypatch.delitem(sys.modules, "block_sparse_attn", raising=False)
        assert cb.active_backend() == "unresolved"
        assert cb.ensure_bsa_available() == "hip"
        mod = sys.modules["block_sparse_attn"]
        assert mod.__version__ == cb.STUB_VERSION and cb.active_backend() == "hip"
        assert callable(mod.block_sparse_attn_func)
    other = types.ModuleType("block_sparse_attn")
    other.__version__ = "2.0"
    monkeypatch.setitem(sys.modules, "block_sparse_attn", other)
    assert cb.active_backend() == "bsa"


@pytest.mark.parametrize("kw", [dict(streaming_info=1), dict(is_causal=True),
                                dict(dropout_p=0.1), dict(return_attn_probs=True)])
def test_bsa_stub_rejects_unsupported(kw):
    from flashvsr_sm89_ops.compat_bsa import _hip_block_sparse_attn_func
    args = dict(q=None, k=None, v=None, cu_seqlens_q=None, cu_seqlens_k=None, head_mask_type=None,
                streaming_info=None, attn_mask=None, max_seqlen_q=0, max_seqlen_k=0)
    args.update(kw)
    with pytest.raises(NotImplementedError):
        _hip_block_sparse_attn_func(**args)


# ----------------------------------------------------------------------------- integrate

def make_fake_dit():
    """A stand-in for diffsynth.models.wan_video_dit: the rebound classes with
    the upstream forward signatures, stock forwards that compute the upstream
    math in torch (CrossAttention, DiTBlock) and record that they ran, and the
    stock helpers."""
    dit = types.ModuleType("fake_wan_video_dit")
    dit.stock_calls = []

    class SelfAttention(torch.nn.Module):
        def forward(self, x, freqs, f=None, h=None, w=None, local_num=None, topk=None,
                    train_img=False, block_id=None, kv_len=None, is_full_block=False,
                    is_stream=False, pre_cache_k=None, pre_cache_v=None, local_range=9):
            dit.stock_calls.append("SelfAttention")
            raise NotImplementedError("stock self-attention is not modelled here")

    class CrossAttention(torch.nn.Module):
        def forward(self, x, y, is_stream=False):
            dit.stock_calls.append("CrossAttention")
            return self.o(self.attn(self.norm_q(self.q(x)), self.cache_k, self.cache_v))

    class DiTBlock(torch.nn.Module):
        def __init__(self, dim=16):
            super().__init__()
            self.modulation = torch.nn.Parameter(torch.randn(1, 6, dim) * 0.1)
            self.norm1 = torch.nn.LayerNorm(dim, eps=1e-6, elementwise_affine=False)
            self.norm2 = torch.nn.LayerNorm(dim, eps=1e-6, elementwise_affine=False)
            self.norm3 = torch.nn.LayerNorm(dim, eps=1e-6)

        def forward(self, x, context, t_mod, freqs, f, h, w, local_num=None, topk=None,
                    train_img=False, block_id=None, kv_len=None, is_full_block=False,
                    is_stream=False, pre_cache_k=None, pre_cache_v=None, local_range=9):
            dit.stock_calls.append("DiTBlock")
            sh, sc, g, sh2, sc2, g2 = (self.modulation + t_mod).chunk(6, dim=1)
            a, ck, cv = self.self_attn(dit.modulate(self.norm1(x), sh, sc), freqs, f, h, w,
                                       local_num, topk, train_img, block_id, kv_len=kv_len,
                                       is_stream=is_stream, pre_cache_k=pre_cache_k,
                                       pre_cache_v=pre_cache_v, local_range=local_range)
            x = self.gate(x, g, a)
            x = x + self.cross_attn(self.norm3(x), context, is_stream=is_stream)
            x = self.gate(x, g2, self.ffn(dit.modulate(self.norm2(x), sh2, sc2)))
            return (x, ck, cv) if is_stream else x

        def gate(self, x, gate, residual):
            return x + gate * residual

    class WindowPartition3D:
        @staticmethod
        def partition(x, win):
            raise NotImplementedError

    dit.SelfAttention, dit.CrossAttention, dit.DiTBlock = SelfAttention, CrossAttention, DiTBlock
    dit.WindowPartition3D = WindowPartition3D
    dit.generate_draft_block_mask = lambda *a, **k: None
    dit.modulate = lambda x, shift, scale: x * (1 + scale) + shift
    return dit


class FakePipe:
    def __init__(self):
        self.model = torch.nn.Module()

    def denoising_model(self):
        return self.model


def test_drift_guard():
    from flashvsr_sm89_ops.integrate import _check_dit_structure
    dit = make_fake_dit()
    _check_dit_structure(dit)
    del dit.SelfAttention
    with pytest.raises(RuntimeError, match="no SelfAttention"):
        _check_dit_structure(dit)
    dit = make_fake_dit()

    class DiTBlock:
        def forward(self, x, context):
            pass
    dit.DiTBlock = DiTBlock
    with pytest.raises(RuntimeError, match="lacks args"):
        _check_dit_structure(dit)
    dit = make_fake_dit()
    del dit.generate_draft_block_mask
    with pytest.raises(RuntimeError, match="generate_draft_block_mask"):
        _check_dit_structure(dit)


def test_enable_wiring_flags_and_idempotence(monkeypatch, capsys):
    import flashvsr_sm89_ops as f
    from flashvsr_sm89_ops import integrate
    dit = make_fake_dit()
    stock = {n: getattr(dit, n).forward for n in ("SelfAttention", "CrossAttention", "DiTBlock")}
    monkeypatch.setenv("FS89_FP8", "")
    applied = f.enable(FakePipe(), dit_module=dit)
    assert applied == {"fused_rope": True, "fused_adaln": True, "lcsa_backend": "hip"}
    assert dit.SelfAttention.forward is not stock["SelfAttention"] and dit._FS89_PATCHED
    assert dit._FS89_STOCK == stock          # the upstream forwards, captured before rebinding
    assert dit.FUSED_ROPE_FN is f.fused_rms_rope
    assert dit.FUSED_ADALN == (f.fused_ln_modulate, f.fused_gate_add)
    assert "[flashvsr-mi355x-ops] enabled" in capsys.readouterr().out
    rebound = dit.DiTBlock.forward
    monkeypatch.setenv("FS89_FUSED_ROPE", "0")
    monkeypatch.setenv("FS89_FUSED_ADALN", "0")
    applied = f.enable(FakePipe(), dit_module=dit, verbose=False)
    assert applied["fused_rope"] is False and dit.FUSED_ROPE_FN is None and dit.FUSED_ADALN is None
    assert dit.DiTBlock.forward is rebound  # not rebound twice
    assert dit._FS89_STOCK == stock          # still the upstream ones, not the rebound ones
    with pytest.raises(ValueError):
        f.enable(FakePipe(), dit_module=dit, scale_granularity="block")
    monkeypatch.setitem(sys.modules, "diffsynth", None)
    with pytest.raises(ImportError, match="wan_video_dit"):
        integrate.enable(FakePipe())


def test_stock_branch_dit_block_on_cpu(monkeypatch):
    """With the fused flags off, the rebound DiTBlock.forward is the upstream
    forward captured by enable(): AdaLN(shift, scale) order, gate,
    cross-attention residual."""
    import flashvsr_sm89_ops as f
    dit = make_fake_dit()
    monkeypatch.setenv("FS89_FP8", "")
    monkeypatch.setenv("FS89_FUSED_ROPE", "0")
    monkeypatch.setenv("FS89_FUSED_ADALN", "0")
    f.enable(FakePipe(), dit_module=dit, verbose=False)
    blk = dit.DiTBlock(16)
    seen = {}

    def self_attn(x, *a, **k):
        seen["attn_in"] = x
        return x * 2, None, None
    blk.self_attn = self_attn
    blk.cross_attn = lambda x, ctx, is_stream=False: x * 0 + 1
    blk.ffn = lambda x: x - 1
    x = torch.randn(1, 5, 16)
    t_mod = torch.randn(1, 6, 16) * 0.1
    out, ck, cv = blk(x, None, t_mod, None, 1, 1, 5, is_stream=True)
    assert dit.stock_calls == ["DiTBlock"] and ck is None and cv is None
    sh, sc, g, sh2, sc2, g2 = (blk.modulation + t_mod).chunk(6, dim=1)
    ln = torch.nn.functional.layer_norm
    a_in = ln(x, (16,), eps=1e-6) * (1 + sc) + sh
    torch.testing.assert_close(seen["attn_in"], a_in)
    x1 = x + g * (a_in * 2)
    x1 = x1 + (ln(x1, (16,), weight=blk.norm3.weight, bias=blk.norm3.bias, eps=1e-6) * 0 + 1)
    ref = x1 + g2 * ((ln(x1, (16,), eps=1e-6) * (1 + sc2) + sh2) - 1)
    torch.testing.assert_close(out, ref)


def test_stock_self_attention_when_rope_off(monkeypatch):
    """FS89_FUSED_ROPE=0: the rebound SelfAttention.forward hands every
    argument to the upstream forward by name."""
    import flashvsr_sm89_ops as f
    dit = make_fake_dit()
    got = {}

    def upstream(self, x, freqs, f=None, h=None, w=None, local_num=None, topk=None,
                 train_img=False, block_id=None, kv_len=None, is_full_block=False,
                 is_stream=False, pre_cache_k=None, pre_cache_v=None, local_range=9):
        got.update(locals())
        return "stock"
    dit.SelfAttention.forward = upstream
    monkeypatch.setenv("FS89_FP8", "")
    monkeypatch.setenv("FS89_FUSED_ROPE", "0")
    f.enable(FakePipe(), dit_module=dit, verbose=False)
    sa = dit.SelfAttention()
    x = torch.zeros(1, 4, 8)
    assert sa(x, "fr", 2, 1, 2, 3, 4, True, 5, kv_len=6, is_full_block=True, is_stream=True,
              pre_cache_k="k", pre_cache_v="v", local_range=7) == "stock"
    assert got["x"] is x and (got["freqs"], got["f"], got["h"], got["w"]) == ("fr", 2, 1, 2)
    assert (got["local_num"], got["topk"], got["train_img"], got["block_id"]) == (3, 4, True, 5)
    assert (got["kv_len"], got["is_full_block"], got["is_stream"]) == (6, True, True)
    assert (got["pre_cache_k"], got["pre_cache_v"], got["local_range"]) == ("k", "v", 7)


def test_fused_self_attention_checks_stream_geometry(monkeypatch):
    """The fused self-attention keeps the upstream preconditions: a stream
    starts with 6 latent frames, continues with 2, and L == f*h*w."""
    import flashvsr_sm89_ops as f
    dit = make_fake_dit()
    monkeypatch.setenv("FS89_FP8", "")
    f.enable(FakePipe(), dit_module=dit, verbose=False)
    sa = dit.SelfAttention()
    sa.head_dim = 128
    x = torch.zeros(1, 2 * 8 * 8, 256)
    with pytest.raises(AssertionError, match="f == 6"):
        sa(x, None, 2, 8, 8, is_stream=True)
    with pytest.raises(AssertionError, match="f == 2"):
        sa(torch.zeros(1, 6 * 64, 256), None, 6, 8, 8, is_stream=True, pre_cache_k=x, pre_cache_v=x)
    with pytest.raises(AssertionError, match="sequence length"):
        sa(x, None, 2, 8, 4)


def test_window_token_map_matches_partition():
    from flashvsr_sm89_ops.block import window_token_map
    from oracle import oracle as O
    f, h, w = 4, 16, 24
    x = np.arange(f * h * w, dtype=np.float32).reshape(1, f, h, w, 1)
    xw = O.window_partition(x).reshape(-1)
    assert np.array_equal(window_token_map(f, h, w).numpy(), xw.astype(np.int32))


def test_stock_branch_cross_attention_on_cpu(monkeypatch):
    """FS89_FUSED_ROPE=0: the rebound CrossAttention.forward is the upstream
    forward (stock RMSNorm, the DiT's own attention over the cached K/V)."""
    import flashvsr_sm89_ops as f
    dit = make_fake_dit()
    monkeypatch.setenv("FS89_FP8", "")
    monkeypatch.setenv("FS89_FUSED_ROPE", "0")
    f.enable(FakePipe(), dit_module=dit, verbose=False)
    ca = dit.CrossAttention()
    ca.q = torch.nn.Linear(16, 16)
    ca.o = torch.nn.Linear(16, 16)
    ca.norm_q = lambda t: t * 3
    ca.num_heads = 2
    ca.cache_k, ca.cache_v = torch.randn(1, 7, 16), torch.randn(1, 7, 16)
    seen = {}

    def attn(q, k, v):
        seen["args"] = (q, k, v)
        return q + 1
    ca.attn = attn
    x = torch.randn(1, 5, 16)
    out = ca(x, None)
    assert dit.stock_calls == ["CrossAttention"]
    q, k, v = seen["args"]
    torch.testing.assert_close(q, ca.q(x) * 3)
    assert k is ca.cache_k and v is ca.cache_v
    torch.testing.assert_close(out, ca.o(ca.q(x) * 3 + 1))


def test_fused_cross_attention_keeps_dit_attention_where_kernel_does_not_apply(monkeypatch):
    """FS89_FUSED_ROPE on: q's RMSNorm goes through FUSED_ROPE_FN (rope=False);
    shapes the HIP attention does not cover (here CPU tensors) use the DiT's
    own attention; a missing prompt cache is refused."""
    import flashvsr_sm89_ops as f
    from flashvsr_sm89_ops.cross_attn import supported
    dit = make_fake_dit()
    monkeypatch.setenv("FS89_FP8", "")
    f.enable(FakePipe(), dit_module=dit, verbose=False)
    calls = []

    def fake_rms(x, weight, freqs, eps=1e-6, rope=True, head_dim=128):
        calls.append((freqs, eps, rope))
        return x * 3
    monkeypatch.setattr(dit, "FUSED_ROPE_FN", fake_rms)
    ca = dit.CrossAttention()
    ca.q, ca.o = torch.nn.Linear(16, 16), torch.nn.Linear(16, 16)
    ca.norm_q = torch.nn.Module()
    ca.norm_q.weight, ca.norm_q.eps = torch.ones(16), 1e-5
    ca.num_heads = 2
    ca.cache_k, ca.cache_v = torch.randn(1, 7, 16), torch.randn(1, 7, 16)
    ca.attn = lambda q, k, v: q + 1
    x = torch.randn(1, 5, 16)
    out = ca(x, None)
    assert calls == [(None, 1e-5, False)] and dit.stock_calls == []
    torch.testing.assert_close(out, ca.o(ca.q(x) * 3 + 1))
    assert not supported(ca.q(x), ca.cache_k, ca.cache_v, 2)
    ca.cache_k = None
    with pytest.raises(AssertionError, match="init_cross_kv"):
        ca(x, None)


def _dit_like(dim=16, ffn=32, seed=0):
    """Two DiT blocks' worth of Linears; the same seed gives the same weights
    (the same checkpoint)."""
    torch.manual_seed(seed)
    m = torch.nn.Module()
    m.blocks = torch.nn.ModuleList()
    for _ in range(2):
        b = torch.nn.Module()
        b.self_attn = torch.nn.Module()
        for n in "qkvo":
            setattr(b.self_attn, n, torch.nn.Linear(dim, dim))
        b.ffn = torch.nn.Sequential(torch.nn.Linear(dim, ffn), torch.nn.GELU(),
                                    torch.nn.Linear(ffn, dim, bias=False))
        m.blocks.append(b)
    return m


def _stored_for(model, per_channel, seed=0):
    g = torch.Generator().manual_seed(seed)
    out = {}
    for name, mod in model.named_modules():
        if isinstance(mod, torch.nn.Linear):
            N, K = mod.weight.shape
            codes = torch.randint(0, 256, (N, K), generator=g, dtype=torch.int64).to(torch.uint8)
            scales = torch.rand(N if per_channel else 1, generator=g) + 0.01
            bias = mod.bias.detach().to(torch.bfloat16) if mod.bias is not None else None
            out[name] = (codes, scales, bias)
    return out


@pytest.mark.parametrize("per_channel", [False, True])
def test_fp8_weights_save_load_roundtrip(tmp_path, per_channel):
    """Stored codes and scales come back bit for bit; conversion from them
    quantises nothing (so it runs here, without the GPU library)."""
    from flashvsr_sm89_ops.fp8_linear import (FP8Linear, convert_linears_fp8, load_fp8_weights,
                                              save_fp8_weights)
    model = _dit_like()
    stored = _stored_for(model, per_channel)
    n = convert_linears_fp8(model, parts=("self", "ffn"), per_channel=per_channel, stored=stored)
    assert n == 12
    for name, (codes, scales, bias) in stored.items():
        mod = model.get_submodule(name)
        assert isinstance(mod, FP8Linear) and mod.weight.dtype == torch.float8_e4m3fn
        assert torch.equal(mod.weight.view(torch.uint8), codes)
        assert torch.equal(mod.w_scale.reshape(-1), scales)
        assert mod.per_channel == per_channel and (mod.w_scale.dim() == 0) != per_channel
    path = str(tmp_path / "w.safetensors")
    assert save_fp8_weights(model, path) == 12
    back = load_fp8_weights(path)
    assert set(back) == set(stored)
    for name, (codes, scales, bias) in stored.items():
        c2, s2, b2 = back[name]
        assert torch.equal(c2, codes) and torch.equal(s2, scales)
        assert (b2 is None) == (bias is None) and (bias is None or torch.equal(b2, bias))
    fresh = _dit_like()
    assert convert_linears_fp8(fresh, parts=("self", "ffn"), per_channel=per_channel,
                               stored=back) == 12
    for name in stored:
        assert torch.equal(fresh.get_submodule(name).weight.view(torch.uint8),
                           model.get_submodule(name).weight.view(torch.uint8))


def test_fp8_weights_rejects_mismatch(tmp_path):
    from flashvsr_sm89_ops.fp8_linear import convert_linears_fp8, load_fp8_weights
    model = _dit_like()
    stored = _stored_for(model, per_channel=True)
    with pytest.raises(ValueError, match="granularity"):
        convert_linears_fp8(_dit_like(), parts=("self",), per_channel=False, stored=stored)
    stored["blocks.0.self_attn.q"] = (torch.zeros(3, 16, dtype=torch.uint8), torch.ones(3), None)
    with pytest.raises(ValueError, match="shape"):
        convert_linears_fp8(_dit_like(), parts=("self",), per_channel=True, stored=stored)
    from safetensors.torch import save_file
    other = str(tmp_path / "other.safetensors")
    save_file({"x": torch.zeros(2)}, other)
    with pytest.raises(ValueError, match="not a"):
        load_fp8_weights(other)


def test_fp8_weights_from_other_checkpoint_refused(tmp_path):
    """A weight file saved from one checkpoint is refused for a model of the
    same architecture whose weights (or biases) differ: the per-module source
    fingerprints in the file's metadata do not match."""
    from flashvsr_sm89_ops.fp8_linear import (convert_linears_fp8, load_fp8_weights,
                                              save_fp8_weights, source_fingerprint)
    src = _dit_like(seed=0)
    convert_linears_fp8(src, parts=("self", "ffn"), stored=_stored_for(src, per_channel=False))
    path = str(tmp_path / "w.safetensors")
    save_fp8_weights(src, path)
    back = load_fp8_weights(path)
    assert convert_linears_fp8(_dit_like(seed=0), parts=("self", "ffn"), stored=back) == 12
    with pytest.raises(ValueError, match="fingerprint"):
        convert_linears_fp8(_dit_like(seed=1), parts=("self", "ffn"), stored=back)
    bias_only = _dit_like(seed=0)
    with torch.no_grad():
        bias_only.blocks[1].ffn[0].bias[3] += 1e-3
    with pytest.raises(ValueError, match="blocks.1.ffn.0"):
        convert_linears_fp8(bias_only, parts=("self", "ffn"), stored=back)
    # the fingerprint sees a swap of two weights (a plain sum would not)
    w = torch.randn(4, 8)
    w2 = w.clone()
    w2[0, 0], w2[3, 7] = w[3, 7], w[0, 0]
    assert source_fingerprint(w, None) != source_fingerprint(w2, None)
    assert source_fingerprint(w, None) == source_fingerprint(w.clone(), None)


def test_enable_loads_stored_fp8_weights(tmp_path, monkeypatch):
    import flashvsr_sm89_ops as f
    from flashvsr_sm89_ops.fp8_linear import convert_linears_fp8, save_fp8_weights
    src = _dit_like(seed=4)
    convert_linears_fp8(src, parts=("self", "ffn"), stored=_stored_for(src, per_channel=False))
    path = str(tmp_path / "w.safetensors")
    save_fp8_weights(src, path)
    pipe = FakePipe()
    pipe.model = _dit_like(seed=4)
    monkeypatch.setenv("FS89_FP8", "self")
    monkeypatch.setenv("FS89_FP8_WEIGHTS", path)
    applied = f.enable(pipe, dit_module=make_fake_dit(), verbose=False)
    assert applied["fp8_weights"] == "loaded" and applied["fp8_linears"] == 8
    assert torch.equal(pipe.model.blocks[1].self_attn.o.weight.view(torch.uint8),
                       src.blocks[1].self_attn.o.weight.view(torch.uint8))


def test_window_path_shape_guard():
    """The copy-free self-attention path (F2) takes batch-1 bf16 GPU input in
    whole 2x8x8 windows only; anything else keeps the reference's sequence."""
    from flashvsr_sm89_ops.integrate import _window_path_ok
    x = torch.empty(1, 2 * 16 * 24, 256, dtype=torch.bfloat16)
    assert not _window_path_ok(x, 2, 16, 24, 128)          # on the CPU
    # a stand-in exposing is_cuda, so the shape rules can be checked without a GPU
    class T:
        def __init__(self, shape, dtype=torch.bfloat16):
            self.shape, self.dtype, self.is_cuda = shape, dtype, True
    assert _window_path_ok(T((1, 768, 256)), 2, 16, 24, 128)
    assert not _window_path_ok(T((2, 768, 256)), 2, 16, 24, 128)           # batch 2
    assert not _window_path_ok(T((1, 768, 256), torch.float32), 2, 16, 24, 128)
    assert not _window_path_ok(T((1, 3 * 16 * 24, 256)), 3, 16, 24, 128)  # odd frames
    assert not _window_path_ok(T((1, 2 * 12 * 24, 256)), 2, 12, 24, 128)  # h % 8
    assert not _window_path_ok(T((1, 768, 256)), 2, 16, 24, 64)            # head_dim
    assert not _window_path_ok(T((1, 768, 3072)), 2, 16, 24, 128)          # D > 1536


def test_kv_store_appends_in_place_and_copies_foreign_caches():
    """The copy-free self-attention's K/V store (integrate._kv_buffers), on
    CPU tensors: the cache it returns, passed back unchanged, gets the next
    chunk appended behind it in the same storage; a cache from elsewhere, or
    a full store, is copied into a new store once."""
    from flashvsr_sm89_ops.integrate import _kv_buffers
    D, L = 8, 4
    mod = types.SimpleNamespace(_fs89_kv=None)
    like = torch.empty(0, dtype=torch.bfloat16)
    kb, vb = _kv_buffers(mod, None, None, 0, L, D, like, True)   # first chunk
    assert kb.shape == (L, D) and mod._fs89_kv[0].shape[0] == L + 4 * L
    kb.copy_(torch.arange(L * D).view(L, D))
    vb.copy_(-torch.arange(L * D).view(L, D))
    ck, cv = kb[2:], vb[2:]                                       # the cache handed out
    k2, v2 = _kv_buffers(mod, ck, cv, 2, L, D, like, True)       # appended in place
    assert k2.untyped_storage().data_ptr() == kb.untyped_storage().data_ptr()
    assert torch.equal(k2[:2], ck) and torch.equal(v2[:2], cv) and k2.shape == (2 + L, D)
    foreign = ck.clone()
    k3, v3 = _kv_buffers(mod, foreign, cv.clone(), 2, L, D, like, True)
    assert k3.untyped_storage().data_ptr() != kb.untyped_storage().data_ptr()
    assert torch.equal(k3[:2], foreign)
    # fill the new store: 2 cached + 5 chunks of L fit in 2 + L + 4L rows; the next one does not
    ck, cv = k3[-2:], v3[-2:]
    base = k3.untyped_storage().data_ptr()
    for step in range(4):
        kk, vv = _kv_buffers(mod, ck, cv, 2, L, D, like, True)
        assert kk.untyped_storage().data_ptr() == base
        kk[2:].fill_(step)  # the new chunk's rows (the kernel would write them)
        vv[2:].fill_(-step)
        ck, cv = kk[-2:], vv[-2:]
    kk, vv = _kv_buffers(mod, ck, cv, 2, L, D, like, True)
    assert kk.untyped_storage().data_ptr() != base and torch.equal(kk[:2], ck)
    assert torch.equal(vv[:2], cv)
    # outside a stream no room is kept and nothing is remembered
    kb, _ = _kv_buffers(mod, None, None, 0, L, D, like, False)
    assert mod._fs89_kv is None and kb.untyped_storage().nbytes() == L * D * 2


def test_qkv_fusion_weight_assembly():
    """integrate._qkv_fused: one [3N, K] weight for the q/k/v FP8Linears,
    per-tensor scales expanded to per-column vectors of the same value,
    biases concatenated; rebuilt when a weight changes in place; refused
    when the three cannot share one GEMM (mixed activation granularity or
    bias presence, a non-FP8 projection)."""
    from flashvsr_sm89_ops.fp8_linear import FP8Linear
    from flashvsr_sm89_ops.integrate import _qkv_fused
    g = torch.Generator().manual_seed(0)

    def lin(scale, bias=True, per_token=False):
        w8 = torch.randint(0, 120, (4, 8), generator=g, dtype=torch.uint8)
        b = torch.randn(4, generator=g).to(torch.bfloat16) if bias else None
        return FP8Linear.from_quantized(w8, scale, b, per_token=per_token)

    mod = types.SimpleNamespace(q=lin(torch.tensor(0.5)), k=lin(torch.tensor(0.25)),
                                v=lin(torch.tensor([1.0, 2.0, 3.0, 4.0])))
    w3, s3, b3, per_token = _qkv_fused(mod)
    assert w3.shape == (12, 8) and not per_token
    assert torch.equal(w3.view(torch.uint8), torch.cat([mod.q.weight, mod.k.weight,
                                                          mod.v.weight]).view(torch.uint8))
    assert torch.equal(s3, torch.tensor([0.5] * 4 + [0.25] * 4 + [1.0, 2.0, 3.0, 4.0]))
    assert torch.equal(b3, torch.cat([mod.q.bias, mod.k.bias, mod.v.bias]))
    assert _qkv_fused(mod)[0] is w3                       # cached
    with torch.no_grad():
        mod.k.weight.view(torch.uint8).zero_()            # in-place change: rebuilt
    assert not torch.equal(_qkv_fused(mod)[0].view(torch.uint8), w3.view(torch.uint8))
    assert _qkv_fused(types.SimpleNamespace(q=mod.q, k=mod.k, v=lin(torch.tensor(1.0),
                                                                   per_token=True))) is None
    assert _qkv_fused(types.SimpleNamespace(q=mod.q, k=mod.k, v=lin(torch.tensor(1.0),
                                                                   bias=False))) is None
    assert _qkv_fused(types.SimpleNamespace(q=mod.q, k=mod.k, v=torch.nn.Linear(8, 4))) is None


def test_rope_table_cache_follows_tensor_identity():
    """The complex128 -> (cos, sin) table cache never serves a table to a
    different freqs tensor, even one allocated at a freed tensor's address,
    and rebuilds after an in-place change."""
    from flashvsr_sm89_ops.fused_rms_rope import _freqs_table
    g = torch.Generator().manual_seed(3)
    for _ in range(20):
        ang = torch.rand(48, 64, generator=g, dtype=torch.float64) * 6.28
        fr = torch.polar(torch.ones_like(ang), ang)           # complex128, like Wan's freqs
        t = _freqs_table(fr)
        want = torch.view_as_real(fr.to(torch.complex64))
        assert torch.equal(t, want)
        assert _freqs_table(fr) is t                          # same live tensor: cached
        del fr, t                                             # the next one may reuse the address
    fr = torch.polar(torch.ones(8, 64, dtype=torch.float64), torch.zeros(8, 64, dtype=torch.float64))
    t0 = _freqs_table(fr)
    fr.mul_(1j)                                               # in place: rotate by 90 degrees
    t1 = _freqs_table(fr)
    assert t1 is not t0 and torch.equal(t1, torch.view_as_real(fr.to(torch.complex64)))


def test_qkv_fusion_not_fooled_by_reused_addresses():
    """A q/k/v FP8Linear replaced by a new one (whose tensors may sit at the
    freed tensors' addresses, version 0 again) rebuilds the fused weight."""
    import gc
    from flashvsr_sm89_ops.fp8_linear import FP8Linear
    from flashvsr_sm89_ops.integrate import _qkv_fused
    g = torch.Generator().manual_seed(1)

    def lin(fill):
        w8 = torch.full((4, 8), fill, dtype=torch.uint8)
        return FP8Linear.from_quantized(w8, torch.tensor(0.5), torch.zeros(4, dtype=torch.bfloat16))

    mod = types.SimpleNamespace(q=lin(1), k=lin(2), v=lin(3))
    for fill in range(4, 24):
        _qkv_fused(mod)
        mod.k = None
        gc.collect()
        mod.k = lin(fill)
        w3 = _qkv_fused(mod)[0]
        assert torch.equal(w3[4:8].view(torch.uint8), torch.full((4, 8), fill, dtype=torch.uint8))


def test_bsa_wrapper_size_checks():
    """Host-side checks of block_sparse_attention_strided that run before the
    launch: tensor extents at the given strides, the block index's size and
    dtype (a mismatch would make the kernel read out of bounds)."""
    from flashvsr_sm89_ops.lcsa.hip_lcsa import _check_extent, _check_index
    H, D, NQ = 2, 128, 3
    q = torch.empty(NQ * 128, H * D, dtype=torch.bfloat16)
    _check_extent(q, NQ * 128, H * D, D, H, D, "q")
    _check_extent(q[1:], NQ * 128 - 1, H * D, D, H, D, "q")            # a view: its own extent
    with pytest.raises(ValueError, match="q: 384 tokens"):
        _check_extent(q[1:], NQ * 128, H * D, D, H, D, "q")
    with pytest.raises(ValueError, match="storage holds"):
        _check_extent(q, NQ * 128, H * D, D, H + 1, D, "q")           # one head too many
    # column slice of a fused [L, 3D] tensor: rows 3D apart, the last slice ends at the end
    qkv = torch.empty(NQ * 128, 3 * H * D, dtype=torch.bfloat16)
    _check_extent(qkv[:, 2 * H * D:], NQ * 128, 3 * H * D, D, H, D, "v")
    with pytest.raises(ValueError):
        _check_extent(qkv[:, 2 * H * D + 8:], NQ * 128, 3 * H * D, D, H, D, "v")
    sel = torch.zeros(H, NQ, 4, dtype=torch.int32)
    cnt = torch.zeros(H, NQ, dtype=torch.int32)
    _check_index(sel, cnt, 4, H, NQ)
    with pytest.raises(ValueError, match="does not cover"):
        _check_index(sel, cnt, 5, H, NQ)                                # maxk beyond sel rows
    with pytest.raises(ValueError, match="does not cover"):
        _check_index(sel, cnt[:, :2].contiguous(), 4, H, NQ)
    with pytest.raises(TypeError):
        _check_index(sel.long(), cnt, 4, H, NQ)
    with pytest.raises(ValueError, match="contiguous"):
        _check_index(sel.transpose(0, 1), cnt, 4, H, NQ)


def test_convert_ffn_fp8_swap_and_assertion():
    """convert_ffn_fp8 (reference fp8_ffn.py:99-115): every blocks.<i>.ffn
    Sequential over FP8Linears becomes an FP8FFN holding those two modules;
    FFNs whose Linears are not FP8 yet raise AssertionError; a second call
    replaces nothing; modules outside blocks.<i>.ffn are untouched."""
    from flashvsr_sm89_ops.fp8_ffn import FP8FFN, convert_ffn_fp8
    from flashvsr_sm89_ops.fp8_linear import FP8Linear, convert_linears_fp8
    plain = _dit_like()
    with pytest.raises(AssertionError, match="blocks.0.ffn"):
        convert_ffn_fp8(plain)
    model = _dit_like()
    model.head = torch.nn.Sequential(torch.nn.Linear(16, 16), torch.nn.GELU(),
                                     torch.nn.Linear(16, 16))
    convert_linears_fp8(model, parts=("ffn",), stored=_stored_for(model, per_channel=False))
    ups = [b.ffn[0] for b in model.blocks]
    downs = [b.ffn[2] for b in model.blocks]
    assert convert_ffn_fp8(model) == 2
    for b, up, down in zip(model.blocks, ups, downs):
        assert isinstance(b.ffn, FP8FFN) and b.ffn.lin0 is up and b.ffn.lin2 is down
        assert isinstance(up, FP8Linear) and isinstance(down, FP8Linear)
    assert isinstance(model.head, torch.nn.Sequential)
    assert convert_ffn_fp8(model) == 0


def _gpu_only(fn, *a, **k):
    """A call whose arguments pass every host-side check reaches the GPU
    check, which rejects CPU tensors."""
    with pytest.raises(RuntimeError, match="GPU only"):
        fn(*a, **k)


def test_fp8_gemm_size_checks():
    """fp8_gemm rejects, before any launch, every operand whose size the
    kernel would trust: bias length, out's shape / dtype / column stride,
    the row-max partials' length and the gate-add residual and gate (the
    checks torch._scaled_mm makes behind reference fp8_linear.py:28-30)."""
    from flashvsr_sm89_ops import _lib
    from flashvsr_sm89_ops.fp8_linear import fp8_gemm
    M, N, K = 5, 300, 64
    e4 = torch.float8_e4m3fn
    x8, w8 = torch.zeros(M, K, dtype=e4), torch.zeros(N, K, dtype=e4)
    s, ws = torch.ones(M), torch.ones(N)
    bf = torch.bfloat16
    _gpu_only(fp8_gemm, x8, s, w8, ws, torch.zeros(N, dtype=bf))
    with pytest.raises(ValueError, match="bias"):
        fp8_gemm(x8, s, w8, ws, torch.zeros(N - 1, dtype=bf))
    with pytest.raises(ValueError, match="bias"):
        fp8_gemm(x8, s, w8, ws, torch.zeros(1, N, dtype=bf))
    with pytest.raises(ValueError, match="K mismatch"):
        fp8_gemm(x8, s, torch.zeros(N, K + 16, dtype=e4), ws)
    with pytest.raises(ValueError, match="scale"):
        fp8_gemm(x8, torch.ones(M + 1), w8, ws)
    # out: shape, dtype, unit column stride; a wider row stride is fine
    _gpu_only(fp8_gemm, x8, s, w8, ws, out=torch.empty(M, N + 8, dtype=bf)[:, :N])
    with pytest.raises(ValueError, match="out must be"):
        fp8_gemm(x8, s, w8, ws, out=torch.empty(M, N - 1, dtype=bf))
    with pytest.raises(ValueError, match="out must be"):
        fp8_gemm(x8, s, w8, ws, out=torch.empty(N, M, dtype=bf).t())
    with pytest.raises(TypeError, match="out"):
        fp8_gemm(x8, s, w8, ws, out=torch.empty(M, N, dtype=torch.float16))
    with pytest.raises(ValueError, match="epilogue"):
        fp8_gemm(x8, s, w8, ws, epilogue=7)
    # row maxima: M * ceil(N / 128) fp32
    parts = (N + 127) // 128
    _gpu_only(fp8_gemm, x8, s, w8, ws, epilogue=_lib.EPI_ROWMAX,
              amax_part=torch.empty(M, parts))
    with pytest.raises(ValueError, match="amax_part"):
        fp8_gemm(x8, s, w8, ws, epilogue=_lib.EPI_ROWMAX)
    with pytest.raises(ValueError, match="amax_part"):
        fp8_gemm(x8, s, w8, ws, epilogue=_lib.EPI_ROWMAX, amax_part=torch.empty(M * parts - 1))
    # gate-add: res [M, N] with out's row stride, gate [N]
    res, gate = torch.zeros(M, N, dtype=bf), torch.zeros(N, dtype=bf)
    _gpu_only(fp8_gemm, x8, s, w8, ws, epilogue=_lib.EPI_GATE_ADD, res=res, gate=gate)
    with pytest.raises(ValueError, match="gate-add epilogue needs"):
        fp8_gemm(x8, s, w8, ws, epilogue=_lib.EPI_GATE_ADD, res=res)
    with pytest.raises(ValueError, match="res must be"):
        fp8_gemm(x8, s, w8, ws, epilogue=_lib.EPI_GATE_ADD, res=res[:-1], gate=gate)
    with pytest.raises(ValueError, match="res must be"):   # row stride differs from out's
        fp8_gemm(x8, s, w8, ws, out=torch.empty(M, N + 8, dtype=bf)[:, :N],
                 epilogue=_lib.EPI_GATE_ADD, res=res, gate=gate)
    with pytest.raises(ValueError, match="gate must"):
        fp8_gemm(x8, s, w8, ws, epilogue=_lib.EPI_GATE_ADD, res=res, gate=gate[:-1])


def test_row_op_size_checks():
    """fused_gate_add checks the residual against x; the RMSNorm(+RoPE)
    entry points check the weight length against D;
    FP8Linear.from_quantized checks the bias length."""
    from flashvsr_sm89_ops.fp8_linear import FP8Linear
    from flashvsr_sm89_ops.fused_adaln import fused_gate_add
    from flashvsr_sm89_ops.fused_rms_rope import (fused_rms_rope, fused_rms_rope_qk,
                                                  fused_rms_rope_qkv_rows)
    bf = torch.bfloat16
    B, L, D = 1, 6, 256
    x = torch.zeros(B, L, D, dtype=bf)
    gate = torch.zeros(B, 1, D, dtype=bf)
    _gpu_only(fused_gate_add, x, gate, torch.zeros_like(x))
    with pytest.raises(ValueError, match="residual"):
        fused_gate_add(x, gate, torch.zeros(B, L - 1, D, dtype=bf))
    w = torch.ones(D, dtype=bf)
    _gpu_only(fused_rms_rope, x, w, None, rope=False)
    with pytest.raises(ValueError, match="RMSNorm weight"):
        fused_rms_rope(x, torch.ones(D - 2, dtype=bf), None, rope=False)
    _gpu_only(fused_rms_rope_qk, x, x, w, w, None)
    with pytest.raises(ValueError, match="RMSNorm weight"):
        fused_rms_rope_qk(x, x, w, torch.ones(D + 2, dtype=bf), None)
    kv = torch.zeros(L, D, dtype=bf)
    rows = torch.arange(L, dtype=torch.int32)
    _gpu_only(fused_rms_rope_qkv_rows, x, x, x, w, w, None, kv, kv.clone(), rows)
    with pytest.raises(ValueError, match="RMSNorm weight"):
        fused_rms_rope_qkv_rows(x, x, x, torch.ones(1, dtype=bf), w, None, kv, kv.clone(), rows)
    codes = torch.zeros(8, 16, dtype=torch.float8_e4m3fn)
    FP8Linear.from_quantized(codes, torch.ones(8), torch.zeros(8, dtype=bf))
    with pytest.raises(ValueError, match="bias"):
        FP8Linear.from_quantized(codes, torch.ones(8), torch.zeros(7, dtype=bf))


def test_per_token_ffn_guard():
    """The DiT block feeds per-token codes straight into the FFN GEMMs only
    when both FFN linears quantise activations per token; an FFN converted
    with per-tensor activation scales keeps FP8FFN.forward."""
    from flashvsr_sm89_ops.fp8_ffn import FP8FFN
    from flashvsr_sm89_ops.fp8_linear import FP8Linear
    from flashvsr_sm89_ops.integrate import _per_token_ffn

    def lin(n, k, per_token):
        return FP8Linear.from_quantized(torch.zeros(n, k, dtype=torch.float8_e4m3fn),
                                        torch.ones(n), per_token=per_token)
    assert _per_token_ffn(FP8FFN(lin(32, 16, True), lin(16, 32, True)))
    assert not _per_token_ffn(FP8FFN(lin(32, 16, False), lin(16, 32, False)))
    assert not _per_token_ffn(FP8FFN(lin(32, 16, True), lin(16, 32, False)))
    assert not _per_token_ffn(torch.nn.Sequential())


def test_enable_rewrites_old_format_fp8_weights(tmp_path, monkeypatch):
    """A weight file of an earlier format version is not an error for
    enable(): it warns, quantises again and overwrites the file with the
    current format; a file that is not an FP8 weight file at all is still
    refused (nothing of the user's is overwritten)."""
    import flashvsr_sm89_ops as f
    from safetensors import safe_open
    from safetensors.torch import save_file
    from flashvsr_sm89_ops.fp8_linear import FP8_WEIGHTS_FORMAT, FP8WeightsFormatError, \
        load_fp8_weights
    path = str(tmp_path / "w.safetensors")
    save_file({"blocks.0.self_attn.q.weight": torch.zeros(2, 2, dtype=torch.uint8)}, path,
              metadata={"format": "flashvsr-fp8-weights/1"})
    with pytest.raises(FP8WeightsFormatError, match="delete it"):
        load_fp8_weights(path)
    # quantising needs the GPU: on the CPU the conversion takes stand-in codes
    import flashvsr_sm89_ops.integrate as integ
    real = integ.convert_linears_fp8

    def convert(model, parts, per_channel, per_token, stored):
        assert stored is None                         # the old file was not used
        return real(model, parts=parts, per_channel=per_channel, per_token=per_token,
                    stored=_stored_for(model, per_channel))
    monkeypatch.setattr(integ, "convert_linears_fp8", convert)
    pipe = FakePipe()
    pipe.model = _dit_like(seed=4)
    monkeypatch.setenv("FS89_FP8", "self")
    monkeypatch.setenv("FS89_FP8_WEIGHTS", path)
    with pytest.warns(UserWarning, match="quantising again"):
        applied = f.enable(pipe, dit_module=make_fake_dit(), verbose=False)
    assert applied["fp8_weights"] == "saved" and applied["fp8_linears"] == 8
    with safe_open(path, framework="pt") as fh:
        assert fh.metadata()["format"] == FP8_WEIGHTS_FORMAT
    other = str(tmp_path / "other.safetensors")
    save_file({"x": torch.zeros(2)}, other)
    pipe2 = FakePipe()
    pipe2.model = _dit_like(seed=4)
    monkeypatch.setenv("FS89_FP8_WEIGHTS", other)
    with pytest.raises(ValueError, match="not a"):
        f.enable(pipe2, dit_module=make_fake_dit(), verbose=False)


def test_bsa_window_entry_argument_checks():
    """fvsr_bsa_fwd_window rejects a grid that is not whole (2, 8, 8)
    windows covering NQ blocks, and raster k/v with NK != NQ, before anything
    is launched (so fake pointers are never touched); the Python wrapper
    raises ValueError for the same cases."""
    from flashvsr_sm89_ops import _lib
    from flashvsr_sm89_ops.lcsa.hip_lcsa import block_sparse_attention_strided
    L = _lib.lib()
    p = 16

    def call(frames, height, width, NQ=12, NK=12, kv_raster=1, H=2):
        return L.fvsr_bsa_fwd_window(p, p, p, p, 256, 128, 256, 128, 256, 128, p, p, NK, H, NQ,
                                     NK, 128, 0.1, frames, height, width, kv_raster, None)
    assert call(3, 16, 24) == _lib.FVSR_EINVAL           # odd frame count
    assert call(4, 12, 24) == _lib.FVSR_EINVAL           # height not a multiple of 8
    assert call(4, 16, 20) == _lib.FVSR_EINVAL           # width not a multiple of 8
    assert call(4, 16, 32) == _lib.FVSR_EINVAL           # 16 windows, NQ = 12
    assert call(4, 16, 24, NK=13) == _lib.FVSR_EINVAL    # raster k/v: NK must equal NQ
    assert call(4, 16, 24, NQ=0, NK=0) == _lib.FVSR_EINVAL
    assert call(0, 16, 24, NQ=0, NK=0, H=2) == _lib.FVSR_OK   # nothing to do
    bf = torch.bfloat16
    q = torch.zeros(1536, 256, dtype=bf)
    sel = torch.zeros(2, 12, 12, dtype=torch.int32)
    cnt = torch.zeros(2, 12, dtype=torch.int32)
    with pytest.raises(ValueError, match="window grid"):
        block_sparse_attention_strided(q, q, q, None, heads=2, head_dim=128, q_strides=(256, 128),
                                       kv_strides=(256, 128), out=q, index=(sel, cnt, 12),
                                       window=(4, 16, 32, True))
    with pytest.raises(ValueError, match="not both"):
        block_sparse_attention_strided(q, q, q, None, heads=2, head_dim=128, q_strides=(256, 128),
                                       kv_strides=(256, 128), out=q, index=(sel, cnt, 12),
                                       window=(4, 16, 24, True), q_map=cnt, kv_map=cnt)
