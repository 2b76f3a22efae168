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
    """A stand-in for diffsynth.models.wan_video_dit with the rebound classes,
    stock helpers in torch, and the upstream forward signatures."""
    dit = types.ModuleType("fake_wan_video_dit")

    class SelfAttention(torch.nn.Module):
        def forward(self, x, freqs, f=None, h=None, w=None, local_num=None, topk=None,
                    train_img=False, block_id=None, kv_len=None, is_full_block=False,
                    is_stream=False, pre_cache_k=None, pre_cache_v=None, local_range=9):
            raise AssertionError("stock forward must be rebound")

    class CrossAttention(torch.nn.Module):
        def forward(self, x, y, is_stream=False):
            raise AssertionError

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
            raise AssertionError

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
    stock = dit.SelfAttention.forward
    monkeypatch.setenv("FS89_FP8", "")
    applied = f.enable(FakePipe(), dit_module=dit)
    assert applied == {"fused_rope": True, "fused_adaln": True, "lcsa_backend": "hip"}
    assert dit.SelfAttention.forward is not stock and dit._FS89_PATCHED
    assert dit.FUSED_ROPE_FN is f.fused_rms_rope
    assert dit.FUSED_ADALN == (f.fused_ln_modulate, f.fused_gate_add)
    assert "[flashvsr-mi355x-ops] enabled" in capsys.readouterr().out
    rebound = dit.DiTBlock.forward
    monkeypatch.setenv("FS89_FUSED_ROPE", "0")
    monkeypatch.setenv("FS89_FUSED_ADALN", "0")
    applied = f.enable(FakePipe(), dit_module=dit, verbose=False)
    assert applied["fused_rope"] is False and dit.FUSED_ROPE_FN is None and dit.FUSED_ADALN is None
    assert dit.DiTBlock.forward is rebound  # not rebound twice
    with pytest.raises(ValueError):
        f.enable(FakePipe(), dit_module=dit, scale_granularity="block")
    monkeypatch.setitem(sys.modules, "diffsynth", None)
    with pytest.raises(ImportError, match="wan_video_dit"):
        integrate.enable(FakePipe())


def test_stock_branch_dit_block_on_cpu(monkeypatch):
    """With the fused flags off, the rebound DiTBlock.forward is the stock
    math: AdaLN(shift, scale) order, gate, cross-attention residual."""
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
    out = blk(x, None, t_mod, None, 1, 1, 5)
    sh, sc, g, sh2, sc2, g2 = (blk.modulation + t_mod).chunk(6, dim=1)
    ln = torch.nn.functional.layer_norm
    a_in = ln(x, (16,), eps=1e-6) * (1 + sc) + sh
    torch.testing.assert_close(seen["attn_in"], a_in)
    x1 = x + g * (a_in * 2)
    x1 = x1 + (ln(x1, (16,), weight=blk.norm3.weight, bias=blk.norm3.bias, eps=1e-6) * 0 + 1)
    ref = x1 + g2 * ((ln(x1, (16,), eps=1e-6) * (1 + sc2) + sh2) - 1)
    torch.testing.assert_close(out, ref)


def test_window_token_map_matches_partition():
    from flashvsr_sm89_ops.block import window_token_map
    from oracle import oracle as O
    f, h, w = 4, 16, 24
    x = np.arange(f * h * w, dtype=np.float32).reshape(1, f, h, w, 1)
    xw = O.window_partition(x).reshape(-1)
    assert np.array_equal(window_token_map(f, h, w).numpy(), xw.astype(np.int32))


def test_stock_branch_cross_attention_on_cpu(monkeypatch):
    """The rebound CrossAttention.forward keeps the DiT's own attention where
    the HIP kernel does not apply (here: CPU tensors), with the stock RMSNorm
    when the fused flag is off (integrate.py:132-143)."""
    import flashvsr_sm89_ops as f
    from flashvsr_sm89_ops.cross_attn import supported
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
    q, k, v = seen["args"]
    torch.testing.assert_close(q, ca.q(x) * 3)
    assert k is ca.cache_k and v is ca.cache_v
    torch.testing.assert_close(out, ca.o(ca.q(x) * 3 + 1))
    assert not supported(q, k, v, 2)


def _dit_like(dim=16, ffn=32):
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


def test_enable_loads_stored_fp8_weights(tmp_path, monkeypatch):
    import flashvsr_sm89_ops as f
    from flashvsr_sm89_ops.fp8_linear import convert_linears_fp8, save_fp8_weights
    src = _dit_like()
    convert_linears_fp8(src, parts=("self", "ffn"), stored=_stored_for(src, per_channel=False))
    path = str(tmp_path / "w.safetensors")
    save_fp8_weights(src, path)
    pipe = FakePipe()
    pipe.model = _dit_like()
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
