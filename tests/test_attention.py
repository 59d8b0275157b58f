"""Attention fusion (``Config.fused_attention``, an opt-in schedule change):
what the pass fuses and refuses, the oracle's execution of the fused kernel
against float64 attention, and the generated MFMA kernel's shape."""

from __future__ import annotations

import math

import pytest
import torch
import torch.nn as nn

from mlc.api import build_pipeline
from mlc.bench.models import build
from mlc.codegen.hip_backend import build_module
from mlc.config import Config
from mlc.ir.capture import capture
from mlc.kernels import AttentionKernel
from mlc.passes.memory_planning import verify
from mlc.runtime import native
from oracle import compile_reference
from workload_cache import graph_of

ATTN = Config(fused_attention=True, cuda_graphs=False)
ALL = Config(fused_attention=True, merge_parallel_gemms=True, gemm_epilogue=True,
             layout_selection=True, cuda_graphs=False)


class Attention(nn.Module):
    """softmax(q k^T / sqrt(d) + mask) v over [B, H, T, D] heads."""

    def forward(self, q, k, v, mask):
        scores = (q @ k.transpose(-2, -1)) / math.sqrt(q.shape[-1]) + mask
        return scores.softmax(dim=-1) @ v


class ScoresOut(Attention):
    def forward(self, q, k, v, mask):
        scores = (q @ k.transpose(-2, -1)) / math.sqrt(q.shape[-1]) + mask
        return scores.softmax(dim=-1) @ v, scores


class LogSoftmax(Attention):
    """Not an ``exp(x - max) / sum`` row: only the single-pass kernel, which
    renders any reduction, could take it."""

    def forward(self, q, k, v, mask):
        scores = (q @ k.transpose(-2, -1)) / math.sqrt(q.shape[-1]) + mask
        return torch.log_softmax(scores.float(), dim=-1).to(q.dtype) @ v


def _inputs(b, h, t, tk, d, dtype=torch.float16, seed=0):
    g = torch.Generator().manual_seed(seed)
    q = torch.randn(b, h, t, d, generator=g).to(dtype)
    k = torch.randn(b, h, tk, d, generator=g).to(dtype)
    v = torch.randn(b, h, tk, d, generator=g).to(dtype)
    mask = torch.where(torch.rand(b, 1, 1, tk, generator=g) < 0.2, -10000.0, 0.0).to(dtype)
    return q, k, v, mask


def _attention(sched):
    return [k for k in sched.kernels if isinstance(k, AttentionKernel)]


@pytest.mark.parametrize("key,cfg,n", [("C2", Config(fused_attention=True), 12),
                                       ("C3", Config(fused_attention=True), 12),
                                       ("C4", Config(fused_attention=True), 12),
                                       ("C2", ALL, 12), ("C4", ALL, 12),
                                       ("C5", Config(fused_attention=True), 12),
                                       ("C1", Config(fused_attention=True), 0)])
def test_workloads_fuse_every_layer(key, cfg, n):
    base = build_pipeline(graph_of(key), Config())
    sched = build_pipeline(graph_of(key), cfg)
    assert len(_attention(sched)) == n
    if n:
        # three kernels became one per layer
        assert len(sched.kernels) <= len(base.kernels) - 2 * n
        assert not verify(list(sched.plan.live_ranges.values()), sched.plan.offsets)
        live = {v.buffer.name for k in sched.kernels for v in k.reads() + k.writes()}
        for a in _attention(sched):
            assert a.softmax.inputs[a.score_slot].value.buffer.name not in live
            assert a.softmax.outputs[0].value.buffer.name not in live


def test_refused_when_scores_escape_or_shapes_do_not_fit():
    q, k, v, m = _inputs(1, 2, 32, 32, 64)
    assert len(_attention(build_pipeline(capture(ScoresOut(), (q, k, v, m)), ATTN))) == 0
    q, k, v, m = _inputs(1, 2, 160, 160, 64)  # too long to hold, not whole 64-key blocks
    assert len(_attention(build_pipeline(capture(Attention(), (q, k, v, m)), ATTN))) == 0
    q, k, v, m = _inputs(1, 2, 32, 256, 64)  # key-blocked, but not a softmax
    assert len(_attention(build_pipeline(capture(LogSoftmax(), (q, k, v, m)), ATTN))) == 0
    assert len(_attention(build_pipeline(capture(Attention(), (q, k, v, m)), ATTN))) == 1
    q, k, v, m = _inputs(1, 2, 32, 32, 64, torch.float32)
    assert len(_attention(build_pipeline(capture(Attention(), (q, k, v, m)), ATTN))) == 0
    q, k, v, m = _inputs(1, 2, 32, 32, 64, torch.bfloat16)  # the bf16 MFMA takes these
    assert len(_attention(build_pipeline(capture(Attention(), (q, k, v, m)), ATTN))) == 1
    q, k, v, m = _inputs(1, 2, 32, 48, 64)  # keys not a multiple of 32
    assert len(_attention(build_pipeline(capture(Attention(), (q, k, v, m)), ATTN))) == 0
    q, k, v, m = _inputs(1, 2, 32, 32, 48)  # head size not a multiple of 32
    assert len(_attention(build_pipeline(capture(Attention(), (q, k, v, m)), ATTN))) == 0


@pytest.mark.parametrize("shape", [(2, 3, 32, 32, 64), (1, 2, 80, 96, 32), (1, 1, 16, 128, 128),
                                   (1, 2, 48, 256, 64), (2, 1, 16, 192, 32)])
def test_oracle_fused_attention_matches_float64(shape):
    """The oracle's fused kernel (fp32 products rounded to fp16 scores, the
    reduction's steps, fp16 probabilities, fp32 products) against attention
    computed in float64 from the same fp16 inputs: within 2e-3 of the largest
    output, and as close as the unfused schedule's oracle. A transposed
    operand, a dropped scale or mask, or a wrong row mapping fails this."""
    args = _inputs(*shape)
    model = Attention()
    sched = build_pipeline(capture(model, args), ATTN)
    assert len(_attention(sched)) == 1
    got = compile_reference(model, args, ATTN)(*args)
    unfused = compile_reference(model, args, Config(cuda_graphs=False))(*args)
    exact = model(*(a.double() for a in args))
    scale = exact.abs().max().item()
    err = (got.double() - exact).abs().max().item() / scale
    err_unfused = (unfused.double() - exact).abs().max().item() / scale
    print(shape, f"fused oracle vs float64 {err:.2e}, unfused {err_unfused:.2e}")
    assert err <= 2e-3


@pytest.mark.parametrize("shape", [(2, 3, 32, 32, 64), (1, 2, 80, 96, 32), (1, 2, 48, 256, 64),
                                   (2, 1, 16, 192, 128)])
def test_oracle_bf16_fused_attention_matches_float64(shape):
    """The same check in bf16 (8 significand bits, so the bar is wider):
    within 1.5e-2 of the largest output and within twice the unfused
    schedule's error."""
    args = _inputs(*shape, dtype=torch.bfloat16, seed=3)
    model = Attention()
    sched = build_pipeline(capture(model, args), ATTN)
    assert [a.q.dtype for a in _attention(sched)] == [torch.bfloat16]
    got = compile_reference(model, args, ATTN)(*args)
    unfused = compile_reference(model, args, Config(cuda_graphs=False))(*args)
    exact = model(*(a.double() for a in args))
    scale = exact.abs().max().item()
    err = (got.double() - exact).abs().max().item() / scale
    err_unfused = (unfused.double() - exact).abs().max().item() / scale
    assert err <= 1.5e-2
    assert err <= max(1.5e-2, 2 * err_unfused)


def test_bf16_kernels_bind_the_bf16_types():
    """The emitter writes one kernel text over ``e16``/``v8``/``v4``; a bf16
    head binds them to ``__bf16`` vectors, whose ``mlc::mfma_16x16x32``
    overload is the bf16 MFMA."""
    for shape in ((2, 3, 32, 32, 64), (1, 2, 48, 256, 64)):
        args = _inputs(*shape, dtype=torch.bfloat16)
        sched = build_pipeline(capture(Attention(), args), ATTN)
        mod = build_module(sched, ATTN)
        body = mod.functions[mod.launches[_attention(sched)[0].name].symbol]
        assert "using e16 = __bf16;" in body and "using v8 = mlc::bf16x8;" in body
        assert "mlc::f16" not in body and "half" not in body


def test_oracle_fused_models_match_unfused():
    for name in ("bert-small", "gpt-small"):
        model, args = build(name, 2, 32, "cpu", torch.float16)
        base = compile_reference(model, args, Config(cuda_graphs=False))(*args)
        got = compile_reference(model, args, ATTN)(*args)
        torch.testing.assert_close(got.float(), base.float(), rtol=1e-2, atol=5e-2)


def test_generated_kernel_shape():
    sched = build_pipeline(graph_of("C2"), ALL)
    mod = build_module(sched, ALL)
    att = _attention(sched)
    specs = {mod.launches[a.name].symbol for a in att}
    assert len(specs) == 1, "every layer shares one attention function"
    spec = mod.launches[att[0].name]
    assert spec.meta["kind"] == "attention"
    # 12 heads: two waves per workgroup, four workgroups per head
    assert spec.block == 128 and spec.grid == 12 * 4
    assert spec.lds_bytes <= 64 * 1024
    body = mod.functions[spec.symbol]
    assert body.count("mlc::mfma_16x16x32(") == 2 and "using e16 = mlc::f16;" in body
    assert "__syncthreads();" in body and body.index("__syncthreads();") < body.index("return;")
    # C2's merged-qkv views are unit-stride along the head dim: 128-bit LDS stores
    assert body.count("*reinterpret_cast<v8*>(") == 2


def test_attention_module_cross_compiles_for_gfx950(tmp_path, monkeypatch):
    monkeypatch.setenv("MLC_CACHE_DIR", str(tmp_path))
    for shape, dt in (((1, 2, 80, 96, 32), torch.float16), ((2, 3, 32, 32, 64), torch.float16),
                      ((1, 2, 48, 256, 64), torch.bfloat16)):
        args = _inputs(*shape, dtype=dt)
        sched = build_pipeline(capture(Attention(), args), ATTN)
        mod = build_module(sched, ATTN)
        _, obj = native.compile_code_object(mod.source)
        assert obj.stat().st_size > 0


def test_operand_producers_write_the_mfma_layouts():
    """At batch > 1 BERT's K and V come from this compiler's own copy
    kernels; the pass has them write K as [bh][key][d] and V as
    [bh][d][key], so staging needs no transposing LDS stores."""
    sched = build_pipeline(graph_of("C4"), ALL)
    mod = build_module(sched, ALL)
    for a in _attention(sched):
        assert a.kt.layout.strides == (128 * 64, 1, 64)
        assert a.v.layout.strides == (128 * 64, 1, 128)
        body = mod.functions[mod.launches[a.name].symbol]
        # Q, K and V^T: one 128-bit LDS store per pack, K's rows in the key
        # order the score MFMAs read (mlc::krow), V^T unpermuted
        assert body.count("*reinterpret_cast<v8*>(") == 3 and "[u][j]" not in body
        assert body.count("*reinterpret_cast<v8*>(ks + mlc::krow(r) * ") == 1
        assert "*reinterpret_cast<v8*>(vt + r + c * " in body
        assert body.count("*reinterpret_cast<const v8*>(vrow") == 1
    assert not verify(list(sched.plan.live_ranges.values()), sched.plan.offsets)


def test_relaid_out_operands_compute_the_same_values(monkeypatch):
    """Moving K and V to other layouts changes where values are stored, not
    what is computed: the oracle's result is bit-identical with and without
    the relayout."""
    import mlc.passes.attention as attention

    model, args = build("bert-small", 2, 32, "cpu", torch.float16)
    sched = build_pipeline(capture(model, args), ATTN)
    assert all(a.v.layout.strides[1] == 1 for a in _attention(sched))
    got = compile_reference(model, args, ATTN)(*args)
    monkeypatch.setattr(attention, "_relayout_operands", lambda kernels, outputs: kernels)
    sched = build_pipeline(capture(model, args), ATTN)
    assert all(a.v.layout.strides[2] == 1 for a in _attention(sched))
    want = compile_reference(model, args, ATTN)(*args)
    assert torch.equal(got, want)


def test_context_copy_folds_into_the_attention_stores():
    """BERT's context copy ``[B*H, T, Dh] -> [B, T, H, Dh]`` only permutes the
    attention output, so the fused kernel writes the copy's buffer through
    the permutation and the copy disappears."""
    for key, n_pointwise in (("C2", 15), ("C4", 51)):
        sched = build_pipeline(graph_of(key), ALL)
        assert sched.counts()["pointwise"] == n_pointwise
        for a in _attention(sched):
            assert [n.op for n in a.nodes][-1] == "aten.clone.default"
            assert a.outputs[0].index.render().endswith("* 768 + (idx % 64))")
    # the oracle stores through the same permutation: compare with eager
    model, args = build("bert-small", 2, 32, "cpu", torch.float16)
    sched = build_pipeline(capture(model, args), ATTN)
    assert all(not a.outputs[0].index.is_identity() for a in _attention(sched))
    with torch.no_grad():
        want = model(*args)
    got = compile_reference(model, args, ATTN)(*args)
    torch.testing.assert_close(got.float(), want.float(), rtol=1e-2, atol=5e-2)


def test_long_rows_use_the_key_blocked_kernel():
    """GPT-2 b32 s512 (512 keys) is key-blocked: 64-key blocks streamed
    through LDS, next block's loads (K, V and the mask) in flight, one
    division by the row sum at the end; the scores and probabilities (201 MB
    each per layer) are gone from the arena."""
    base = build_pipeline(graph_of("C5"), Config())
    sched = build_pipeline(graph_of("C5"), Config(fused_attention=True))
    mod = build_module(sched, Config(fused_attention=True))
    att = _attention(sched)
    spec = mod.launches[att[0].name]
    assert spec.meta["mode"] == "blocked" and spec.meta["key_block"] == 64
    body = mod.functions[spec.symbol]
    assert "m_run" in body and "l_run" in body and "ml_run" in body
    # exponents in log2 units against the rounded RN(m log2 e): one fma each
    assert "__builtin_amdgcn_exp2f(__builtin_fmaf(x[t][i], 0x1.715476p+0f, -ml_sub))" in body
    assert body.count("__syncthreads();") == 3
    # 4 query tiles of 128 per head: tile j is the half-tiles j and 7 - j, so
    # under the causal mask every workgroup has the same unmasked keys
    assert "const int qa = (q0 / 128) * 64, qb = (7 - q0 / 128) * 64;" in body
    assert "const int qw = w < 4 ? qa + w * 16 : qb + (w - 4) * 16;" in body
    assert sched.arena_bytes < base.arena_bytes // 2


class _NoMask(nn.Module):
    def forward(self, q, k, v):
        return ((q @ k.transpose(-2, -1)) / math.sqrt(q.shape[-1])).softmax(-1) @ v


class _WhereMask(nn.Module):
    def forward(self, q, k, v, keep):
        s = (q @ k.transpose(-2, -1)) / math.sqrt(q.shape[-1])
        s = torch.where(keep, s, torch.tensor(torch.finfo(torch.float16).min, dtype=s.dtype))
        return s.softmax(-1) @ v


class _Fp32Softmax(nn.Module):
    def forward(self, q, k, v):
        s = (q @ k.transpose(-2, -1)) / math.sqrt(q.shape[-1])
        return s.float().softmax(-1).half() @ v


class _ScaledQ(nn.Module):
    def forward(self, q, k, v):
        return ((q * (1.0 / math.sqrt(q.shape[-1]))) @ k.transpose(-2, -1)).softmax(-1) @ v


class _MaskedFill(nn.Module):
    def forward(self, q, k, v, keep):
        s = (q @ k.transpose(-2, -1)) / math.sqrt(q.shape[-1])
        return s.masked_fill(~keep, float("-inf")).softmax(-1) @ v


def attention_patterns(t=128, tk=128):
    """How models write attention: no mask, a boolean causal mask through
    ``where`` or ``masked_fill``, the softmax in fp32, the scale on q."""
    q, k, v, _ = _inputs(2, 4, t, tk, 64)
    keep = torch.tril(torch.ones(t, tk, dtype=torch.bool), diagonal=tk - t)[None, None]
    return [("no_mask", _NoMask(), (q, k, v)), ("where_bool", _WhereMask(), (q, k, v, keep)),
            ("fp32_softmax", _Fp32Softmax(), (q, k, v)), ("scaled_q", _ScaledQ(), (q, k, v)),
            ("masked_fill", _MaskedFill(), (q, k, v, keep))]


def exact_attention(name, args):
    """float64 attention for a pattern of ``attention_patterns``."""
    q, k, v = (a.double() for a in args[:3])
    s = (q @ k.transpose(-2, -1)) / math.sqrt(q.shape[-1])
    if len(args) > 3:
        s = s.masked_fill(~args[3], float("-inf"))
    return s.softmax(-1) @ v


@pytest.mark.parametrize("tk", [128, 256])
def test_common_attention_patterns_fuse(tk):
    """Each way of writing attention becomes one attention kernel (single pass
    at 128 keys, key-blocked at 256), and the oracle's fused kernel is within
    2e-3 of float64."""
    for name, model, args in attention_patterns(tk, tk):
        sched = build_pipeline(capture(model, args), ATTN)
        assert len(_attention(sched)) == 1, name
        got = compile_reference(model, args, ATTN)(*args)
        exact = exact_attention(name, args)
        err = ((got.double() - exact).abs().max() / exact.abs().max()).item()
        assert err <= 2e-3, (name, err)


class _OffsetMask(nn.Module):
    """An additive fp16 mask read through a column slice at offset ``off``."""

    def __init__(self, off):
        super().__init__()
        self.off = off

    def forward(self, q, k, v, mask):
        tk = k.shape[-2]
        s = (q @ k.transpose(-2, -1)) / math.sqrt(q.shape[-1]) + mask[..., self.off:self.off + tk]
        return s.softmax(-1) @ v


def offset_mask_case(off, t=128, tk=128):
    q, k, v, _ = _inputs(2, 2, t, tk, 64)
    causal = torch.triu(torch.full((t, tk + 8), float("-inf")), diagonal=1 + off)
    return _OffsetMask(off), (q, k, v, causal.to(torch.float16)[None, None])


@pytest.mark.parametrize("tk", [128, 256])
@pytest.mark.parametrize("off,form", [(0, "mlc::pack<mlc::f16, 8>"), (4, "mlc::pack<mlc::f16, 4>"),
                                      (1, "for (int j = 0; j < 8; ++j)")])
def test_mask_words_load_at_the_widest_aligned_width(off, form, tk):
    """A lane's 8 mask words per 32-key chunk are one 16-byte load when the
    mask's rows are 16-byte aligned, two 8-byte loads at 8-byte alignment
    (a column slice at offset 4), and one load per word otherwise."""
    model, args = offset_mask_case(off, tk, tk)
    sched = build_pipeline(capture(model, args), ATTN)
    mod = build_module(sched, ATTN)
    att = _attention(sched)
    assert len(att) == 1
    body = mod.functions[mod.launches[att[0].name].symbol]
    assert form in body
    for wider in ("mlc::pack<mlc::f16, 8>", "mlc::pack<mlc::f16, 4>"):
        if wider == form:
            break
        assert f"const {wider} w_" not in body


def test_shifted_fast_exp_only_for_the_row_max():
    """``exp_fast_shift`` folds the rounding of ``m log2 e`` into a factor the
    normalisation cancels, which holds only when ``m`` is the row's maximum
    (an ``x - rowmax(x)`` of ``nonpositive_args``); the exp of any other
    difference is ``exp_fast`` of the rounded difference."""
    from mlc.codegen.hip_attention import _FastExpRenderer
    from mlc.ir.scalar import Call, Load

    diff = Call("sub", (Load(0), Load(1)))
    e = Call("exp", (diff,))

    def render(nonpos):
        r = _FastExpRenderer(lambda s: (f"x{s}", "float"), lambda n: (n, "float"), nonpos=nonpos)
        return r(e)[0]

    assert render(frozenset()) == "mlc::exp_fast((x0 - x1))"
    assert render(frozenset({diff})) == "mlc::exp_fast_shift(x0, x1)"
