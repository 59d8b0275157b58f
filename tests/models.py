"""Small models the suite compiles under every pass configuration.

Each exercises one thing the front end must get right: pointwise chains of
two inputs, broadcasting operands, an FFN with LayerNorm and GELU, a masked
softmax, LayerNorm followed by an affine of its own, fused-projection
attention, a pre-norm transformer block at two batch shapes, masking with
where/clamp/compare/cast into a reduction, and one producer with several
consumers (the recompute case). Seeded 0; the golden schedules were written
by the reference compiler from exactly these modules
(``tests/golden/dump_reference.py``).
"""

import torch
import torch.nn as nn
import torch.nn.functional as F


class TwoInputChain(nn.Module):
    """Pointwise ops over two same-shaped inputs, one fused kernel."""

    def forward(self, a, b):
        s = torch.sigmoid(a) * b - 0.5
        return torch.relu(s + a * a) / (1.0 + b.abs())


class BiasScaleTanh(nn.Module):
    """A [16] bias and an [8, 1] scale broadcast over [4, 8, 16]."""

    def forward(self, x, bias, scale):
        return torch.tanh(scale * x - bias) + 0.25


class FeedForward(nn.Module):
    """LayerNorm -> Linear -> GELU -> Linear, plus the residual."""

    def __init__(self, width=32, hidden=64):
        super().__init__()
        self.norm = nn.LayerNorm(width)
        self.up = nn.Linear(width, hidden)
        self.down = nn.Linear(hidden, width)

    def forward(self, x):
        return self.down(F.gelu(self.up(self.norm(x)))) + x


class ScaledMaskedSoftmax(nn.Module):
    """Scale, add a [B, 1, 1, T] mask, softmax over the last dim."""

    def forward(self, scores, mask):
        return torch.softmax(scores / 8.0 + mask, dim=-1)


class NormThenAffine(nn.Module):
    """LayerNorm with its own affine, then a second elementwise affine."""

    def __init__(self, width=32):
        super().__init__()
        self.norm = nn.LayerNorm(width)
        self.gain = nn.Parameter(torch.randn(width))
        self.shift = nn.Parameter(torch.randn(width))

    def forward(self, x):
        return self.shift + self.gain * self.norm(x)


class FusedQKVAttention(nn.Module):
    """One projection to q, k and v, split into heads, softmax attention,
    heads merged back and projected."""

    def __init__(self, width=32, heads=4):
        super().__init__()
        self.heads = heads
        self.in_proj = nn.Linear(width, 3 * width)
        self.out_proj = nn.Linear(width, width)

    def forward(self, x):
        b, t, w = x.shape
        dh = w // self.heads
        q, k, v = (p.reshape(b, t, self.heads, dh).permute(0, 2, 1, 3)
                   for p in self.in_proj(x).split(w, dim=-1))
        weights = torch.softmax(q @ k.transpose(2, 3) * dh ** -0.5, dim=-1)
        merged = (weights @ v).permute(0, 2, 1, 3).reshape(b, t, w)
        return self.out_proj(merged)


class PreNormBlock(nn.Module):
    """x + attn(norm(x)), then + mlp(norm(x))."""

    def __init__(self, width=32, heads=4):
        super().__init__()
        self.norm_a = nn.LayerNorm(width)
        self.attn = FusedQKVAttention(width, heads)
        self.norm_m = nn.LayerNorm(width)
        self.mlp_in = nn.Linear(width, 4 * width)
        self.mlp_out = nn.Linear(4 * width, width)

    def forward(self, x):
        h = x + self.attn(self.norm_a(x))
        return h + self.mlp_out(F.gelu(self.mlp_in(self.norm_m(h))))


class WhereClampSum(nn.Module):
    """A comparison mask, where with a filled tensor, clamp, a cast of a
    comparison, and a row sum."""

    def forward(self, x, gate):
        picked = torch.where(gate < 0.3, torch.full_like(x, 5e3), x)
        positive = (x > 0).to(x.dtype)
        return (picked.clamp(-2.0, 2.0) * positive).sum(dim=-1)


class SharedProducer(nn.Module):
    """One cheap producer read by three consumers."""

    def forward(self, x):
        e = torch.exp(x * -0.25)
        return (e + 2.0) * (e * 3.0) - (e - 1.0)


def all_models():
    """(name, module, example inputs) for every model, seeded 0."""
    torch.manual_seed(0)
    return [
        ("two_input_chain", TwoInputChain(), (torch.randn(4, 16), torch.randn(4, 16))),
        ("bias_scale_tanh", BiasScaleTanh(),
         (torch.randn(4, 8, 16), torch.randn(16), torch.randn(8, 1))),
        ("feed_forward", FeedForward(), (torch.randn(4, 32),)),
        ("masked_softmax", ScaledMaskedSoftmax(), (torch.randn(2, 4, 8, 8), torch.randn(2, 1, 1, 8))),
        ("norm_affine", NormThenAffine(), (torch.randn(6, 32),)),
        ("attention", FusedQKVAttention(), (torch.randn(2, 8, 32),)),
        ("pre_norm_block", PreNormBlock(), (torch.randn(2, 8, 32),)),
        ("pre_norm_block_b8", PreNormBlock(), (torch.randn(8, 16, 32),)),
        ("where_clamp_sum", WhereClampSum(), (torch.randn(4, 8), torch.rand(4, 8))),
        ("shared_producer", SharedProducer(), (torch.randn(6, 12),)),
    ]


def get(name):
    return next(t for t in all_models() if t[0] == name)
