"""The measured workloads as plain PyTorch modules (imports torch only).

From BASELINE.json's configurations:

* BERT-base: a post-norm encoder -- word, position and token-type
  embeddings summed and normalised; 12 layers of self-attention (separate q,
  k, v projections, an additive padding mask of ``(1 - mask) * min(fp32)``)
  and an erf-GELU MLP, each added back and LayerNorm'd (eps 1e-12); a tanh
  pooler over the first token. Hidden 768, 12 heads, FFN 3072, vocabulary
  30522, 512 positions.
* GPT-2 small: a pre-norm decoder -- token and position embeddings; 12
  blocks of causal self-attention (one fused qkv projection, an additive
  ``min(fp32)`` upper-triangle mask) and an erf-GELU MLP around pre-norms
  (eps 1e-5); a final norm and an untied vocabulary head. Hidden 768, 12
  heads, vocabulary 50257, 1024 positions.
* the FFN block of config 1: ``fc2(gelu_tanh(fc1(LayerNorm(x + r))))``.

Small variants (4 layers, width 512, 8 heads, vocabulary 8192) keep tests
fast. ``build`` seeds 0; ``init="normal"`` gives Linear and Embedding
weights N(0, 0.02), biases 0 and LayerNorm (1, 0) as the configurations
prescribe.
"""

from __future__ import annotations

from dataclasses import dataclass

import torch
import torch.nn as nn
import torch.nn.functional as F

FP32_MIN = torch.finfo(torch.float32).min


@dataclass(frozen=True)
class Shape:
    """Sizes of one transformer stack."""

    vocab: int
    positions: int
    layers: int = 12
    heads: int = 12
    width: int = 768
    ffn: int = 3072
    eps: float = 1e-12


class Attention(nn.Module):
    """Multi-head self-attention over ``[B, T, width]`` with an additive mask
    that broadcasts over ``[B, heads, T, T]``. ``fused`` keeps q, k and v in
    one projection (GPT-2), otherwise three (BERT); the output projection is
    the caller's."""

    def __init__(self, s: Shape, fused: bool):
        super().__init__()
        self.heads, self.head_width = s.heads, s.width // s.heads
        if fused:
            self.qkv = nn.Linear(s.width, 3 * s.width)
        else:
            self.q, self.k, self.v = (nn.Linear(s.width, s.width) for _ in range(3))
        self.fused = fused

    def _per_head(self, t: torch.Tensor) -> torch.Tensor:
        b, n, _ = t.shape
        return t.view(b, n, self.heads, self.head_width).transpose(1, 2)

    def forward(self, x: torch.Tensor, mask: torch.Tensor) -> torch.Tensor:
        if self.fused:
            q, k, v = self.qkv(x).chunk(3, dim=-1)
        else:
            q, k, v = self.q(x), self.k(x), self.v(x)
        q, k, v = self._per_head(q), self._per_head(k), self._per_head(v)
        scores = q @ k.transpose(-2, -1) / self.head_width ** 0.5 + mask
        ctx = scores.softmax(dim=-1) @ v
        b, _, n, _ = ctx.shape
        return ctx.transpose(1, 2).reshape(b, n, -1)


class EncoderLayer(nn.Module):
    """Post-norm: ``norm(x + attn(x))`` then ``norm(x + mlp(x))``."""

    def __init__(self, s: Shape):
        super().__init__()
        self.attn = Attention(s, fused=False)
        self.attn_proj = nn.Linear(s.width, s.width)
        self.attn_norm = nn.LayerNorm(s.width, eps=s.eps)
        self.mlp_in = nn.Linear(s.width, s.ffn)
        self.mlp_out = nn.Linear(s.ffn, s.width)
        self.mlp_norm = nn.LayerNorm(s.width, eps=s.eps)

    def forward(self, x, mask):
        x = self.attn_norm(x + self.attn_proj(self.attn(x, mask)))
        return self.mlp_norm(x + self.mlp_out(F.gelu(self.mlp_in(x))))


class BertEncoder(nn.Module):
    def __init__(self, s: Shape):
        super().__init__()
        self.tokens = nn.Embedding(s.vocab, s.width)
        self.places = nn.Embedding(s.positions, s.width)
        self.segments = nn.Embedding(2, s.width)
        self.embed_norm = nn.LayerNorm(s.width, eps=s.eps)
        self.layers = nn.ModuleList(EncoderLayer(s) for _ in range(s.layers))
        self.pool = nn.Linear(s.width, s.width)
        self.register_buffer("place_ids", torch.arange(s.positions), persistent=False)

    def forward(self, input_ids, attention_mask):
        n = input_ids.shape[1]
        segment_ids = torch.zeros_like(input_ids)  # one segment: token type 0
        x = self.tokens(input_ids) + self.places(self.place_ids[:n]) + self.segments(segment_ids)
        x = self.embed_norm(x)
        mask = (1.0 - attention_mask[:, None, None, :]) * FP32_MIN
        for layer in self.layers:
            x = layer(x, mask)
        return torch.tanh(self.pool(x[:, 0]))


class DecoderBlock(nn.Module):
    """Pre-norm: ``x + attn(norm(x))`` then ``x + mlp(norm(x))``."""

    def __init__(self, s: Shape):
        super().__init__()
        self.attn_norm = nn.LayerNorm(s.width, eps=s.eps)
        self.attn = Attention(s, fused=True)
        self.attn_proj = nn.Linear(s.width, s.width)
        self.mlp_norm = nn.LayerNorm(s.width, eps=s.eps)
        self.mlp_in = nn.Linear(s.width, s.ffn)
        self.mlp_out = nn.Linear(s.ffn, s.width)

    def forward(self, x, mask):
        x = x + self.attn_proj(self.attn(self.attn_norm(x), mask))
        return x + self.mlp_out(F.gelu(self.mlp_in(self.mlp_norm(x))))


class GPT2Decoder(nn.Module):
    def __init__(self, s: Shape):
        super().__init__()
        self.tokens = nn.Embedding(s.vocab, s.width)
        self.places = nn.Embedding(s.positions, s.width)
        self.blocks = nn.ModuleList(DecoderBlock(s) for _ in range(s.layers))
        self.final_norm = nn.LayerNorm(s.width, eps=s.eps)
        self.lm_head = nn.Linear(s.width, s.vocab, bias=False)
        future = torch.ones(s.positions, s.positions).triu(1) * FP32_MIN
        self.register_buffer("future", future[None, None], persistent=False)
        self.register_buffer("place_ids", torch.arange(s.positions), persistent=False)

    def forward(self, input_ids):
        n = input_ids.shape[1]
        x = self.tokens(input_ids) + self.places(self.place_ids[:n])
        mask = self.future[:, :, :n, :n]
        for block in self.blocks:
            x = block(x, mask)
        return self.lm_head(self.final_norm(x))


class FFNBlock(nn.Module):
    """``fc2(gelu_tanh(fc1(LayerNorm(x + r))))``."""

    def __init__(self, d: int = 768, ff: int = 3072, eps: float = 1e-12):
        super().__init__()
        self.ln = nn.LayerNorm(d, eps=eps)
        self.fc1 = nn.Linear(d, ff)
        self.fc2 = nn.Linear(ff, d)

    def forward(self, x, r):
        return self.fc2(F.gelu(self.fc1(self.ln(x + r)), approximate="tanh"))


BERT_BASE = Shape(vocab=30522, positions=512)
GPT2_SMALL = Shape(vocab=50257, positions=1024, eps=1e-5)
_SMALL = dict(layers=4, heads=8, width=512, ffn=2048, vocab=8192)


def _ids_and_mask(vocab):
    return lambda b, t, dev: (torch.randint(0, vocab, (b, t), device=dev),
                              torch.ones(b, t, device=dev))


def _ids(vocab):
    return lambda b, t, dev: (torch.randint(0, vocab, (b, t), device=dev),)


#: name -> (model factory, input factory, default sequence length)
SUITE = {
    "bert-base": (lambda: BertEncoder(BERT_BASE), _ids_and_mask(BERT_BASE.vocab), 128),
    "bert-small": (lambda: BertEncoder(Shape(positions=512, **_SMALL)), _ids_and_mask(8192), 128),
    "gpt2-small": (lambda: GPT2Decoder(GPT2_SMALL), _ids(GPT2_SMALL.vocab), 128),
    "gpt-small": (lambda: GPT2Decoder(Shape(positions=256, eps=1e-5, **_SMALL)), _ids(8192), 128),
    "ffn-block": (FFNBlock, lambda b, t, dev: (torch.randn(b, t, 768, device=dev),
                                               torch.randn(b, t, 768, device=dev)), 128),
}


def normal_init_(model: nn.Module, std: float = 0.02) -> nn.Module:
    """Linear/Embedding weights ~ N(0, std), biases 0, LayerNorm (1, 0)."""
    with torch.no_grad():
        for m in model.modules():
            if isinstance(m, nn.LayerNorm):
                nn.init.ones_(m.weight)
                nn.init.zeros_(m.bias)
            elif isinstance(m, (nn.Linear, nn.Embedding)):
                m.weight.normal_(0.0, std)
                if getattr(m, "bias", None) is not None:
                    nn.init.zeros_(m.bias)
    return model


def ffn_block_config1(seed: int = 0):
    """BASELINE config 1 exactly: x, r ~ N(0,1) [1,128,768]; gamma ~ N(1,0.02),
    beta ~ N(0,0.02); W1, W2 ~ N(0,0.02); b1 = b2 = 0; eps 1e-12."""
    torch.manual_seed(seed)
    m = FFNBlock().eval()
    with torch.no_grad():
        m.ln.weight.normal_(1.0, 0.02)
        m.ln.bias.normal_(0.0, 0.02)
        for fc in (m.fc1, m.fc2):
            fc.weight.normal_(0.0, 0.02)
            fc.bias.zero_()
    return m, (torch.randn(1, 128, 768), torch.randn(1, 128, 768))


def build(name: str, batch: int, seq: int | None = None, device: str | torch.device = "cpu",
          dtype: torch.dtype = torch.float32, init: str = "default"):
    """Model and inputs, seeded 0 (``init="normal"``: the N(0, 0.02) scheme).
    A reduced ``dtype`` applies to weights and float inputs, not to ids."""
    make_model, make_inputs, default_seq = SUITE[name]
    torch.manual_seed(0)
    model = make_model().eval()
    if init == "normal":
        normal_init_(model)
    model = model.to(device)
    args = make_inputs(batch, seq or default_seq, device)
    if dtype != torch.float32:
        model = model.to(dtype)
        args = tuple(a.to(dtype) if a.is_floating_point() else a for a in args)
    return model, args
