"""Workload definitions: BERT-base (post-norm encoder) and GPT-2 small
(pre-norm causal decoder) in plain PyTorch, plus the single FFN block.

The architectures are the reference's benchmark models
(``mlc/bench/models.py:87-224``) so export produces the same graph and the
compiler the same schedule: post-norm BERT with an additive
``(1 - mask) * finfo(fp32).min`` attention mask, erf-GELU and a tanh pooler;
pre-norm GPT-2 with a ``finfo(fp32).min`` causal mask buffer. Weights are
synthetic: ``build`` seeds 0 and, with ``init="normal"``, sets Linear and
Embedding weights to N(0, 0.02), biases to 0, LayerNorm to (1, 0).
"""

from __future__ import annotations

import math
from dataclasses import dataclass

import torch
import torch.nn as nn
import torch.nn.functional as F


@dataclass
class BertConfig:
    vocab_size: int = 30522
    max_position: int = 512
    n_layer: int = 12
    n_head: int = 12
    d_model: int = 768
    d_ff: int = 3072
    eps: float = 1e-12


@dataclass
class GPTConfig:
    vocab_size: int = 50257
    block_size: int = 1024
    n_layer: int = 12
    n_head: int = 12
    d_model: int = 768
    eps: float = 1e-5


class BertSelfAttention(nn.Module):
    def __init__(self, cfg: BertConfig):
        super().__init__()
        self.n_head = cfg.n_head
        self.d_head = cfg.d_model // cfg.n_head
        self.query = nn.Linear(cfg.d_model, cfg.d_model)
        self.key = nn.Linear(cfg.d_model, cfg.d_model)
        self.value = nn.Linear(cfg.d_model, cfg.d_model)

    def _split_heads(self, x):
        b, t, _ = x.shape
        return x.view(b, t, self.n_head, self.d_head).transpose(1, 2)

    def forward(self, x, mask):
        q = self._split_heads(self.query(x))
        k = self._split_heads(self.key(x))
        v = self._split_heads(self.value(x))
        scores = (q @ k.transpose(-2, -1)) / math.sqrt(self.d_head) + mask
        probs = scores.softmax(dim=-1)
        b, t, _ = x.shape
        return (probs @ v).transpose(1, 2).reshape(b, t, -1)


class BertLayer(nn.Module):
    def __init__(self, cfg: BertConfig):
        super().__init__()
        self.attn = BertSelfAttention(cfg)
        self.attn_out = nn.Linear(cfg.d_model, cfg.d_model)
        self.ln1 = nn.LayerNorm(cfg.d_model, eps=cfg.eps)
        self.fc1 = nn.Linear(cfg.d_model, cfg.d_ff)
        self.fc2 = nn.Linear(cfg.d_ff, cfg.d_model)
        self.ln2 = nn.LayerNorm(cfg.d_model, eps=cfg.eps)

    def forward(self, x, mask):
        x = self.ln1(x + self.attn_out(self.attn(x, mask)))
        return self.ln2(x + self.fc2(F.gelu(self.fc1(x))))


class Bert(nn.Module):
    def __init__(self, cfg: BertConfig = BertConfig()):
        super().__init__()
        self.cfg = cfg
        self.word_emb = nn.Embedding(cfg.vocab_size, cfg.d_model)
        self.pos_emb = nn.Embedding(cfg.max_position, cfg.d_model)
        self.type_emb = nn.Embedding(2, cfg.d_model)
        self.emb_ln = nn.LayerNorm(cfg.d_model, eps=cfg.eps)
        self.layers = nn.ModuleList(BertLayer(cfg) for _ in range(cfg.n_layer))
        self.pooler = nn.Linear(cfg.d_model, cfg.d_model)
        self.register_buffer("positions", torch.arange(cfg.max_position), persistent=False)

    def forward(self, input_ids, attention_mask):
        _, t = input_ids.shape
        x = (self.word_emb(input_ids) + self.pos_emb(self.positions[:t])
             + self.type_emb(torch.zeros_like(input_ids)))
        x = self.emb_ln(x)
        mask = (1.0 - attention_mask[:, None, None, :]) * torch.finfo(torch.float32).min
        for layer in self.layers:
            x = layer(x, mask)
        return torch.tanh(self.pooler(x[:, 0]))


class CausalSelfAttention(nn.Module):
    def __init__(self, cfg: GPTConfig):
        super().__init__()
        self.n_head = cfg.n_head
        self.d_head = cfg.d_model // cfg.n_head
        self.qkv = nn.Linear(cfg.d_model, 3 * cfg.d_model)
        self.proj = nn.Linear(cfg.d_model, cfg.d_model)

    def forward(self, x, causal):
        b, t, d = x.shape
        q, k, v = self.qkv(x).chunk(3, dim=-1)
        heads = (b, t, self.n_head, self.d_head)
        q = q.view(heads).transpose(1, 2)
        k = k.view(heads).transpose(1, 2)
        v = v.view(heads).transpose(1, 2)
        scores = (q @ k.transpose(-2, -1)) / math.sqrt(self.d_head) + causal[:, :, :t, :t]
        probs = scores.softmax(dim=-1)
        return self.proj((probs @ v).transpose(1, 2).reshape(b, t, d))


class GPTBlock(nn.Module):
    def __init__(self, cfg: GPTConfig):
        super().__init__()
        self.ln1 = nn.LayerNorm(cfg.d_model, eps=cfg.eps)
        self.attn = CausalSelfAttention(cfg)
        self.ln2 = nn.LayerNorm(cfg.d_model, eps=cfg.eps)
        self.fc1 = nn.Linear(cfg.d_model, 4 * cfg.d_model)
        self.fc2 = nn.Linear(4 * cfg.d_model, cfg.d_model)

    def forward(self, x, causal):
        x = x + self.attn(self.ln1(x), causal)
        return x + self.fc2(F.gelu(self.fc1(self.ln2(x))))


class GPT(nn.Module):
    def __init__(self, cfg: GPTConfig = GPTConfig()):
        super().__init__()
        self.cfg = cfg
        self.tok_emb = nn.Embedding(cfg.vocab_size, cfg.d_model)
        self.pos_emb = nn.Embedding(cfg.block_size, cfg.d_model)
        self.blocks = nn.ModuleList(GPTBlock(cfg) for _ in range(cfg.n_layer))
        self.ln_f = nn.LayerNorm(cfg.d_model, eps=cfg.eps)
        self.head = nn.Linear(cfg.d_model, cfg.vocab_size, bias=False)
        tril = torch.tril(torch.ones(cfg.block_size, cfg.block_size))
        causal = (1.0 - tril) * torch.finfo(torch.float32).min
        self.register_buffer("causal", causal.view(1, 1, cfg.block_size, cfg.block_size),
                             persistent=False)
        self.register_buffer("positions", torch.arange(cfg.block_size), persistent=False)

    def forward(self, input_ids):
        _, t = input_ids.shape
        x = self.tok_emb(input_ids) + self.pos_emb(self.positions[:t])
        for block in self.blocks:
            x = block(x, self.causal)
        return self.head(self.ln_f(x))


class FFNBlock(nn.Module):
    """``fc2(gelu_tanh(fc1(LayerNorm(x + r))))``."""

    def __init__(self, d: int = 768, ff: int = 3072, eps: float = 1e-12):
        super().__init__()
        self.ln = nn.LayerNorm(d, eps=eps)
        self.fc1 = nn.Linear(d, ff)
        self.fc2 = nn.Linear(ff, d)

    def forward(self, x, r):
        return self.fc2(F.gelu(self.fc1(self.ln(x + r)), approximate="tanh"))


def _bert_inputs(vocab):
    return lambda b, t, dev: (torch.randint(0, vocab, (b, t), device=dev),
                              torch.ones(b, t, device=dev))


def _gpt_inputs(vocab):
    return lambda b, t, dev: (torch.randint(0, vocab, (b, t), device=dev),)


#: name -> (model builder, input builder, default sequence length)
SUITE = {
    "bert-base": (lambda: Bert(BertConfig()), _bert_inputs(30522), 128),
    "bert-small": (lambda: Bert(BertConfig(n_layer=4, n_head=8, d_model=512, d_ff=2048,
                                           vocab_size=8192)), _bert_inputs(8192), 128),
    "gpt2-small": (lambda: GPT(GPTConfig()), _gpt_inputs(50257), 128),
    "gpt-small": (lambda: GPT(GPTConfig(n_layer=4, n_head=8, d_model=512, vocab_size=8192,
                                        block_size=256)), _gpt_inputs(8192), 128),
    "ffn-block": (lambda: FFNBlock(),
                  lambda b, t, dev: (torch.randn(b, t, 768, device=dev),
                                     torch.randn(b, t, 768, device=dev)), 128),
}


def normal_init_(model: nn.Module, std: float = 0.02) -> nn.Module:
    """Linear/Embedding weights ~ N(0, std), biases 0, LayerNorm (1, 0)."""
    with torch.no_grad():
        for m in model.modules():
            if isinstance(m, (nn.Linear, nn.Embedding)):
                m.weight.normal_(0.0, std)
                if getattr(m, "bias", None) is not None:
                    m.bias.zero_()
            elif isinstance(m, nn.LayerNorm):
                m.weight.fill_(1.0)
                m.bias.zero_()
    return model


def ffn_block_config1(seed: int = 0):
    """BASELINE config 1 exactly: x, r ~ N(0,1) [1,128,768]; gamma ~ N(1,0.02),
    beta ~ N(0,0.02); W1, W2 ~ N(0,0.02); b1 = b2 = 0; eps 1e-12."""
    torch.manual_seed(seed)
    m = FFNBlock().eval()
    with torch.no_grad():
        m.ln.weight.normal_(1.0, 0.02)
        m.ln.bias.normal_(0.0, 0.02)
        m.fc1.weight.normal_(0.0, 0.02)
        m.fc1.bias.zero_()
        m.fc2.weight.normal_(0.0, 0.02)
        m.fc2.bias.zero_()
    x = torch.randn(1, 128, 768)
    r = torch.randn(1, 128, 768)
    return m, (x, r)


def build(name: str, batch: int, seq: int | None = None, device: str | torch.device = "cpu",
          dtype: torch.dtype = torch.float32, init: str = "default"):
    """Model and inputs, seeded 0. ``dtype`` halves weights and float inputs;
    index tensors stay integral."""
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
