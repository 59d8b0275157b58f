"""The measured configurations, as concrete seeded workloads.

C1  single FFN block, fp32, [1,128,768] (LayerNorm(x+r) -> Linear 768->3072
    -> tanh-GELU -> Linear 3072->768); runnable on the CPU oracle.
C2  BERT-base fp16 b1 s128.
C3  GPT-2 small fp16 b1 s128.
C4  BERT-base fp16 b32 s128.
C5  GPT-2 small fp16 b32 s512.
C2-fp32  BERT-base fp32 b1 s128 (compiled by the reference's GPU check too;
    a parity case for the fp32 bar, not a benchmark line).

BERT/GPT weights: Linear and Embedding ~ N(0, 0.02), biases 0, LayerNorm
(1, 0); inputs are ``input_ids ~ U[0, vocab)`` (and an all-ones attention
mask for BERT), all seeded 0.
"""

from __future__ import annotations

from dataclasses import dataclass

import torch

from .models import build, ffn_block_config1


@dataclass(frozen=True)
class Workload:
    key: str
    model: str
    batch: int
    seq: int
    dtype: torch.dtype
    description: str


WORKLOADS = {
    "C1": Workload("C1", "ffn-block", 1, 128, torch.float32,
                   "FFN block fp32 x,r[1,128,768]: LN -> fc1 -> tanh-GELU -> fc2"),
    "C2": Workload("C2", "bert-base", 1, 128, torch.float16, "BERT-base fp16 b1 s128"),
    "C3": Workload("C3", "gpt2-small", 1, 128, torch.float16, "GPT-2 small fp16 b1 s128"),
    "C4": Workload("C4", "bert-base", 32, 128, torch.float16, "BERT-base fp16 b32 s128"),
    "C5": Workload("C5", "gpt2-small", 32, 512, torch.float16, "GPT-2 small fp16 b32 s512"),
    "C2-fp32": Workload("C2-fp32", "bert-base", 1, 128, torch.float32, "BERT-base fp32 b1 s128"),
}


def make(key: str, device: str | torch.device = "cpu"):
    """(model, example inputs) of a workload on ``device``, seeded 0."""
    w = WORKLOADS[key]
    # built on the CPU and then moved, so every device sees the same draws
    if w.model == "ffn-block":
        model, args = ffn_block_config1(0)
    else:
        model, args = build(w.model, w.batch, w.seq, "cpu", w.dtype, init="normal")
    return model.to(device), tuple(a.to(device) for a in args)
