"""The parity oracle (test infrastructure; never imported by the product).

``compile_reference`` runs the product's front end (capture, fusion,
lowering, planning) and executes the resulting kernel IR on the CPU with the
torch reference runner, mirroring what ``mlc.compile`` does with the
reference's torch backend (``mlc/runtime/executor.py:28-38``).
"""

from __future__ import annotations

import sys
from pathlib import Path

_PKG = Path(__file__).resolve().parents[1] / "mlc-compiler_amd"
if str(_PKG) not in sys.path:
    sys.path.insert(0, str(_PKG))

import torch  # noqa: E402

from .torch_reference import (TorchReferenceRunner, eval_expr, run_kernel,  # noqa: E402,F401
                              run_pointwise, run_reduction)


def compile_reference(model, example_inputs, config=None, device="cpu"):
    """``mlc.compile`` with the oracle executing every generated kernel."""
    from mlc.api import build_pipeline
    from mlc.config import Config
    from mlc.ir.capture import capture
    from mlc.runtime.executor import CompiledModel

    cfg = config or Config()
    graph = capture(model, tuple(example_inputs))
    schedule = build_pipeline(graph, cfg)
    return CompiledModel(graph, schedule, cfg, torch.device(device), runner=TorchReferenceRunner())
