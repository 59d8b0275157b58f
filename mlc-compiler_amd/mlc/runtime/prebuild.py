"""Compile the kernel modules of known workloads ahead of time.

``mlc.compile`` generates and compiles one HIP module per schedule; the code
object is cached by content (``native.compile_code_object``). Running this
before shipping a tree fills the cache for the configurations the test suite,
the smoke run and the benchmark compile, so those runs only load code
objects. It changes nothing about what runs: a cache miss compiles the same
source.

    python -m mlc.runtime.prebuild [C1 C2 ...]
"""

from __future__ import annotations

import sys
import time

import torch

from ..api import build_pipeline
from ..bench.workloads import WORKLOADS, make
from ..codegen.hip_backend import build_module
from ..config import Config
from ..ir.capture import capture
from . import native

FAST = Config(merge_parallel_gemms=True, gemm_epilogue=True, layout_selection=True)
ATTENTION = Config(fused_attention=True)
ALL = Config(merge_parallel_gemms=True, gemm_epilogue=True, layout_selection=True,
             fused_attention=True)

#: every (workload, config) pair a committed caller compiles
DEFAULT = [("C1", Config()), ("C2", Config()), ("C3", Config()), ("C4", Config()),
           ("C5", Config()), ("C2-fp32", Config()), ("C2", Config(max_persistent_row=64)),
           ("C2", Config(gemm_epilogue=True)), ("C3", Config(gemm_epilogue=True)),
           ("C4", Config(gemm_epilogue=True)), ("C4", Config(layout_selection=True)),
           ("C5", Config(layout_selection=True)),
           ("C4", Config(layout_selection=True, gemm_epilogue=True)),
           ("C2", FAST), ("C4", FAST), ("C2", ATTENTION), ("C3", ATTENTION),
           ("C4", ATTENTION), ("C5", ATTENTION), ("C2", ALL), ("C3", ALL), ("C4", ALL),
           ("C5", ALL)]
# the planned / unplanned pairs the exactness tests compile (the unplanned
# schedule is the planned one, so each pair shares its code object)
DEFAULT += [(key, cfg) for key in ("C2", "C3", "C4")
            for cfg in (Config(reduction_fusion=False, cuda_graphs=False), Config(cuda_graphs=False))]


def prebuild(items=None, verbose: bool = True) -> None:
    from ..bench.copy_ceiling import SOURCE as COPY_CEILING

    native.compile_code_object(COPY_CEILING)
    for key, cfg in (items or DEFAULT):
        t0 = time.time()
        model, args = make(key, "cpu")
        graph = capture(model, args)
        schedule = build_pipeline(graph, cfg)
        module = build_module(schedule, cfg)
        _, obj = native.compile_code_object(module.source)
        if verbose:
            print(f"prebuild {key} max_row={cfg.max_persistent_row}: {len(module.functions)} "
                  f"functions -> {obj.name} ({time.time() - t0:.1f}s)", flush=True)
        del model, args, graph, schedule
        torch.cuda.empty_cache() if torch.cuda.is_available() else None


if __name__ == "__main__":
    keys = sys.argv[1:] or None
    prebuild([(k, Config()) for k in keys] if keys else None)
    if keys is None:
        print("workloads:", ", ".join(WORKLOADS))
