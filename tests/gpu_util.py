"""Helpers shared by the GPU parity tests.

Error measure used throughout: ``max|got - want| / max|want|`` over the whole
output (the largest error relative to the output's largest magnitude).
"""

from __future__ import annotations

import torch

from mlc.kernels import ExternKernel
from mlc.runtime.executor import run_extern


def rel_err(got: torch.Tensor, want: torch.Tensor) -> float:
    got = got.detach().double().cpu()
    want = want.detach().double().cpu()
    scale = want.abs().max().item()
    if scale == 0.0:
        return got.abs().max().item()
    return (got - want).abs().max().item() / scale


def flat_outputs(out):
    if isinstance(out, (list, tuple)):
        return [t for o in out for t in flat_outputs(o)]
    return [out]


def lockstep(schedule, graph, params_cpu: dict, inputs_cpu, hip_runtime, check=None,
             device="cuda", limit=None):
    """Run ``schedule`` twice in lockstep: the oracle on the CPU, and every
    generated kernel also through the HIP runtime on inputs copied from the
    oracle's buffers, so each kernel is compared on identical inputs.

    Extern ops run on the GPU (torch) and their results are copied back, so
    both sides see the same library results. ``check(kernel, name, got,
    want)`` is called for every output of every generated kernel. Returns the
    oracle's buffer table.
    """
    from oracle import run_kernel

    cpu: dict[str, torch.Tensor] = {n: t.clone() for n, t in params_cpu.items()}
    for v, t in zip(graph.inputs, inputs_cpu):
        cpu[v.buffer.name] = t.reshape(-1).clone()
    kernels = schedule.kernels if limit is None else schedule.kernels[:limit]
    for k in kernels:
        for v in list(k.reads()) + list(k.writes()):
            if v.buffer.name not in cpu:
                cpu[v.buffer.name] = torch.zeros(v.buffer.numel, dtype=v.buffer.dtype)
    for k in kernels:
        names_in = {v.buffer.name for v in k.reads()}
        names_out = {v.buffer.name for v in k.writes()}
        gpu = {n: cpu[n].to(device) for n in names_in | names_out}
        if isinstance(k, ExternKernel):
            bound = hip_runtime.bind_native_extern(k, gpu)
            if bound is not None:
                # a native template of an extern op must match torch bit for bit
                mine = {n: t.clone() for n, t in gpu.items()}
                bound = hip_runtime.bind_native_extern(k, mine)
                hip_runtime.run_bound(bound)
            run_extern(k, gpu)
            torch.cuda.synchronize()
            for n in names_out:
                cpu[n] = gpu[n].cpu()
                if bound is not None:
                    assert torch.equal(mine[n].cpu(), cpu[n]), f"{k.summary()}: native != torch"
            if bound is not None:
                hip_runtime.check_errors()
            continue
        run_kernel(k, cpu)
        hip_runtime.launch(k, gpu)
        torch.cuda.synchronize()
        if check is not None:
            for n in sorted(names_out):
                check(k, n, gpu[n].cpu(), cpu[n])
    return cpu
