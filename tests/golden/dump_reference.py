"""Write golden fixtures from the reference compiler (run in the build
container only; the GPU box never has the reference).

What the fixtures pin, per case: the schedule (kernel kinds, order, operand
buffers and rendered index strings, reduce kinds, row outputs), the arena
size, lower bound, unplanned total and every arena offset, plus -- for the
toy models -- the reference's torch-backend outputs. Nothing else pins these:
the published numbers only give kernel counts and arena totals.

The models are this repository's own (``tests/models.py`` and
``mlc-compiler_amd/mlc/bench/models.py``, which import torch only), loaded by
file path and compiled by the reference compiler.

Usage (from the repository root)::

    python tests/golden/dump_reference.py /root/reference tests/golden/reference_schedules.json
    python tests/golden/dump_reference.py /root/reference tests/golden --config1

The second form writes only BASELINE config 1 (the FFN block, fp32, seeded 0,
built by ``ffn_block_config1``): ``reference_config1.json`` (schedule, arena
plan, output shape) and ``reference_config1_out.npy`` (the reference's
torch-backend output on the CPU, float32).

    python tests/golden/dump_reference.py /root/reference tests/golden --outputs

The third form writes ``reference_outputs_fp16.npz``: the reference's
torch-backend outputs on the CPU for BASELINE configs 2-5 (BERT-base fp16 b1
and b32 pooled outputs in full; GPT-2 small fp16 b1 logits as every 101st
element of the flattened tensor, plus each of its 128 rows' sum and maximum
in float64; GPT-2 b32 s512 logits as every 10007th element plus each of its
16,384 rows' maximum), from this repository's seeded workloads.

The reference is imported from the path given; the script runs in its own
process so the reference's ``mlc`` package never meets this repository's.
"""

from __future__ import annotations

import importlib.util
import json
import pathlib
import sys

REPO = pathlib.Path(__file__).resolve().parents[2]


def _load(path: pathlib.Path, name: str):
    spec = importlib.util.spec_from_file_location(name, path)
    module = importlib.util.module_from_spec(spec)
    sys.modules[name] = module  # dataclasses look their module up by name
    spec.loader.exec_module(module)
    return module


def _describe(sched):
    from mlc.kernels import ExternKernel, PointwiseKernel, ReductionKernel

    out = []
    for k in sched.kernels:
        d = {"name": k.name, "summary": k.summary()}
        if isinstance(k, ExternKernel):
            d["kind"] = "extern"
            d["op"] = k.node.op
            d["inputs"] = [v.buffer.name for v in k.inputs]
            d["outputs"] = [v.buffer.name for v in k.outputs]
        else:
            d["kind"] = "pointwise" if isinstance(k, PointwiseKernel) else "reduction"
            d["inputs"] = [[a.value.buffer.name, str(a.dtype), a.index.render()] for a in k.inputs]
            d["outputs"] = [[a.value.buffer.name, str(a.dtype), a.index.render()] for a in k.outputs]
            d["ops"] = [n.op for n in k.nodes]
            if isinstance(k, PointwiseKernel):
                d["space"] = list(k.space)
                d["body"] = [[t, repr(e)] for t, e in k.body]
            else:
                d["row_space"] = list(k.row_space)
                d["reduce_space"] = list(k.reduce_space)
                d["reduces"] = [r.kind for r in k.reduces]
                d["steps"] = [[s.name, type(s).__name__, repr(s.expr)] for s in k.steps]
                d["row_outputs"] = sorted(k.row_outputs)
                d["two_pass"] = bool(k.two_pass)
            d["out_expr"] = {n: repr(e) for n, e in sorted(k.out_expr.items())}
        out.append(d)
    return out


def _plan(sched):
    p = sched.plan
    return {"mode": p.mode, "arena_bytes": p.arena_bytes, "peak_bytes": p.peak_bytes,
            "total_bytes": p.total_bytes, "offsets": dict(sorted(p.offsets.items()))}


def main(ref_root: str, out_path: str) -> None:
    sys.path.insert(0, ref_root)
    import torch

    import mlc
    from mlc.api import build_pipeline
    from mlc.config import Config
    from mlc.ir.capture import capture

    all_models = _load(REPO / "tests" / "models.py", "repo_toy_models").all_models
    build = _load(REPO / "mlc-compiler_amd" / "mlc" / "bench" / "models.py",
                  "repo_bench_models").build

    configs = {
        "no_fusion": Config(elementwise_fusion=False, recompute=False, reduction_fusion=False,
                            memory_planning=False, cuda_graphs=False),
        "elementwise": Config(reduction_fusion=False, recompute=False, memory_planning=False,
                              cuda_graphs=False),
        "planned": Config(reduction_fusion=False, cuda_graphs=False),
        "all_passes": Config(cuda_graphs=False),
        "streamed": Config(cuda_graphs=False, max_persistent_row=4),
        "graphs": Config(),
    }
    result = {"torch": torch.__version__, "toy": {}, "bench": {}}

    for name, model, args in all_models():
        entry = {}
        for cname, cfg in configs.items():
            g = capture(model, args)
            sched = build_pipeline(g, cfg)
            rec = {"kernels": _describe(sched), "plan": _plan(sched),
                   "counts": sched.counts(), "graph_nodes": len(g.nodes)}
            if cname in ("all_passes", "streamed", "no_fusion"):
                torch.manual_seed(0)
                got = mlc.compile(model, args, cfg)(*args)
                outs = got if isinstance(got, (list, tuple)) else [got]
                rec["outputs"] = [o.detach().double().reshape(-1).tolist() for o in outs]
                rec["output_shapes"] = [list(o.shape) for o in outs]
            entry[cname] = rec
        result["toy"][name] = entry

    bench_cases = [
        ("bert-base", 1, 128, torch.float16),
        ("bert-base", 32, 128, torch.float16),
        ("bert-base", 1, 128, torch.float32),
        ("gpt2-small", 1, 128, torch.float16),
        ("gpt2-small", 32, 128, torch.float16),
        ("gpt2-small", 32, 512, torch.float16),
        ("gpt-small", 1, 32, torch.float32),
        ("gpt-small", 2, 32, torch.float32),
        ("bert-small", 1, 32, torch.float32),
        ("bert-small", 2, 32, torch.float32),
    ]
    for mname, batch, seq, dt in bench_cases:
        model, args = build(mname, batch, seq, "cpu", dt)
        g = capture(model, args)
        for cname in ("graphs", "streamed64"):
            cfg = Config() if cname == "graphs" else Config(max_persistent_row=64)
            if cname == "streamed64" and not (mname == "bert-base" and batch == 1 and dt == torch.float16):
                continue
            g = capture(model, args)
            sched = build_pipeline(g, cfg)
            key = f"{mname}|b{batch}|s{seq}|{str(dt).replace('torch.', '')}|{cname}"
            result["bench"][key] = {"kernels": _describe(sched), "plan": _plan(sched),
                                    "counts": sched.counts(), "graph_nodes": len(g.nodes)}
            print(key, sched.counts(), sched.plan.arena_bytes, flush=True)

    with open(out_path, "w") as f:
        json.dump(result, f, indent=0, sort_keys=True)


def main_config1(ref_root: str, out_dir: str) -> None:
    sys.path.insert(0, ref_root)
    import numpy as np
    import torch

    import mlc
    from mlc.api import build_pipeline
    from mlc.config import Config
    from mlc.ir.capture import capture

    ffn = _load(REPO / "mlc-compiler_amd" / "mlc" / "bench" / "models.py",
                "repo_bench_models").ffn_block_config1
    model, args = ffn(0)
    cfg = Config()
    g = capture(model, args)
    sched = build_pipeline(g, cfg)
    compiled = mlc.compile(model, args, cfg)
    out = compiled(*args).detach()
    record = {"torch": torch.__version__, "backend": compiled.backend,
              "kernels": _describe(sched), "plan": _plan(sched), "counts": sched.counts(),
              "graph_nodes": len(g.nodes), "output_shape": list(out.shape),
              "output_dtype": str(out.dtype).replace("torch.", "")}
    out_dir = pathlib.Path(out_dir)
    with open(out_dir / "reference_config1.json", "w") as f:
        json.dump(record, f, indent=1, sort_keys=True)
    np.save(out_dir / "reference_config1_out.npy", out.float().numpy().reshape(-1))
    print("config1", sched.counts(), sched.plan.arena_bytes, flush=True)


def main_outputs(ref_root: str, out_dir: str) -> None:
    sys.path.insert(0, ref_root)
    import numpy as np
    import torch

    import mlc
    from mlc.config import Config

    build = _load(REPO / "mlc-compiler_amd" / "mlc" / "bench" / "models.py",
                  "repo_bench_models").build
    arrays = {"torch_version": np.array(torch.__version__)}
    for key, name, batch, seq in (("C2", "bert-base", 1, 128), ("C4", "bert-base", 32, 128),
                                  ("C3", "gpt2-small", 1, 128), ("C5", "gpt2-small", 32, 512)):
        model, args = build(name, batch, seq, "cpu", torch.float16, init="normal")
        compiled = mlc.compile(model, args, Config())
        out = compiled(*args)
        out = (out if isinstance(out, torch.Tensor) else out[0]).detach()
        arrays[f"{key}_shape"] = np.array(list(out.shape))
        if key == "C3":
            flat = out.reshape(-1)
            arrays[f"{key}_sample"] = flat[::101].numpy()
            rows = out.double().reshape(-1, out.shape[-1])
            arrays[f"{key}_row_sum"] = rows.sum(dim=1).numpy()
            arrays[f"{key}_row_max"] = rows.max(dim=1).values.numpy()
        elif key == "C5":
            arrays[f"{key}_sample"] = out.reshape(-1)[::10007].numpy()
            arrays[f"{key}_row_max"] = out.reshape(-1, out.shape[-1]).max(dim=1).values.numpy()
        else:
            arrays[f"{key}_out"] = out.numpy()
        print(key, compiled.backend, tuple(out.shape), out.dtype, flush=True)
    np.savez_compressed(pathlib.Path(out_dir) / "reference_outputs_fp16.npz", **arrays)


if __name__ == "__main__":
    if len(sys.argv) > 3 and sys.argv[3] == "--config1":
        main_config1(sys.argv[1], sys.argv[2])
    elif len(sys.argv) > 3 and sys.argv[3] == "--outputs":
        main_outputs(sys.argv[1], sys.argv[2])
    else:
        main(sys.argv[1], sys.argv[2])
