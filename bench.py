"""Benchmark: BERT-base fp16 s128 ms/forward (b1 and b32) through hipGraph
replay, and the fused kernels' HBM bandwidth against the MI355X peak.

    python bench.py [--gpus 1] [--steps K] [--warmup W] [--no-cpu-baseline] [--no-cpu-c5]
                    [--no-variants]

One step is one forward of the compiled model (one hipGraph replay: every
generated kernel plus every extern library call) over inputs already resident
in HBM. ``value`` is ms per forward at b1; b32 (config 4)
is timed the same way and reported beside it. The roofline object covers the
dominant fused kernel at b32 (the function moving the most algorithmic bytes
per forward), timed with hipEvents on its launch stream, with its
counter-measured traffic from the committed PMC summary in ``profiles/``;
``fused_b32`` aggregates every fused kernel (and ``fused_kernels`` under
``schedule_variants.gpt2_b32_s512.reference`` does the same for GPT-2 b32 s512,
whose launches are 4-30x larger). Beside each kernel figure,
``copy_ceiling`` times a plain packed copy kernel of the same algorithmic
bytes the same way: the practical ceiling once each launch's fixed cost is
counted.
The per-kernel loop launches a kernel back to back on the same buffers, so
after the first launch its inputs are cache-resident (the 256 MB Infinity
Cache holds them). ``fused_b32_in_forward`` prices the kernels where they run:
it decomposes the forward's hipGraph (the generated kernels' excess over empty
graph nodes, and their cost with their launches, against the library GEMMs
alone; ``mlc.bench.launch_floor``), and ``roofline.in_forward`` gives the
dominant kernel's excess per launch the same way.
``schedule_variants`` times the opt-in schedule changes (never the headline
value). The CPU baseline is the oracle (the kernel IR executed with torch on
the host) on a bounded number of forwards of every config. ``parity`` holds the
GPU outputs' distance from that oracle and from the reference compiler's own
outputs (a committed fixture). Prints one JSON line.
"""

from __future__ import annotations

import argparse
import json
import os
import pathlib
import statistics
import sys
import time

ROOT = pathlib.Path(__file__).resolve().parent
for _p in (ROOT / "mlc-compiler_amd", ROOT):
    if str(_p) not in sys.path:
        sys.path.insert(0, str(_p))

METRIC = "BERT-base fp16 s128 ms/forward b1&b32; fused-kernel HBM GB/s vs peak"


def _time_replays(compiled, inputs, steps: int, warmup: int):
    import torch

    for _ in range(max(1, warmup)):
        compiled(*inputs)  # the first call captures the hipGraph
    torch.cuda.synchronize()
    stream = torch.cuda.current_stream()
    starts = [torch.cuda.Event(enable_timing=True) for _ in range(steps)]
    ends = [torch.cuda.Event(enable_timing=True) for _ in range(steps)]
    total0 = torch.cuda.Event(enable_timing=True)
    total1 = torch.cuda.Event(enable_timing=True)
    torch.cuda.synchronize()
    total0.record(stream)
    for i in range(steps):
        starts[i].record(stream)
        compiled(*inputs)
        ends[i].record(stream)
    total1.record(stream)
    torch.cuda.synchronize()
    per = sorted(s.elapsed_time(e) for s, e in zip(starts, ends))
    return {
        "ms_per_step": total0.elapsed_time(total1) / steps,
        "median_ms": statistics.median(per),
        "p10_ms": per[max(0, int(0.1 * len(per)) - 1)] if len(per) >= 10 else per[0],
    }


_CEILING = None


def _copy_period_us(nbytes: int, iters: int) -> float:
    """Back-to-back launch period of a plain packed copy moving ``nbytes``
    (half read, half written), timed like the kernel table
    (``mlc.bench.copy_ceiling``)."""
    import torch

    from mlc.bench.copy_ceiling import CopyCeiling

    global _CEILING
    if _CEILING is None:
        _CEILING = CopyCeiling(torch.cuda.current_device())
    return _CEILING.period_us(nbytes, iters, torch.cuda.current_stream().cuda_stream)


def _copy_ceiling(nbytes: int, kernel_us: float, iters: int) -> dict:
    copy_us = _copy_period_us(nbytes, iters)
    return {"copy_us": round(copy_us, 3), "copy_gbs": round(nbytes / copy_us / 1e3, 1),
            "kernel_vs_copy": round(copy_us / kernel_us, 4)}


def _kernel_table(compiled, iters: int):
    """(kernel, symbol, algorithmic bytes, avg ms) of every generated kernel,
    each launched ``iters`` times back to back and timed with hipEvents on
    the launch stream.

    Each kernel is timed on its real inputs: the forward's plan is replayed up
    to that kernel first. Planned buffers are reused across the forward, so
    after a whole forward a kernel's input slot holds some later tensor, and
    data-dependent work (erf takes one of two branches per element) would be
    timed on the wrong data. A generated kernel never writes its own inputs,
    so repeating it leaves them intact."""
    import torch

    from mlc.bench.roofline import algorithmic_bytes
    from mlc.kernels import ExternKernel
    from mlc.runtime.executor import NativeCall, run_bound_extern

    rt = compiled._module
    stream = torch.cuda.current_stream().cuda_stream
    plan = compiled._plan
    rows = []
    replayed = 0
    for i, (k, (kind, payload)) in enumerate(zip(compiled.schedule.kernels, plan)):
        native = kind == "extern" and isinstance(payload, NativeCall)
        if isinstance(k, ExternKernel) and not native:
            continue
        for kind_j, payload_j in plan[replayed:i]:
            if kind_j == "extern":
                run_bound_extern(payload_j)
            elif kind_j == "kernel":
                rt.run_bound(payload_j)
        replayed = i
        bound = payload.bound if native else payload
        ms = rt.time_bound(bound, iters, stream)
        rows.append((k, rt.launch_table[k.name].symbol, algorithmic_bytes(k), ms, bound))
    torch.cuda.synchronize()
    return rows


def _per_symbol(rows) -> dict:
    per_symbol = {}
    for k, sym, nbytes, ms, _ in rows:
        agg = per_symbol.setdefault(sym, {"total_bytes": 0, "bytes": nbytes, "launch_ms": [],
                                          "kernel": k})
        agg["total_bytes"] += nbytes
        agg["launch_ms"].append(ms)
    return per_symbol


def _dominant(rows) -> str:
    """The generated function moving the most algorithmic bytes per forward
    (a property of the schedule, not of one timing run)."""
    per_symbol = _per_symbol(rows)
    return max(per_symbol, key=lambda s: per_symbol[s]["total_bytes"])


def _fused_aggregate(rows, iters: int) -> dict:
    """Every generated kernel of one forward (``_kernel_table`` rows), summed:
    algorithmic bytes over the sum of launch times, and the same launches as
    plain copies of each kernel's bytes (the ceiling once each launch's fixed
    cost is counted)."""
    from mlc.bench.roofline import HBM_PEAK_GBS

    fused_bytes = sum(r[2] for r in rows)
    fused_ms = sum(r[3] for r in rows)
    fused_gbs = fused_bytes / (fused_ms * 1e-3) / 1e9
    copy_of = {b: _copy_period_us(b, iters) for b in {r[2] for r in rows}}
    copy_ms = sum(copy_of[r[2]] for r in rows) / 1e3
    return {"kernels": len(rows), "algorithmic_bytes": fused_bytes, "ms": round(fused_ms, 4),
            "achieved": round(fused_gbs, 1), "frac": round(fused_gbs / HBM_PEAK_GBS, 4),
            "copy_ceiling_ms": round(copy_ms, 4), "kernels_vs_copy": round(copy_ms / fused_ms, 4)}


def _in_forward(compiled, inputs, rows, dom_sym: str, replays: int) -> dict:
    """What the generated kernels cost inside the b32 forward (hipGraph
    replays through ``mlc.bench.launch_floor``): the forward against the same
    graph with every generated kernel an empty node (their excess over an
    empty node) and against the library calls alone (their cost with their
    launches); the dominant function's own excess per launch the same way."""
    from mlc.bench.launch_floor import decompose_compiled
    from mlc.bench.roofline import HBM_PEAK_GBS

    d = decompose_compiled(compiled, inputs, replays, families=[dom_sym], shapes=False,
                           log=lambda line: print(f"# {line}", file=sys.stderr, flush=True))
    fused_bytes = sum(r[2] for r in rows)

    def rate(ms):
        gbs = fused_bytes / (ms * 1e-3) / 1e9
        return round(ms, 4), round(gbs, 1), round(gbs / HBM_PEAK_GBS, 4)

    excess = rate(d["full"] - d["base"])
    with_launch = rate(d["full"] - d["library_only"])
    fam, n, fam_ms = d["families"][0]
    nbytes = next(r[2] for r in rows if r[1] == dom_sym)
    per_launch_us = fam_ms * 1e3 / n
    gbs = nbytes / per_launch_us / 1e3
    return {
        "forward_ms": round(d["full"], 4), "library_calls_only_ms": round(d["library_only"], 4),
        "library_calls_plus_empty_ms": round(d["base"], 4), "generated_kernels": d["generated"],
        "algorithmic_bytes": fused_bytes,
        "excess_over_empty_nodes": dict(zip(("ms", "achieved", "frac"), excess)),
        "with_launches": dict(zip(("ms", "achieved", "frac"), with_launch)),
        "dominant": {"symbol": fam, "launches": n, "excess_us_per_launch": round(per_launch_us, 3),
                     "achieved": round(gbs, 1), "frac": round(gbs / HBM_PEAK_GBS, 4)},
        "replays": replays}


def _attention_row(compiled, iters: int) -> dict:
    """Average launch time and algorithmic bandwidth of the fused attention
    kernel (every layer shares one function)."""
    from mlc.bench.roofline import HBM_PEAK_GBS
    from mlc.kernels import AttentionKernel

    rows = [r for r in _kernel_table(compiled, iters) if isinstance(r[0], AttentionKernel)]
    if not rows:
        return {}
    ms = statistics.mean(r[3] for r in rows)
    gbs = rows[0][2] / (ms * 1e-3) / 1e9
    return {"symbol": rows[0][1], "launch_us": round(ms * 1e3, 3),
            "bytes_per_launch": rows[0][2], "achieved_gbs": round(gbs, 1),
            "frac": round(gbs / HBM_PEAK_GBS, 4), "traffic": _measured_traffic(rows[0][1]),
            "copy_ceiling": _copy_ceiling(rows[0][2], ms * 1e3, iters)}


def _measured_traffic(symbol: str):
    """Counter-measured HBM bytes per launch of ``symbol`` from the committed
    PMC summary (FETCH_SIZE and WRITE_SIZE, each scaled by what it reads for a
    plain copy of known size), or None when that summary is for other code."""
    for path in sorted((ROOT / "profiles").glob("*.md")):
        for line in path.read_text().splitlines():
            parts = line.split()
            if len(parts) == 3 and parts[0] == "traffic_bytes_per_launch" and parts[1] == symbol:
                return int(parts[2])
    return None


def _cpu_model() -> str:
    """The host CPU's model name, as ``lscpu`` reports it."""
    import subprocess

    try:
        out = subprocess.run(["lscpu"], capture_output=True, text=True, timeout=10).stdout
    except (OSError, subprocess.SubprocessError):
        return "unknown"
    for line in out.splitlines():
        if line.startswith("Model name:"):
            return line.split(":", 1)[1].strip()
    return "unknown"


def _time_cpu(fn, args, warmup: int, min_runs: int, budget_s: float):
    for _ in range(warmup):
        out = fn(*args)
    times = []
    t_end = time.perf_counter() + budget_s
    while len(times) < min_runs or (time.perf_counter() < t_end and len(times) < 200):
        t0 = time.perf_counter()
        out = fn(*args)
        times.append(time.perf_counter() - t0)
    return statistics.median(times), times, out


def _cpu_baseline(hip_outputs: dict, budget_s: float, with_c5: bool = True):
    """The CPU oracle (the kernel IR executed with torch on the host, fp32
    math, fp16 storage; its own CPU GEMMs) timed on the host's cores for
    every BASELINE config: 2 (the headline), 1, 3 and 4 with 2 warm-ups (1
    for config 4) then the median of the timed forwards
    (``mlc/bench/runner.py:106-110``); config 5 (GPT-2 b32 s512, about 30 s
    per forward on 16 threads) as one forward with no warm-up. Its outputs
    double as the parity check of the GPU results timed above
    (``hip_outputs``): max error relative to the oracle output's largest
    magnitude."""
    import torch

    from mlc.bench.workloads import make
    from oracle import compile_reference

    threads = os.cpu_count() or 1
    torch.set_num_threads(threads)
    timed = {}
    parity = {}
    plan = [("C2", 2, 5, budget_s), ("C1", 2, 5, 2.0), ("C3", 2, 5, 2.0), ("C4", 1, 3, 0.0)]
    if with_c5:
        plan.append(("C5", 0, 1, 0.0))
    for key, warmup, min_runs, budget in plan:
        model, args = make(key, "cpu")
        ref = compile_reference(model, args)
        med, times, out = _time_cpu(ref, args, warmup, min_runs, budget)
        timed[key] = (med, times)
        if key in hip_outputs:
            want = out.double()
            got = hip_outputs[key].double()
            parity[key] = round((got - want).abs().max().item() / want.abs().max().item(), 6)
        del model, args, ref
    med, times = timed["C2"]
    return {
        "value": round(med * 1e3, 3),
        "unit": "ms/forward",
        "cores": torch.get_num_threads(),
        "kind": "port",
        "cpu_model": _cpu_model(),
        "sample": (f"CPU oracle (kernel IR executed with torch, fp16 storage, fp32 math) on "
                   f"BASELINE config 2, BERT-base fp16 b1 s128: median of {len(times)} forwards "
                   f"after 2 warm-ups, {sum(times):.1f}s of CPU work, os.cpu_count()={threads}"),
        "other_configs_ms_per_forward": {
            key: {"median_ms": round(timed[key][0] * 1e3, 3), "runs": len(timed[key][1]),
                  "warmup": next(w for k, w, _, _ in plan if k == key)}
            for key in timed if key != "C2"},
    }, parity


def _reference_fixture_errors(hip_outputs: dict) -> dict:
    """The GPU outputs timed above against the reference compiler's own
    outputs for configs 2-4 (``tests/golden/reference_outputs_fp16.npz``,
    written by the reference's torch backend on a CPU): max error relative to
    the reference's largest magnitude; GPT-2's logits on the fixture's sample
    of every 101st value."""
    import numpy as np
    import torch

    path = ROOT / "tests" / "golden" / "reference_outputs_fp16.npz"
    if not path.exists():
        return {}
    ref = np.load(path, allow_pickle=False)
    errs = {}
    for key in ("C2", "C3", "C4"):
        got = hip_outputs.get(key)
        if got is None:
            continue
        if key == "C3":
            got, want = got.reshape(-1)[::101], torch.from_numpy(ref["C3_sample"]).float()
        else:
            want = torch.from_numpy(ref[f"{key}_out"]).float()
        got, want = got.double(), want.double()
        errs[key] = round((got - want).abs().max().item() / want.abs().max().item(), 6)
    errs["bar"] = {"C2": 2e-3, "C3": 2e-3, "C4": 3e-3}
    errs["north_star_bar"] = 2e-3
    return errs


def main() -> int:
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=50)
    ap.add_argument("--warmup", type=int, default=20)
    ap.add_argument("--kernel-iters", type=int, default=50)
    ap.add_argument("--cpu-budget", type=float, default=12.0)
    ap.add_argument("--floor-replays", type=int, default=100,
                    help="graph replays per decomposition graph of the b32 in-forward figure")
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--no-cpu-c5", action="store_true",
                    help="leave config 5 (one ~30 s CPU forward) out of the CPU baseline")
    ap.add_argument("--no-variants", action="store_true",
                    help="skip the schedule variants (the reference schedule only)")
    opts = ap.parse_args()
    if opts.gpus != 1:
        print(f"bench.py runs on one GPU: the compiled model replays one hipGraph on one device "
              f"and this build has no multi-GPU path (asked for --gpus {opts.gpus})",
              file=sys.stderr)
        return 2

    import torch

    import mlc
    from mlc.bench.roofline import HBM_PEAK_GBS, forward_bytes
    from mlc.bench.workloads import make
    from mlc.config import Config

    torch.cuda.set_device(0)
    results = {}
    tables = {}
    outputs = {}
    for key in ("C2", "C3", "C4"):
        model, inputs = make(key, "cuda")
        compiled = mlc.compile(model, inputs, Config())
        results[key] = _time_replays(compiled, inputs, opts.steps, opts.warmup)
        if key in ("C2", "C3", "C4"):
            out = compiled(*inputs)
            outputs[key] = (out if isinstance(out, torch.Tensor) else out[0]).float().cpu()
        results[key]["kernels"] = compiled.schedule.counts()
        results[key]["graph_nodes"] = compiled._module.graph_nodes()
        results[key]["arena_bytes"] = compiled.schedule.arena_bytes
        results[key]["forward_bytes"] = forward_bytes(compiled.schedule)
        if key == "C4":
            rows = tables[key] = _kernel_table(compiled, opts.kernel_iters)
            results[key]["dominant"] = _dominant(rows)
            results[key]["in_forward"] = _in_forward(compiled, inputs, rows,
                                                     results[key]["dominant"], opts.floor_replays)
        print(f"# {key}: {results[key]}", file=sys.stderr, flush=True)
        del compiled, model, inputs
        torch.cuda.empty_cache()

    FAST = Config(merge_parallel_gemms=True, gemm_epilogue=True, layout_selection=True)
    ATTENTION = Config(fused_attention=True)
    ALL = Config(merge_parallel_gemms=True, gemm_epilogue=True, layout_selection=True,
                 fused_attention=True)
    # opt-in schedule changes, measured beside the reference schedule
    # (different kernel schedules, so never the headline value)
    variants = {}
    variant_runs = () if opts.no_variants else (
                           ("gemm_epilogue", "C2", Config(gemm_epilogue=True)),
                           ("gemm_epilogue", "C4", Config(gemm_epilogue=True)),
                           ("layout_selection", "C4", Config(layout_selection=True)),
                           ("layout_selection+gemm_epilogue", "C4",
                            Config(layout_selection=True, gemm_epilogue=True)),
                           ("all: merged qkv GEMM+epilogue+layout", "C2", FAST),
                           ("all: merged qkv GEMM+epilogue+layout", "C4", FAST),
                           ("fused_attention", "C2", ATTENTION),
                           ("fused_attention", "C4", ATTENTION),
                           ("all + fused_attention", "C2", ALL),
                           ("all + fused_attention", "C3", ALL),
                           ("all + fused_attention", "C4", ALL),
                           # GPT-2 b32 s512 (config 5): the key-blocked attention kernel
                           ("gpt2_b32_s512", "C5", Config()),
                           ("gpt2_b32_s512", "C5", ALL))
    for name, key, cfg in variant_runs:
        model, inputs = make(key, "cuda")
        compiled = mlc.compile(model, inputs, cfg)
        r = _time_replays(compiled, inputs, opts.steps, opts.warmup)
        entry = {"ms_per_forward": round(r["ms_per_step"], 4),
                 "kernels": compiled.schedule.counts()}
        if cfg.fused_attention:
            entry["attention_kernel"] = _attention_row(compiled, opts.kernel_iters)
        if key == "C5" and not cfg.fused_attention:
            # every generated kernel of the reference schedule, launches of 50-403 MB
            entry["fused_kernels"] = _fused_aggregate(_kernel_table(compiled, 10), 10)
        if key == "C5":
            slot = "all + fused_attention" if cfg.fused_attention else "reference"
        else:
            slot = {"C2": "b1", "C3": "gpt2_b1", "C4": "b32"}[key]
        variants.setdefault(name, {})[slot] = entry
        del compiled, model, inputs
        torch.cuda.empty_cache()

    rows = tables["C4"]
    per_symbol = _per_symbol(rows)
    dom_sym = results["C4"]["dominant"]
    dom = per_symbol[dom_sym]
    in_forward = results["C4"]["in_forward"]
    launch_ms = statistics.mean(dom["launch_ms"])
    achieved = dom["bytes"] / (launch_ms * 1e-3) / 1e9

    line = {
        "metric": METRIC,
        "value": round(results["C2"]["ms_per_step"], 4),
        "unit": "ms/forward",
        "n_gpus": 1,
        "steps": opts.steps,
        "warmup": opts.warmup,
        "ms_per_step": round(results["C2"]["ms_per_step"], 4),
        "higher_is_better": False,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "fp16",
        "data": "synthetic: weights N(0,0.02), input_ids U[0,30522), all-ones mask, seed 0",
        "config": {
            "workload": "BERT-base fp16 b1 s128, one hipGraph replay per forward (config 2)",
            "global_batch": 1, "seq_len": 128, "parallelism": "none (1 GPU)",
            "b1": {k: results["C2"][k] for k in ("median_ms", "p10_ms", "kernels", "graph_nodes",
                                                 "arena_bytes")},
            "b32": {"ms_per_forward": round(results["C4"]["ms_per_step"], 4),
                    **{k: results["C4"][k] for k in ("median_ms", "p10_ms", "kernels",
                                                     "graph_nodes", "arena_bytes")}},
            # BASELINE config 3, GPT-2 small fp16 b1 s128 (reference on A40: 1.141 ms)
            "gpt2_b1": {"ms_per_forward": round(results["C3"]["ms_per_step"], 4),
                        **{k: results["C3"][k] for k in ("median_ms", "p10_ms", "kernels",
                                                         "graph_nodes", "arena_bytes")}},
        },
        "schedule_variants": variants,
        # the whole forward (library GEMMs included) against its bytes-moved floor
        "e2e_roofline": {
            b: {"algorithmic_bytes": results[key]["forward_bytes"],
                "floor_ms": round(results[key]["forward_bytes"] / (HBM_PEAK_GBS * 1e6), 4),
                "frac": round(results[key]["forward_bytes"] / (HBM_PEAK_GBS * 1e6)
                              / results[key]["ms_per_step"], 4)}
            for b, key in (("b1", "C2"), ("b32", "C4"))},
        "roofline": {
            "bound": "hbm",
            "kernel": f"{dom_sym}: {dom['kernel'].summary().split(': ', 1)[1]} (b32)",
            "bytes_per_launch": dom["bytes"],
            "launch_us": round(launch_ms * 1e3, 3),
            "achieved": round(achieved, 1),
            "peak": HBM_PEAK_GBS,
            "unit": "GB/s",
            "frac": round(achieved / HBM_PEAK_GBS, 4),
            "traffic": _measured_traffic(dom_sym),
            "copy_ceiling": _copy_ceiling(dom["bytes"], launch_ms * 1e3, opts.kernel_iters),
            # the same function inside the forward: its excess over an empty
            # graph node
            "in_forward": in_forward["dominant"],
        },
        # every generated kernel of the b32 forward, two ways: back-to-back
        # launches on the same buffers, and inside the forward
        "fused_b32": _fused_aggregate(rows, opts.kernel_iters),
        "fused_b32_in_forward": {k: v for k, v in in_forward.items() if k != "dominant"},
        "cpu_baseline": None,
        "parity": None,
    }
    if not opts.no_cpu_baseline:
        line["cpu_baseline"], checked = _cpu_baseline(outputs, opts.cpu_budget,
                                                      with_c5=not opts.no_cpu_c5)
        # BERT's pooled output is the one output held to 3e-3 instead of the
        # north-star 2e-3: fp16 rounding flips saturate the 12-layer hidden
        # state, and the oracle is as far from itself across devices
        line["parity"] = {"bert_pooled_vs_oracle": {
            "b1": checked.get("C2"), "b32": checked.get("C4"), "bar": 3e-3,
            "north_star_bar": 2e-3,
            "measure": "max|hip - oracle| / max|oracle|, oracle on the CPU (its own GEMMs)"}}
    line["parity"] = line["parity"] or {}
    line["parity"]["vs_reference_outputs"] = _reference_fixture_errors(outputs)
    print(json.dumps(line), flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
