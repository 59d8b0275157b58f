"""What a generated kernel costs depending on which kernel wrote its input.

    rocprofv3 --kernel-trace --output-format csv -d OUT -o t -- \\
        python mlc-compiler_amd/mlc/bench/producer.py run
    python mlc-compiler_amd/mlc/bench/producer.py split OUT

``run`` compiles BERT-base fp16 b32 (config 4) on the reference schedule,
replays the plan up to the first softmax (so its scores are real), and then
launches that softmax ``--iters`` times in each of three ways: right after
the hipBLASLt batched GEMM (``bmm``) that writes the scores in the forward;
right after a torch copy that writes the same bytes into the same buffer; and
right after itself. ``split`` reads the kernel trace and prints, for each
way, the dispatch count, the median and mean traced duration of the softmax,
and the median idle gap before it.
"""

from __future__ import annotations

import argparse
import csv
import pathlib
import statistics
import sys

ROOT = pathlib.Path(__file__).resolve().parents[3]
for _p in (ROOT / "mlc-compiler_amd", ROOT):
    if str(_p) not in sys.path:
        sys.path.insert(0, str(_p))


def run(iters: int) -> None:
    import torch

    import mlc
    from mlc.bench.workloads import make
    from mlc.config import Config
    from mlc.kernels import ReductionKernel
    from mlc.runtime.executor import run_bound_extern

    model, inputs = make("C4", "cuda")
    compiled = mlc.compile(model, inputs, Config(cuda_graphs=False))
    compiled(*inputs)
    torch.cuda.synchronize()
    plan, kernels, rt = compiled._plan, compiled.schedule.kernels, compiled._module
    i = next(j for j, k in enumerate(kernels)
             if isinstance(k, ReductionKernel) and k.reduce_numel == 128 and plan[j][0] == "kernel")
    if plan[i - 1][0] != "extern":
        raise RuntimeError(f"the softmax's producer is not a library call: {kernels[i - 1].summary()}")
    for kind, payload in plan[:i]:
        if kind == "extern":
            run_bound_extern(payload)
        elif kind == "kernel":
            rt.run_bound(payload)
    torch.cuda.synchronize()
    scores = compiled._resident[kernels[i].inputs[0].value.buffer.name]
    saved = scores.clone()
    softmax, producer = plan[i][1], plan[i - 1][1]
    print(f"softmax {rt.launch_table[kernels[i].name].symbol}; producer {kernels[i - 1].summary()}",
          flush=True)
    for _ in range(iters):
        run_bound_extern(producer)
        rt.run_bound(softmax)
        scores.copy_(saved)
        rt.run_bound(softmax)
        rt.run_bound(softmax)
    torch.cuda.synchronize()


def split(out_dir: str, symbol: str | None) -> str:
    rows = []
    for f in pathlib.Path(out_dir).rglob("*kernel_trace.csv"):
        with open(f) as fh:
            rows += list(csv.DictReader(fh))
    rows.sort(key=lambda r: int(r["Start_Timestamp"]))
    if symbol is None:
        # the generated function launched most often
        counts: dict[str, int] = {}
        for r in rows:
            if r["Kernel_Name"].startswith("mlc_"):
                counts[r["Kernel_Name"]] = counts.get(r["Kernel_Name"], 0) + 1
        symbol = max(counts, key=counts.get)
    by: dict[str, list[tuple[float, float]]] = {}
    for prev, r in zip(rows, rows[1:]):
        if r["Kernel_Name"] != symbol:
            continue
        before = prev["Kernel_Name"]
        if before == symbol:
            kind = "after itself"
        elif before.startswith("Cijk") or "gemm" in before.lower():
            kind = "after the library bmm"
        elif "copy" in before.lower() or "elementwise" in before.lower():
            kind = "after a torch copy"
        else:
            kind = f"after {before[:40]}"
        dur = (int(r["End_Timestamp"]) - int(r["Start_Timestamp"])) / 1e3
        gap = (int(r["Start_Timestamp"]) - int(prev["End_Timestamp"])) / 1e3
        by.setdefault(kind, []).append((dur, gap))
    lines = [f"`{symbol}`", "",
             "| predecessor | n | median us | mean us | median gap before, us |",
             "|---|---:|---:|---:|---:|"]
    for kind, v in by.items():
        d, g = [x for x, _ in v], [y for _, y in v]
        lines.append(f"| {kind} | {len(d)} | {statistics.median(d):.2f} | "
                     f"{statistics.mean(d):.2f} | {statistics.median(g):.2f} |")
    return "\n".join(lines)


def main() -> int:
    ap = argparse.ArgumentParser()
    sub = ap.add_subparsers(dest="cmd", required=True)
    r = sub.add_parser("run")
    r.add_argument("--iters", type=int, default=20)
    s = sub.add_parser("split")
    s.add_argument("out_dir")
    s.add_argument("--symbol")
    opts = ap.parse_args()
    if opts.cmd == "run":
        run(opts.iters)
    else:
        print(split(opts.out_dir, opts.symbol))
    return 0


if __name__ == "__main__":
    sys.exit(main())
