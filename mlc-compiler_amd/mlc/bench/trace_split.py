"""Split a ``rocprofv3 --kernel-trace`` by what ran just before each
generated-kernel dispatch:

* ``loop``: the same kernel (a back-to-back timing loop, such as
  ``bench.py``'s per-kernel table: the inputs stay cache-resident after the
  first launch);
* ``after fill``: a torch fill kernel (a measurement that writes a large
  buffer before a launch to evict the caches);
* ``in sequence``: anything else -- a library GEMM or another generated
  kernel, as inside a forward (the hipGraph replays, and the plan prefixes a
  timing loop replays before each kernel).

    python mlc-compiler_amd/mlc/bench/trace_split.py <kernel_trace.csv> [--bytes BYTES.json]

Prints a markdown table: per generated function, the dispatch count and the
mean traced duration of each class that occurs (and, with ``--bytes``, a JSON
map from symbol to algorithmic bytes per launch, each class's fraction of
8 TB/s).
"""

from __future__ import annotations

import argparse
import csv
import json
import statistics
import sys

HBM_PEAK_GBS = 8000.0
KINDS = ("loop", "after fill", "in sequence")


def classify(rows: list[dict]) -> dict[str, dict[str, list[float]]]:
    rows = sorted(rows, key=lambda r: int(r["Start_Timestamp"]))
    out: dict[str, dict[str, list[float]]] = {}
    prev = None
    for r in rows:
        name = r["Kernel_Name"]
        if name.startswith("mlc_") and prev is not None:
            before = prev["Kernel_Name"]
            if before == name:
                kind = "loop"
            elif "FillFunctor" in before:
                kind = "after fill"
            else:
                kind = "in sequence"
            us = (int(r["End_Timestamp"]) - int(r["Start_Timestamp"])) / 1e3
            out.setdefault(name, {}).setdefault(kind, []).append(us)
        prev = r
    return out


def report(split, nbytes: dict | None = None) -> str:
    kinds = [k for k in KINDS if any(k in d for d in split.values())]
    head = "| symbol | " + " | ".join(f"{k}: n, avg us" for k in kinds) + " |"
    if nbytes:
        head += " " + " | ".join(f"{k}: of 8 TB/s" for k in kinds) + " |"
    lines = [head, "|---" * (1 + len(kinds) * (2 if nbytes else 1)) + "|"]
    for sym in sorted(split, key=lambda s: -(nbytes or {}).get(s, 0)):
        cells, fracs = [], []
        for k in kinds:
            v = split[sym].get(k, [])
            cells.append(f"{len(v)}, {statistics.mean(v):.2f}" if v else "0, -")
            if nbytes and v and sym in nbytes:
                fracs.append(f"{nbytes[sym] / statistics.mean(v) / 1e3 / HBM_PEAK_GBS:.3f}")
            elif nbytes:
                fracs.append("-")
        line = f"| `{sym}` | " + " | ".join(cells) + " |"
        if nbytes:
            line += " " + " | ".join(fracs) + " |"
        lines.append(line)
    return "\n".join(lines)


def main() -> int:
    ap = argparse.ArgumentParser()
    ap.add_argument("trace")
    ap.add_argument("--bytes", default=None, help="JSON file: symbol -> algorithmic bytes")
    opts = ap.parse_args()
    with open(opts.trace) as f:
        split = classify(list(csv.DictReader(f)))
    nbytes = json.load(open(opts.bytes)) if opts.bytes else None
    print(report(split, nbytes))
    return 0


if __name__ == "__main__":
    sys.exit(main())
