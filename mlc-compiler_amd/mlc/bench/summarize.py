"""Turn rocprofv3 CSV output into the markdown summaries kept in ``profiles/``.

    python mlc-compiler_amd/mlc/bench/summarize.py traffic --workload C4 \\
        --fetch DIR --write DIR --trace DIR [--config every] --title TEXT -o profiles/X.md
    python mlc-compiler_amd/mlc/bench/summarize.py stats --trace DIR --command TEXT \\
        --title TEXT -o profiles/X.md
    python mlc-compiler_amd/mlc/bench/summarize.py counters --kind valu|stalls \\
        --workload C4 --pmc DIR [--pmc DIR] --trace DIR --title TEXT -o profiles/X.md

``traffic``: the ``FETCH_SIZE`` and ``WRITE_SIZE`` runs of ``traffic.py --kernel
all`` (one counter per run) and a kernel trace of the same tool. Each counter
is scaled by what it reads for the plain 1 GiB copy the tool launches first
(true bytes / counter bytes), averaged over every dispatch of a generated
function, and set beside that function's algorithmic bytes per launch (the
reference cost model's ``traffic()``); the time is the traced average of its
back-to-back launches. The summary ends with one machine-readable line per
function, ``traffic_bytes_per_launch <symbol> <bytes>``, which ``bench.py``
reads for its ``traffic`` field.

``stats``: a kernel trace (``--kernel-trace --stats``) of ``bench.py``: the top
of rocprofv3's own per-kernel table, then every generated function of BERT
b32 with its dispatches split by what ran just before (``trace_split``: the
timing loop, or in sequence as in a forward).

``counters``: per generated function, the means of a ``--pmc`` run's counters
over its launches inside the forward: VALU issue against traced time
(``--kind valu``), or the shares of its waves' lifetime spent waiting and the
texture-path stall cycles (``--kind stalls``).

Symbols are matched to kernels by compiling the workload's schedule on the CPU
(the symbol is a hash of the generated function's body).
"""

from __future__ import annotations

import argparse
import collections
import csv
import pathlib
import statistics
import sys

ROOT = pathlib.Path(__file__).resolve().parents[3]
for _p in (ROOT / "mlc-compiler_amd", ROOT):
    if str(_p) not in sys.path:
        sys.path.insert(0, str(_p))

HBM_PEAK_GBS = 8000.0
COPY_BYTES = 1 << 30  # traffic.py's plain copy: 1 GiB read and 1 GiB written


def _show(path: str) -> str:
    """``path`` as the summaries quote it: relative to the repository as ``$R/...``."""
    p = pathlib.Path(path).resolve()
    try:
        return "$R/" + str(p.relative_to(ROOT.resolve()))
    except ValueError:
        return str(path)


def _csv(directory: str, suffix: str) -> list[dict]:
    found = sorted(pathlib.Path(directory).rglob(f"*{suffix}"))
    if not found:
        raise SystemExit(f"no *{suffix} under {directory}")
    with open(found[0]) as f:
        return list(csv.DictReader(f))


def schedule_symbols(workload: str, every: bool = False) -> dict:
    """symbol -> [kernel, algorithmic bytes per launch, launches per forward]
    for the generated functions of a workload's schedule (embedding gathers
    left out: their bytes depend on the ids)."""
    from mlc.api import build_pipeline
    from mlc.bench.roofline import algorithmic_bytes
    from mlc.bench.workloads import make
    from mlc.codegen.hip_backend import build_module
    from mlc.config import Config
    from mlc.ir.capture import capture

    cfg = (Config(merge_parallel_gemms=True, gemm_epilogue=True, layout_selection=True,
                  fused_attention=True) if every else Config())
    model, args = make(workload, "cpu")
    schedule = build_pipeline(capture(model, args), cfg)
    module = build_module(schedule, cfg)
    info: dict = {}
    for k in schedule.kernels:
        spec = module.launches.get(k.name)
        if spec is None or spec.meta.get("kind") == "embedding":
            continue
        entry = info.setdefault(spec.symbol, [k, algorithmic_bytes(k), 0])
        entry[2] += 1
    return info


def _counter_bytes(rows: list[dict]) -> tuple[float, dict[str, list[float]]]:
    """(scale to true bytes, symbol -> counter KiB per dispatch)."""
    copy = [float(r["Counter_Value"]) for r in rows
            if "copyBuffer" in r["Kernel_Name"] and float(r["Counter_Value"]) > 4e5]
    if not copy:
        raise SystemExit("the counter run holds no 1 GiB copy to scale by")
    per: dict[str, list[float]] = collections.defaultdict(list)
    for r in rows:
        per[r["Kernel_Name"].split("(")[0].strip()].append(float(r["Counter_Value"]))
    return COPY_BYTES / (statistics.mean(copy) * 1024), per


def _loop_us(trace: list[dict]) -> dict[str, list[float]]:
    trace = sorted(trace, key=lambda r: int(r["Start_Timestamp"]))
    loop: dict[str, list[float]] = collections.defaultdict(list)
    for before, r in zip(trace, trace[1:]):
        if before["Kernel_Name"] == r["Kernel_Name"]:
            loop[r["Kernel_Name"]].append((int(r["End_Timestamp"]) - int(r["Start_Timestamp"])) / 1e3)
    return loop


def traffic(opts) -> str:
    info = schedule_symbols(opts.workload, opts.config == "every")
    fscale, fetch = _counter_bytes(_csv(opts.fetch, "counter_collection.csv"))
    wscale, write = _counter_bytes(_csv(opts.write, "counter_collection.csv"))
    loop = _loop_us(_csv(opts.trace, "kernel_trace.csv"))
    rows = []
    for sym, (k, alg, n) in info.items():
        if not fetch.get(sym) or not write.get(sym):
            continue
        counted = (statistics.mean(fetch[sym]) * fscale + statistics.mean(write[sym]) * wscale) * 1024
        us = statistics.mean(loop[sym]) if loop.get(sym) else float("nan")
        rows.append((n * us, n, sym, k, alg, counted, us))
    rows.sort(key=lambda r: -r[0])
    flag = " --config every" if opts.config == "every" else ""
    tool = "python3 -u $R/mlc-compiler_amd/mlc/bench/traffic.py --kernel all" + flag
    L = [f"# HBM traffic (PMC) of every generated kernel: {opts.title}", "",
         "Commands (run from `/tmp` on the MI355X box, repository at `$R`; one counter per run):",
         "", "```",
         f"rocprofv3 --pmc FETCH_SIZE --output-format csv -d {_show(opts.fetch)} -o t -- \\",
         f"    {tool} --workload {opts.workload} --iters 3",
         f"rocprofv3 --pmc WRITE_SIZE --output-format csv -d {_show(opts.write)} -o t -- \\",
         f"    {tool} --workload {opts.workload} --iters 3",
         f"rocprofv3 --kernel-trace --stats --output-format csv -d {_show(opts.trace)} -o t -- \\",
         f"    {tool} --workload {opts.workload} --iters 20 --copy-mib 64",
         f"python3 $R/mlc-compiler_amd/mlc/bench/summarize.py traffic --workload {opts.workload} "
         f"--config {opts.config} --fetch {_show(opts.fetch)} --write {_show(opts.write)} "
         f"--trace {_show(opts.trace)} --title '{opts.title}' -o <summary.md>",
         "```", "",
         "`traffic.py --kernel all` launches a plain 1 GiB fp16 copy five times, runs one forward, "
         "then, for every generated kernel in schedule order, replays the plan up to it (so it runs "
         "on its real inputs) and launches it `--iters` more times. Counters are averaged over every "
         "dispatch of a function and scaled by what they read for the copy (true bytes / counter "
         f"bytes: FETCH {fscale:.4f}, WRITE {wscale:.4f}). Time is the traced average of the "
         "back-to-back launches of the third run (inputs resident in the MALL after the first "
         "launch; tracing adds about 10% per dispatch); GB/s is counter bytes over that time. "
         "Embedding gathers are left out (their algorithmic bytes depend on the ids).", "",
         "| n | symbol | kernel | algorithmic MB | counter MB | counter / alg. | traced us | "
         "counter GB/s | of 8 TB/s |",
         "|---:|---|---|---:|---:|---:|---:|---:|---:|"]
    tot_alg = tot_cnt = tot_us = 0.0
    for _, n, sym, k, alg, counted, us in rows:
        gbs = counted / (us * 1e-6) / 1e9
        desc = k.summary().split(": ", 1)[1][:56]
        L.append(f"| {n} | `{sym}` | {desc} | {alg / 1e6:.2f} | {counted / 1e6:.2f} | "
                 f"{counted / alg:.3f} | {us:.2f} | {gbs:.0f} | {gbs / HBM_PEAK_GBS:.3f} |")
        tot_alg += n * alg
        tot_cnt += n * counted
        tot_us += n * us
    nk = sum(r[1] for r in rows)
    L += ["", f"All {nk} generated kernels of a forward (embeddings aside): {tot_cnt / 1e9:.3f} GB "
          f"counted against {tot_alg / 1e9:.3f} GB algorithmic ({tot_cnt / tot_alg:.3f}x), "
          f"{tot_us / 1e3:.3f} ms traced, {tot_cnt / (tot_us * 1e-6) / 1e9:.0f} GB/s "
          f"({tot_cnt / (tot_us * 1e-6) / 1e9 / HBM_PEAK_GBS:.3f} of 8 TB/s)."]
    L += ["", "Machine-readable lines (counter bytes per launch, read by `bench.py` for its "
          "`traffic` fields):", ""]
    L += [f"traffic_bytes_per_launch {sym} {int(round(counted))}"
          for _, n, sym, k, alg, counted, us in rows]
    return "\n".join(L) + "\n"


def stats(opts) -> str:
    from mlc.bench.trace_split import classify, report

    table = _csv(opts.trace, "kernel_stats.csv")
    trace = _csv(opts.trace, "kernel_trace.csv")
    info = schedule_symbols("C4")
    nbytes = {sym: v[1] for sym, v in info.items()}
    L = [f"# Kernel trace: {opts.title}", "", "Command (run from `/tmp` on the MI355X box, "
         "repository at `$R`):", "", "```", opts.command,
         f"python3 $R/mlc-compiler_amd/mlc/bench/summarize.py stats --trace {_show(opts.trace)} "
         "--command '<the command above>' --title '<title>' -o <summary.md>",
         "```", "", "`mlc_*` are this build's generated kernels; `Cijk_*` are hipBLASLt GEMMs "
         "(torch extern `mm.out`/`bmm.out`).", "",
         "| calls | avg us | % time | kernel |", "|---:|---:|---:|---|"]
    for r in table[:opts.top]:
        name = r["Name"] if len(r["Name"]) <= 90 else r["Name"][:87] + "..."
        L.append(f"| {r['Calls']} | {float(r['AverageNs']) / 1e3:.2f} | {float(r['Percentage']):.2f} "
                 f"| `{name}` |")
    split = {s: v for s, v in classify(trace).items() if s in info}
    L += ["", "Generated functions of the BERT b32 reference schedule, their dispatches split by "
          "what ran just before each (`trace_split.py`): `loop`, the same kernel (the timing "
          "loop: inputs cache-resident after the first launch); `in sequence`, a library GEMM or "
          "another generated kernel, as inside a forward (the hipGraph replays, and the plan "
          "prefixes the timing loop replays). Fractions are algorithmic bytes per launch over "
          "the mean traced duration.", "", report(split, nbytes), "",
          "| symbol | launches per forward | kernel | algorithmic MB |", "|---|---:|---|---:|"]
    for sym, (k, alg, n) in sorted(info.items(), key=lambda kv: -kv[1][1] * kv[1][2]):
        L.append(f"| `{sym}` | {n} | {k.summary().split(': ', 1)[1][:60]} | {alg / 1e6:.2f} |")
    return "\n".join(L) + "\n"


def _counters(directories: list[str]) -> dict:
    """symbol -> counter name -> [(dispatch id, value)] over several PMC runs."""
    by: dict = collections.defaultdict(lambda: collections.defaultdict(list))
    for d in directories:
        for r in _csv(d, "counter_collection.csv"):
            by[r["Kernel_Name"].split("(")[0].strip()][r["Counter_Name"]].append(
                (int(r["Dispatch_Id"]), float(r["Counter_Value"])))
    return by


#: cycles per wave64 fp32 VALU instruction on a 16-lane SIMD (packed fp32 off),
#: SIMDs on the chip, and the shader clock used to turn issue counts into time
VALU_CYCLES, SIMDS, CLOCK_HZ = 4, 1024, 2.4e9

VALU_COUNTERS = ("SQ_WAVES SQ_INSTS_VALU SQ_INSTS_SALU SQ_INSTS_VMEM_RD SQ_INSTS_VMEM_WR "
                 "SQ_INSTS_LDS SQ_BUSY_CYCLES SQ_WAVE_CYCLES",
                 "SQ_INSTS_VALU_ADD_F32 SQ_INSTS_VALU_CVT SQ_INSTS_VALU_FMA_F32 "
                 "SQ_INSTS_VALU_MFMA_F32 SQ_INSTS_VALU_MUL_F32 SQ_INSTS_VALU_TRANS_F16 "
                 "SQ_INSTS_VALU_TRANS_F32")
STALL_COUNTERS = ("SQ_WAVES SQ_WAVE_CYCLES SQ_BUSY_CYCLES SQ_WAIT_ANY SQ_WAIT_INST_ANY "
                  "SQ_ACTIVE_INST_VALU SQ_ACTIVE_INST_ANY SQ_INSTS_VALU",
                  "TA_BUSY_avr TA_DATA_STALLED_BY_TC_CYCLES_sum TCP_PENDING_STALL_CYCLES_sum "
                  "TCP_TCR_TCP_STALL_CYCLES_sum TCP_READ_TAGCONFLICT_STALL_CYCLES_sum "
                  "TCP_TCP_TA_DATA_STALL_CYCLES_sum GRBM_GUI_ACTIVE")


def counters(opts) -> str:
    """``valu``: VALU issue against traced time per generated function;
    ``stalls``: where its waves wait. Each counter is the mean over the
    function's first ``n`` dispatches (``n`` = its launches per forward:
    ``traffic.py`` runs one whole forward before its timing loops, so those
    are the launches inside the forward, on their real inputs)."""
    info = schedule_symbols(opts.workload, opts.config == "every")
    by = _counters(opts.pmc)
    loop = _loop_us(_csv(opts.trace, "kernel_trace.csv"))
    sets = VALU_COUNTERS if opts.kind == "valu" else STALL_COUNTERS
    tool = ("python3 -u $R/mlc-compiler_amd/mlc/bench/traffic.py --kernel all"
            + (" --config every" if opts.config == "every" else "")
            + f" --workload {opts.workload}")
    L = [f"# {opts.title}", "", "Commands (run from `/tmp` on the MI355X box, repository at "
         "`$R`; one counter set per run):", "", "```"]
    for d, names in zip(opts.pmc, sets):
        L += [f"rocprofv3 --pmc {names} --output-format csv -d {_show(d)} -o v -- \\",
              f"    {tool} --iters 3 --copy-mib 64"]
    L += [f"rocprofv3 --kernel-trace --stats --output-format csv -d {_show(opts.trace)} -o t -- "
          "\\", f"    {tool} --iters 20 --copy-mib 64",
          f"python3 $R/mlc-compiler_amd/mlc/bench/summarize.py counters --kind {opts.kind} "
          f"--workload {opts.workload} --config {opts.config} "
          + " ".join(f"--pmc {_show(d)}" for d in opts.pmc)
          + f" --trace {_show(opts.trace)} --title '<title>' -o <summary.md>", "```", ""]
    rows = []
    for sym, (k, nbytes, n) in info.items():
        c = by.get(sym)
        if not c:
            continue
        def f(name, c=c, n=n):
            return statistics.mean(v for _, v in sorted(c[name])[:n])

        t = statistics.mean(loop[sym]) if loop.get(sym) else float("nan")
        rows.append((n, sym, k.summary().split(": ", 1)[1], nbytes, f, t))
    rows.sort(key=lambda r: -r[0] * (r[5] if r[5] == r[5] else 0))
    if opts.kind == "valu":
        L += ["Counters are each function's launches inside the forward (real inputs); the time "
              "is the traced average of its back-to-back launches (tracing adds about 0.8 us). "
              "VALU issue time = `SQ_INSTS_VALU` x 4 cycles (a wave64 fp32 VALU instruction on a "
              "16-lane SIMD; packed fp32 is off) / 1024 SIMDs / 2.4 GHz: the time the kernel "
              "would take if it did nothing but issue its vector ALU instructions on every SIMD "
              "of the chip. The `SQ_INSTS_VALU_*` classes are per wave; `v_fma_mix_f32` counts "
              "as FMA_F32.", "",
              "| n | symbol | kernel | MB / launch | waves | VALU / wave | TRANS | FMA | ADD | MUL "
              "| CVT | VMEM / wave | VALU issue us | traced us |",
              "|---:|---|---|---:|---:|---:|---:|---:|---:|---:|---:|---:|---:|---:|"]
        for n, sym, summ, nbytes, f, t in rows:
            waves = f("SQ_WAVES")
            valu = f("SQ_INSTS_VALU")
            def per(name, f=f, waves=waves):
                return f(name) / waves

            issue = valu * VALU_CYCLES / SIMDS / CLOCK_HZ * 1e6
            vmem = (f("SQ_INSTS_VMEM_RD") + f("SQ_INSTS_VMEM_WR")) / waves
            L.append(f"| {n} | `{sym}` | {summ[:50]} | {nbytes / 1e6:.2f} | {waves:.0f} | "
                     f"{valu / waves:.1f} | {per('SQ_INSTS_VALU_TRANS_F32'):.1f} | "
                     f"{per('SQ_INSTS_VALU_FMA_F32'):.1f} | {per('SQ_INSTS_VALU_ADD_F32'):.1f} | "
                     f"{per('SQ_INSTS_VALU_MUL_F32'):.1f} | {per('SQ_INSTS_VALU_CVT'):.1f} | "
                     f"{vmem:.1f} | {issue:.2f} | {t:.2f} |")
    else:
        L += ["Each function's launches inside the forward (real inputs). The SQ columns are "
              "shares of the waves' lifetime (`SQ_WAVE_CYCLES`): waiting on anything "
              "(`SQ_WAIT_ANY`), waiting for an instruction's dependency (`SQ_WAIT_INST_ANY`), "
              "issuing VALU work, issuing anything. The TA/TCP columns are cycles per GPU-active "
              "cycle (`GRBM_GUI_ACTIVE`), summed over the chip's instances (`TA_BUSY_avr` "
              "averaged): texture-address busy, texture-address data stalled by the L2 "
              "(`TA_DATA_STALLED_BY_TC`), vector L1 stalled on pending misses "
              "(`TCP_PENDING_STALL`), on the L2 return path (`TCP_TCR_TCP_STALL`), on tag "
              "conflicts, and on the TA data path.", "",
              "| n | symbol | kernel | waves | wait any | wait inst | VALU | issue any | TA busy "
              "| TA data stalled by L2 | TCP pending stall | TCP L2-return stall | TCP tag conflict "
              "| TCP TA-data stall |",
              "|---:|---|---|---:|---:|---:|---:|---:|---:|---:|---:|---:|---:|---:|"]
        for n, sym, summ, nbytes, f, t in rows:
            wc, g = f("SQ_WAVE_CYCLES"), f("GRBM_GUI_ACTIVE")
            L.append(f"| {n} | `{sym}` | {summ[:44]} | {f('SQ_WAVES'):.0f} | "
                     f"{f('SQ_WAIT_ANY') / wc:.0%} | {f('SQ_WAIT_INST_ANY') / wc:.0%} | "
                     f"{f('SQ_ACTIVE_INST_VALU') / wc:.0%} | {f('SQ_ACTIVE_INST_ANY') / wc:.0%} | "
                     f"{f('TA_BUSY_avr') / g:.2f} | {f('TA_DATA_STALLED_BY_TC_CYCLES_sum') / g:.2f} | "
                     f"{f('TCP_PENDING_STALL_CYCLES_sum') / g:.2f} | "
                     f"{f('TCP_TCR_TCP_STALL_CYCLES_sum') / g:.2f} | "
                     f"{f('TCP_READ_TAGCONFLICT_STALL_CYCLES_sum') / g:.2f} | "
                     f"{f('TCP_TCP_TA_DATA_STALL_CYCLES_sum') / g:.2f} |")
    return "\n".join(L) + "\n"


def main() -> int:
    ap = argparse.ArgumentParser()
    sub = ap.add_subparsers(dest="what", required=True)
    t = sub.add_parser("traffic")
    t.add_argument("--workload", required=True)
    t.add_argument("--config", choices=("reference", "every"), default="reference")
    t.add_argument("--fetch", required=True)
    t.add_argument("--write", required=True)
    t.add_argument("--trace", required=True)
    t.add_argument("--title", required=True)
    t.add_argument("-o", "--out", required=True)
    s = sub.add_parser("stats")
    s.add_argument("--trace", required=True)
    s.add_argument("--command", required=True, help="the traced command, quoted in the summary")
    s.add_argument("--title", required=True)
    s.add_argument("--top", type=int, default=30)
    s.add_argument("-o", "--out", required=True)
    c = sub.add_parser("counters")
    c.add_argument("--kind", choices=("valu", "stalls"), required=True)
    c.add_argument("--workload", required=True)
    c.add_argument("--config", choices=("reference", "every"), default="reference")
    c.add_argument("--pmc", action="append", required=True,
                   help="a PMC run's output directory (the counter sets of --kind, in order)")
    c.add_argument("--trace", required=True)
    c.add_argument("--title", required=True)
    c.add_argument("-o", "--out", required=True)
    opts = ap.parse_args()
    text = {"traffic": traffic, "stats": stats, "counters": counters}[opts.what](opts)
    pathlib.Path(opts.out).write_text(text)
    print(text[-1500:])
    return 0


if __name__ == "__main__":
    sys.exit(main())
