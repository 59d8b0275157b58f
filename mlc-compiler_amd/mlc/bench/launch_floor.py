"""Where a small-batch forward's time goes: hipGraphs of empty kernel nodes
against the compiled schedule.

    python mlc-compiler_amd/mlc/bench/launch_floor.py --workload C2 [--replays 200]
    python mlc-compiler_amd/mlc/bench/launch_floor.py --workload C2 --shapes

Every graph below is captured with the same C ABI the executor uses
(``mlc_graph_begin`` / ``mlc_launch`` / ``mlc_graph_end``) and replayed
``--replays`` times back to back; the figure is the mean per replay (hipEvents
on the replay stream):

* ``empty x N``: N nodes of a kernel with no body, one 64-thread workgroup
  each, N = the forward's node count -- the floor of a graph that size;
* ``empty, real grids``: the same nodes with each generated kernel's own grid
  and workgroup size (the cost of dispatching its waves);
* ``library calls + empty``: the forward with every generated kernel (and the
  native embedding gather) replaced by a one-workgroup empty node, the
  library GEMMs real -- what the forward would cost if the fused kernels
  were free;
* ``library calls only``: the GEMMs alone;
* ``forward``: every node real (the executor's graph, re-captured here);
* per kernel family (one generated function, every layer's launch of it):
  that family real and every other generated kernel empty. Its excess over
  ``library calls + empty`` is what the family costs above an empty node.

Replacing a kernel by an empty one leaves its outputs stale; the GEMMs that
read them take the same time on any values.
"""

from __future__ import annotations

import argparse
import ctypes
import pathlib
import struct
import sys

ROOT = pathlib.Path(__file__).resolve().parents[3]
for _p in (ROOT / "mlc-compiler_amd", ROOT):
    if str(_p) not in sys.path:
        sys.path.insert(0, str(_p))

EMPTY_SOURCE = """#include <hip/hip_runtime.h>
extern "C" __global__ void __launch_bounds__(1024) mlc_empty(const void* p) { (void)p; }
"""


class _Graph:
    """One context holding one captured graph."""

    def __init__(self, lib, native, device: int) -> None:
        self.lib, self.native = lib, native
        self.ctx = ctypes.c_void_p()
        native.check(lib.mlc_ctx_create(device, ctypes.byref(self.ctx)), "mlc_ctx_create")

    def capture(self, stream, body) -> None:
        import torch

        self.native.check(self.lib.mlc_graph_begin(self.ctx, stream.cuda_stream), "mlc_graph_begin")
        try:
            with torch.cuda.stream(stream):
                body(stream.cuda_stream)
        finally:
            self.native.check(self.lib.mlc_graph_end(self.ctx), "mlc_graph_end")

    def nodes(self) -> int:
        n = ctypes.c_size_t()
        self.native.check(self.lib.mlc_graph_node_count(self.ctx, ctypes.byref(n)), "node count")
        return n.value

    def time(self, stream, replays: int) -> float:
        """Mean ms per replay of ``replays`` back-to-back replays."""
        import torch

        for _ in range(10):
            self.native.check(self.lib.mlc_graph_replay(self.ctx, stream.cuda_stream), "replay")
        stream.synchronize()
        samples = []
        for _ in range(3):
            t0, t1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
            t0.record(stream)
            for _ in range(replays):
                self.native.check(self.lib.mlc_graph_replay(self.ctx, stream.cuda_stream), "replay")
            t1.record(stream)
            t1.synchronize()
            samples.append(t0.elapsed_time(t1) / replays)
        return min(samples)

    def close(self) -> None:
        self.lib.mlc_ctx_destroy(self.ctx)


def decompose(workload: str, replays: int = 200, blas: str | None = None):
    import torch

    import mlc
    from mlc.bench.workloads import make
    from mlc.config import Config

    device = torch.device("cuda", 0)
    torch.cuda.set_device(device)
    if blas:
        torch.backends.cuda.preferred_blas_library(blas)
    model, inputs = make(workload, device)
    compiled = mlc.compile(model, inputs, Config())
    d = decompose_compiled(compiled, inputs, replays)
    d.update(workload=workload, blas=blas)
    return d


def decompose_compiled(compiled, inputs, replays: int = 200, families=None, shapes: bool = True,
                       log=print):
    """The graphs above for an already compiled model (``families``: the
    generated functions to time one by one, every one when None; ``shapes``:
    also the all-empty graphs; ``log``: where progress lines go)."""
    import torch

    from mlc.runtime import native
    from mlc.runtime.hip_runtime import Bound

    index = compiled.device.index
    device = torch.device("cuda", torch.cuda.current_device() if index is None else index)
    lib = native.load_library()
    compiled(*inputs)
    torch.cuda.synchronize()
    rt = compiled._module

    _, obj = native.compile_code_object(EMPTY_SOURCE)
    image = obj.read_bytes()
    ctx0 = ctypes.c_void_p()
    native.check(lib.mlc_ctx_create(device.index, ctypes.byref(ctx0)), "mlc_ctx_create")
    mod = ctypes.c_void_p()
    native.check(lib.mlc_module_load(ctx0, ctypes.create_string_buffer(image, len(image)), len(image),
                                     ctypes.byref(mod)), "mlc_module_load")
    empty = ctypes.c_void_p()
    native.check(lib.mlc_function(mod, b"mlc_empty", ctypes.byref(empty)), "mlc_function")
    dummy = torch.zeros(64, device=device)
    empty_args = struct.pack("<Q", dummy.data_ptr())

    # (kind, bound launch or library call, family symbol) in schedule order
    entries = []
    for k, (kind, payload) in zip(compiled.schedule.kernels, compiled._plan):
        if kind == "kernel":
            entries.append(("gen", payload, rt.launch_table[k.name].symbol))
        elif kind == "extern" and getattr(payload, "module", None) is rt:
            entries.append(("gen", payload.bound, rt.launch_table[k.name].symbol))
        elif kind == "extern":
            entries.append(("lib", payload, None))
    n_gen = sum(1 for e in entries if e[0] == "gen")
    n_lib = len(entries) - n_gen

    def launch(b: Bound, s):
        if b.grid:
            native.check(lib.mlc_launch(b.fn, b.grid, b.block, b.lds, b.args, len(b.args), s), b.name)

    def launch_empty(s, grid=1, block=64):
        native.check(lib.mlc_launch(empty, grid, block, 0, empty_args, len(empty_args), s), "empty")

    def body(real_gen, real_lib=True, empty_for_gen=True, real_grids=False):
        def run(s):
            for kind, p, fam in entries:
                if kind == "lib":
                    if real_lib:
                        p.run()
                    elif empty_for_gen:
                        launch_empty(s)
                elif real_gen(fam):
                    launch(p, s)
                elif empty_for_gen and not (real_grids and p.grid == 0):
                    launch_empty(s, p.grid if real_grids else 1, p.block if real_grids else 64)
        return run

    # the executor's own graph first: the variants below run the embedding
    # gathers on stale ids (their id producers replaced by empty nodes), which
    # flags the compiled model's invalid-input word
    t0, t1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    for _ in range(10):
        compiled(*inputs)
    torch.cuda.synchronize()
    t0.record()
    for _ in range(replays):
        compiled(*inputs)
    t1.record()
    t1.synchronize()
    executor_ms = t0.elapsed_time(t1) / replays
    log(f"executor graph replay: {executor_ms * 1e3:.1f} us per forward")

    stream = torch.cuda.Stream(device)
    results = []

    def measure(label, run, note=""):
        g = _Graph(lib, native, device.index)
        try:
            g.capture(stream, run)
            ms = g.time(stream, replays)
            results.append((label, g.nodes(), ms, note))
        finally:
            g.close()
        log(f"{label}: {results[-1][1]} nodes, {ms * 1e3:.1f} us per replay")
        return ms

    n = len(entries)
    if shapes:
        measure(f"empty x {n}", lambda s: [launch_empty(s) for _ in range(n)])
        measure(f"empty x {n}, real grids", body(lambda f: False, real_lib=False, real_grids=True))
    base = measure(f"library calls ({n_lib}) + empty ({n_gen})", body(lambda f: False))
    library = measure(f"library calls only ({n_lib})", body(lambda f: False, empty_for_gen=False))
    full = measure("forward (every node real)", body(lambda f: True))
    launches_of = {}
    for kind, p, fam in entries:
        if kind == "gen":
            launches_of.setdefault(fam, []).append(p)
    fam_rows = []
    for fam, launches in launches_of.items():
        if families is not None and fam not in families:
            continue
        ms = measure(f"family {fam} real", body(lambda f, fam=fam: f == fam))
        fam_rows.append((fam, len(launches), ms - base))
    torch.cuda.synchronize()
    rt.clear_errors()
    lib.mlc_module_unload(mod)
    lib.mlc_ctx_destroy(ctx0)
    summaries = {}
    for k in compiled.schedule.kernels:
        spec = rt.launch_table.get(k.name)
        if spec is not None and spec.symbol not in summaries:
            summaries[spec.symbol] = k.summary().split(": ", 1)[-1][:60]
    return {"entries": n, "generated": n_gen, "library": n_lib, "results": results,
            "families": fam_rows, "base": base, "library_only": library, "full": full,
            "executor": executor_ms, "summaries": summaries, "replays": replays}


def report(d) -> str:
    L = [f"| graph | nodes | us per replay |", "|---|---:|---:|"]
    for label, nodes, ms, _ in d["results"]:
        if not label.startswith("family"):
            L.append(f"| {label} | {nodes} | {ms * 1e3:.1f} |")
    L.append(f"| executor's graph (`CompiledModel.__call__`, input copy included) | | "
             f"{d['executor'] * 1e3:.1f} |")
    L += ["", "| family (generated function) | launches | excess over empty nodes, us | per launch, us | kernel |",
          "|---|---:|---:|---:|---|"]
    total = 0.0
    for fam, n, ex in sorted(d["families"], key=lambda r: -r[2]):
        total += ex
        L.append(f"| `{fam}` | {n} | {ex * 1e3:.1f} | {ex * 1e3 / n:.2f} | {d['summaries'].get(fam, '')} |")
    L.append(f"| sum of families | | {total * 1e3:.1f} | | |")
    L.append(f"| forward - (library calls + empty) | | {(d['full'] - d['base']) * 1e3:.1f} | | |")
    return "\n".join(L)


def shape_sweep(workload: str, shapes, replays: int = 200):
    """Forward time (executor graph replay) with the pointwise and reduction
    workgroup sizes set to each ``(pointwise, reduction)`` pair."""
    import torch

    import mlc
    from mlc.bench.workloads import make
    from mlc.codegen import hip_backend
    from mlc.config import Config

    saved = hip_backend.POINTWISE_TUNING["block"], hip_backend.REDUCTION_TUNING["block"]
    rows = []
    try:
        for pw, red in shapes:
            hip_backend.POINTWISE_TUNING["block"] = pw
            hip_backend.REDUCTION_TUNING["block"] = red
            model, inputs = make(workload, "cuda")
            compiled = mlc.compile(model, inputs, Config())
            for _ in range(20):
                compiled(*inputs)
            torch.cuda.synchronize()
            best = float("inf")
            for _ in range(3):
                t0, t1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
                t0.record()
                for _ in range(replays):
                    compiled(*inputs)
                t1.record()
                t1.synchronize()
                best = min(best, t0.elapsed_time(t1) / replays)
            rows.append((pw, red, best))
            print(f"{workload} pointwise {pw} / reduction {red} threads: {best * 1e3:.1f} us per forward",
                  flush=True)
            del compiled, model, inputs
    finally:
        hip_backend.POINTWISE_TUNING["block"], hip_backend.REDUCTION_TUNING["block"] = saved
    return rows


SHAPES = [(512, 128), (256, 128), (128, 128), (64, 128), (128, 64), (128, 256), (512, 64)]


def main() -> int:
    ap = argparse.ArgumentParser()
    ap.add_argument("--workload", default="C2")
    ap.add_argument("--replays", type=int, default=200)
    ap.add_argument("--blas", default=None,
                    help="torch's preferred BLAS library for the GEMMs (torch.backends.cuda."
                         "preferred_blas_library: cublas = rocBLAS, cublaslt = hipBLASLt)")
    ap.add_argument("--shapes", action="store_true",
                    help="instead: the forward under each workgroup-size pair of SHAPES")
    opts = ap.parse_args()
    if opts.shapes:
        shape_sweep(opts.workload, SHAPES, opts.replays)
        return 0
    d = decompose(opts.workload, opts.replays, opts.blas)
    print(report(d), flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
