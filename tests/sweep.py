"""Random-program sweeps beyond the committed seeds (test infrastructure; not
collected by pytest). Four modes:

    python tests/sweep.py lower START COUNT      # CPU: every program and its wide
                                                 # form captured, scheduled and
                                                 # rendered under four pass
                                                 # configurations each; no hipcc
    python tests/sweep.py compile START COUNT    # CPU: the GPU cases' modules built
                                                 # with hipcc into the code-object cache
    python tests/sweep.py gpu START COUNT        # MI355X: each case through the HIP
                                                 # path against the oracle
    python tests/sweep.py attention START COUNT  # MI355X: the fused-attention variant

A case per seed: the program under the default passes, streamed reductions,
its wide form, graph replay and layout selection; the wide form with long
streamed rows (even seeds); a random transformer stack; a random extern
chain. ``gpu`` prints ``OK``/``BAD`` with the worst error per case, at the bar
of the narrowest dtype each chain stores (``fuzz_programs.TOLERANCE``) for
programs, 1e-5 / 2e-3 / 2.5e-2 (fp32 / fp16 / bf16) for stacks and extern
chains; ``lower`` and ``compile`` print every exception. A failure is
reported, not raised, so one run covers the whole range.
"""

from __future__ import annotations

import pathlib
import sys
import time

ROOT = pathlib.Path(__file__).resolve().parents[1]
for _p in (ROOT / "mlc-compiler_amd", ROOT, ROOT / "tests"):
    if str(_p) not in sys.path:
        sys.path.insert(0, str(_p))

WORKERS = 6


def _configs():
    from mlc.config import Config

    plain = Config(cuda_graphs=False)
    layout = Config(cuda_graphs=False, layout_selection=True)
    no_fusion = Config(elementwise_fusion=False, recompute=False, reduction_fusion=False,
                       memory_planning=False, cuda_graphs=False)
    # a name starting "wide" runs the program's wide form (rows of 700-4099)
    return {"default": plain, "graph": Config(),
            "streamed": Config(cuda_graphs=False, max_persistent_row=16),
            "layout": layout, "no_fusion": no_fusion,
            "wide": plain, "wide_streamed": Config(cuda_graphs=False, max_persistent_row=512),
            "wide_layout": layout, "wide_no_fusion": no_fusion}


def gpu_cases(start: int, count: int):
    for seed in range(start, start + count):
        for cname in ("default", "streamed", "wide", "graph", "layout"):
            yield ("program", seed, cname)
        if seed % 2 == 0:
            yield ("program", seed, "wide_streamed")
        yield ("stack", seed, "default")
        yield ("extern", seed, "default")


def _build(kind: str, seed: int, cname: str):
    import fuzz_programs as fp

    if kind == "program":
        return fp.program(seed, wide=cname.startswith("wide")) + (None,)
    if kind == "stack":
        return fp.block_case(seed)
    return fp.extern_case(seed)


def _lower_one(job):
    """(job, error or None): build one module; with ``hip`` also compile it."""
    case, hip = job
    from mlc.api import build_pipeline
    from mlc.codegen.hip_backend import build_module
    from mlc.ir.capture import capture
    from mlc.runtime import native

    kind, seed, cname = case
    cfg = _configs()[cname]
    try:
        model, args, _ = _build(kind, seed, cname)
        mod = build_module(build_pipeline(capture(model, args), cfg), cfg)
        if hip and mod.functions:
            native.compile_code_object(mod.source)
    except Exception as exc:  # noqa: BLE001 - the sweep reports every failure
        return case, f"{type(exc).__name__}: {exc}"
    return case, None


def _pool(jobs) -> int:
    from concurrent.futures import ProcessPoolExecutor

    bad = 0
    with ProcessPoolExecutor(WORKERS) as ex:
        for case, err in ex.map(_lower_one, jobs):
            if err is not None:
                bad += 1
                print("FAIL", case, err, flush=True)
    return bad


def lower(start: int, count: int) -> int:
    names = ("default", "streamed", "layout", "no_fusion",
             "wide", "wide_streamed", "wide_layout", "wide_no_fusion")
    jobs = [(("program", s, c), False) for s in range(start, start + count) for c in names]
    bad = _pool(jobs)
    print(f"done: {len(jobs)} modules, {bad} failing", flush=True)
    return bad


def compile_all(start: int, count: int) -> int:
    jobs = [(case, True) for case in gpu_cases(start, count)]
    bad = _pool(jobs)
    print(f"done: {len(jobs)} modules compiled, {bad} failing", flush=True)
    return bad


def gpu(start: int, count: int) -> int:
    import torch

    import fuzz_programs as fp
    import mlc
    from oracle import compile_reference

    bars = {torch.float32: 1e-5, torch.float16: 2e-3, torch.bfloat16: 2.5e-2}
    configs = _configs()
    bad, t0, n = 0, time.time(), 0
    for kind, seed, cname in gpu_cases(start, count):
        n += 1
        cfg = configs[cname]
        model, args, desc = _build(kind, seed, cname)
        print(f"... {kind} seed {seed} {cname}", flush=True)
        want = compile_reference(model, args, cfg)(*args)
        want = want if isinstance(want, (list, tuple)) else (want,)
        dev = tuple(a.cuda() for a in args)
        if isinstance(model, torch.nn.Module):
            model = model.cuda()
        got = mlc.compile(model, dev, cfg)(*dev)
        got = got if isinstance(got, (list, tuple)) else (got,)
        torch.cuda.synchronize()
        worst, ok = 0.0, True
        chains = model.chains if kind == "program" else [None] * len(want)
        for c, g, w in zip(chains, got, want):
            e = fp.max_rel_error(g.cpu(), w)
            worst = max(worst, e)
            bar = fp.tolerance(c) if c is not None else bars[w.dtype]
            ok &= g.shape == w.shape and g.dtype == w.dtype and e <= bar
        bad += not ok
        print(f"{'OK ' if ok else 'BAD'} {kind} seed {seed} {cname}: worst {worst:.2e} "
              f"{desc or ''} [{time.time() - t0:.0f}s]", flush=True)
    print(f"done: {n} cases, {bad} failing", flush=True)
    return bad


def attention(start: int, count: int) -> int:
    """The fused-attention variant on random problems (fp16 every seed, bf16
    even seeds) against the oracle's fused kernel: 2e-3 (fp16), 1e-2 (bf16)."""
    import torch

    import fuzz_programs as fp
    import mlc
    from mlc.config import Config
    from oracle import compile_reference

    cfg = Config(fused_attention=True, cuda_graphs=False)
    bars = {torch.float16: 2e-3, torch.bfloat16: 1e-2}
    bad, n, t0 = 0, 0, time.time()
    for seed in range(start, start + count):
        for dt in (torch.float16, torch.bfloat16) if seed % 2 == 0 else (torch.float16,):
            n += 1
            model, args, desc = fp.attention_case(seed, dt)
            print(f"... {seed} {desc}", flush=True)
            want = compile_reference(model, args, cfg)(*args)
            dev = tuple(a.cuda() for a in args)
            compiled = mlc.compile(model, dev, cfg)
            kinds = [spec.meta["kind"] for spec in compiled._module.launch_table.values()]
            got = compiled(*dev)
            torch.cuda.synchronize()
            err = fp.max_rel_error(got.cpu(), want)
            ok = (kinds.count("attention") == 1 and bool(torch.isfinite(got).all())
                  and err <= bars[dt])
            bad += not ok
            print(f"{'OK ' if ok else 'BAD'} {seed} {desc}: err {err:.2e} "
                  f"[{time.time() - t0:.0f}s]", flush=True)
    print(f"done: {n} cases, {bad} failing", flush=True)
    return bad


def main() -> int:
    mode, start, count = sys.argv[1], int(sys.argv[2]), int(sys.argv[3])
    run = {"lower": lower, "compile": compile_all, "gpu": gpu, "attention": attention}[mode]
    run(start, count)
    return 0


if __name__ == "__main__":
    sys.exit(main())
