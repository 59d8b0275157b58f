"""Launches for counter-measured HBM traffic (run under ``rocprofv3 --pmc``).

    rocprofv3 --pmc FETCH_SIZE --output-format csv -d OUT -o fetch -- \\
        python mlc-compiler_amd/mlc/bench/traffic.py
    rocprofv3 --pmc WRITE_SIZE ... (same)

It launches, ``--iters`` times each (with ``--kernel all``, each kernel after
the plan is replayed up to it, so on its real inputs):

1. a plain device copy of ``--copy-mib`` MiB (torch ``copy_``), whose true
   traffic is known (that many bytes read and written): the counters' scale
   factor is what they read for it divided by the true bytes;
2. with ``--kernel gelu`` (the default), the dominant fused kernel of
   BERT-base fp16 b32 (config 4) -- the generated function with the most
   device time per forward, fc1 bias + GELU -- on the buffers of a compiled
   model, after one full forward; with ``--kernel attention``, the fused
   attention kernel of the same model compiled with every schedule variant
   on (``merge_parallel_gemms``, ``gemm_epilogue``, ``layout_selection``,
   ``fused_attention``); with ``--kernel all``, every generated kernel of
   the reference schedule at config 4 (for per-kernel counters such as
   ``SQ_INSTS_VALU``), or of the schedule with every variant on with
   ``--config every``. ``--workload`` picks another configuration (default
   config 4).

It prints each kernel's symbol and algorithmic bytes per launch so the
counter CSV can be matched to them.
"""

from __future__ import annotations

import argparse
import pathlib
import sys

ROOT = pathlib.Path(__file__).resolve().parents[3]
for _p in (ROOT / "mlc-compiler_amd", ROOT):
    if str(_p) not in sys.path:
        sys.path.insert(0, str(_p))


def main() -> int:
    ap = argparse.ArgumentParser()
    ap.add_argument("--iters", type=int, default=5)
    ap.add_argument("--copy-mib", type=int, default=1024)
    ap.add_argument("--kernel", choices=("gelu", "attention", "all"), default="gelu")
    ap.add_argument("--workload", default="C4", help="workload key (default C4)")
    ap.add_argument("--config", choices=("reference", "every"), default="reference",
                    help="schedule for --kernel all: the reference's, or every variant on")
    opts = ap.parse_args()

    import torch

    import mlc
    from mlc.bench.roofline import algorithmic_bytes
    from mlc.bench.workloads import make
    from mlc.config import Config
    from mlc.kernels import AttentionKernel, PointwiseKernel
    from mlc.runtime.executor import run_bound_extern

    torch.cuda.set_device(0)
    n = opts.copy_mib * (1 << 20) // 2
    src = torch.randn(n, device="cuda", dtype=torch.float32).half()
    dst = torch.empty_like(src)
    torch.cuda.synchronize()
    for _ in range(opts.iters):
        dst.copy_(src)
    torch.cuda.synchronize()
    print(f"copy: {2 * n} bytes read + {2 * n} bytes written per launch", flush=True)

    model, inputs = make(opts.workload, "cuda")
    if opts.kernel == "gelu":
        cfg = Config(cuda_graphs=False)

        def wanted(k):
            return (isinstance(k, PointwiseKernel)
                    and any(nd.op == "aten.erf.default" for nd in k.nodes))
    elif opts.kernel == "attention":
        cfg = Config(cuda_graphs=False, merge_parallel_gemms=True, gemm_epilogue=True,
                     layout_selection=True, fused_attention=True)

        def wanted(k):
            return isinstance(k, AttentionKernel)
    else:
        cfg = Config(cuda_graphs=False)
        if opts.config == "every":
            cfg = Config(cuda_graphs=False, merge_parallel_gemms=True, gemm_epilogue=True,
                         layout_selection=True, fused_attention=True)

        def wanted(k):
            return True
    compiled = mlc.compile(model, inputs, cfg)
    compiled(*inputs)
    torch.cuda.synchronize()
    rt = compiled._module
    plan = compiled._plan
    found = [(i, k, p) for i, (k, (kind, p)) in enumerate(zip(compiled.schedule.kernels, plan))
             if kind == "kernel" and wanted(k)]
    if opts.kernel != "all":
        found = found[-1:]
    replayed = 0
    for i, k, bound in found:
        if opts.kernel == "all":
            # the plan up to this kernel first, so it runs on its real inputs
            # (the arena's slots are reused; erf's work depends on its data)
            for kind_j, payload_j in plan[replayed:i]:
                if kind_j == "extern":
                    run_bound_extern(payload_j)
                elif kind_j == "kernel":
                    rt.run_bound(payload_j)
            replayed = i
        for _ in range(opts.iters):
            rt.run_bound(bound)
        torch.cuda.synchronize()
        print(f"{opts.kernel}: {rt.launch_table[k.name].symbol} {k.summary()} "
              f"algorithmic_bytes={algorithmic_bytes(k)}", flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
