"""Launches for counter-measured HBM traffic (run under ``rocprofv3 --pmc``).

    rocprofv3 --pmc FETCH_SIZE --output-format csv -d OUT -o fetch -- \\
        python mlc-compiler_amd/mlc/bench/traffic.py
    rocprofv3 --pmc WRITE_SIZE ... (same)

It launches, ``--iters`` times each:

1. a plain device copy of ``--copy-mib`` MiB (torch ``copy_``), whose true
   traffic is known (that many bytes read and written): the counters' scale
   factor is what they read for it divided by the true bytes;
2. the dominant fused kernel of BERT-base fp16 b32 (config 4) -- the
   generated function with the most device time per forward, fc1 bias +
   GELU -- on the buffers of a compiled model, after one full forward.

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
    opts = ap.parse_args()

    import torch

    import mlc
    from mlc.bench.roofline import algorithmic_bytes
    from mlc.bench.workloads import make
    from mlc.config import Config
    from mlc.kernels import PointwiseKernel

    torch.cuda.set_device(0)
    n = opts.copy_mib * (1 << 20) // 2
    src = torch.randn(n, device="cuda", dtype=torch.float32).half()
    dst = torch.empty_like(src)
    torch.cuda.synchronize()
    for _ in range(opts.iters):
        dst.copy_(src)
    torch.cuda.synchronize()
    print(f"copy: {2 * n} bytes read + {2 * n} bytes written per launch", flush=True)

    model, inputs = make("C4", "cuda")
    compiled = mlc.compile(model, inputs, Config(cuda_graphs=False))
    compiled(*inputs)
    torch.cuda.synchronize()
    rt = compiled._module
    gelu = [(k, p) for k, (kind, p) in zip(compiled.schedule.kernels, compiled._plan)
            if kind == "kernel" and isinstance(k, PointwiseKernel)
            and any(nd.op == "aten.erf.default" for nd in k.nodes)]
    k, bound = gelu[-1]
    for _ in range(opts.iters):
        rt.run_bound(bound)
    torch.cuda.synchronize()
    print(f"dominant: {rt.launch_table[k.name].symbol} {k.summary()} "
          f"algorithmic_bytes={algorithmic_bytes(k)}", flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
