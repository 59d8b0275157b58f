"""Write the reference compiler's behaviour on front-end edge cases to a
fixture (run in the build container only; the GPU box never has the
reference).

Each case is a small program at the edge of the reduction-fusion frame rules:
a row output that reads a row-constant operand, a reshape of the row shape,
shapes that right-align onto the element shape (among them a LayerNorm whose
batch is 1 and whose rows are as long as the sequence), a permutation that
passes the reshape test, a [1, 1] scalar added before a transpose makes its
row shape a reshape, an operand broadcast against a keepdim row value whose
size-1 dim a view moved, and zero-element inputs (no rows, or rows of no
columns). Per case the fixture records what the reference does:
the exception it raises (type and message), or its schedule (kernel
summaries, operand buffers and index strings) and whether its torch backend's
outputs agree with eager PyTorch (or the error its torch backend raises). Nothing else pins the front end there: the
reference's own tests do not reach these shapes.

Usage (from the repository root)::

    python tests/golden/dump_edge_cases.py /root/reference tests/golden/reference_edge_cases.json
"""

from __future__ import annotations

import json
import sys


def cases():
    """(name, module, inputs): the programs; shared with the tests that read
    the fixture."""
    import torch
    import torch.nn.functional as F

    class RowOutputReadsOperand(torch.nn.Module):
        def forward(self, x, y):
            return torch.clamp(x.sum(dim=0, keepdim=True) + y, -0.5, 0.7)

    class ReshapedRowOperand(torch.nn.Module):
        def forward(self, x, y):
            return torch.minimum(F.silu(x), y).transpose(0, 1).mean(dim=1)

    class RightAlignedRowResult(torch.nn.Module):
        def forward(self, x, y):
            return torch.rsqrt(torch.minimum(x.amax(dim=1), y).float())

    class PermutedElementProducer(torch.nn.Module):
        def forward(self, x):
            t = torch.cos(x).transpose(2, 0)
            return F.layer_norm(t, (t.shape[-1],))

    class PermutedRowValue(torch.nn.Module):
        def forward(self, x, y):
            return torch.sqrt((x.mean(dim=3, keepdim=True) + y).permute(1, 2, 3, 0).abs())

    class LayerNormRowMatchesTrailing(torch.nn.Module):
        def forward(self, x):
            return F.layer_norm(x, (x.shape[-1],))

    class ScalarOperandTransposedRow(torch.nn.Module):
        def forward(self, x, y):
            return (torch.relu(x) + y).transpose(0, 1).sum(dim=1, keepdim=True)

    class MovedKeepdimRow(torch.nn.Module):
        def forward(self, x, y):
            return torch.reciprocal(x.sum(dim=2, keepdim=True).transpose(2, 1).abs() + 1.0) - y

    class AffineRelu(torch.nn.Module):
        def forward(self, x):
            return torch.relu(x * 2.0 + 1.0)

    class Softmax(torch.nn.Module):
        def forward(self, x):
            return torch.softmax(x, dim=-1)

    class RowSum(torch.nn.Module):
        def forward(self, x):
            return x.sum(dim=-1)

    g = torch.Generator().manual_seed(0)

    def rn(*s, dt=torch.float32):
        return torch.randn(*s, generator=g).to(dt)

    return [
        ("row_output_reads_operand", RowOutputReadsOperand(), (rn(128), rn(1))),
        ("reshaped_row_operand", ReshapedRowOperand(),
         (rn(1, 100, dt=torch.float16), rn(1, 100, dt=torch.float16))),
        ("right_aligned_row_result", RightAlignedRowResult(),
         (rn(3, 3, 9, 128, dt=torch.float16), rn(1, 1, 1, dt=torch.float16))),
        ("permuted_element_producer", PermutedElementProducer(), (rn(7, 24, 5, 16),)),
        ("permuted_row_value", PermutedRowValue(), (rn(16, 3, 64, 5), rn(3, 64, 1))),
        ("layer_norm_row_matches_trailing", LayerNormRowMatchesTrailing(), (rn(1, 128, 128),)),
        ("layer_norm_b2", LayerNormRowMatchesTrailing(), (rn(2, 128, 128),)),
        ("scalar_operand_transposed_row", ScalarOperandTransposedRow(), (rn(1, 100), rn(1, 1))),
        ("moved_keepdim_row", MovedKeepdimRow(), (rn(3, 50, 4), rn(3, 1, 1))),
        # zero-element inputs: no rows, or rows of no columns
        ("empty_rows_pointwise", AffineRelu(), (rn(0, 16),)),
        ("empty_rows_softmax", Softmax(), (rn(0, 16),)),
        ("empty_rows_sum", RowSum(), (rn(0, 16),)),
        ("empty_rows_layer_norm", LayerNormRowMatchesTrailing(), (rn(0, 16),)),
        ("empty_cols_sum", RowSum(), (rn(4, 0),)),
        ("empty_cols_softmax", Softmax(), (rn(4, 0),)),
    ]


def main(ref_root: str, out_path: str) -> None:
    sys.path.insert(0, ref_root)
    import torch

    import mlc
    from mlc.api import build_pipeline
    from mlc.config import Config
    from mlc.ir.capture import capture

    result = {"torch": torch.__version__, "cases": {}}
    cfg = Config(cuda_graphs=False)
    for name, model, args in cases():
        rec = {}
        try:
            sched = build_pipeline(capture(model, args), cfg)
        except Exception as e:  # the reference's own error is the fixture
            rec["error"] = [type(e).__name__, str(e)]
            result["cases"][name] = rec
            print(name, "raises", type(e).__name__, flush=True)
            continue
        rec["kernels"] = [
            {"summary": k.summary(),
             "inputs": [[a.value.buffer.name, a.index.render()] for a in getattr(k, "inputs", [])
                        if hasattr(a, "index")],
             "outputs": [[a.value.buffer.name, a.index.render()] for a in getattr(k, "outputs", [])
                         if hasattr(a, "index")]}
            for k in sched.kernels]
        torch.manual_seed(0)
        try:
            got = mlc.compile(model, args, cfg)(*args)
        except Exception as e:  # its torch backend's own failure
            rec["run_error"] = [type(e).__name__, str(e)]
            result["cases"][name] = rec
            print(name, "compiles; its torch backend raises", type(e).__name__, flush=True)
            continue
        with torch.no_grad():
            want = model(*args)
        rec["finite"] = bool(torch.isfinite(got.float()).all())
        rec["matches_eager"] = bool(torch.allclose(got.float(), want.float(), rtol=1e-2, atol=1e-2))
        result["cases"][name] = rec
        print(name, "compiles; finite", rec["finite"], "matches eager", rec["matches_eager"],
              flush=True)

    with open(out_path, "w") as f:
        json.dump(result, f, indent=1, sort_keys=True)


if __name__ == "__main__":
    main(sys.argv[1], sys.argv[2])
