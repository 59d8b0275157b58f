"""Compiler configuration: every pass flag, the cost-model constants and the
backend selector.

Reference behaviour followed: ``mlc/config.py:14-80``. Defaults are identical,
so the same model compiles to the same schedule and arena. ``backend`` takes
``"hip"`` (the MI355X backend) in place of the reference's ``"triton"``;
``"auto"`` selects it for a GPU device.
"""

from __future__ import annotations

from dataclasses import dataclass, replace as _dc_replace


@dataclass
class Config:
    # passes
    elementwise_fusion: bool = True
    recompute: bool = True
    reduction_fusion: bool = True
    memory_planning: bool = True
    #: replay the schedule as one captured hipGraph
    cuda_graphs: bool = True
    #: fold a bias add that would be a kernel of its own back into the GEMM
    #: before it (addmm: hipBLASLt's bias epilogue). A schedule change, so it
    #: is off by default, where the schedule is the reference's.
    gemm_epilogue: bool = False
    #: merge a pointwise producer into the copy that re-lays its output out
    #: (q/k/v written straight in the bmm layout). A schedule change, off by
    #: default.
    layout_selection: bool = False
    #: merge linear layers that read the same activation (BERT's q/k/v) into
    #: one GEMM over concatenated weights. A graph rewrite, off by default.
    merge_parallel_gemms: bool = False
    #: one MFMA kernel per batch-head for bmm -> softmax -> bmm (scores and
    #: probabilities never stored). A schedule change, off by default.
    fused_attention: bool = False

    #: bind the arena to the runtime library's static device array
    #: (``mlc_slab_static``: no hipMalloc, at most 64 MiB, shared by every
    #: model on the GPU that sets it, so their calls must not overlap)
    #: instead of a slab of its own. Changes no schedule.
    static_arena: bool = False
    #: wait for every call to finish and raise ``ExecutionError`` in that
    #: same call when it met an invalid input (an embedding id outside its
    #: table). Costs one stream synchronize per call. Off: the error is
    #: raised by the next call or by ``check_errors()``. Changes no schedule.
    sync_input_checks: bool = False

    # codegen
    pointwise_block: int = 1024
    #: longest row a persistent reduction holds; longer rows are streamed
    max_persistent_row: int = 16384
    #: declared for interface parity; reductions always accumulate in fp32
    fp32_accumulate: bool = True

    # cost model (bytes of HBM traffic are the currency)
    flops_per_byte: float = 20.0
    launch_overhead_bytes: float = 4.5e6
    graph_launch_overhead_bytes: float = 1.1e6
    max_recompute_ops: int = 32

    # misc
    backend: str = "auto"  # "auto" | "hip"
    debug: bool = False

    @property
    def effective_launch_bytes(self) -> float:
        """What one saved launch is worth given whether launches are replayed."""
        if self.cuda_graphs:
            return self.graph_launch_overhead_bytes
        return self.launch_overhead_bytes

    def replace(self, **kw) -> "Config":
        return _dc_replace(self, **kw)


#: every pass off: the baseline per-pass attribution is measured against
NO_FUSION = Config(elementwise_fusion=False, recompute=False, reduction_fusion=False,
                   memory_planning=False, cuda_graphs=False)

#: elementwise fusion only
ELEMENTWISE_ONLY = Config(reduction_fusion=False)
