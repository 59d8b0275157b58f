"""The compiled model: a fixed buffer table, a resolved launch plan, a graph.

Calling a :class:`CompiledModel` copies the inputs into fixed device
buffers and replays one captured hipGraph of the whole schedule (generated
kernels through ``libmlc_hip.so``, library calls through torch), then hands
back views of the output buffers.

Memory (``_Buffers``):

* params are uploaded once and stay resident, each a flat 1-D tensor;
* planned intermediates are slices of the arena -- one ``hipMalloc`` slab, or
  the library's static array -- at the planner's offsets, so every pointer a
  kernel sees is the same on every call (what makes capture valid);
* inputs are copied into buffers of their own each call, never aliased;
* outputs alias storage the next call overwrites (clone to keep one).

With ``memory_planning`` off the plan is "eager": intermediates are allocated
just before the kernel that writes them and dropped after their last reader,
and nothing is captured.

Library calls (``ExternCall``) are resolved once against the buffer table:
when the op has an ``.out`` overload taking exactly its arguments plus
``out`` (read off the schemas, never by calling it) the result is written
straight into its buffer; otherwise the op is called and its result copied.
The HIP runtime may claim an op with a native kernel instead (``NativeCall``:
the bounds-checked embedding gather).

Behaviour kept from the reference runtime (``mlc/runtime/executor.py:41-474``):
the input checks and their messages, output aliasing, the eager mode, three
warm-up runs before capture, per-kernel profiling. The runner of generated
kernels is pluggable so the tests can execute the same plan with the CPU
oracle; the product only ever selects the HIP runtime and raises without a
GPU.
"""

from __future__ import annotations

from dataclasses import dataclass
from typing import Any, Sequence

import torch

from ..config import Config
from ..ir.graph import Graph, Value
from ..kernels import ExternKernel, Schedule


class ExecutionError(Exception):
    pass


def select_backend(cfg: Config, device: torch.device) -> str:
    """``"hip"``, for a ROCm GPU device (torch names it ``cuda``)."""
    if cfg.backend not in ("auto", "hip"):
        raise ExecutionError(f"backend {cfg.backend!r} is not built here; this build runs 'hip'")
    if device.type != "cuda":
        raise ExecutionError(
            f"the HIP backend runs on a ROCm GPU (torch device 'cuda'), not on {device}; "
            "running the kernel IR on the CPU is the test oracle's job, not the product's")
    return "hip"


# --------------------------------------------------------------------------
# library calls
# --------------------------------------------------------------------------

def _materialise(a, buffers: dict[str, torch.Tensor]):
    """Graph values inside an argument structure -> tensor views."""
    if isinstance(a, Value):
        return a.layout.as_torch(buffers[a.buffer.name])
    if isinstance(a, (list, tuple)):
        return type(a)(_materialise(x, buffers) for x in a)
    return a


def out_variant(node):
    """The op's ``.out`` overload when its schema is the default overload's
    arguments followed by ``out`` (cached in ``node.meta``), else None."""
    if "out_variant" not in node.meta:
        node.meta["out_variant"] = _find_out_overload(node)
    return node.meta["out_variant"]


def _find_out_overload(node):
    target = node.meta.get("target")
    if not node.op.startswith("aten.") or len(node.outputs) != 1 or not hasattr(target, "_schema"):
        return None
    packet = getattr(torch.ops.aten, node.op.split(".")[1], None)
    candidate = getattr(packet, "out", None)
    try:
        default_args = [a.name for a in target._schema.arguments]
        out_args = [a.name for a in candidate._schema.arguments]
    except AttributeError:
        return None
    return candidate if out_args == default_args + ["out"] else None


@dataclass
class ExternCall:
    """A torch op bound to the buffer table: run() writes its buffers."""

    target: Any
    overload: Any  # the .out overload, or None
    args: list
    kwargs: dict
    dest: torch.Tensor | None
    outs: list[torch.Tensor]

    def run(self) -> None:
        if self.overload is not None:
            self.overload(*self.args, **self.kwargs, out=self.dest)
            return
        result = self.target(*self.args, **self.kwargs)
        for buf, r in zip(self.outs, result if isinstance(result, (list, tuple)) else [result]):
            buf.copy_(r.contiguous().reshape(-1))

    def functional(self) -> "ExternCall":
        return ExternCall(self.target, None, self.args, self.kwargs, None, self.outs)


@dataclass
class NativeCall:
    """A library op the runtime implements with a kernel of its own."""

    module: Any
    bound: Any

    def run(self) -> None:
        self.module.run_bound(self.bound)


def bind_extern(k: ExternKernel, buffers: dict[str, torch.Tensor], module=None):
    """Resolve a library call against the buffer table without running it."""
    claim = getattr(module, "bind_native_extern", None)
    bound = claim(k, buffers) if claim is not None else None
    if bound is not None:
        return NativeCall(module, bound)
    node = k.node
    target = node.meta.get("target")
    if target is None:
        raise ExecutionError(f"{node.op}: no torch op to dispatch to")
    overload = out_variant(node)
    dest = None
    if overload is not None:
        out = node.outputs[0]
        dest = out.layout.as_torch(buffers[out.buffer.name])
    return ExternCall(target, overload, [_materialise(a, buffers) for a in node.args],
                      {n: _materialise(v, buffers) for n, v in node.kwargs.items()}, dest,
                      [buffers[o.buffer.name] for o in node.outputs])


def run_bound_extern(call) -> None:
    call.run()


def run_extern(k: ExternKernel, buffers: dict[str, torch.Tensor], module=None) -> None:
    """Bind and run one library call (the unplanned path). An ``.out``
    overload that rejects this call is dropped for the node, which then runs
    functionally and is copied into its buffer."""
    call = bind_extern(k, buffers, module)
    if isinstance(call, ExternCall) and call.overload is not None:
        try:
            call.run()
            return
        except (RuntimeError, TypeError):
            k.node.meta["out_variant"] = None
            call = call.functional()
    call.run()


# --------------------------------------------------------------------------
# buffers
# --------------------------------------------------------------------------

class _Buffers:
    """The model's device memory: resident params, fixed inputs, the arena."""

    def __init__(self, model: "CompiledModel") -> None:
        self.model = model
        graph, schedule = model.graph, model.schedule
        self.live = {v.buffer.name for v in (*graph.inputs, *graph.outputs)}
        for k in schedule.kernels:
            self.live.update(v.buffer.name for v in (*k.reads(), *k.writes()))
        self.params = {v.buffer.name: graph.param_tensors[v.name].to(model.device).contiguous()
                       .reshape(-1) for v in graph.params}
        self.arena: torch.Tensor | None = None
        self.table: dict[str, torch.Tensor] | None = None
        self.inputs: list[torch.Tensor] = []

    def empty(self, b) -> torch.Tensor:
        return torch.empty(b.numel, dtype=b.dtype, device=self.model.device)

    def _base(self) -> dict[str, torch.Tensor]:
        """Resident params and every live buffer outside the arena's reach."""
        table = {n: t for n, t in self.params.items() if n in self.live}
        for b in self.model.graph.buffers():
            if b.name not in table and not b.plannable and b.name in self.live:
                table[b.name] = self.empty(b)
        return table

    def per_call(self, inputs: Sequence[torch.Tensor]) -> dict[str, torch.Tensor]:
        """Eager mode: the caller's inputs used in place, intermediates come
        and go with the alloc/free plan."""
        table = self._base()
        for v, t in zip(self.model.graph.inputs, inputs):
            table[v.buffer.name] = t.to(self.model.device).contiguous().reshape(-1)
        return table

    def resident(self, inputs: Sequence[torch.Tensor]) -> dict[str, torch.Tensor]:
        """The fixed table (built on first use) with this call's inputs
        copied in."""
        model = self.model
        if self.table is None:
            table = self._base()
            for v in model.graph.inputs:
                table[v.buffer.name] = torch.empty(v.buffer.numel, dtype=v.dtype,
                                                   device=model.device)
            for k in model.schedule.kernels:
                if k.name in model._constants:
                    for v in k.writes():
                        table.setdefault(v.buffer.name, self.empty(v.buffer))
            self._place_in_arena(table)
            self.table = table
            self.inputs = [table[v.buffer.name] for v in model.graph.inputs]
        for dst, src in zip(self.inputs, inputs):
            dst.copy_(src.reshape(-1), non_blocking=True)
        return self.table

    def _place_in_arena(self, table: dict[str, torch.Tensor]) -> None:
        plan = self.model.schedule.plan
        offsets = plan.offsets if plan is not None else {}
        arena = self.get_arena()
        for b in self.model.graph.buffers():
            if b.name in table or b.name not in self.live:
                continue
            at = offsets.get(b.name)
            table[b.name] = self.empty(b) if at is None else arena[at:at + b.nbytes].view(b.dtype)

    def get_arena(self) -> torch.Tensor:
        need = max(self.model.schedule.arena_bytes, 1)
        if self.arena is None or self.arena.numel() < need:
            make = getattr(self.model._module, "arena", None)
            self.arena = make(need) if make is not None else torch.empty(
                need, dtype=torch.uint8, device=self.model.device)
        return self.arena


# --------------------------------------------------------------------------
# the model
# --------------------------------------------------------------------------

def _alloc_count(device) -> int:
    return int(torch.cuda.memory_stats(device).get("allocation.all.allocated", 0))


class CompiledModel:
    """A compiled graph, called like the module it came from."""

    def __init__(self, graph: Graph, schedule: Schedule, cfg: Config, device: torch.device,
                 runner: Any = None) -> None:
        self.graph, self.schedule, self.cfg = graph, schedule, cfg
        self.device = torch.device(device)
        if runner is None:
            self.backend = select_backend(cfg, self.device)
            from .hip_runtime import HipRuntime

            self._module = HipRuntime(schedule, cfg, self.device)
        else:
            self.backend, self._module = getattr(runner, "name", "custom"), runner
        # library calls reading no tensor always give the same result: they run
        # once, into memory of their own, when the plan is resolved (one with
        # no out= form would otherwise allocate inside the captured graph)
        self._constants = {k.name for k in schedule.kernels
                           if isinstance(k, ExternKernel) and not k.reads()}
        self._buffers = _Buffers(self)
        self._plan: list | None = None
        self._runs: list | None = None
        self._captured = False
        self._capture_stream = None
        self._static_outputs: Any = None

    # state the tests and the bench inspect
    params = property(lambda self: self._buffers.params)
    _arena = property(lambda self: self._buffers.arena)
    _resident = property(lambda self: self._buffers.table)

    # -- inputs and outputs ---------------------------------------------------
    def _check_inputs(self, inputs: Sequence[torch.Tensor]) -> None:
        expected = self.graph.inputs
        if len(inputs) != len(expected):
            raise ExecutionError(f"expected {len(expected)} inputs, got {len(inputs)}")
        for v, t in zip(expected, inputs):
            if tuple(t.shape) != v.shape:
                raise ExecutionError(
                    f"input {v.name}: compiled for {v.shape}, called with {tuple(t.shape)}")

    def _collect(self, table: dict[str, torch.Tensor]):
        """Views of the outputs (aliasing storage the next call overwrites),
        in the structure the module returned them."""
        outs = [v.layout.as_torch(table[v.buffer.name]) for v in self.graph.outputs]
        spec = self.graph.meta.get("out_spec")
        if spec is not None:
            from torch.utils._pytree import tree_unflatten

            try:
                return tree_unflatten(outs, spec)
            except Exception:
                pass
        return outs[0] if len(outs) == 1 else tuple(outs)

    # -- the plan ---------------------------------------------------------------
    def _resolve(self, table: dict[str, torch.Tensor]) -> None:
        """Bind every kernel once: ``[(kind, payload)]`` in schedule order,
        with kind "const" (already run), "extern" or "kernel"."""
        if self._plan is not None:
            return
        plan = []
        for k in self.schedule.kernels:
            if k.name in self._constants:
                call = bind_extern(k, table, self._module)
                call.run()
                plan.append(("const", call))
            elif isinstance(k, ExternKernel):
                plan.append(("extern", bind_extern(k, table, self._module)))
            else:
                plan.append(("kernel", self._module.bind(k, table)))
        self._plan = plan
        group = getattr(self._module, "compile_runs", None)
        self._runs = group(plan) if group is not None else plan

    def run_one(self, k, table: dict[str, torch.Tensor]) -> None:
        if isinstance(k, ExternKernel):
            run_extern(k, table, self._module)
        else:
            self._module.launch(k, table)

    def run_kernels(self, table: dict[str, torch.Tensor]) -> None:
        """One pass of the schedule over ``table`` (through the resolved plan
        when ``table`` is the resident one)."""
        if self._plan is not None and table is self._buffers.table:
            for kind, payload in self._runs:
                if kind == "extern":
                    payload.run()
                elif kind == "kernel":
                    self._module.run_bound(payload)
        else:
            for k in self.schedule.kernels:
                self.run_one(k, table)
        fetch = getattr(self._module, "fetch_errors", None)
        if fetch is not None:
            fetch()

    def forward(self, *inputs: torch.Tensor):
        """One uncaptured run."""
        self._check_inputs(inputs)
        plan = self.schedule.plan
        if plan is not None and plan.mode == "eager":
            table = self._buffers.per_call(inputs)
            for i, k in enumerate(self.schedule.kernels):
                for b in plan.alloc_at.get(i, ()):
                    if b.name in self._buffers.live:
                        table[b.name] = self._buffers.empty(b)
                self.run_one(k, table)
                for name in plan.free_at.get(i, ()):
                    table.pop(name, None)
            fetch = getattr(self._module, "fetch_errors", None)
            if fetch is not None:
                fetch()
            return self._collect(table)
        table = self._buffers.resident(inputs)
        self._resolve(table)
        self.run_kernels(table)
        return self._collect(table)

    def __call__(self, *inputs: torch.Tensor):
        self._raise_pending()
        if not (self.cfg.cuda_graphs and self.device.type == "cuda"):
            out = self.forward(*inputs)
        else:
            if not self._captured:
                self._capture(inputs)
            self._check_inputs(inputs)
            for dst, src in zip(self._buffers.inputs, inputs):
                dst.copy_(src.reshape(-1), non_blocking=True)
            self._module.replay(torch.cuda.current_stream(self.device).cuda_stream)
            out = self._static_outputs
        if self.cfg.sync_input_checks:
            self.check_errors()
        return out

    # -- capture ----------------------------------------------------------------
    def _capture(self, inputs) -> None:
        """Three warm-up runs on a side stream (modules loaded, library
        workspaces allocated), then one run captured into the context's
        hipGraph. Capture must allocate nothing: every library call writes a
        pre-bound slice, and an allocation is reported with its culprits."""
        self._check_inputs(inputs)
        table = self._buffers.resident(inputs)
        self._resolve(table)
        side = torch.cuda.Stream(self.device)
        side.wait_stream(torch.cuda.current_stream(self.device))
        with torch.cuda.stream(side):
            for _ in range(3):
                self.run_kernels(table)
            side.synchronize()
            before = _alloc_count(self.device)
            self._module.capture_begin(side.cuda_stream)
            try:
                self.run_kernels(table)
            finally:
                self._module.capture_end()
            grew = _alloc_count(self.device) - before
        torch.cuda.current_stream(self.device).wait_stream(side)
        if grew:
            raise ExecutionError(f"{grew} device allocation(s) during graph capture would leave "
                                 "the graph pointing at memory it does not own; allocating "
                                 f"plan entries: {self._allocating_entries(side)}")
        self._capture_stream = side
        self._captured = True
        self._static_outputs = self._collect(table)

    def _allocating_entries(self, stream) -> list[str]:
        culprits = []
        with torch.cuda.stream(stream):
            for kernel, (kind, payload) in zip(self.schedule.kernels, self._plan):
                before = _alloc_count(self.device)
                if kind == "extern":
                    payload.run()
                elif kind == "kernel":
                    self._module.run_bound(payload)
                if _alloc_count(self.device) != before:
                    culprits.append(kernel.summary())
        stream.synchronize()
        return culprits

    # -- invalid inputs -------------------------------------------------------
    def _raise_pending(self) -> None:
        """Raise for an invalid input (an embedding id outside its table) that
        an earlier, completed call met. The native gather cannot raise where
        torch's ``aten.embedding`` would, so it flags the id in a device word
        that every run copies back asynchronously; the flag is cleared before
        raising, so the call after the exception runs normally."""
        poll = getattr(self._module, "pending_error", None)
        msg = poll() if poll is not None else None
        if msg is not None:
            self._module.clear_errors()
            raise ExecutionError(msg)

    def check_errors(self) -> None:
        """Wait for every call so far to finish and raise
        :class:`ExecutionError` if one of them met an invalid input."""
        fetch = getattr(self._module, "fetch_errors", None)
        if fetch is None:
            return
        fetch()
        if self.device.type == "cuda":
            torch.cuda.synchronize(self.device)
        self._raise_pending()

    # -- profiling and introspection --------------------------------------------
    def profile_kernels(self, inputs, iters: int = 20) -> list[tuple]:
        """``(name, summary, ms)`` per kernel in schedule order, each timed in
        place on the launch stream: generated kernels by the runtime's
        hipEvents, library calls by torch events."""
        if self.device.type != "cuda":
            raise ExecutionError("profiling kernels needs the GPU")
        table = self._buffers.resident(inputs)
        self._resolve(table)
        for _ in range(3):
            self.run_kernels(table)
        torch.cuda.synchronize(self.device)
        stream = torch.cuda.current_stream(self.device)
        rows = []
        for kernel, (kind, payload) in zip(self.schedule.kernels, self._plan):
            if kind == "kernel":
                ms = self._module.time_bound(payload, iters, stream.cuda_stream)
            else:
                for _ in range(3):
                    payload.run()
                start, end = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
                start.record(stream)
                for _ in range(iters):
                    payload.run()
                end.record(stream)
                end.synchronize()
                ms = start.elapsed_time(end) / iters
            rows.append((kernel.name, kernel.summary(), ms))
        return rows

    def source(self) -> str:
        """The generated module text (``mlc/runtime/executor.py:354-358``)."""
        return self._module.source

    def source_path(self):
        return getattr(self._module, "path", None)

    def __repr__(self) -> str:  # pragma: no cover - debug aid
        return (f"CompiledModel({self.graph.name}, {len(self.schedule)} kernels, "
                f"backend={self.backend}, device={self.device})")
