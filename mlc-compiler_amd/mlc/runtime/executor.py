"""Runtime: the buffer table, the pre-resolved launch plan and graph replay.

Every buffer is a flat 1-D tensor; shapes and strides live in the IR. Params
are resident, inputs are copied into fixed buffers, intermediates are slices
of the arena (one ``hipMalloc`` slab on the GPU), outputs alias storage the
next call overwrites. The plan is resolved once; on the GPU consecutive
generated kernels run as one native launch range and the whole schedule
(generated kernels and extern library calls) is captured into one hipGraph.

Reference behaviour followed: ``mlc/runtime/executor.py:28-474`` (buffer
liveness, resident table, arena binding, extern ``.out`` dispatch decided from
the schema, output aliasing, the eager alloc/free mode, 3 warm-up runs before
capture, per-kernel profiling). The generated-kernel runner is pluggable so
the test suite can execute the same plan with the CPU oracle; the product
itself only ever selects the HIP runner and fails loudly without one.
"""

from __future__ import annotations

from typing import Any, Sequence

import torch

from ..config import Config
from ..ir.graph import Graph, Value
from ..kernels import ExternKernel, Schedule


class ExecutionError(Exception):
    pass


def select_backend(cfg: Config, device: torch.device) -> str:
    if cfg.backend not in ("auto", "hip"):
        raise ExecutionError(f"unknown backend {cfg.backend!r}; this build provides 'hip'")
    if device.type != "cuda":
        raise ExecutionError(
            f"the HIP backend runs on a ROCm GPU (torch device 'cuda'); got {device}. "
            "CPU execution of the kernel IR is the parity oracle's job, not the product's")
    return "hip"


class CompiledModel:
    """A compiled graph, callable like the module it came from."""

    def __init__(self, graph: Graph, schedule: Schedule, cfg: Config, device: torch.device,
                 runner: Any = None) -> None:
        self.graph = graph
        self.schedule = schedule
        self.cfg = cfg
        self.device = torch.device(device)
        if runner is None:
            self.backend = select_backend(cfg, self.device)
            from .hip_runtime import HipRuntime

            self._module = HipRuntime(schedule, cfg, self.device)
        else:
            self.backend = getattr(runner, "name", "custom")
            self._module = runner

        self.params: dict[str, torch.Tensor] = {}
        for v in graph.params:
            t = graph.param_tensors[v.name]
            self.params[v.buffer.name] = t.to(self.device).contiguous().reshape(-1)

        self._arena: torch.Tensor | None = None
        self._live = self._live_buffers()
        # externs reading no tensor (``aten.scalar_tensor``, ``full``, ...):
        # their result never changes, so they run once when the plan is
        # built, into memory of their own, and are not replayed. One that
        # allocates (no ``out=`` form) would otherwise allocate inside the
        # captured graph.
        self._constants = {k.name for k in schedule.kernels
                           if isinstance(k, ExternKernel) and not k.reads()}
        self._resident: dict[str, torch.Tensor] | None = None
        self._plan: list | None = None
        self._runs: list | None = None
        self._static_inputs_flat: list[torch.Tensor] | None = None
        self._captured = False
        self._capture_stream = None
        self._static_inputs: list[torch.Tensor] | None = None
        self._static_outputs: Any = None

    # -- allocation -----------------------------------------------------------
    def _live_buffers(self) -> set[str]:
        live = {v.buffer.name for v in self.graph.inputs}
        live |= {v.buffer.name for v in self.graph.outputs}
        for k in self.schedule.kernels:
            live |= {v.buffer.name for v in k.reads()}
            live |= {v.buffer.name for v in k.writes()}
        return live

    def _check_inputs(self, inputs: Sequence[torch.Tensor]) -> None:
        if len(inputs) != len(self.graph.inputs):
            raise ExecutionError(f"expected {len(self.graph.inputs)} inputs, got {len(inputs)}")
        for v, t in zip(self.graph.inputs, inputs):
            if tuple(t.shape) != v.shape:
                raise ExecutionError(
                    f"input {v.name}: compiled for {v.shape}, called with {tuple(t.shape)}")

    def _empty(self, b) -> torch.Tensor:
        return torch.empty(b.numel, dtype=b.dtype, device=self.device)

    def _bind_resident(self, inputs: Sequence[torch.Tensor]) -> dict[str, torch.Tensor]:
        """Unplanned mode: params, this call's inputs and the non-plannable
        buffers (intermediates come and go per the alloc/free plan)."""
        self._check_inputs(inputs)
        buffers = {n: t for n, t in self.params.items() if n in self._live}
        for v, t in zip(self.graph.inputs, inputs):
            buffers[v.buffer.name] = t.to(self.device).contiguous().reshape(-1)
        for b in self.graph.buffers():
            if b.name in buffers or b.plannable or b.name not in self._live:
                continue
            buffers[b.name] = self._empty(b)
        return buffers

    def _get_arena(self) -> torch.Tensor:
        need = max(self.schedule.arena_bytes, 1)
        if self._arena is None or self._arena.numel() < need:
            make = getattr(self._module, "arena", None)
            if make is not None:
                self._arena = make(need)
            else:
                self._arena = torch.empty(need, dtype=torch.uint8, device=self.device)
        return self._arena

    def _bind_arena(self, buffers: dict[str, torch.Tensor]) -> None:
        plan = self.schedule.plan
        arena = self._get_arena()
        for b in self.graph.buffers():
            if b.name in buffers or b.name not in self._live:
                continue
            offset = plan.offsets.get(b.name) if plan is not None else None
            if offset is None:
                buffers[b.name] = self._empty(b)
            else:
                buffers[b.name] = arena[offset:offset + b.nbytes].view(b.dtype)

    def _resident_buffers(self, inputs: Sequence[torch.Tensor]) -> dict[str, torch.Tensor]:
        """The buffer table, built once; inputs are copied into fixed buffers
        so every pointer is stable for the life of the model."""
        self._check_inputs(inputs)
        if self._resident is None:
            buffers = {n: t for n, t in self.params.items() if n in self._live}
            for b in self.graph.buffers():
                if b.name in buffers or b.plannable or b.name not in self._live:
                    continue
                buffers[b.name] = self._empty(b)
            for v in self.graph.inputs:
                buffers[v.buffer.name] = torch.empty(v.buffer.numel, dtype=v.dtype,
                                                     device=self.device)
            for k in self.schedule.kernels:
                if k.name in self._constants:
                    for v in k.writes():
                        buffers.setdefault(v.buffer.name, self._empty(v.buffer))
            self._bind_arena(buffers)
            self._resident = buffers
            self._static_inputs_flat = [buffers[v.buffer.name] for v in self.graph.inputs]
        for dst, t in zip(self._static_inputs_flat, inputs):
            dst.copy_(t.reshape(-1), non_blocking=True)
        return self._resident

    # -- execution --------------------------------------------------------------
    def _build_plan(self, buffers: dict[str, torch.Tensor]) -> list:
        plan: list = []
        for k in self.schedule.kernels:
            if k.name in self._constants:
                bound = bind_extern(k, buffers, self._module)
                run_bound_extern(bound)
                plan.append(("const", bound))
            elif isinstance(k, ExternKernel):
                plan.append(("extern", bind_extern(k, buffers, self._module)))
            else:
                plan.append(("kernel", self._module.bind(k, buffers)))
        compile_runs = getattr(self._module, "compile_runs", None)
        self._runs = compile_runs(plan) if compile_runs is not None else plan
        return plan

    def _ensure_plan(self, buffers) -> None:
        if self._plan is None:
            self._plan = self._build_plan(buffers)

    def run_kernels(self, buffers: dict[str, torch.Tensor]) -> None:
        if self._plan is None or buffers is not self._resident:
            for k in self.schedule.kernels:
                self.run_one(k, buffers)
        else:
            run = self._module.run_bound
            for kind, payload in self._runs:
                if kind == "extern":
                    run_bound_extern(payload)
                elif kind == "kernel":
                    run(payload)
        fetch = getattr(self._module, "fetch_errors", None)
        if fetch is not None:
            fetch()

    def run_one(self, k, buffers: dict[str, torch.Tensor]) -> None:
        if isinstance(k, ExternKernel):
            run_extern(k, buffers, self._module)
        else:
            self._module.launch(k, buffers)

    def _run_eager(self, buffers: dict[str, torch.Tensor], plan) -> None:
        for i, k in enumerate(self.schedule.kernels):
            for b in plan.alloc_at.get(i, ()):
                if b.name in self._live:
                    buffers[b.name] = self._empty(b)
            self.run_one(k, buffers)
            for name in plan.free_at.get(i, ()):
                buffers.pop(name, None)

    def forward(self, *inputs: torch.Tensor):
        plan = self.schedule.plan
        if plan is not None and plan.mode == "eager":
            buffers = self._bind_resident(inputs)
            self._run_eager(buffers, plan)
            return self._collect(buffers)
        buffers = self._resident_buffers(inputs)
        self._ensure_plan(buffers)
        self.run_kernels(buffers)
        return self._collect(buffers)

    def _collect(self, buffers: dict[str, torch.Tensor]):
        """Views of the output buffers; they alias storage the next call
        overwrites (clone a result that must outlive the next call)."""
        outs = [v.layout.as_torch(buffers[v.buffer.name]) for v in self.graph.outputs]
        spec = self.graph.meta.get("out_spec")
        if spec is not None:
            from torch.utils._pytree import tree_unflatten

            try:
                return tree_unflatten(outs, spec)
            except Exception:
                pass
        return outs[0] if len(outs) == 1 else tuple(outs)

    def __call__(self, *inputs: torch.Tensor):
        self._raise_pending()
        if self.cfg.cuda_graphs and self.device.type == "cuda":
            return self._call_captured(inputs)
        return self.forward(*inputs)

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

    # -- graph replay -----------------------------------------------------------
    def _call_captured(self, inputs):
        if not self._captured:
            self._capture(inputs)
        else:
            self._check_inputs(inputs)
        for dst, src in zip(self._static_inputs, inputs):
            dst.copy_(src.reshape(-1), non_blocking=True)
        self._module.replay(torch.cuda.current_stream(self.device).cuda_stream)
        return self._static_outputs

    def _capture(self, inputs) -> None:
        """Warm up three times on a side stream (kernels loaded, library
        workspaces allocated), then capture one run into the context's
        hipGraph. Capture must not allocate: every extern writes into a
        pre-bound slice, and an allocation during capture is an error."""
        buffers = self._resident_buffers(inputs)
        self._ensure_plan(buffers)
        side = torch.cuda.Stream(self.device)
        side.wait_stream(torch.cuda.current_stream(self.device))
        with torch.cuda.stream(side):
            for _ in range(3):
                self.run_kernels(buffers)
            side.synchronize()
            before = _alloc_count(self.device)
            self._module.capture_begin(side.cuda_stream)
            try:
                self.run_kernels(buffers)
            finally:
                self._module.capture_end()
            after = _alloc_count(self.device)
        torch.cuda.current_stream(self.device).wait_stream(side)
        if after != before:
            culprits = self._allocating_entries(side)
            raise ExecutionError(f"{after - before} device allocation(s) happened during graph "
                                 "capture; the captured graph would reference memory it does not "
                                 f"own (allocating entries: {culprits})")
        self._capture_stream = side
        self._captured = True
        self._static_inputs = [buffers[v.buffer.name] for v in self.graph.inputs]
        self._static_outputs = self._collect(buffers)

    def _allocating_entries(self, stream) -> list[str]:
        """Plan entries that allocate device memory each time they run."""
        found = []
        with torch.cuda.stream(stream):
            for kernel, (kind, payload) in zip(self.schedule.kernels, self._plan):
                before = _alloc_count(self.device)
                if kind == "extern":
                    run_bound_extern(payload)
                elif kind == "kernel":
                    self._module.run_bound(payload)
                if _alloc_count(self.device) != before:
                    found.append(kernel.summary())
        stream.synchronize()
        return found

    def profile_kernels(self, inputs, iters: int = 20) -> list[tuple]:
        """(name, summary, ms) per kernel, each timed in place on the launch
        stream with events, in schedule order."""
        if self.device.type != "cuda":
            raise ExecutionError("kernel profiling needs a GPU device")
        buffers = self._resident_buffers(inputs)
        self._ensure_plan(buffers)
        for _ in range(3):
            self.run_kernels(buffers)
        torch.cuda.synchronize(self.device)
        out = []
        stream = torch.cuda.current_stream(self.device)
        for kernel, (kind, payload) in zip(self.schedule.kernels, self._plan):
            if kind == "kernel":
                ms = self._module.time_bound(payload, iters, stream.cuda_stream)
            else:
                for _ in range(3):
                    run_bound_extern(payload)
                start = torch.cuda.Event(enable_timing=True)
                end = torch.cuda.Event(enable_timing=True)
                start.record(stream)
                for _ in range(iters):
                    run_bound_extern(payload)
                end.record(stream)
                end.synchronize()
                ms = start.elapsed_time(end) / iters
            out.append((kernel.name, kernel.summary(), ms))
        return out

    # -- introspection ------------------------------------------------------------
    def source(self) -> str:
        """The generated module text (``mlc/runtime/executor.py:354-358``)."""
        return self._module.source

    def source_path(self):
        return getattr(self._module, "path", None)

    def __repr__(self) -> str:  # pragma: no cover
        return (f"CompiledModel({self.graph.name}, {len(self.schedule)} kernels, "
                f"backend={self.backend}, device={self.device})")


def _alloc_count(device) -> int:
    stats = torch.cuda.memory_stats(device)
    return int(stats.get("allocation.all.allocated", 0))


# ----------------------------------------------------------------------------
# extern dispatch
# ----------------------------------------------------------------------------

def _materialise(a, buffers):
    if isinstance(a, Value):
        return a.layout.as_torch(buffers[a.buffer.name])
    if isinstance(a, (list, tuple)):
        return type(a)(_materialise(x, buffers) for x in a)
    return a


def bind_extern(k: ExternKernel, buffers: dict[str, torch.Tensor], module=None):
    """Resolve an extern call against the fixed buffer table (never runs it).
    A runner may claim the op with a native kernel (``bind_native_extern``)."""
    node = k.node
    native = getattr(module, "bind_native_extern", None)
    if native is not None:
        bound = native(k, buffers)
        if bound is not None:
            return ("native", module, bound)
    target = node.meta.get("target")
    if target is None:
        raise ExecutionError(f"{node.op} has no dispatch target")
    args = [_materialise(a, buffers) for a in node.args]
    kwargs = {n: _materialise(v, buffers) for n, v in node.kwargs.items()}
    variant = out_variant(node)
    dest = None
    if variant is not None:
        out = node.outputs[0]
        dest = out.layout.as_torch(buffers[out.buffer.name])
    outs = [buffers[o.buffer.name] for o in node.outputs]
    return ("torch", target, variant, args, kwargs, dest, outs)


def run_bound_extern(bound) -> None:
    if bound[0] == "native":
        _, module, payload = bound
        module.run_bound(payload)
        return
    _, target, variant, args, kwargs, dest, outs = bound
    if variant is not None:
        variant(*args, **kwargs, out=dest)
        return
    result = target(*args, **kwargs)
    results = result if isinstance(result, (list, tuple)) else [result]
    for buf, r in zip(outs, results):
        buf.copy_(r.contiguous().reshape(-1))


def out_variant(node):
    """The op's ``.out`` overload when it takes exactly the default overload's
    arguments plus ``out`` (decided from the schema, never by calling it)."""
    if "out_variant" in node.meta:
        return node.meta["out_variant"]
    found = None
    target = node.meta.get("target")
    if (node.op.startswith("aten.") and len(node.outputs) == 1 and target is not None
            and hasattr(target, "_schema")):
        packet = getattr(torch.ops.aten, node.op.split(".")[1], None)
        overload = getattr(packet, "out", None) if packet is not None else None
        if overload is not None and _same_arguments(target, overload):
            found = overload
    node.meta["out_variant"] = found
    return found


def _same_arguments(default, out_overload) -> bool:
    try:
        want = [a.name for a in default._schema.arguments]
        have = [a.name for a in out_overload._schema.arguments]
    except AttributeError:
        return False
    return have[:len(want)] == want and have[len(want):] == ["out"]


def run_extern(k: ExternKernel, buffers: dict[str, torch.Tensor], module=None) -> None:
    """Dispatch one extern op through the flat buffers (unplanned path). An
    ``.out`` overload that rejects the call is dropped for this node and the
    op runs functionally, copied into its buffer."""
    bound = bind_extern(k, buffers, module)
    if bound[0] == "torch" and bound[2] is not None:
        _, target, variant, args, kwargs, dest, outs = bound
        try:
            variant(*args, **kwargs, out=dest)
            return
        except (RuntimeError, TypeError):
            k.node.meta["out_variant"] = None
            bound = ("torch", target, None, args, kwargs, None, outs)
    run_bound_extern(bound)
