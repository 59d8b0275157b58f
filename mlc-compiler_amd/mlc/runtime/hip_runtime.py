"""Load and launch the generated HIP module through ``libmlc_hip.so``.

The counterpart of the reference's ``TritonRuntime``
(``mlc/runtime/triton_runtime.py:60-97``) behind the same seam: it is built
from a schedule, exposes ``source`` (the module text, a ``str``), ``path``
(where that text was written) and ``launch_table``, resolves a
kernel against the buffer table once (``bind``) and launches it
(``launch``/``run_bound``) on torch's current stream. On top of that it owns
the per-model native state the MI355X design adds:

* one context per compiled model (device binding, the arena slab, the graph);
* the arena as one ``hipMalloc`` slab, handed to torch through DLPack so the
  extern library calls write into the same memory (``arena``);
* the pre-resolved plan as a native launch table: consecutive generated
  kernels run as one ``mlc_plan_run`` call (``compile_runs``);
* hipGraph capture and replay of the whole schedule (``capture_begin``,
  ``capture_end``, ``replay``);
* hipEvent timing of one bound kernel in place (``time_bound``);
* the invalid-input word: the native embedding gather flags an id outside
  its table there (torch raises ``IndexError`` for one); every run enqueues
  an asynchronous copy of the word to pinned host memory (``fetch_errors``,
  captured into the graph too) and ``pending_error`` reads that copy without
  waiting for the device.
"""

from __future__ import annotations

import ctypes
import struct
from dataclasses import dataclass

import torch

from ..codegen.hip_backend import LaunchSpec, build_module
from ..config import Config
from ..kernels import ExternKernel, Kernel, Schedule
from . import native

_CAPSULE_NAME = b"dltensor"
_PyCapsule_New = ctypes.pythonapi.PyCapsule_New
_PyCapsule_New.restype = ctypes.py_object
_PyCapsule_New.argtypes = [ctypes.c_void_p, ctypes.c_char_p, ctypes.c_void_p]


@dataclass
class Bound:
    """One generated kernel resolved against the buffer table."""

    name: str
    fn: int
    grid: int
    block: int
    lds: int
    args: bytes


@dataclass
class Range:
    """Entries ``[begin, end)`` of the native launch plan."""

    plan: int
    begin: int
    end: int


def _stream() -> int:
    return torch.cuda.current_stream().cuda_stream


class HipRuntime:
    name = "hip"

    def __init__(self, schedule: Schedule, cfg: Config, device: torch.device) -> None:
        if device.type != "cuda":
            raise native.NativeError(f"HipRuntime needs a ROCm GPU device, got {device}")
        self.device = device
        self.index = device.index if device.index is not None else torch.cuda.current_device()
        self.lib = native.load_library()
        self.module = build_module(schedule, cfg)
        #: the generated HIP module text (``TritonRuntime.source``)
        self.source: str = self.module.source
        self.launch_table: dict[str, LaunchSpec] = self.module.launches
        self.path, self.code_object_path = native.compile_code_object(self.source)
        image = self.code_object_path.read_bytes()

        self._ctx = ctypes.c_void_p()
        native.check(self.lib.mlc_ctx_create(self.index, ctypes.byref(self._ctx)), "mlc_ctx_create")
        self._mod = ctypes.c_void_p()
        buf = ctypes.create_string_buffer(image, len(image))
        native.check(self.lib.mlc_module_load(self._ctx, buf, len(image), ctypes.byref(self._mod)),
                     "mlc_module_load")
        self.functions: dict[str, int] = {}
        for symbol in sorted({s.symbol for s in self.launch_table.values()}):
            fn = ctypes.c_void_p()
            native.check(self.lib.mlc_function(self._mod, symbol.encode(), ctypes.byref(fn)),
                         f"mlc_function({symbol})")
            self.functions[symbol] = fn.value
        self._plans: list[ctypes.c_void_p] = []
        self._arena_tensor: torch.Tensor | None = None
        self._static_arena = bool(getattr(cfg, "static_arena", False))
        #: device address of the context's invalid-input word, if a kernel
        #: of this module can flag one (the native embedding gather)
        self._error_word: int | None = None
        if any(spec.meta.get("error_word") for spec in self.launch_table.values()):
            word = ctypes.c_void_p()
            native.check(self.lib.mlc_error_word(self._ctx, ctypes.byref(word)), "mlc_error_word")
            self._error_word = word.value

    # -- the reference seam ---------------------------------------------------

    def bind(self, k: Kernel, buffers: dict[str, torch.Tensor]) -> Bound:
        """Resolve a launch once: function handle, geometry and the packed
        kernel arguments (``in0..in{n-1}, out0..out{m-1}`` buffer base
        pointers, ``mlc/runtime/triton_runtime.py:67-83``)."""
        if isinstance(k, ExternKernel):
            raise TypeError("extern kernels do not go through the HIP runtime")
        spec = self.launch_table[k.name]
        ptrs = []
        for a in list(k.inputs) + list(k.outputs):
            t = buffers[a.value.buffer.name]
            if t.device.type != "cuda":
                raise native.NativeError(f"{k.name}: buffer {a.value.buffer.name} is on {t.device}")
            if t.dtype != a.value.buffer.dtype or t.numel() < a.value.buffer.numel:
                raise native.NativeError(
                    f"{k.name}: buffer {a.value.buffer.name} is {t.dtype}[{t.numel()}], the kernel "
                    f"was generated for {a.value.buffer.dtype}[{a.value.buffer.numel}]")
            if t.data_ptr() % 16:
                raise native.NativeError(f"{k.name}: buffer {a.value.buffer.name} is not 16-byte "
                                         "aligned; the kernel's packed accesses assume it is")
            ptrs.append(t.data_ptr())
        args = struct.pack(f"<{len(ptrs)}Q", *ptrs)
        return Bound(k.name, self.functions[spec.symbol], spec.grid, spec.block, spec.lds_bytes,
                     args)

    def bind_native_extern(self, k: ExternKernel, buffers: dict[str, torch.Tensor]) -> Bound | None:
        """An extern op this module implements natively (``aten.embedding``),
        resolved like a generated kernel; ``None`` leaves it to the library."""
        spec = self.launch_table.get(k.name)
        if spec is None:
            return None
        ptrs = []
        for name, dtype, numel in zip(spec.meta["buffers"], spec.meta["dtypes"],
                                      spec.meta["numels"]):
            t = buffers[name]
            if t.device.type != "cuda" or t.dtype != dtype or t.numel() < numel:
                raise native.NativeError(f"{k.name}: buffer {name} is {t.dtype}[{t.numel()}] on "
                                         f"{t.device}, expected {dtype}[{numel}] on the GPU")
            if t.data_ptr() % 16:
                raise native.NativeError(f"{k.name}: buffer {name} is not 16-byte aligned")
            ptrs.append(t.data_ptr())
        if spec.meta.get("error_word"):
            ptrs.append(self._error_word)
        return Bound(k.name, self.functions[spec.symbol], spec.grid, spec.block, spec.lds_bytes,
                     struct.pack(f"<{len(ptrs)}Q", *ptrs))

    # -- invalid inputs ------------------------------------------------------------
    @property
    def flags_errors(self) -> bool:
        """Whether a kernel of this module can flag an invalid input."""
        return self._error_word is not None

    def fetch_errors(self, stream: int | None = None) -> None:
        """Enqueue the copy of the invalid-input word to its pinned host
        mirror on ``stream`` (torch's current stream by default). It is
        issued after a run's kernels, so under capture it becomes the graph's
        last node."""
        if self._error_word is not None:
            native.check(self.lib.mlc_error_fetch(self._ctx, _stream() if stream is None
                                                  else stream), "mlc_error_fetch")

    def pending_error(self) -> str | None:
        """The message for an invalid input flagged by a completed run, read
        from the host mirror without waiting for the device; ``None`` if no
        completed run flagged one. Runs still in flight are seen by a later
        call."""
        if self._error_word is None:
            return None
        value = ctypes.c_int32()
        native.check(self.lib.mlc_error_poll(self._ctx, ctypes.byref(value)), "mlc_error_poll")
        if value.value == 0:
            return None
        return ("an embedding id was outside its table (torch raises IndexError for such an "
                "id); the rows it addressed were written as zeros")

    def clear_errors(self) -> None:
        """Wait for the device, then zero the word and its mirror."""
        if self._error_word is not None:
            native.check(self.lib.mlc_error_clear(self._ctx), "mlc_error_clear")

    def check_errors(self) -> None:
        """Synchronize, fetch the word, and raise :class:`native.NativeError`
        if any run so far flagged an invalid input (clearing the flag)."""
        if self._error_word is None:
            return
        self.fetch_errors()
        torch.cuda.synchronize(self.device)
        msg = self.pending_error()
        if msg is not None:
            self.clear_errors()
            raise native.NativeError(msg)

    def launch(self, k: Kernel, buffers: dict[str, torch.Tensor]) -> None:
        self.run_bound(self.bind(k, buffers))

    def run_bound(self, payload) -> None:
        if isinstance(payload, Bound) and payload.grid == 0:
            return  # a reduction over zero rows: nothing to launch
        if isinstance(payload, Range):
            native.check(self.lib.mlc_plan_run(payload.plan, payload.begin, payload.end, _stream()),
                         "mlc_plan_run")
            return
        native.check(self.lib.mlc_launch(payload.fn, payload.grid, payload.block, payload.lds,
                                         payload.args, len(payload.args), _stream()),
                     f"mlc_launch({payload.name})")

    # -- the pre-resolved plan ----------------------------------------------------
    def compile_runs(self, plan: list) -> list:
        """Turn ``[(kind, payload)]`` into runs where every maximal sequence of
        generated kernels is one ``Range`` of a native launch plan."""
        def native_of(kind, payload):
            if kind == "kernel":
                return payload if payload.grid else None
            if kind == "extern" and getattr(payload, "module", None) is self:
                return payload.bound  # a library op this module claimed
            return None

        kernels = [b for b in (native_of(kind, p) for kind, p in plan) if b is not None]
        handle = ctypes.c_void_p()
        native.check(self.lib.mlc_plan_create(self._ctx, len(kernels), ctypes.byref(handle)),
                     "mlc_plan_create")
        self._plans.append(handle)
        for i, b in enumerate(kernels):
            native.check(self.lib.mlc_plan_set(handle, i, b.fn, b.grid, b.block, b.lds, b.args,
                                               len(b.args)), "mlc_plan_set")
        runs: list = []
        i = 0
        for kind, payload in plan:
            if native_of(kind, payload) is not None:
                if runs and runs[-1][0] == "kernel":
                    runs[-1][1].end = i + 1
                else:
                    runs.append(("kernel", Range(handle.value, i, i + 1)))
                i += 1
            else:
                runs.append((kind, payload))
        return runs

    # -- arena -----------------------------------------------------------------
    def arena(self, nbytes: int) -> torch.Tensor:
        """The arena: one ``hipMalloc`` slab of at least ``nbytes``, or with
        ``Config(static_arena=True)`` the library's static device array
        (``mlc_slab_static``, nothing allocated), as a uint8 tensor that
        aliases it (DLPack, no copy)."""
        if self._arena_tensor is not None and self._arena_tensor.numel() >= nbytes:
            return self._arena_tensor
        self._arena_tensor = None
        ptr = ctypes.c_void_p()
        if self._static_arena:
            native.check(self.lib.mlc_slab_static(self._ctx, nbytes, ctypes.byref(ptr)),
                         "mlc_slab_static")
        else:
            native.check(self.lib.mlc_slab_alloc(self._ctx, nbytes, ctypes.byref(ptr)),
                         "mlc_slab_alloc")
        managed = ctypes.c_void_p()
        native.check(self.lib.mlc_slab_dlpack(self._ctx, ctypes.byref(managed)), "mlc_slab_dlpack")
        capsule = _PyCapsule_New(managed, _CAPSULE_NAME, None)
        t = torch.utils.dlpack.from_dlpack(capsule)
        if t.data_ptr() != ptr.value or t.device.type != "cuda":
            raise native.NativeError("the slab's DLPack export does not alias the slab")
        self._arena_tensor = t
        return t

    # -- graph -----------------------------------------------------------------
    def capture_begin(self, stream: int) -> None:
        native.check(self.lib.mlc_graph_begin(self._ctx, stream), "mlc_graph_begin")

    def capture_end(self) -> None:
        native.check(self.lib.mlc_graph_end(self._ctx), "mlc_graph_end")

    def replay(self, stream: int) -> None:
        native.check(self.lib.mlc_graph_replay(self._ctx, stream), "mlc_graph_replay")

    def graph_nodes(self) -> int:
        n = ctypes.c_size_t()
        native.check(self.lib.mlc_graph_node_count(self._ctx, ctypes.byref(n)),
                     "mlc_graph_node_count")
        return n.value

    # -- profiling -------------------------------------------------------------
    def time_bound(self, payload: Bound, iters: int, stream: int) -> float:
        """Average ms of ``iters`` back-to-back launches of one bound kernel,
        timed with hipEvents on ``stream``."""
        if payload.grid == 0:
            return 0.0
        handle = ctypes.c_void_p()
        native.check(self.lib.mlc_plan_create(self._ctx, 1, ctypes.byref(handle)), "mlc_plan_create")
        try:
            native.check(self.lib.mlc_plan_set(handle, 0, payload.fn, payload.grid, payload.block,
                                               payload.lds, payload.args, len(payload.args)),
                         "mlc_plan_set")
            ms = ctypes.c_float()
            native.check(self.lib.mlc_time_entry(handle, 0, iters, stream, ctypes.byref(ms)),
                         "mlc_time_entry")
            return float(ms.value)
        finally:
            self.lib.mlc_plan_destroy(handle)

    def synchronize(self) -> None:
        native.check(self.lib.mlc_device_synchronize(self._ctx), "mlc_device_synchronize")

    def close(self) -> None:
        lib = self.lib
        for p in self._plans:
            lib.mlc_plan_destroy(p)
        self._plans = []
        self._arena_tensor = None
        # the context owns the graph that names the module's functions: it goes first
        if getattr(self, "_ctx", None) is not None and self._ctx.value:
            lib.mlc_ctx_destroy(self._ctx)
            self._ctx = None
        if getattr(self, "_mod", None) is not None and self._mod.value:
            lib.mlc_module_unload(self._mod)
            self._mod = None

    def __del__(self) -> None:
        try:
            self.close()
        except Exception:
            pass
