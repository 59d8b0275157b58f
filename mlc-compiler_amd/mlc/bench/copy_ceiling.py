"""The practical ceiling for a bandwidth-bound kernel: a plain packed copy.

A generated kernel's launch period is ``fixed cost + bytes / bandwidth``. On
MI355X the fixed cost of a launch (dispatch, ramp, drain and the cache
write-back between dependent kernels) is about 1.5 us, which is as long as
moving 12 MB at full bandwidth. The fraction of 8 TB/s alone therefore
understates kernels of BERT's sizes. This module times the cheapest kernel that
moves the same bytes: a copy with the pointwise template's geometry (512-thread
workgroups, one 16-byte pack per thread), launched back to back through the
same C ABI as the generated kernels. Dividing its period by a kernel's period
gives how close that kernel is to a copy.
"""

from __future__ import annotations

import ctypes
import struct

from ..runtime import native

SOURCE = """// Plain packed copy: the bandwidth ceiling generated kernels are compared with.
#include "mlc_cdna4.h"
extern "C" __global__ void __launch_bounds__(512)
mlc_copy_ceiling(const mlc::f16x8* __restrict__ src, mlc::f16x8* __restrict__ dst,
                 uint32_t packs) {
  const uint32_t i = blockIdx.x * 512u + threadIdx.x;
  if (i < packs) dst[i] = src[i];
}
"""

BLOCK = 512


class CopyCeiling:
    """Times packed copies on one device; one instance loads the module once."""

    def __init__(self, device_index: int = 0) -> None:
        self.lib = native.load_library()
        _, obj = native.compile_code_object(SOURCE)
        image = obj.read_bytes()
        self._ctx = ctypes.c_void_p()
        native.check(self.lib.mlc_ctx_create(device_index, ctypes.byref(self._ctx)),
                     "mlc_ctx_create")
        self._mod = ctypes.c_void_p()
        buf = ctypes.create_string_buffer(image, len(image))
        native.check(self.lib.mlc_module_load(self._ctx, buf, len(image), ctypes.byref(self._mod)),
                     "mlc_module_load")
        fn = ctypes.c_void_p()
        native.check(self.lib.mlc_function(self._mod, b"mlc_copy_ceiling", ctypes.byref(fn)),
                     "mlc_function(mlc_copy_ceiling)")
        self._fn = fn.value
        self._cache: dict[int, float] = {}

    def period_us(self, nbytes: int, iters: int, stream: int) -> float:
        """Average launch period (us) of a copy reading ``nbytes / 2`` and
        writing ``nbytes / 2`` bytes (16-byte packs)."""
        if nbytes in self._cache:
            return self._cache[nbytes]
        import torch

        packs = max(1, nbytes // 32)
        src = torch.ones(packs * 8, dtype=torch.float16, device="cuda")
        dst = torch.empty_like(src)
        args = struct.pack("<QQI", src.data_ptr(), dst.data_ptr(), packs)
        grid = -(-packs // BLOCK)
        plan = ctypes.c_void_p()
        native.check(self.lib.mlc_plan_create(self._ctx, 1, ctypes.byref(plan)), "mlc_plan_create")
        try:
            native.check(self.lib.mlc_plan_set(plan, 0, self._fn, grid, BLOCK, 0, args, len(args)),
                         "mlc_plan_set")
            ms = ctypes.c_float()
            native.check(self.lib.mlc_time_entry(plan, 0, iters, stream, ctypes.byref(ms)),
                         "mlc_time_entry")
        finally:
            self.lib.mlc_plan_destroy(plan)
        torch.cuda.synchronize()
        self._cache[nbytes] = float(ms.value) * 1e3
        return self._cache[nbytes]

    def close(self) -> None:
        if self._ctx:
            self.lib.mlc_ctx_destroy(self._ctx)
            self.lib.mlc_module_unload(self._mod)
            self._ctx = None
