"""The arena for callers that cannot allocate (``mlc_slab_static``).

Through the C ABI: the entry point hands back the library's static device
array (256-byte aligned, one address for every context on the GPU), leaves
the device's free memory unchanged, and rejects a request beyond
``MLC_STATIC_SLAB_BYTES`` with ``MLC_E_RANGE`` and a message. End to end: a
model whose arena is the static array computes what the same model with its
own ``hipMalloc`` slab (``mlc_slab_alloc``) computes, on two calls in a row,
the second with a smaller input (half the tokens, a smaller arena) that
reuses the array the first call left its contents in.
"""

from __future__ import annotations

import ctypes

import pytest
import torch

import mlc
from mlc.bench.models import FFNBlock
from mlc.config import Config
from mlc.runtime import native

pytestmark = pytest.mark.gpu

MLC_E_RANGE = -10002
MLC_E_STATE = -10003


def _ctx(lib):
    ctx = ctypes.c_void_p()
    native.check(lib.mlc_ctx_create(0, ctypes.byref(ctx)), "mlc_ctx_create")
    return ctx


def _static_address(lib) -> int:
    ctx = _ctx(lib)
    try:
        ptr = ctypes.c_void_p()
        native.check(lib.mlc_slab_static(ctx, 256, ctypes.byref(ptr)), "mlc_slab_static")
        return ptr.value
    finally:
        lib.mlc_ctx_destroy(ctx)


def test_static_slab_entry_point_through_the_c_abi():
    torch.cuda.init()
    lib = native.load_library()
    a, b = _ctx(lib), _ctx(lib)
    try:
        free_before = torch.cuda.mem_get_info(0)[0]
        pa, pb = ctypes.c_void_p(), ctypes.c_void_p()
        assert lib.mlc_slab_static(a, 3 << 20, ctypes.byref(pa)) == 0
        assert lib.mlc_slab_static(b, native.STATIC_SLAB_BYTES, ctypes.byref(pb)) == 0
        assert torch.cuda.mem_get_info(0)[0] == free_before
        assert pa.value and pa.value % 256 == 0 and pa.value == pb.value
        # asking again is a no-op; asking for more than the array holds fails cleanly
        again = ctypes.c_void_p()
        assert lib.mlc_slab_static(a, 1 << 20, ctypes.byref(again)) == 0
        assert again.value == pa.value
        c = _ctx(lib)
        try:
            big = ctypes.c_void_p()
            assert lib.mlc_slab_static(c, native.STATIC_SLAB_BYTES + 1,
                                       ctypes.byref(big)) == MLC_E_RANGE
            assert b"static arena holds" in lib.mlc_last_error()
            # a context that already holds an allocated slab keeps it
            own = ctypes.c_void_p()
            native.check(lib.mlc_slab_alloc(c, 4096, ctypes.byref(own)), "mlc_slab_alloc")
            assert lib.mlc_slab_static(c, 4096, ctypes.byref(big)) == MLC_E_STATE
        finally:
            lib.mlc_ctx_destroy(c)
        # the other direction: a context on the static array keeps it for
        # requests it holds and never replaces it with an allocated slab
        grown = ctypes.c_void_p()
        assert lib.mlc_slab_alloc(a, 1 << 20, ctypes.byref(grown)) == 0
        assert grown.value == pa.value
        assert lib.mlc_slab_alloc(a, native.STATIC_SLAB_BYTES + 1,
                                  ctypes.byref(grown)) == MLC_E_STATE
    finally:
        lib.mlc_ctx_destroy(a)
        lib.mlc_ctx_destroy(b)


def _ffn(seq: int):
    """BASELINE config 1's FFN block (fp32, LN -> fc1 -> tanh-GELU -> fc2)
    over ``seq`` tokens, seeded."""
    torch.manual_seed(0)
    model = FFNBlock().eval()
    with torch.no_grad():
        model.ln.weight.normal_(1.0, 0.02)
        model.ln.bias.normal_(0.0, 0.02)
        model.fc1.weight.normal_(0.0, 0.02)
        model.fc2.weight.normal_(0.0, 0.02)
    x, r = torch.randn(1, seq, 768), torch.randn(1, seq, 768)
    return model.cuda(), (x.cuda(), r.cuda())


@pytest.mark.parametrize("graphs", [True, False], ids=["graph", "plan"])
def test_static_arena_matches_allocated_slab(graphs):
    lib = native.load_library()
    address = _static_address(lib)
    for seq in (128, 64):
        model, args = _ffn(seq)
        want = mlc.compile(model, args, Config(cuda_graphs=graphs))(*args).clone()
        compiled = mlc.compile(model, args, Config(cuda_graphs=graphs, static_arena=True))
        got = compiled(*args)
        torch.cuda.synchronize()
        arena = compiled.schedule.arena_bytes
        assert 0 < arena <= native.STATIC_SLAB_BYTES
        assert compiled._arena.data_ptr() == address
        err = (got - want).abs().max().item() / want.abs().max().item()
        print(f"seq {seq}: arena {arena} B at the static array, rel err vs own slab {err:.2e}, "
              f"bit-identical {torch.equal(got, want)}")
        assert err <= 1e-5
        assert torch.equal(got, want)
        del compiled, model
