"""Native pieces of the HIP backend.

* ``libmlc_hip.so`` -- the C ABI declared in ``include/mlc_hip.h`` (contexts,
  code-object modules, the arena slab, launch plans, hipGraph capture and
  replay, hipEvent timing), built from ``csrc/mlc_hip.cpp`` with ``hipcc`` and
  loaded with ``ctypes``.
* gfx950 code objects of generated kernel modules, compiled with
  ``hipcc --genco`` and kept in a content-addressed cache, keyed by the
  source, the device template header, the compile flags and the compiler
  version (the role of ``mlc/runtime/triton_runtime.py:29-44``'s hashed module
  files).

There is no fallback: if the library or the compiler is missing the call
raises, so nothing can silently run elsewhere.
"""

from __future__ import annotations

import ctypes
import functools
import hashlib
import os
import pathlib
import shutil
import subprocess

PKG = pathlib.Path(__file__).resolve().parents[1]          # .../mlc
ROOT = PKG.parent                                           # .../mlc-compiler_amd
REPO = ROOT.parent
CSRC = ROOT / "csrc"
INCLUDE = REPO / "include"
TEMPLATES = PKG / "codegen" / "templates"
LIB_PATH = pathlib.Path(__file__).resolve().parent / "libmlc_hip.so"

ARCH = "gfx950"
#: flags for every piece of HIP code built here. Packed-fp32 instructions are
#: switched off; contraction is off so each fp32 operation rounds on its own,
#: exactly as the op-by-op reference evaluation does.
HIP_FLAGS = [
    "-O3", f"--offload-arch={ARCH}", "-std=c++17",
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-ffp-contract=off",
]


#: size of the library's static arena (``MLC_STATIC_SLAB_BYTES`` in the header)
STATIC_SLAB_BYTES = 64 << 20


class NativeError(RuntimeError):
    """A failure inside libmlc_hip.so or while building native code."""


def hipcc() -> str:
    exe = os.environ.get("HIPCC") or shutil.which("hipcc") or "/opt/rocm/bin/hipcc"
    if not os.path.exists(exe):
        raise NativeError("hipcc not found: the HIP backend compiles its kernels with hipcc")
    return exe


@functools.lru_cache(maxsize=None)
def compiler_version() -> str:
    out = subprocess.run([hipcc(), "--version"], capture_output=True, text=True, check=True)
    return out.stdout


def _run(cmd: list[str]) -> None:
    proc = subprocess.run(cmd, capture_output=True, text=True)
    if proc.returncode != 0:
        raise NativeError(f"command failed ({proc.returncode}): {' '.join(cmd)}\n"
                          f"{proc.stdout}\n{proc.stderr}")


# ---------------------------------------------------------------------------
# the runtime library
# ---------------------------------------------------------------------------

def build_library(force: bool = True) -> pathlib.Path:
    """Compile ``libmlc_hip.so`` in-tree (next to this file)."""
    src = CSRC / "mlc_hip.cpp"
    if not force and LIB_PATH.exists() and LIB_PATH.stat().st_mtime >= src.stat().st_mtime:
        return LIB_PATH
    tmp = LIB_PATH.with_name(LIB_PATH.name + f".tmp{os.getpid()}")
    _run([hipcc(), "-x", "hip", *HIP_FLAGS, "-fPIC", "-shared", f"-I{INCLUDE}",
          str(src), "-o", str(tmp)])
    tmp.replace(LIB_PATH)
    return LIB_PATH


_c_int, _c_u32, _c_size, _vp = ctypes.c_int, ctypes.c_uint32, ctypes.c_size_t, ctypes.c_void_p
_pvp = ctypes.POINTER(ctypes.c_void_p)

SIGNATURES = {
    "mlc_version": ([], _c_int),
    "mlc_ctx_create": ([_c_int, _pvp], _c_int),
    "mlc_ctx_destroy": ([_vp], _c_int),
    "mlc_module_load": ([_vp, _vp, _c_size, _pvp], _c_int),
    "mlc_module_unload": ([_vp], _c_int),
    "mlc_function": ([_vp, ctypes.c_char_p, _pvp], _c_int),
    "mlc_slab_alloc": ([_vp, _c_size, _pvp], _c_int),
    "mlc_slab_static": ([_vp, _c_size, _pvp], _c_int),
    "mlc_slab_dlpack": ([_vp, _pvp], _c_int),
    "mlc_launch": ([_vp, _c_u32, _c_u32, _c_u32, _vp, _c_size, _vp], _c_int),
    "mlc_plan_create": ([_vp, _c_int, _pvp], _c_int),
    "mlc_plan_set": ([_vp, _c_int, _vp, _c_u32, _c_u32, _c_u32, _vp, _c_size], _c_int),
    "mlc_plan_run": ([_vp, _c_int, _c_int, _vp], _c_int),
    "mlc_plan_destroy": ([_vp], _c_int),
    "mlc_graph_begin": ([_vp, _vp], _c_int),
    "mlc_graph_end": ([_vp], _c_int),
    "mlc_graph_replay": ([_vp, _vp], _c_int),
    "mlc_graph_node_count": ([_vp, ctypes.POINTER(_c_size)], _c_int),
    "mlc_time_entry": ([_vp, _c_int, _c_int, _vp, ctypes.POINTER(ctypes.c_float)], _c_int),
    "mlc_error_word": ([_vp, _pvp], _c_int),
    "mlc_error_fetch": ([_vp, _vp], _c_int),
    "mlc_error_poll": ([_vp, ctypes.POINTER(ctypes.c_int32)], _c_int),
    "mlc_error_clear": ([_vp], _c_int),
    "mlc_device_synchronize": ([_vp], _c_int),
    "mlc_last_error": ([], ctypes.c_char_p),
}


@functools.lru_cache(maxsize=None)
def load_library() -> ctypes.CDLL:
    """The runtime library, with every C-ABI signature declared. Raises if
    it was not built (``__graft_entry__.build()`` or ``build_library()``)."""
    if not LIB_PATH.exists():
        raise NativeError(f"{LIB_PATH} is missing: build it first (python -c "
                          "'import __graft_entry__ as g; g.build()')")
    lib = ctypes.CDLL(str(LIB_PATH))
    for name, (args, res) in SIGNATURES.items():
        fn = getattr(lib, name)
        fn.argtypes = args
        fn.restype = res
    return lib


def check(rc: int, what: str = "") -> None:
    """Raise :class:`NativeError` carrying the library's message if ``rc`` is
    not 0."""
    if rc != 0:
        msg = load_library().mlc_last_error().decode(errors="replace")
        raise NativeError(f"{what or 'libmlc_hip'} failed ({rc}): {msg}")


# ---------------------------------------------------------------------------
# code objects of generated modules
# ---------------------------------------------------------------------------

def cache_dir() -> pathlib.Path:
    """``MLC_CACHE_DIR`` if set, else ``.mlc_cache`` at the repository root
    (so code objects built here travel with the tree), else ``~/.cache/mlc``."""
    root = os.environ.get("MLC_CACHE_DIR")
    candidates = [pathlib.Path(root)] if root else [REPO / ".mlc_cache",
                                                    pathlib.Path.home() / ".cache" / "mlc"]
    for path in candidates:
        try:
            path.mkdir(parents=True, exist_ok=True)
            if os.access(path, os.W_OK):
                return path
        except OSError:
            continue
    raise NativeError(f"no writable kernel cache directory among {candidates}")


def _template_text() -> str:
    return "".join(p.read_text() for p in sorted(TEMPLATES.glob("*.h")))


def module_key(source: str) -> str:
    h = hashlib.sha256()
    for part in (source, _template_text(), " ".join(HIP_FLAGS), compiler_version()):
        h.update(part.encode())
        h.update(b"\0")
    return h.hexdigest()[:24]


def compile_code_object(source: str) -> tuple[pathlib.Path, pathlib.Path]:
    """(source path, code-object path) for ``source``, compiling on a cache
    miss. Files are written then renamed, so a concurrent reader never sees a
    partial object."""
    key = module_key(source)
    d = cache_dir()
    src = d / f"mlc_kernels_{key}.hip"
    obj = d / f"mlc_kernels_{key}.hsaco"
    if not src.exists() or src.read_text() != source:
        tmp = src.with_name(src.name + f".{os.getpid()}.tmp")
        tmp.write_text(source)
        tmp.replace(src)
    if not obj.exists():
        tmp = obj.with_name(obj.name + f".{os.getpid()}.tmp")
        _run([hipcc(), "--genco", *HIP_FLAGS, f"-I{TEMPLATES}", "-x", "hip", str(src),
              "-o", str(tmp)])
        tmp.replace(obj)
    return src, obj
