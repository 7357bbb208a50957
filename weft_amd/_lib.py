"""ctypes binding of the in-tree ``libweft_hip.so``.

The library is the product: there is no fallback.  ``load()`` raises if the
shared library has not been built (``python -m weft_amd.build`` or
``__graft_entry__.build()``).  Argument types come from the library's own ABI
metadata (``weft_hip_artifact``): one ``c_void_p`` per View parameter, then one
``c_size_t`` per shape parameter, as Weft's CompiledKernel binds generated
symbols (python/weft/runtime/compiler.py:91-96).
"""
from __future__ import annotations

import ctypes
import json
import threading
from pathlib import Path

LIB_PATH = Path(__file__).resolve().parent / "libweft_hip.so"

_lock = threading.Lock()
_lib: ctypes.CDLL | None = None
_artifact: dict | None = None


class LibraryMissing(RuntimeError):
    pass


def _share_torch_hip_runtime() -> None:
    """Import torch (when installed) before dlopen-ing libweft_hip.

    PyTorch-ROCm ships its own libamdhip64 with the same SONAME
    (libamdhip64.so.7) as /opt/rocm's.  Loaded after torch, libweft_hip binds
    to torch's copy and the process has one HIP runtime; loaded first, torch
    would bring in a second HIP/HSA runtime and device discovery fails.
    """
    try:
        import torch  # noqa: F401
    except ImportError:
        pass


def load() -> ctypes.CDLL:
    global _lib, _artifact
    with _lock:
        if _lib is None:
            _share_torch_hip_runtime()
            if not LIB_PATH.exists():
                raise LibraryMissing(
                    f"{LIB_PATH} is not built; run python -m weft_amd.build (hipcc, gfx950)")
            lib = ctypes.CDLL(str(LIB_PATH))
            lib.weft_hip_artifact.restype = ctypes.c_char_p
            lib.weft_hip_version.restype = ctypes.c_char_p
            lib.weft_hip_error_string.restype = ctypes.c_char_p
            lib.weft_hip_error_string.argtypes = [ctypes.c_int]
            lib.weft_hip_set_stream.argtypes = [ctypes.c_void_p]
            lib.weft_hip_set_stream.restype = ctypes.c_int
            lib.weft_hip_get_stream.restype = ctypes.c_void_p
            lib.weft_hip_set_tile_binding.argtypes = [ctypes.c_char_p, ctypes.c_size_t]
            lib.weft_hip_set_tile_binding.restype = ctypes.c_int
            lib.weft_hip_clear_tile_bindings.argtypes = []
            lib.weft_hip_clear_tile_bindings.restype = None
            lib.weft_hip_get_last_error.restype = ctypes.c_int
            lib.weft_hip_synchronize.restype = ctypes.c_int
            lib.weft_hip_device_count.restype = ctypes.c_int
            lib.weft_hip_device_arch.argtypes = [ctypes.c_int, ctypes.c_char_p, ctypes.c_size_t]
            lib.weft_hip_device_arch.restype = ctypes.c_int
            lib.weft_hip_set_launch_log.argtypes = [ctypes.c_int]
            lib.weft_hip_set_launch_log.restype = ctypes.c_int
            lib.weft_hip_launch_log.argtypes = [ctypes.c_char_p, ctypes.c_size_t]
            lib.weft_hip_launch_log.restype = ctypes.c_size_t
            lib.weft_hip_probe_empty.argtypes = []
            lib.weft_hip_probe_empty.restype = None
            lib.weft_hip_probe_read.argtypes = [ctypes.c_void_p, ctypes.c_size_t, ctypes.c_void_p, ctypes.c_int]
            lib.weft_hip_probe_read.restype = None
            lib.weft_hip_probe_read_shape.argtypes = [ctypes.c_void_p, ctypes.c_size_t, ctypes.c_void_p,
                                                      ctypes.c_int, ctypes.c_int, ctypes.c_int, ctypes.c_int]
            lib.weft_hip_probe_read_shape.restype = None
            lib.weft_hip_probe_write_shape.argtypes = [ctypes.c_void_p, ctypes.c_size_t, ctypes.c_int, ctypes.c_int,
                                                       ctypes.c_int, ctypes.c_int]
            lib.weft_hip_probe_write_shape.restype = None
            lib.weft_hip_probe_mfma.argtypes = [ctypes.c_int, ctypes.c_int, ctypes.c_int, ctypes.c_void_p]
            lib.weft_hip_probe_mfma.restype = None
            _bind_ggml(lib)
            artifact = json.loads(lib.weft_hip_artifact())
            for kernel in artifact["kernels"]:
                fn = getattr(lib, kernel["symbol"])
                fn.argtypes = ([ctypes.c_void_p] * len(kernel["arguments"]) +
                               [ctypes.c_size_t] * len(kernel["shape_parameters"]))
                fn.restype = None
                # artifact-phase functions of a derived weight layout
                # (lib/Target/Emission/Emitter.h:231-272)
                if hasattr(lib, kernel["symbol"] + "_W_pack"):
                    size = getattr(lib, kernel["symbol"] + "_W_packed_size")
                    size.argtypes = [ctypes.c_size_t, ctypes.c_size_t]
                    size.restype = ctypes.c_size_t
                    pack = getattr(lib, kernel["symbol"] + "_W_pack")
                    pack.argtypes = [ctypes.c_void_p, ctypes.c_void_p, ctypes.c_size_t, ctypes.c_size_t]
                    pack.restype = None
            _artifact = artifact
            _lib = lib
        return _lib


def _bind_ggml(lib: ctypes.CDLL) -> None:
    """Types of the GGML MUL_MAT boundary (weft_ggml_*)."""
    i32, i64, sz, vp = ctypes.c_int32, ctypes.c_int64, ctypes.c_size_t, ctypes.c_void_p
    for name, args, res in (("weft_ggml_type_size", [i32], sz), ("weft_ggml_blck_size", [i32], i64),
                            ("weft_ggml_row_size", [i32, i64], sz),
                            ("weft_ggml_vec_dot_type", [i32], i32),
                            ("weft_ggml_mul_mat_work_size", [vp, vp], sz),
                            ("weft_ggml_mul_mat", [vp, vp, vp, vp, sz], ctypes.c_int),
                            ("weft_ggml_mul_mat_id_work_size", [vp, vp, vp], sz),
                            ("weft_ggml_mul_mat_id", [vp, vp, vp, vp, vp, sz], ctypes.c_int),
                            ("weft_ggml_mul_mat_id_noalloc", [vp, vp, vp, vp], ctypes.c_int)):
        fn = getattr(lib, name)
        fn.argtypes, fn.restype = args, res


def artifact() -> dict:
    load()
    assert _artifact is not None
    return _artifact


def kernel_metadata(symbol: str) -> dict:
    for kernel in artifact()["kernels"]:
        if kernel["symbol"] == symbol:
            return kernel
    raise KeyError(symbol)


class HipError(RuntimeError):
    def __init__(self, code: int, where: str) -> None:
        self.code = code
        msg = load().weft_hip_error_string(code).decode()
        super().__init__(f"{where}: hip error {code} ({msg})")


def check(where: str) -> None:
    """Raise the calling thread's recorded launch error, if any."""
    code = load().weft_hip_get_last_error()
    if code != 0:
        raise HipError(code, where)


def set_stream(handle: int | None) -> None:
    load().weft_hip_set_stream(ctypes.c_void_p(handle or 0))


def synchronize() -> None:
    code = load().weft_hip_synchronize()
    if code != 0:
        load().weft_hip_get_last_error()
        raise HipError(code, "synchronize")


def launch_log() -> list[str]:
    """Kernels this thread launched through the library since the last read.
    The library keeps the log only once a thread asks for it, so the first
    call turns it on for this thread (and returns what is there: nothing)."""
    lib = load()
    lib.weft_hip_set_launch_log(1)
    n = lib.weft_hip_launch_log(None, 0)
    buf = ctypes.create_string_buffer(n + 1)
    lib.weft_hip_launch_log(buf, n + 1)
    return [k for k in buf.value.decode().split(",") if k]
