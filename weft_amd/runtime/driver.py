"""Toolchain and execution target (the reference's
python/weft/runtime/driver.py:17-85) for the HIP library.

The reference discovers a RISC-V host through ``weft-compile
--query-native-target`` and compiles each kernel with the system C compiler.
Here the kernels are prebuilt into libweft_hip; the "toolchain" is that
library and discovery asks it for the visible HIP devices.
"""
from __future__ import annotations

import ctypes
import os
import sys
from dataclasses import dataclass
from pathlib import Path

from weft_amd.diagnostics import WeftError


class CompilationError(WeftError):
    pass


@dataclass(frozen=True)
class Toolchain:
    library: str = ""

    def resolve(self) -> "Toolchain":
        from weft_amd import _lib

        path = Path(self.library) if self.library else _lib.LIB_PATH
        if not path.exists():
            raise CompilationError(f"native toolchain is unavailable: {path} is not built")
        if path.resolve() != _lib.LIB_PATH.resolve():
            raise CompilationError("only the in-tree libweft_hip is supported")
        return Toolchain(str(path.resolve()))


@dataclass(frozen=True)
class HipTarget:
    gfx_arch: str
    wavefront_size: int
    xlen: int
    device: int

    @classmethod
    def discover(cls, toolchain: Toolchain) -> "HipTarget":
        from weft_amd import _lib

        lib = _lib.load()
        count = lib.weft_hip_device_count()
        if count <= 0:
            raise CompilationError("native discovery found no HIP device")
        device = _current_device()
        buf = ctypes.create_string_buffer(64)
        if lib.weft_hip_device_arch(device, buf, 64) != 0:
            raise CompilationError("native discovery could not read the device architecture")
        target = cls(buf.value.decode().split(":")[0], 64, ctypes.sizeof(ctypes.c_void_p) * 8, device)
        target.check_execution()
        return target

    def check_execution(self) -> None:
        if sys.platform != "linux" or sys.byteorder != "little":
            raise CompilationError("native execution requires little-endian Linux")
        if ctypes.sizeof(ctypes.c_void_p) * 8 != self.xlen:
            raise CompilationError("process pointer ABI disagrees with the compiled target")
        if self.gfx_arch != "gfx950":
            raise CompilationError(f"libweft_hip is built for gfx950, the device is {self.gfx_arch}")


def _current_device() -> int:
    env = os.environ.get("WEFT_HIP_DEVICE")
    if env is not None:
        return int(env)
    try:
        import torch

        if torch.cuda.is_available():
            return torch.cuda.current_device()
    except ImportError:
        pass
    return 0
