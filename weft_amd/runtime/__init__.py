"""HIP-target runtime with the surface of the reference's weft.runtime
(python/weft/runtime/__init__.py): Buffer, CompileOptions, CompiledKernel,
compile, jit, Toolchain, CompilationError, plus HipTarget in the role of
NativeTarget."""
from .buffer import Buffer
from .compiler import CompiledKernel, CompileOptions, JITKernel, compile, jit
from .driver import CompilationError, HipTarget, Toolchain

__all__ = [
    "Buffer", "CompilationError", "CompiledKernel", "CompileOptions", "HipTarget", "JITKernel",
    "Toolchain", "compile", "jit",
]
