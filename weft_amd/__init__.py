"""weft_amd: MI355X (gfx950) implementation of Weft's quantized mul_mat path.

``libweft_hip.so`` (built from ``csrc/`` by ``weft_amd.build``) exports the
reference's generated-kernel symbols behind Weft's C ABI; ``weft_amd.runtime``
mirrors ``weft.runtime`` (Buffer / CompileOptions / CompiledKernel / compile /
jit) on top of it for device buffers.
"""
from ._lib import LIB_PATH, LibraryMissing, artifact, kernel_metadata, load

__all__ = ["LIB_PATH", "LibraryMissing", "artifact", "kernel_metadata", "load"]
