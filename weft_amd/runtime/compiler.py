"""compile / jit / CompiledKernel for libweft_hip, with the semantics of the
reference's python/weft/runtime/compiler.py:36-254.

``CompiledKernel.__call__`` performs the reference's pre-call ABI checks in
the same order and with the same exception types (Encoding -> TypeError;
rank, extent, storage, alignment, alias -> ValueError; read-only output ->
TypeError; closed -> RuntimeError) and adds the device ones (host storage ->
TypeError, wrong device -> ValueError).  It then calls the exported symbol
through ctypes with raw device pointers and size_t shapes, raises any launch
error the library recorded, and by default synchronizes the stream so that
"returns => result visible" holds as for the reference's host C kernels.
"""
from __future__ import annotations

import ctypes
import math
import threading
from collections.abc import Mapping
from dataclasses import dataclass, field
from types import MappingProxyType

from weft_amd.kernels import KernelDefinition

from .buffer import Buffer
from .driver import CompilationError, HipTarget, Toolchain


def _interleave_rows(encoding: str) -> int:
    """Cohort size of a derived row-interleave encoding such as ``Q4K_I[16]``
    (examples/formats/ggml.py:286-290), 0 for any other encoding."""
    head, sep, tail = encoding.partition("_I[")
    if not sep or not head or not tail.endswith("]") or not tail[:-1].isdecimal():
        return 0
    return int(tail[:-1])


def _freeze(value):
    if isinstance(value, dict):
        return MappingProxyType({key: _freeze(item) for key, item in value.items()})
    if isinstance(value, list):
        return tuple(_freeze(item) for item in value)
    return value


_RVV_DEFAULTS = {"lmul_eighths": 8, "unroll": 1, "pipeline_depth": 1, "scalar_load_prime": 0,
                 "partial_combine_policy": "independent-multilevel",
                 "record_axis_policy": "within-record", "max_widening_combine_groups": 2}


@dataclass(frozen=True)
class CompileOptions:
    """The reference's CompileOptions (compiler.py:36-67).  ``meta`` holds
    source bindings; the RISC-V physical bindings are kept for drop-in
    compatibility and must stay at their defaults on gfx950."""

    meta: Mapping[str, int] = field(default_factory=dict)
    lmul_eighths: int = 8
    unroll: int = 1
    pipeline_depth: int = 1
    scalar_load_prime: int = 0
    partial_combine_policy: str = "independent-multilevel"
    record_axis_policy: str = "within-record"
    max_widening_combine_groups: int = 2
    matrix_extension: str = "none"

    def __post_init__(self) -> None:
        values = dict(self.meta)
        if any(not isinstance(name, str) or not name.isidentifier() or
               type(value) is not int or value <= 0 for name, value in values.items()):
            raise ValueError("source bindings must be named positive integers")
        object.__setattr__(self, "meta", MappingProxyType(values))

    def arguments(self) -> list[str]:
        return [f"--meta={name}={value}" for name, value in sorted(self.meta.items())]


class CompiledKernel:
    def __init__(self, definition: KernelDefinition, metadata: dict, target: HipTarget,
                 options: CompileOptions) -> None:
        from weft_amd import _lib

        if metadata["gfx_arch"] != target.gfx_arch:
            raise CompilationError("compiled artifact disagrees with its discovered target")
        # the artifact records the source bindings it was compiled with, sorted
        # by name (lib/Target/ConvertWeftToRISCV.cpp:944-954)
        metadata = dict(metadata, bindings=dict(sorted(options.meta.items())))
        self.metadata = _freeze(metadata)
        self.target = target
        self.options = options
        self.definition = definition
        self.synchronize = True
        self._lock = threading.RLock()
        self._signature = definition.signature
        self._lib = _lib
        self._function = getattr(_lib.load(), metadata["symbol"])
        self.closed = False

    def __call__(self, *args: object, **kwargs: object) -> None:
        with self._lock:
            if self.closed:
                raise RuntimeError("the compiled kernel has been closed")
            self.target.check_execution()
            dimensions = {}
            for name in self.metadata["shape_parameters"]:
                if name in kwargs and name not in self._signature.parameters:
                    value = kwargs.pop(name)
                    if type(value) is not int or not 0 <= value < 1 << self.target.xlen:
                        raise ValueError(f"shape parameter {name} must fit the target unsigned index ABI")
                    dimensions[name] = value
            bound = self._signature.bind(*args, **kwargs)
            bound.apply_defaults()
            buffers = []
            spans = []
            for parameter in self.metadata["arguments"]:
                value = bound.arguments[parameter["name"]]
                buffer = value if isinstance(value, Buffer) else Buffer(value)
                if buffer.encoding != parameter["encoding"]:
                    raise TypeError(
                        f"{parameter['name']} requires {parameter['encoding']}, got {buffer.encoding}")
                if len(buffer.shape) != len(parameter["shape"]):
                    raise ValueError(f"{parameter['name']} has the wrong logical rank")
                for spelling, extent in zip(parameter["shape"], buffer.shape):
                    if extent >= 1 << self.target.xlen:
                        raise ValueError(f"{parameter['name']} extent cannot be represented by the target ABI")
                    if spelling.isdecimal():
                        expected = int(spelling)
                    elif spelling in dimensions:
                        expected = dimensions[spelling]
                    else:
                        dimensions[spelling] = extent
                        expected = extent
                    if extent != expected:
                        raise ValueError(f"{parameter['name']} disagrees with extent {spelling}={expected}")
                elements = parameter["record_elements"]
                if buffer.shape and buffer.shape[-1] % elements:
                    raise ValueError(f"{parameter['name']} does not contain complete Encoding records")
                cohort = _interleave_rows(parameter["encoding"])
                if cohort and buffer.shape and buffer.shape[0] % cohort:
                    # the interleave builder needs whole row cohorts
                    # (doc/dsl/encoding-and-artifacts.md:209)
                    raise ValueError(f"{parameter['name']} rows are not whole {cohort}-row cohorts")
                required = math.prod(buffer.shape) // elements * parameter["storage_bytes"]
                if required > buffer.nbytes:
                    raise ValueError(f"{parameter['name']} storage is shorter than its logical View")
                if required and buffer.address % parameter["alignment"]:
                    raise ValueError(f"{parameter['name']} does not meet its Encoding alignment")
                if parameter["writable"] and buffer.readonly:
                    raise TypeError(f"{parameter['name']} requires writable storage")
                if required and buffer.device is None:
                    raise TypeError(f"{parameter['name']} is host memory; libweft_hip takes device storage")
                if required and buffer.device != self.target.device:
                    raise ValueError(f"{parameter['name']} lives on device {buffer.device}, "
                                     f"the kernel runs on device {self.target.device}")
                for other, begin, end, alias_set in spans:
                    if required and parameter["alias_set"] != alias_set and (
                            buffer.address < end and begin < buffer.address + required):
                        raise ValueError(f"{parameter['name']} aliases {other} across declared alias groups")
                if required:
                    spans.append((parameter["name"], buffer.address,
                                  buffer.address + required, parameter["alias_set"]))
                buffers.append(buffer)
            self._function(*(ctypes.c_void_p(buffer.address) for buffer in buffers),
                           *(dimensions[name] for name in self.metadata["shape_parameters"]))
            self._lib.check(self.metadata["symbol"])
            if self.synchronize:
                self._lib.synchronize()

    def close(self) -> None:
        with self._lock:
            if self.closed:
                return
            self.closed = True
            self._function = None


class _Compiler:
    def __init__(self, toolchain: Toolchain) -> None:
        self.toolchain = toolchain
        self.target = HipTarget.discover(toolchain)
        self._cache: dict[tuple, CompiledKernel] = {}
        self._lock = threading.RLock()

    def compile(self, definition: KernelDefinition, options: CompileOptions) -> CompiledKernel:
        from weft_amd import _lib

        if not isinstance(definition, KernelDefinition):
            raise TypeError("compile expects a weft_amd kernel definition")
        if options.matrix_extension != "none":
            raise NotImplementedError("native discovery does not expose vendor matrix capabilities")
        for name, default in _RVV_DEFAULTS.items():
            if getattr(options, name) != default:
                raise CompilationError(f"RISC-V physical binding {name} has no gfx950 meaning")
        # every wl.auto extent needs one concrete binding; other names are
        # accepted and recorded (lib/Target/ConvertWeftToRISCV.cpp:730-745).
        # The gfx950 kernels' tiles are fixed by their hand-written code, so
        # a binding selects an artifact identity, not a different tiling.
        for name in definition.source_bindings:
            if name not in options.meta:
                raise CompilationError(
                    f"source auto parameter '{name}' requires one concrete --meta binding")
        key = (definition, tuple(options.arguments()))
        with self._lock:
            self.target.check_execution()
            cached = self._cache.get(key)
            if cached is not None and not cached.closed:
                return cached
            try:
                metadata = _lib.kernel_metadata(definition.__name__)
            except KeyError:
                raise CompilationError(f"libweft_hip exports no kernel {definition.__name__}") from None
            names = [a["name"] for a in metadata["arguments"]]
            if tuple(names) != definition.parameters:
                raise CompilationError(f"{definition.__name__}: library ABI {names} disagrees with "
                                       f"the definition {list(definition.parameters)}")
            kernel = CompiledKernel(definition, dict(metadata), self.target, options)
            self._cache[key] = kernel
            return kernel


_compilers: dict[tuple, _Compiler] = {}
_compilers_lock = threading.RLock()


def compile(definition: KernelDefinition, *, options: CompileOptions | None = None,
            toolchain: Toolchain | None = None) -> CompiledKernel:
    selected = (Toolchain() if toolchain is None else toolchain).resolve()
    from .driver import _current_device

    identity = (selected, _current_device())
    with _compilers_lock:
        compiler = _compilers.get(identity)
        if compiler is None:
            compiler = _Compiler(selected)
            _compilers[identity] = compiler
    return compiler.compile(definition, CompileOptions() if options is None else options)


class JITKernel:
    def __init__(self, definition: KernelDefinition, options: CompileOptions,
                 toolchain: Toolchain) -> None:
        if not isinstance(definition, KernelDefinition):
            raise TypeError("jit expects a weft_amd kernel definition")
        self.definition = definition
        self.options = options
        self.toolchain = toolchain
        self.compiled: CompiledKernel | None = None
        self._lock = threading.RLock()

    def __call__(self, *args: object, **kwargs: object) -> None:
        with self._lock:
            if self.compiled is None:
                self.compiled = compile(self.definition, options=self.options, toolchain=self.toolchain)
            compiled = self.compiled
        compiled(*args, **kwargs)


def jit(definition: KernelDefinition, *, options: CompileOptions | None = None,
        toolchain: Toolchain | None = None) -> JITKernel:
    return JITKernel(definition, CompileOptions() if options is None else options,
                     Toolchain() if toolchain is None else toolchain)
