"""compile / jit / CompiledKernel over libweft_hip.

The drop-in surface is the reference's python/weft/runtime/compiler.py:36-254:
the names ``CompileOptions``, ``CompiledKernel``, ``compile``, ``JITKernel``
and ``jit``, their signatures, and the exception type and message each
pre-call check raises (Encoding -> TypeError; rank, extent, records, storage,
alignment, alias -> ValueError; read-only output -> TypeError; closed ->
RuntimeError; compile-time problems -> CompilationError).

The implementation is this library's own.  The kernels are prebuilt, so
"compiling" resolves a kernel definition to an exported symbol and turns the
symbol's ABI metadata (``weft_hip_artifact``) into an ``_AbiPlan``: one
``_Slot`` per pointer argument with its checks precomputed, plus the shape
parameters.  A call binds the Python arguments, lets every slot check its
Buffer against a shared table of extents and a table of claimed byte ranges,
launches through ctypes with device pointers and size_t shapes, raises any
error the library recorded, and by default synchronizes the library's stream
so that "returns => result visible" holds as for the reference's host C.
On top of the reference checks a slot rejects host storage (TypeError) and
storage on another device (ValueError).
"""
from __future__ import annotations

import ctypes
import functools
import math
import threading
from collections.abc import Mapping
from dataclasses import dataclass, field
from types import MappingProxyType

from weft_amd.kernels import KernelDefinition

from .buffer import Buffer
from .driver import CompilationError, HipTarget, Toolchain, _current_device


# --------------------------------------------------------------- metadata
@functools.singledispatch
def _immutable(value):
    """Read-only view of JSON-shaped metadata (dicts become mappings, lists
    tuples, scalars stay)."""
    return value


@_immutable.register(dict)
def _(value):
    return MappingProxyType({k: _immutable(v) for k, v in value.items()})


@_immutable.register(list)
def _(value):
    return tuple(_immutable(v) for v in value)


def _cohort_rows(encoding: str) -> int:
    """Rows per cohort of a row-interleaved derived encoding such as
    ``Q4K_I[16]`` (examples/formats/ggml.py:286-290); 0 for any other."""
    if not encoding.endswith("]") or "_I[" not in encoding:
        return 0
    base, _, count = encoding[:-1].partition("_I[")
    return int(count) if base and count.isdecimal() else 0


# ---------------------------------------------------------------- options
# RISC-V physical bindings of the reference compiler and their defaults; on
# gfx950 they must stay at the defaults (the hand-written kernels have no
# LMUL, unroll or prime to choose)
_PHYSICAL_DEFAULTS = MappingProxyType({
    "lmul_eighths": 8, "unroll": 1, "pipeline_depth": 1, "scalar_load_prime": 0,
    "partial_combine_policy": "independent-multilevel", "record_axis_policy": "within-record",
    "max_widening_combine_groups": 2,
})


@dataclass(frozen=True)
class CompileOptions:
    """Source bindings (``meta``: named positive integers) and the
    reference's physical bindings, field for field (compiler.py:36-67)."""

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
        bindings = {}
        for name, value in dict(self.meta).items():
            valid_name = isinstance(name, str) and name.isidentifier()
            valid_value = type(value) is int and value > 0
            if not (valid_name and valid_value):
                raise ValueError("source bindings must be named positive integers")
            bindings[name] = value
        object.__setattr__(self, "meta", MappingProxyType(bindings))

    def arguments(self) -> list[str]:
        """The bindings as compiler flags, sorted by name (the identity under
        which a compiled kernel is cached)."""
        return ["--meta=%s=%d" % item for item in sorted(self.meta.items())]


# ------------------------------------------------------------- call plan
class _Extents:
    """Shape symbols of one call: fixed by a keyword or by the first View
    that spells them, then checked against every later one."""

    def __init__(self, limit: int) -> None:
        self.limit = limit
        self.values: dict[str, int] = {}

    def fix(self, name: str, value: object) -> None:
        if type(value) is not int or value < 0 or value >= self.limit:
            raise ValueError(f"shape parameter {name} must fit the target unsigned index ABI")
        self.values[name] = value

    def unify(self, owner: str, spelling: str, extent: int) -> None:
        if extent >= self.limit:
            raise ValueError(f"{owner} extent cannot be represented by the target ABI")
        expected = int(spelling) if spelling.isdecimal() else self.values.setdefault(spelling, extent)
        if extent != expected:
            raise ValueError(f"{owner} disagrees with extent {spelling}={expected}")


class _Claims:
    """Byte ranges the call's Views occupy; two ranges of different alias
    sets must not overlap (the ABI's restrict rule, Emitter.h:483-488)."""

    def __init__(self) -> None:
        self.ranges: list[tuple[int, int, object, str]] = []

    def claim(self, owner: str, begin: int, end: int, alias_set: object) -> None:
        for lo, hi, group, name in self.ranges:
            if group != alias_set and begin < hi and lo < end:
                raise ValueError(f"{owner} aliases {name} across declared alias groups")
        self.ranges.append((begin, end, alias_set, owner))


@dataclass(frozen=True)
class _Slot:
    """One pointer argument of the ABI and the checks its Buffer passes."""

    name: str
    encoding: str
    shape: tuple[str, ...]
    record_elements: int
    storage_bytes: int
    alignment: int
    alias_set: object
    writable: bool
    cohort: int

    @classmethod
    def of(cls, argument: Mapping) -> "_Slot":
        return cls(argument["name"], argument["encoding"], tuple(argument["shape"]),
                   argument["record_elements"], argument["storage_bytes"], argument["alignment"],
                   argument["alias_set"], bool(argument["writable"]), _cohort_rows(argument["encoding"]))

    def admit(self, value: object, extents: _Extents, claims: _Claims, device: int) -> int:
        """Check one argument; returns its device address."""
        buf = value if isinstance(value, Buffer) else Buffer(value)
        who = self.name
        if buf.encoding != self.encoding:
            raise TypeError(f"{who} requires {self.encoding}, got {buf.encoding}")
        if len(buf.shape) != len(self.shape):
            raise ValueError(f"{who} has the wrong logical rank")
        for spelling, extent in zip(self.shape, buf.shape):
            extents.unify(who, spelling, extent)
        if buf.shape and buf.shape[-1] % self.record_elements != 0:
            raise ValueError(f"{who} does not contain complete Encoding records")
        if self.cohort and buf.shape and buf.shape[0] % self.cohort != 0:
            # the interleave builds whole row cohorts (doc/dsl/encoding-and-artifacts.md:209)
            raise ValueError(f"{who} rows are not whole {self.cohort}-row cohorts")
        nbytes = math.prod(buf.shape) // self.record_elements * self.storage_bytes
        if nbytes > buf.nbytes:
            raise ValueError(f"{who} storage is shorter than its logical View")
        if nbytes and buf.address % self.alignment != 0:
            raise ValueError(f"{who} does not meet its Encoding alignment")
        if self.writable and buf.readonly:
            raise TypeError(f"{who} requires writable storage")
        if nbytes == 0:
            return buf.address  # an empty View touches no memory
        if buf.device is None:
            raise TypeError(f"{who} is host memory; libweft_hip takes device storage")
        if buf.device != device:
            raise ValueError(f"{who} lives on device {buf.device}, the kernel runs on device {device}")
        claims.claim(who, buf.address, buf.address + nbytes, self.alias_set)
        return buf.address


class _AbiPlan:
    """The argument slots and shape parameters of one exported kernel."""

    def __init__(self, metadata: Mapping, definition: KernelDefinition, target: HipTarget) -> None:
        self.slots = tuple(_Slot.of(a) for a in metadata["arguments"])
        self.shape_parameters = tuple(metadata["shape_parameters"])
        self.signature = definition.signature
        self.target = target

    def bind(self, args: tuple, kwargs: dict) -> tuple[list[int], list[int]]:
        extents = _Extents(1 << self.target.xlen)
        # shape symbols that are not View parameters may come as keywords
        free = {k: kwargs.pop(k) for k in list(kwargs)
                if k in self.shape_parameters and k not in self.signature.parameters}
        for name in self.shape_parameters:
            if name in free:
                extents.fix(name, free[name])
        bound = self.signature.bind(*args, **kwargs)
        bound.apply_defaults()
        claims = _Claims()
        pointers = [slot.admit(bound.arguments[slot.name], extents, claims, self.target.device)
                    for slot in self.slots]
        return pointers, [extents.values[name] for name in self.shape_parameters]


# ---------------------------------------------------------------- kernels
class CompiledKernel:
    """One exported libweft_hip kernel bound to its ABI metadata.  Calling it
    checks the arguments (see _Slot.admit) and launches on the library's
    current stream; ``synchronize`` (default True) waits for the result."""

    def __init__(self, definition: KernelDefinition, metadata: dict, target: HipTarget,
                 options: CompileOptions) -> None:
        from weft_amd import _lib

        if metadata["gfx_arch"] != target.gfx_arch:
            raise CompilationError("compiled artifact disagrees with its discovered target")
        # the artifact records the source bindings it was built for, sorted by
        # name (lib/Target/ConvertWeftToRISCV.cpp:944-954), and which of them
        # no gfx950 launch takes (the library answers per name: NC / MR tile
        # the GEMVs, NC / MC the Q4_K GEMM; KC, NR and the rest are recorded
        # only)
        lib = _lib.load()
        inert = []
        for name in sorted(options.meta):
            if not lib.weft_hip_set_tile_binding(name.encode(), 1):
                inert.append(name)
        lib.weft_hip_clear_tile_bindings()
        self.metadata = _immutable(dict(metadata, bindings=dict(sorted(options.meta.items())),
                                        bindings_without_launch_knob=tuple(inert)))
        self.target = target
        self.options = options
        self.definition = definition
        self.synchronize = True
        self._plan = _AbiPlan(self.metadata, definition, target)
        self._lib = _lib
        self._entry = getattr(_lib.load(), self.metadata["symbol"])
        # the source bindings, set on the library's calling thread for each
        # call (weft_hip_set_tile_binding: NC / MR retile the GEMV launches,
        # NC / MC the Q4_K GEMM's tiles)
        self._tiles = tuple((name.encode(), value) for name, value in self.metadata["bindings"].items())
        self._lock = threading.RLock()

    @property
    def closed(self) -> bool:
        return self._entry is None

    def __call__(self, *args: object, **kwargs: object) -> None:
        with self._lock:
            if self._entry is None:
                raise RuntimeError("the compiled kernel has been closed")
            self.target.check_execution()
            pointers, shapes = self._plan.bind(args, dict(kwargs))
            lib = self._lib.load()
            for name, value in self._tiles:
                lib.weft_hip_set_tile_binding(name, value)
            try:
                self._entry(*map(ctypes.c_void_p, pointers), *shapes)
            finally:
                lib.weft_hip_clear_tile_bindings()
            self._lib.check(self.metadata["symbol"])
            if self.synchronize:
                self._lib.synchronize()

    def close(self) -> None:
        with self._lock:
            self._entry = None


class _Registry:
    """Compiled kernels of one (toolchain, device): a definition plus its
    bindings resolves once and is reused while open (native_jit.py:43-48)."""

    def __init__(self, toolchain: Toolchain, target: HipTarget | None = None) -> None:
        self.toolchain = toolchain
        self.target = target if target is not None else HipTarget.discover(toolchain)
        self._kernels: dict[tuple, CompiledKernel] = {}
        self._lock = threading.RLock()

    def _check_options(self, definition: KernelDefinition, options: CompileOptions) -> None:
        if options.matrix_extension != "none":
            raise NotImplementedError("native discovery does not expose vendor matrix capabilities")
        for name, default in _PHYSICAL_DEFAULTS.items():
            if getattr(options, name) != default:
                raise CompilationError(f"RISC-V physical binding {name} has no gfx950 meaning")
        # every wl.auto extent needs one concrete binding; other names are
        # recorded (lib/Target/ConvertWeftToRISCV.cpp:730-745).  On gfx950
        # NC (weight rows per workgroup) and MR (activation rows per pass)
        # retile the GEMV launches, NC and MC the Q4_K GEMM's tile; the other
        # MFMA GEMMs keep their 64 x 128 tile.
        missing = [name for name in definition.source_bindings if name not in options.meta]
        if missing:
            raise CompilationError(f"source auto parameter '{missing[0]}' requires one concrete --meta binding")

    def resolve(self, definition: KernelDefinition, options: CompileOptions) -> CompiledKernel:
        from weft_amd import _lib

        if not isinstance(definition, KernelDefinition):
            raise TypeError("compile expects a weft_amd kernel definition")
        self._check_options(definition, options)
        key = (definition, tuple(options.arguments()))
        with self._lock:
            self.target.check_execution()
            kernel = self._kernels.get(key)
            if kernel is not None and not kernel.closed:
                return kernel
            try:
                metadata = dict(_lib.kernel_metadata(definition.__name__))
            except KeyError:
                raise CompilationError(f"libweft_hip exports no kernel {definition.__name__}") from None
            exported = tuple(a["name"] for a in metadata["arguments"])
            if exported != definition.parameters:
                raise CompilationError(f"{definition.__name__}: library ABI {list(exported)} disagrees with "
                                       f"the definition {list(definition.parameters)}")
            kernel = self._kernels[key] = CompiledKernel(definition, metadata, self.target, options)
            return kernel


_registries: dict[tuple, _Registry] = {}
_registries_lock = threading.RLock()


def _registry(toolchain: Toolchain | None) -> _Registry:
    chosen = (toolchain or Toolchain()).resolve()
    identity = (chosen, _current_device())
    with _registries_lock:
        if identity not in _registries:
            _registries[identity] = _Registry(chosen)
        return _registries[identity]


def compile(definition: KernelDefinition, *, options: CompileOptions | None = None,
            toolchain: Toolchain | None = None) -> CompiledKernel:
    return _registry(toolchain).resolve(definition, options or CompileOptions())


class JITKernel:
    """A definition compiled on its first call (then reused)."""

    def __init__(self, definition: KernelDefinition, options: CompileOptions,
                 toolchain: Toolchain) -> None:
        if not isinstance(definition, KernelDefinition):
            raise TypeError("jit expects a weft_amd kernel definition")
        self.definition = definition
        self.options = options
        self.toolchain = toolchain
        self.compiled: CompiledKernel | None = None
        self._lock = threading.RLock()

    def _kernel(self) -> CompiledKernel:
        with self._lock:
            if self.compiled is None:
                self.compiled = compile(self.definition, options=self.options, toolchain=self.toolchain)
            return self.compiled

    def __call__(self, *args: object, **kwargs: object) -> None:
        self._kernel()(*args, **kwargs)


def jit(definition: KernelDefinition, *, options: CompileOptions | None = None,
        toolchain: Toolchain | None = None) -> JITKernel:
    return JITKernel(definition, options or CompileOptions(), toolchain or Toolchain())
