"""Host logic of weft_amd.runtime, checked on the CPU.

Mirrors the reference runtime's failure modes (python/weft/runtime/
compiler.py:99-155): every invalid call is rejected before the library is
called, with the reference's exception type.  Device storage is simulated
with objects exposing __cuda_array_interface__ at fake addresses; nothing is
dereferenced, and a call that passes validation without a GPU surfaces the
library's launch error instead of falling back."""
from __future__ import annotations

import numpy as np
import pytest

from weft_amd import _lib, kernels as K
from weft_amd.diagnostics import DefinitionError, LanguageUseError
from weft_amd.runtime import Buffer, CompilationError, CompileOptions, HipTarget, Toolchain
from weft_amd.runtime.compiler import CompiledKernel, _Registry

TARGET = HipTarget("gfx950", 64, 64, 0)


class FakeDev:
    """Device storage descriptor (no memory behind it)."""

    def __init__(self, ptr, shape, typestr="|u1", readonly=False, device=0):
        self.__cuda_array_interface__ = {"shape": tuple(shape), "typestr": typestr,
                                         "data": (ptr, readonly), "version": 3, "strides": None}
        self.device_id = device


def compiled(name):
    return CompiledKernel(K.DEFINITIONS[name], dict(_lib.kernel_metadata(name)), TARGET, CompileOptions())


def q4k_decode_args(n=64, k=512, m=1, base=1 << 20):
    rb = k // 256 * 144
    W = Buffer(FakeDev(base, (n * rb,)), shape=(n, k), encoding="Q4_K")
    X = Buffer(FakeDev(base + (1 << 16), (m, k), "<f4"))
    Xq = Buffer(FakeDev(base + (2 << 16), (m * (k // 256) * 292,)), shape=(m, k), encoding="Q8_K")
    Y = Buffer(FakeDev(base + (3 << 16), (m, n), "<f4"))
    return W, X, Xq, Y


def test_valid_call_reaches_the_library_and_surfaces_its_error():
    fn = compiled("production_mul_mat_q4_k_decode")
    if _lib.load().weft_hip_device_count() > 0:
        pytest.skip("a HIP device is present: the fake pointers must not be launched")
    with pytest.raises(_lib.HipError):
        fn(*q4k_decode_args())


def test_wrong_encoding_is_a_type_error():
    W, X, Xq, Y = q4k_decode_args()
    W2 = Buffer(FakeDev(1 << 20, (64 * 288,)), shape=(64, 512), encoding="Q4_0")
    with pytest.raises(TypeError, match="requires Q4_K"):
        compiled("production_mul_mat_q4_k_decode")(W2, X, Xq, Y)


def test_rank_extent_records_storage_alignment_are_value_errors():
    fn = compiled("production_mul_mat_q4_k_decode")
    W, X, Xq, Y = q4k_decode_args()
    with pytest.raises(ValueError, match="rank"):
        fn(Buffer(FakeDev(1 << 20, (64 * 288,)), shape=(64 * 512,), encoding="Q4_K"), X, Xq, Y)
    with pytest.raises(ValueError, match="disagrees with extent"):
        fn(W, X, Xq, Buffer(FakeDev(5 << 20, (1, 63), "<f4")))
    with pytest.raises(ValueError, match="complete Encoding records"):
        fn(Buffer(FakeDev(1 << 20, (64 * 288,)), shape=(64, 500), encoding="Q4_K"), X, Xq, Y)
    with pytest.raises(ValueError, match="shorter"):
        fn(Buffer(FakeDev(1 << 20, (64 * 288 - 1,)), shape=(64, 512), encoding="Q4_K"), X, Xq, Y)
    with pytest.raises(ValueError, match="alignment"):
        fn(Buffer(FakeDev((1 << 20) + 1, (64 * 288,)), shape=(64, 512), encoding="Q4_K"), X, Xq, Y)


def test_read_only_output_is_a_type_error():
    W, X, Xq, _ = q4k_decode_args()
    Y = Buffer(FakeDev(9 << 20, (1, 64), "<f4", readonly=True))
    with pytest.raises(TypeError, match="writable"):
        compiled("production_mul_mat_q4_k_decode")(W, X, Xq, Y)


def test_alias_across_declared_groups_is_rejected():
    # Xq ("workspace") overlapping W (no group): rejected
    W, X, _, Y = q4k_decode_args()
    Xq = Buffer(FakeDev((1 << 20) + 144, (584,)), shape=(1, 512), encoding="Q8_K")
    with pytest.raises(ValueError, match="aliases W"):
        compiled("production_mul_mat_q4_k_decode")(W, X, Xq, Y)


def test_alias_inside_one_group_is_allowed():
    # W and X are both in alias set 0: overlap passes validation
    fn = compiled("production_mul_mat_q4_k_decode")
    W, _, Xq, Y = q4k_decode_args()
    X = Buffer(FakeDev(1 << 20, (1, 512), "<f4"))
    if _lib.load().weft_hip_device_count() > 0:
        pytest.skip("a HIP device is present")
    with pytest.raises(_lib.HipError):
        fn(W, X, Xq, Y)


def test_host_storage_is_rejected():
    W, X, Xq, _ = q4k_decode_args()
    with pytest.raises(TypeError, match="host memory"):
        compiled("production_mul_mat_q4_k_decode")(W, X, Xq, np.zeros((1, 64), np.float32))


def test_storage_on_another_device_is_rejected():
    W, X, Xq, _ = q4k_decode_args()
    Y = Buffer(FakeDev(9 << 20, (1, 64), "<f4", device=1))
    with pytest.raises(ValueError, match="device 1"):
        compiled("production_mul_mat_q4_k_decode")(W, X, Xq, Y)


def test_shape_keywords_are_checked():
    fn = compiled("production_mul_mat_q4_k_decode")
    with pytest.raises(ValueError, match="disagrees with extent N=65"):
        fn(*q4k_decode_args(), N=65)
    with pytest.raises(ValueError, match="unsigned index"):
        fn(*q4k_decode_args(), K=-1)


def test_closed_kernel_raises():
    fn = compiled("production_mul_mat_q4_k_decode")
    fn.close()
    with pytest.raises(RuntimeError, match="closed"):
        fn(*q4k_decode_args())


def test_definitions_match_library_and_cannot_be_called():
    for name, d in K.DEFINITIONS.items():
        assert tuple(a["name"] for a in _lib.kernel_metadata(name)["arguments"]) == d.parameters
    with pytest.raises(LanguageUseError):
        K.production_mul_mat_q4_k_decode(1, 2, 3, 4)
    with pytest.raises(DefinitionError):
        K.KernelDefinition("x", ("A",), "", {"B": "g"})


def test_compile_options_are_validated():
    with pytest.raises(ValueError):
        CompileOptions(meta={"NC": 0})
    comp = _Registry(Toolchain(), TARGET)
    with pytest.raises(CompilationError, match="RISC-V"):
        comp.resolve(K.production_mul_mat_q4_k_decode, CompileOptions(lmul_eighths=16))
    with pytest.raises(NotImplementedError):
        comp.resolve(K.production_mul_mat_q4_k_decode, CompileOptions(matrix_extension="ime"))
    a = comp.resolve(K.production_mul_mat_q4_k_decode, CompileOptions())
    assert comp.resolve(K.production_mul_mat_q4_k_decode, CompileOptions()) is a  # reuse
    assert dict(a.metadata["bindings"]) == {}


def _compiler():
    return _Registry(Toolchain(), TARGET)


def test_source_bindings_follow_the_reference_compiler():
    """A wl.auto extent needs a binding; other names are accepted and
    recorded sorted; the same bindings reuse one artifact and different ones
    specialize (lib/Target/ConvertWeftToRISCV.cpp:730-745, :944-954;
    examples/repro/weft/native_jit.py:43-50)."""
    comp = _compiler()
    staged = K.production_mul_mat_q4_k_staged
    assert staged.source_bindings == ("KC", "MC", "MR", "NC")
    with pytest.raises(CompilationError, match="'KC' requires one concrete --meta binding"):
        comp.resolve(staged, CompileOptions())
    with pytest.raises(CompilationError, match="'MR' requires"):
        comp.resolve(staged, CompileOptions(meta={"NC": 64, "KC": 512, "MC": 8}))
    # examples/kernels/mul_mat/tuning.json "mul-mat:k1 q4_k prefill"
    tuned = {"NC": 64, "KC": 512, "MC": 8, "MR": 2}
    a = comp.resolve(staged, CompileOptions(meta=tuned))
    assert list(a.metadata["bindings"].items()) == sorted(tuned.items())
    assert comp.resolve(staged, CompileOptions(meta=dict(tuned))) is a
    b = comp.resolve(staged, CompileOptions(meta={**tuned, "MR": 4}))
    assert b is not a and b.metadata["bindings"]["MR"] == 4
    # a kernel without auto extents records whatever it is given
    d = comp.resolve(K.production_mul_mat_q4_k_decode, CompileOptions(meta={"NC": 64}))
    assert dict(d.metadata["bindings"]) == {"NC": 64}
    assert d is not comp.resolve(K.production_mul_mat_q4_k_decode, CompileOptions())
    for name in ("production_mul_mat_q4_0", "production_mul_mat_mxfp4",
                 "production_mul_mat_iq2_xxs_staged"):
        with pytest.raises(CompilationError, match="requires one concrete"):
            comp.resolve(K.DEFINITIONS[name], CompileOptions())


def test_buffer_inference_and_contiguity():
    b = Buffer(np.zeros((3, 4), np.int8))
    assert (b.encoding, b.shape, b.device) == ("dense.i8", (3, 4), None)
    with pytest.raises(ValueError):
        Buffer(np.zeros((4, 4), np.float32)[:, ::2])
    with pytest.raises(TypeError):
        Buffer(FakeDev(1 << 20, (8,), "|V8"))
    with pytest.raises(ValueError):
        Buffer(np.zeros(4, np.uint8), shape=(-1,), encoding="Q4_0")


def test_interleaved_weights_need_whole_row_cohorts():
    fn = compiled("q4_k_q8_k_gemv")
    k = 512
    X = Buffer(FakeDev(2 << 20, (2 * 292,)), shape=(k,), encoding="Q8_K")
    Y = Buffer(FakeDev(3 << 20, (24,), "<f4"))
    W = Buffer(FakeDev(1 << 20, (24 * 288,)), shape=(24, k), encoding="Q4K_I[16]")
    with pytest.raises(ValueError, match="16-row cohorts"):
        fn(W, X, Y)
    # the layout identity is checked like any Encoding
    W = Buffer(FakeDev(1 << 20, (32 * 288,)), shape=(32, k), encoding="Q4_K")
    with pytest.raises(TypeError, match="requires Q4K_I"):
        fn(W, X, Buffer(FakeDev(3 << 20, (32,), "<f4")))
