"""GGML MUL_MAT / MUL_MAT_ID boundary of libweft_hip from Python.

``Tensor`` is the part of ``struct ggml_tensor`` (ggml/include/ggml.h:667-692)
that MUL_MAT reads: type id, ``ne``, byte strides ``nb`` and a device data
pointer.  ``mul_mat`` runs GGML_OP_MUL_MAT with the semantics of
ggml_compute_forward_mul_mat (ggml-cpu/ggml-cpu.c:1245-1443) on the quantized
kernels; where GGML asserts, it raises ``HipError`` (the library launches
nothing).
"""
from __future__ import annotations

import ctypes
from collections.abc import Sequence

from . import _lib

# enum ggml_type (ggml/include/ggml.h:389-431), the types of this path
F32, Q4_0, Q8_0, Q4_K, Q5_K, Q6_K, Q8_K, IQ2_XXS, I32, MXFP4, NVFP4 = 0, 2, 8, 12, 13, 14, 15, 16, 26, 39, 40
Q4_1, Q8_1, IQ2_XS = 3, 9, 17


class Tensor(ctypes.Structure):
    _fields_ = [("type", ctypes.c_int32), ("ne", ctypes.c_int64 * 4),
                ("nb", ctypes.c_size_t * 4), ("data", ctypes.c_void_p)]


def type_size(t: int) -> int:
    return _lib.load().weft_ggml_type_size(t)


def blck_size(t: int) -> int:
    return _lib.load().weft_ggml_blck_size(t)


def row_size(t: int, ne: int) -> int:
    return _lib.load().weft_ggml_row_size(t, ne)


def vec_dot_type(t: int) -> int:
    return _lib.load().weft_ggml_vec_dot_type(t)


def tensor(t: int, ne: Sequence[int], data: int = 0, nb: Sequence[int] | None = None) -> Tensor:
    """A descriptor with GGML's default strides (ggml_new_tensor_impl:
    nb0 = type size, nb1 = nb0 * ne0 / block size, nb_i = nb_{i-1} * ne_{i-1})
    unless ``nb`` is given."""
    ne = list(ne) + [1] * (4 - len(ne))
    if nb is None:
        size = 4 if t == I32 else type_size(t)
        nb = [size, size * ne[0] if t == I32 else row_size(t, ne[0])]
        nb += [nb[1] * ne[1], nb[1] * ne[1] * ne[2]]
    return Tensor(t, (ctypes.c_int64 * 4)(*ne), (ctypes.c_size_t * 4)(*nb), data)


def mul_mat_work_size(src0: Tensor, src1: Tensor) -> int:
    return _lib.load().weft_ggml_mul_mat_work_size(ctypes.byref(src0), ctypes.byref(src1))


def mul_mat(src0: Tensor, src1: Tensor, dst: Tensor, wdata: int = 0, wsize: int = 0) -> None:
    """Enqueue dst = MUL_MAT(src0, src1) on the current stream."""
    lib = _lib.load()
    code = lib.weft_ggml_mul_mat(ctypes.byref(src0), ctypes.byref(src1), ctypes.byref(dst),
                                 ctypes.c_void_p(wdata), wsize)
    if code != 0:
        lib.weft_hip_get_last_error()  # the same error, recorded: clear it
        raise _lib.HipError(code, "weft_ggml_mul_mat")


def mul_mat_id_work_size(src0: Tensor, src1: Tensor, ids: Tensor) -> int:
    return _lib.load().weft_ggml_mul_mat_id_work_size(ctypes.byref(src0), ctypes.byref(src1),
                                                      ctypes.byref(ids))


def mul_mat_id(src0: Tensor, src1: Tensor, ids: Tensor, dst: Tensor, wdata: int = 0,
               wsize: int = 0) -> None:
    """Enqueue dst = MUL_MAT_ID(src0 experts, src1, ids) on the current stream."""
    lib = _lib.load()
    code = lib.weft_ggml_mul_mat_id(ctypes.byref(src0), ctypes.byref(src1), ctypes.byref(ids),
                                    ctypes.byref(dst), ctypes.c_void_p(wdata), wsize)
    if code != 0:
        lib.weft_hip_get_last_error()
        raise _lib.HipError(code, "weft_ggml_mul_mat_id")


# the library's per-device work buffer of mul_mat_id_noalloc (weft_hip.h)
NOALLOC_SCRATCH_BYTES = 32 << 20


def mul_mat_id_noalloc(src0: Tensor, src1: Tensor, ids: Tensor, dst: Tensor) -> None:
    """MUL_MAT_ID without a caller work buffer: the library's per-device
    scratch stands in for it (calls that overlap on one device race)."""
    lib = _lib.load()
    code = lib.weft_ggml_mul_mat_id_noalloc(ctypes.byref(src0), ctypes.byref(src1), ctypes.byref(ids),
                                            ctypes.byref(dst))
    if code != 0:
        lib.weft_hip_get_last_error()
        raise _lib.HipError(code, "weft_ggml_mul_mat_id_noalloc")

