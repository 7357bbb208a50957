"""Borrowed storage with an explicit logical Encoding (the reference's
python/weft/runtime/buffer.py:33-63), extended to device memory.

A Buffer wraps, without copying:
  * a torch tensor (device or host),
  * any object exposing ``__cuda_array_interface__`` (device memory),
  * any object supporting the Python buffer protocol (host memory).
The kernel ABI needs contiguous storage; packed record encodings must be
named explicitly, dense ones are inferred from the element type.
"""
from __future__ import annotations

from collections.abc import Sequence

_TYPESTR = {
    "i1": "i8", "u1": "u8", "i2": "i16", "u2": "u16", "i4": "i32", "u4": "u32",
    "i8": "i64", "u8": "u64", "f2": "f16", "f4": "f32", "f8": "f64", "b1": "i1",
}
_BUFFER_FORMATS = {
    "b": "i8", "B": "u8", "h": "i16", "H": "u16", "i": "i32", "I": "u32",
    "q": "i64", "Q": "u64", "e": "f16", "f": "f32", "d": "f64", "?": "i1",
}


def _torch_info(t):
    import torch

    names = {torch.int8: "i8", torch.uint8: "u8", torch.int16: "i16", torch.int32: "i32",
             torch.int64: "i64", torch.float16: "f16", torch.float32: "f32", torch.float64: "f64",
             torch.bool: "i1"}
    if not t.is_contiguous():
        raise ValueError("the current kernel ABI requires contiguous Encoding storage")
    dense = names.get(t.dtype)
    device = t.device.index if t.device.type == "cuda" else None
    if t.device.type == "cuda" and device is None:
        device = torch.cuda.current_device()
    return (t.data_ptr(), t.numel() * t.element_size(), tuple(t.shape),
            None if dense is None else "dense." + dense, False, device)


def _cai_info(obj):
    cai = obj.__cuda_array_interface__
    shape = tuple(int(s) for s in cai["shape"])
    typestr = cai["typestr"]
    itemsize = int(typestr[2:])
    strides = cai.get("strides")
    if strides is not None:
        expect, acc = [], itemsize
        for extent in reversed(shape):
            expect.append(acc)
            acc *= extent
        if tuple(strides) != tuple(reversed(expect)):
            raise ValueError("the current kernel ABI requires contiguous Encoding storage")
    ptr, readonly = cai["data"]
    n = 1
    for s in shape:
        n *= s
    dense = _TYPESTR.get(typestr[1:])
    return (int(ptr), n * itemsize, shape, None if dense is None else "dense." + dense,
            bool(readonly), int(getattr(obj, "device_id", 0) or 0))


def _buffer_info(obj):
    view = memoryview(obj)
    if not view.c_contiguous:
        raise ValueError("the current kernel ABI requires contiguous Encoding storage")
    import ctypes

    spelling = view.format.lstrip("@=<")
    dense = None
    if spelling in ("l", "L") and view.itemsize in (4, 8):
        dense = ("i" if spelling == "l" else "u") + str(view.itemsize * 8)
    elif spelling in _BUFFER_FORMATS:
        dense = _BUFFER_FORMATS[spelling]
    buf = (ctypes.c_char * view.nbytes).from_buffer(view) if not view.readonly else None
    # read-only host storage: address through the buffer protocol
    address = ctypes.addressof(buf) if buf is not None else _readonly_address(view)
    return (address, view.nbytes, tuple(view.shape), None if dense is None else "dense." + dense,
            bool(view.readonly), None), (view, buf)


def _readonly_address(view):
    import ctypes

    class _PyBuffer(ctypes.Structure):
        _fields_ = [("buf", ctypes.c_void_p), ("obj", ctypes.c_void_p), ("len", ctypes.c_ssize_t),
                    ("itemsize", ctypes.c_ssize_t), ("readonly", ctypes.c_int), ("ndim", ctypes.c_int),
                    ("format", ctypes.c_char_p), ("shape", ctypes.c_void_p),
                    ("strides", ctypes.c_void_p), ("suboffsets", ctypes.c_void_p),
                    ("internal", ctypes.c_void_p)]

    get = ctypes.pythonapi.PyObject_GetBuffer
    get.argtypes = [ctypes.py_object, ctypes.POINTER(_PyBuffer), ctypes.c_int]
    rel = ctypes.pythonapi.PyBuffer_Release
    rel.argtypes = [ctypes.POINTER(_PyBuffer)]
    b = _PyBuffer()
    get(view, ctypes.byref(b), 0)
    try:
        return b.buf
    finally:
        rel(ctypes.byref(b))


class Buffer:
    """A borrowed contiguous storage object with an explicit logical Encoding.

    ``device`` is the HIP device index holding the storage, or None for host
    memory.  libweft_hip kernels take device storage only.
    """

    def __init__(self, data: object, *, shape: Sequence[int] | None = None,
                 encoding: str | None = None) -> None:
        keep = data
        if type(data).__module__.startswith("torch") and hasattr(data, "data_ptr"):
            info = _torch_info(data)
        elif hasattr(data, "__cuda_array_interface__"):
            info = _cai_info(data)
        else:
            info, keep = _buffer_info(data)
        address, nbytes, native_shape, dense, readonly, device = info
        if encoding is None:
            if dense is None:
                raise TypeError("buffer element type needs an explicit Encoding")
            encoding = dense
        if not isinstance(encoding, str) or not encoding:
            raise TypeError("buffer Encoding must be a non-empty layout identity")
        logical_shape = tuple(native_shape if shape is None else shape)
        if any(type(extent) is not int or extent < 0 for extent in logical_shape):
            raise ValueError("logical buffer extents must be non-negative integers")
        self._keep = keep
        self.shape = logical_shape
        self.encoding = encoding
        self.address = int(address or 0)
        self.nbytes = int(nbytes)
        self.readonly = bool(readonly)
        self.device = device

    def __repr__(self) -> str:
        where = "host" if self.device is None else f"hip:{self.device}"
        return f"Buffer({self.encoding}, shape={self.shape}, {self.nbytes} B on {where})"
