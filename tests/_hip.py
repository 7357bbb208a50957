"""GPU test harness: device buffers from torch, calls through the C ABI.

Every call goes through ``libweft_hip``'s exported symbol (ctypes) with raw
device pointers and size_t shapes, exactly as a C caller of the reference's
generated kernels would; torch only allocates and copies device memory.
"""
from __future__ import annotations

import ctypes

import numpy as np

import oracle as o


class Harness:
    def __init__(self) -> None:
        import torch
        from weft_amd import _lib

        if not torch.cuda.is_available():
            raise RuntimeError("no HIP device")
        self.torch = torch
        self.dev = torch.device("cuda:0")
        self.lib = _lib.load()
        self._lib = _lib
        _lib.set_stream(torch.cuda.current_stream().cuda_stream)
        self.grid_i8x8 = self.to_dev(o.iq2xxs_grid().view(np.int8))
        self.grid_xs_i8x8 = self.to_dev(o.iq2xs_grid().view(np.int8))
        self.signs_i8x8 = self.to_dev(o.signs_i8x8())
        self.codebook = self.to_dev(o.kvalues_mxfp4())
        self.scale = self.to_dev(o.e8m0_half_table())
        self.ue4m3 = self.to_dev(o.ue4m3_table())

    # ------------------------------------------------------------ memory
    def to_dev(self, a: np.ndarray, offset: int = 0):
        """Copy a numpy array to the GPU; ``offset`` bytes of slack in front
        give a deliberately misaligned base pointer (see ptr())."""
        a = np.ascontiguousarray(a)
        raw = np.zeros(a.nbytes + offset + 256, np.uint8)
        raw[offset:offset + a.nbytes] = a.view(np.uint8).reshape(-1)
        t = self.torch.from_numpy(raw).to(self.dev)
        return _DevBuf(t, offset, a.nbytes, a.dtype, a.shape)

    def empty(self, nbytes: int, fill: int = 0, offset: int = 0):
        raw = np.full(nbytes + offset + 256, fill, np.uint8)
        t = self.torch.from_numpy(raw).to(self.dev)
        return _DevBuf(t, offset, nbytes, np.uint8, (nbytes,))

    # -------------------------------------------------------------- calls
    def call(self, symbol: str, *args) -> None:
        fn = getattr(self.lib, symbol)
        conv = [a.ptr if isinstance(a, _DevBuf) else a for a in args]
        fn(*conv)
        self.torch.cuda.synchronize()
        self._lib.check(symbol)

    def last_error(self) -> int:
        return self.lib.weft_hip_get_last_error()


class _DevBuf:
    def __init__(self, t, offset, nbytes, dtype, shape):
        self.t = t
        self.offset = offset
        self.nbytes = nbytes
        self.dtype = np.dtype(dtype)
        self.shape = shape

    @property
    def ptr(self) -> int:
        return self.t.data_ptr() + self.offset

    def numpy(self, dtype=None, shape=None) -> np.ndarray:
        raw = self.t.cpu().numpy()[self.offset:self.offset + self.nbytes]
        dt = np.dtype(dtype) if dtype is not None else self.dtype
        arr = raw.view(dt)
        return arr.reshape(shape if shape is not None else (-1,) if dtype else self.shape)
