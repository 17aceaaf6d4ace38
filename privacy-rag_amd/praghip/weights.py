"""The reference's quantized_f12 weight files (int32 .npy [out][in]) through the
C reader (artifacts.hpp:31-49 MappedWeights, quantize_weights.py:60-64)."""
from __future__ import annotations

import ctypes

import numpy as np

from ._lib import check, lib
from ._util import dev_ptr


class MappedWeights:
    """Read-only memory map of one int32 .npy tensor of an exact shape."""

    def __init__(self, path: str, rows: int, cols: int = 0, vector: bool = False):
        h = ctypes.c_void_p()
        check(lib().praghip_weights_open(str(path).encode(), rows, cols, 1 if vector else 0, ctypes.byref(h)))
        self._h = h
        r, c = ctypes.c_size_t(), ctypes.c_size_t()
        check(lib().praghip_weights_shape(h, ctypes.byref(r), ctypes.byref(c)))
        self.rows, self.cols = r.value, c.value

    def _handle(self):
        if self._h is None:
            raise ValueError("weights closed")
        return self._h

    def at(self, r: int, c: int = 0) -> int:
        """Ring word of element (r, c): sign-extended, & (2^59 - 1) (artifacts.hpp:86-92)."""
        v = ctypes.c_uint64()
        check(lib().praghip_weights_at(self._handle(), r, c, ctypes.byref(v)))
        return v.value

    def array(self) -> np.ndarray:
        """Copy of the int32 tensor [rows][cols]."""
        p = lib().praghip_weights_data(self._handle())
        buf = (ctypes.c_int32 * (self.rows * self.cols)).from_address(p)
        return np.frombuffer(buf, dtype=np.int32).reshape(self.rows, self.cols).copy()

    def max_abs(self) -> int:
        v = ctypes.c_uint64()
        check(lib().praghip_weights_max_abs(self._handle(), ctypes.byref(v)))
        return v.value

    def upload(self, dst, stream=None):
        """Copy into a GPU int32 tensor of rows * cols elements (share_gemm with int32 weights)."""
        import torch
        if dst.dtype != torch.int32 or dst.numel() != self.rows * self.cols:
            raise ValueError("E_NPY_SHAPE")
        s = None if stream is None else ctypes.c_void_p(stream.cuda_stream).value
        if s is None:
            s = ctypes.c_void_p(torch.cuda.current_stream(dst.device).cuda_stream).value
        check(lib().praghip_weights_upload(self._handle(), dst.device.index or 0, dev_ptr(dst), s))
        return dst

    def upload_split(self, dst, stream=None):
        """Split on the host into the three signed-byte planes and copy into a GPU
        int8 tensor [3][rows][cols] (share_gemm's pre-split form, w_bits 24)."""
        import torch
        if dst.dtype != torch.int8 or dst.numel() != 3 * self.rows * self.cols:
            raise ValueError("E_NPY_SHAPE")
        s = None if stream is None else ctypes.c_void_p(stream.cuda_stream).value
        if s is None:
            s = ctypes.c_void_p(torch.cuda.current_stream(dst.device).cuda_stream).value
        check(lib().praghip_weights_upload_split(self._handle(), dst.device.index or 0, dev_ptr(dst), s))
        return dst

    def close(self):
        if self._h is not None:
            lib().praghip_weights_close(self._h)
            self._h = None

    def __enter__(self):
        return self

    def __exit__(self, *exc):
        self.close()

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass
