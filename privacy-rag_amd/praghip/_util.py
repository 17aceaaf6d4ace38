"""Pointer and stream hand-off helpers (torch tensors and numpy arrays)."""
from __future__ import annotations

import ctypes

import numpy as np


def host_u64(a) -> np.ndarray:
    a = np.ascontiguousarray(a)
    if a.dtype == np.int64:
        a = a.view(np.uint64)
    if a.dtype != np.uint64:
        a = np.ascontiguousarray(a, dtype=np.uint64)
    return a


def host_ptr(a: np.ndarray) -> int:
    return a.ctypes.data


def dev_ptr(t, dtypes=None) -> int:
    """Device address of a contiguous CUDA/HIP torch tensor."""
    import torch
    if not isinstance(t, torch.Tensor) or not t.is_cuda:
        raise TypeError("expected a torch tensor on the GPU")
    if not t.is_contiguous():
        raise ValueError("tensor must be contiguous")
    if dtypes is not None and t.dtype not in dtypes:
        raise TypeError(f"unexpected dtype {t.dtype}")
    return t.data_ptr()


def stream_handle(stream) -> int | None:
    """hipStream_t of a torch stream (None -> the caller's current stream)."""
    import torch
    if stream is None:
        stream = torch.cuda.current_stream()
    return ctypes.c_void_p(stream.cuda_stream).value


def u64_dtypes():
    import torch
    return (torch.int64, torch.uint64)
