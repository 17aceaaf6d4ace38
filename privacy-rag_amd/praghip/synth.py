"""Seeded synthetic inputs generated on the device (splitmix64 counter stream)."""
from __future__ import annotations

import numpy as np

from ._lib import check, lib, shape_error
from ._util import dev_ptr, host_ptr, stream_handle, u64_dtypes


def fill_residues(t, q, log_n: int, seed: int, stream=None):
    """t: GPU u64 [limbs][2^log_n]; limb l uniform mod q[l % len(q)]."""
    if t.numel() % (1 << log_n):
        raise shape_error("E_FILL_SHAPE")
    qa = np.asarray([int(x) for x in q], dtype=np.uint64)
    check(lib().praghip_fill_residues(t.device.index or 0, dev_ptr(t, u64_dtypes()), t.numel() >> log_n, log_n,
                                      host_ptr(qa), len(qa), seed, stream_handle(stream)))
    return t


def fill_u64(t, seed: int, stream=None):
    check(lib().praghip_fill_u64(t.device.index or 0, dev_ptr(t, u64_dtypes()), t.numel(), seed,
                                 stream_handle(stream)))
    return t


def fill_i8(t, seed: int, stream=None):
    import torch
    check(lib().praghip_fill_i8(t.device.index or 0, dev_ptr(t, (torch.int8,)), t.numel(), seed,
                                stream_handle(stream)))
    return t


def fill_shift(t, seed: int, stream=None):
    """Per-channel shifts in [0, 7] (int8)."""
    import torch
    check(lib().praghip_fill_shift(t.device.index or 0, dev_ptr(t, (torch.int8,)), t.numel(), seed,
                                   stream_handle(stream)))
    return t
