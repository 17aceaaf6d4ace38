"""Party-local share operations over Z_2^64 / Z_2^59 (local_shares.hpp:22-32)."""
from __future__ import annotations

from ._lib import check, lib, shape_error
from ._util import dev_ptr, stream_handle, u64_dtypes


def share_gemm(x, w, y=None, shifts=None, mask_bits: int = 64, stream=None):
    """y[m][n] = ((sum_k x[m][k] * w[n][k]) << shifts[n]) mod 2^mask_bits.

    x: GPU u64 [M][K] shares; w: GPU int8 or int32 [N][K] (the reference's
    [out][in] order; int32 values must lie in [-0x808080, 0x7F7F7F], which holds
    the reference f12 domain |w| <= 2^20); shifts: GPU int8 [N] or None.
    The loop of bfv_matrix.inc:101-105 with mask_bits=59 is the reference ring.
    """
    import torch
    m, k = x.shape
    n, k2 = w.shape
    if k != k2:
        raise ValueError("inner dimensions differ")
    if w.dtype == torch.int8:
        w_bits = 8
    elif w.dtype == torch.int32:
        w_bits = 32
    else:
        raise TypeError("weights must be int8 or int32")
    if y is None:
        y = torch.empty((m, n), dtype=torch.int64, device=x.device)
    if tuple(y.shape) != (m, n) or (shifts is not None and shifts.numel() != n):
        raise shape_error("E_SHARE_SHAPE")
    for t in (x, w, y) + (() if shifts is None else (shifts,)):
        if t.device != x.device:
            raise shape_error("E_SHARE_DEVICE")
    sp = None if shifts is None else dev_ptr(shifts, (torch.int8,))
    check(lib().praghip_share_gemm(x.device.index or 0, dev_ptr(x, u64_dtypes()), dev_ptr(w), w_bits, sp,
                                   dev_ptr(y, u64_dtypes()), m, k, n, mask_bits, stream_handle(stream)))
    return y
