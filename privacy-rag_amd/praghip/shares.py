"""Party-local share operations over Z_2^64 / Z_2^59 (local_shares.hpp:22-32)."""
from __future__ import annotations

import math

from ._lib import check, lib, shape_error
from ._util import dev_ptr, stream_handle, u64_dtypes


def share_gemm(x, w, y=None, shifts=None, mask_bits: int = 64, stream=None):
    """y[m][n] = ((sum_k x[m][k] * w[n][k]) << shifts[n]) mod 2^mask_bits.

    x: GPU u64 [M][K] shares; w: GPU int8 or int32 [N][K] (the reference's
    [out][in] order; int32 values must lie in [-0x808080, 0x7F7F7F], which holds
    the reference f12 domain |w| <= 2^20), or int8 [3][N][K]: such int32
    weights pre-split into signed-byte planes (split_weights,
    MappedWeights.upload_split), the fast form of static weights; shifts:
    GPU int8 [N] or None.  The loop of bfv_matrix.inc:101-105 with
    mask_bits=59 is the reference ring.
    """
    import torch
    m, k = x.shape
    if w.dim() == 3:
        if w.dtype != torch.int8 or w.shape[0] != 3:
            raise TypeError("pre-split weights must be int8 [3][N][K]")
        n, k2 = w.shape[1:]
        w_bits = 24
    else:
        n, k2 = w.shape
        if w.dtype == torch.int8:
            w_bits = 8
        elif w.dtype == torch.int32:
            w_bits = 32
        else:
            raise TypeError("weights must be int8 or int32")
    if k != k2:
        raise ValueError("inner dimensions differ")
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


def share_gemm_valu(x, w, y=None, shifts=None, mask_bits: int = 64, stream=None):
    """share_gemm with int8 weights on VALU dot products instead of the matrix
    cores (the measured alternative to the MFMA kernels); same results."""
    import torch
    m, k = x.shape
    n, k2 = w.shape
    if k != k2 or w.dtype != torch.int8:
        raise ValueError("int8 weights [N][K] expected")
    if y is None:
        y = torch.empty((m, n), dtype=torch.int64, device=x.device)
    sp = None if shifts is None else dev_ptr(shifts, (torch.int8,))
    check(lib().praghip_share_gemm_valu(x.device.index or 0, dev_ptr(x, u64_dtypes()), dev_ptr(w), sp,
                                        dev_ptr(y, u64_dtypes()), m, k, n, mask_bits, stream_handle(stream)))
    return y


def split_weights(w, out=None, stream=None):
    """int32 [N][K] weights in [-0x808080, 0x7F7F7F] on the GPU -> int8
    [3][N][K] signed-byte planes (w = sum_e plane_e 256^e), the w_bits 24
    form of share_gemm."""
    import torch
    if w.dtype != torch.int32 or w.dim() != 2:
        raise TypeError("weights must be int32 [N][K]")
    n, k = w.shape
    if out is None:
        out = torch.empty((3, n, k), dtype=torch.int8, device=w.device)
    if tuple(out.shape) != (3, n, k) or out.dtype != torch.int8:
        raise shape_error("E_SHARE_SHAPE")
    check(lib().praghip_weights_split(w.device.index or 0, dev_ptr(w), dev_ptr(out), n * k, stream_handle(stream)))
    return out


RING_BITS = 59
RING_MASK = (1 << RING_BITS) - 1


def _dev(t):
    return t.device.index or 0


def _out_like(out, shape, like):
    import torch
    if out is None:
        return torch.empty(shape, dtype=torch.int64, device=like.device)
    if out.numel() != math.prod(shape):
        raise shape_error("E_CUDA_SHAPE")
    return out


def ring_add(a, b, out=None, mask_bits: int = RING_BITS, stream=None):
    """(a + b) mod 2^mask_bits on the GPU (local_shares.cu add_kernel)."""
    if a.numel() != b.numel() or a.numel() == 0:
        raise shape_error("E_CUDA_SHAPE")
    out = _out_like(out, tuple(a.shape), a)
    check(lib().praghip_ring_add(_dev(a), dev_ptr(a, u64_dtypes()), dev_ptr(b, u64_dtypes()),
                                 dev_ptr(out, u64_dtypes()), a.numel(), mask_bits, stream_handle(stream)))
    return out


def ring_scale(a, factor: int, out=None, mask_bits: int = RING_BITS, stream=None):
    """(a * factor) mod 2^mask_bits on the GPU (local_shares.cu scale_kernel)."""
    if a.numel() == 0:
        raise shape_error("E_CUDA_SHAPE")
    out = _out_like(out, tuple(a.shape), a)
    check(lib().praghip_ring_scale(_dev(a), dev_ptr(a, u64_dtypes()), int(factor) & (2**64 - 1),
                                   dev_ptr(out, u64_dtypes()), a.numel(), mask_bits, stream_handle(stream)))
    return out


def ring_layout(a, index_map, out=None, stream=None):
    """out[i] = a[index_map[i]] on the GPU (local_shares.cu layout_kernel); index_map: GPU int64."""
    if a.numel() == 0 or index_map.numel() == 0:
        raise shape_error("E_CUDA_SHAPE")
    out = _out_like(out, (index_map.numel(),), a)
    check(lib().praghip_ring_layout(_dev(a), dev_ptr(a, u64_dtypes()), a.numel(), dev_ptr(index_map, u64_dtypes()),
                                    dev_ptr(out, u64_dtypes()), index_map.numel(), stream_handle(stream)))
    return out


def ring_sum_rows(a, columns: int, out=None, mask_bits: int = RING_BITS, stream=None):
    """Row sums of a viewed as [rows][columns], mod 2^mask_bits (local_shares.cu sum_kernel)."""
    if a.numel() == 0 or columns <= 0 or a.numel() % columns:
        raise shape_error("E_CUDA_SHAPE")
    rows = a.numel() // columns
    out = _out_like(out, (rows,), a)
    check(lib().praghip_ring_sum_rows(_dev(a), dev_ptr(a, u64_dtypes()), dev_ptr(out, u64_dtypes()), rows, columns,
                                      mask_bits, stream_handle(stream)))
    return out


def lift59(ring, q, log_n: int, width: int = 0, out=None, stream=None):
    """Centred lift of ring-2^59 words to residues [blocks][len(q)][2^log_n].

    width 0: ring is [blocks][2^log_n] (matrix.cu:23-26); width > 0: ring is
    [blocks][width], written in reverse order below `width` (resident.cu:23-30).
    """
    import numpy as np
    n = 1 << log_n
    per = width if width else n
    if ring.numel() == 0 or ring.numel() % per:
        raise shape_error("E_LIFT_SHAPE")
    blocks = ring.numel() // per
    qa = np.ascontiguousarray(q, dtype=np.uint64)
    out = _out_like(out, (blocks, len(qa), n), ring)
    check(lib().praghip_lift59(_dev(ring), dev_ptr(ring, u64_dtypes()), dev_ptr(out, u64_dtypes()), blocks, log_n,
                               width, qa.ctypes.data, len(qa), stream_handle(stream)))
    return out


def dyadic_mac(a, w, q, out=None, stream=None):
    """out[l] = sum_b a[b][l] * w[b][l % wl] mod q[l % P] (resident.cu accumulate, matrix.cu product).

    a: GPU [blocks][limbs][N], w: GPU [blocks][wl][N], residues below their prime.
    """
    import numpy as np
    blocks, limbs, n = a.shape
    wb, wl, wn = w.shape
    if wb != blocks or wn != n or n & (n - 1):
        raise shape_error("E_DYADIC_SHAPE")
    qa = np.ascontiguousarray(q, dtype=np.uint64)
    out = _out_like(out, (limbs, n), a)
    check(lib().praghip_dyadic_mac(_dev(a), dev_ptr(a, u64_dtypes()), dev_ptr(w, u64_dtypes()),
                                   dev_ptr(out, u64_dtypes()), blocks, limbs, n.bit_length() - 1, wl, qa.ctypes.data,
                                   len(qa), stream_handle(stream)))
    return out


def bfv_delta(q, t_bits: int = RING_BITS):
    """Delta_k = floor(Q/t) mod q_k and r = Q mod t for Q = prod(q), t = 2^t_bits
    (the constants bind_local_shares derives, resident/seal_adapter.cpp:43-53)."""
    Q = 1
    for x in q:
        Q *= int(x)
    t = 1 << t_bits
    return [(Q // t) % int(x) for x in q], Q % t


def local_dot_scale(shares, weights, q, delta=None, r=None, out=None, stream=None):
    """Party-local dot product + BFV Delta scaling (resident.cu:60-74).

    shares: GPU [slots][words] u64, weights: GPU [words] u64 ring words.
    Returns GPU [slots][len(q)]: Delta_k * m + floor((r m + 2^58) / 2^59) mod q_k,
    m = (shares . weights mod 2^64) & (2^59 - 1).
    """
    import numpy as np
    import torch
    slots, words = shares.shape
    if weights.numel() != words:
        raise shape_error("E_LOCAL_SHAPE")
    if delta is None or r is None:
        delta, r = bfv_delta(q)
    qa = np.ascontiguousarray(q, dtype=np.uint64)
    da = np.ascontiguousarray(delta, dtype=np.uint64)
    out = _out_like(out, (slots, len(qa)), shares)
    work = torch.empty(int(lib().praghip_local_dot_workspace_words(slots)), dtype=torch.int64, device=shares.device)
    check(lib().praghip_local_dot_scale(_dev(shares), dev_ptr(shares, u64_dtypes()), dev_ptr(weights, u64_dtypes()),
                                        words, slots, da.ctypes.data, int(r), qa.ctypes.data, len(qa),
                                        dev_ptr(out, u64_dtypes()), dev_ptr(work, u64_dtypes()),
                                        stream_handle(stream)))
    return out


def local_dot_scale_noalloc(shares, weights, q, delta, r, out, stream=None):
    """local_dot_scale through the allocation-free entry point: no workspace,
    no allocation in the call (``out`` is required).  At most 64 slots; calls
    that overlap on one device race on its static scratch."""
    import numpy as np
    slots, words = shares.shape
    if weights.numel() != words or out.numel() < slots * len(q):
        raise shape_error("E_LOCAL_SHAPE")
    qa = np.ascontiguousarray(q, dtype=np.uint64)
    da = np.ascontiguousarray(delta, dtype=np.uint64)
    check(lib().praghip_local_dot_scale_noalloc(_dev(shares), dev_ptr(shares, u64_dtypes()),
                                                dev_ptr(weights, u64_dtypes()), words, slots, da.ctypes.data, int(r),
                                                qa.ctypes.data, len(qa), dev_ptr(out, u64_dtypes()),
                                                stream_handle(stream)))
    return out


class ShareStorage:
    """prag::model::ShareStorage (local_shares.hpp:12-17) from
    LocalShares.allocate: device words of one participant's shares,
    zero-filled; write/read are synchronous; clear() wipes and frees."""

    def __init__(self, words: int, device: int = 0, on_clear=None):
        import ctypes
        h = ctypes.c_void_p()
        check(lib().praghip_storage_allocate(device, int(words), ctypes.byref(h)))
        self._h = h
        self.words = int(words)
        self._on_clear = on_clear

    def write(self, offset: int, words) -> None:
        import numpy as np
        a = np.ascontiguousarray(words, dtype=np.uint64)
        check(lib().praghip_storage_write(self._h, int(offset), a.ctypes.data if a.size else None, a.size))

    def read(self, offset: int, count: int):
        import numpy as np
        out = np.empty(int(count), dtype=np.uint64)
        check(lib().praghip_storage_read(self._h, int(offset), int(count), out.ctypes.data if count else None))
        return out

    @property
    def data_ptr(self) -> int:
        """Device address of word 0 (for the device-pointer entry points)."""
        import ctypes
        p, n = ctypes.c_void_p(), ctypes.c_size_t()
        check(lib().praghip_storage_data(self._h, ctypes.byref(p), ctypes.byref(n)))
        return int(p.value)

    def stats(self):
        import ctypes
        up, down = ctypes.c_uint64(), ctypes.c_uint64()
        check(lib().praghip_storage_stats(self._h, ctypes.byref(up), ctypes.byref(down)))
        return {"uploaded_bytes": up.value, "downloaded_bytes": down.value}

    def _released(self):
        cb, self._on_clear = getattr(self, "_on_clear", None), None
        if cb is not None:
            cb(self)

    def clear(self):
        """ShareStorage::clear: wipe with zeros, synchronise, free (idempotent)."""
        import ctypes
        from ._lib import Cleanup
        c = Cleanup()
        check(lib().praghip_storage_clear(self._h, ctypes.byref(c)))
        if c.closed:
            self._released()
        return c

    def __del__(self):
        h = getattr(self, "_h", None)
        if h:
            lib().praghip_storage_destroy(h)
            self._h = None
            self._released()


class LocalShares:
    """Host-vector mirror of prag::model::LocalShares (local_shares.hpp:22-32).

    Like the reference backend (local_shares.cu:28-31) each call uploads its
    operands, runs one kernel and downloads the result synchronously; words
    above the ring mask are rejected (E_CUDA_WORD), as are empty or mismatched
    shapes (E_CUDA_SHAPE) and out-of-range public maps (E_CUDA_PUBLIC_MAP).
    ``matmul`` adds the party-local share GEMM as a member.
    """

    def __init__(self, device: int = 0):
        import torch
        self.device = torch.device("cuda", device)
        self.kernels = self.uploaded_bytes = self.downloaded_bytes = 0
        self.live_bytes = self.peak_bytes = 0

    def _up(self, v):
        import numpy as np
        import torch
        a = np.ascontiguousarray(v, dtype=np.uint64)
        if a.size == 0:
            raise shape_error("E_CUDA_SHAPE")
        if int(a.max()) > RING_MASK:
            raise shape_error("E_CUDA_WORD")
        self.uploaded_bytes += a.nbytes
        return torch.from_numpy(a.view(np.int64).copy()).to(self.device)

    def _down(self, t):
        import numpy as np
        import torch
        torch.cuda.synchronize(self.device)
        a = t.cpu().numpy().view(np.uint64).copy()
        self.downloaded_bytes += a.nbytes
        self.kernels += 1
        return a

    def add(self, a, b):
        if len(a) != len(b):
            raise shape_error("E_CUDA_SHAPE")
        return self._down(ring_add(self._up(a), self._up(b)))

    def scale(self, a, public_factor: int):
        if int(public_factor) > RING_MASK or int(public_factor) < 0:
            raise shape_error("E_CUDA_SHAPE")
        return self._down(ring_scale(self._up(a), int(public_factor)))

    def layout(self, a, public_indices):
        import numpy as np
        import torch
        idx = np.ascontiguousarray(public_indices, dtype=np.uint64)
        if idx.size == 0 or len(a) == 0:
            raise shape_error("E_CUDA_SHAPE")
        if int(idx.max()) >= len(a):
            raise shape_error("E_CUDA_PUBLIC_MAP")
        x = self._up(a)
        m = torch.from_numpy(idx.view(np.int64).copy()).to(self.device)
        self.uploaded_bytes += idx.nbytes
        return self._down(ring_layout(x, m))

    def sum_rows(self, a, columns: int):
        if columns <= 0 or len(a) == 0 or len(a) % columns:
            raise shape_error("E_CUDA_SHAPE")
        return self._down(ring_sum_rows(self._up(a), columns))

    def matmul(self, x, w, rows: int, inner: int, out: int, mask_bits: int = RING_BITS):
        """Y[rows][out] = X[rows][inner] . W[out][inner]^T mod 2^mask_bits; W int32 f12 weights."""
        import numpy as np
        import torch
        wa = np.ascontiguousarray(w, dtype=np.int32).reshape(out, inner)
        xa = self._up(np.asarray(x).reshape(rows, inner))
        wt = torch.from_numpy(wa).to(self.device)
        self.uploaded_bytes += wa.nbytes
        return self._down(share_gemm(xa.view(rows, inner), wt, mask_bits=mask_bits)).reshape(rows, out)

    def allocate(self, words: int) -> ShareStorage:
        """LocalShares::allocate (local_shares.hpp:29, local_shares.cu:37): a
        zero-filled device ShareStorage of `words` words (E_CUDA_SHAPE for 0)."""
        st = ShareStorage(words, self.device.index or 0, on_clear=self._released)
        self.live_bytes += st.words * 8
        self.peak_bytes = max(self.peak_bytes, self.live_bytes)
        return st

    def _released(self, st):
        self.live_bytes -= st.words * 8

    def stats(self):
        """LocalShareStats (local_shares.hpp:18-21)."""
        return {"kernels": self.kernels, "uploaded_bytes": self.uploaded_bytes,
                "downloaded_bytes": self.downloaded_bytes, "live_bytes": self.live_bytes,
                "peak_bytes": self.peak_bytes}
