"""HE matrix product on resident ciphertexts: mirror of matrix_gpu::Matrix
(matrix.hpp:9-24, matrix.cu:48-81) over praghip_matrix_*."""
from __future__ import annotations

import ctypes
from collections import namedtuple

import numpy as np

from ._lib import Cleanup, MatrixPackingT, check, lib, shape_error
from ._util import dev_ptr, host_u64, stream_handle, u64_dtypes


MatrixPacking = namedtuple("MatrixPacking", "reduction columns returns inputs")


def matrix_packing(batch: int, inner: int, outputs: int, qk_reverse64: bool = False) -> MatrixPacking:
    """prag::matrix_packing / matrix_packing_qk_reverse64 (bfv_layout.hpp:8-27):
    the packing of a batch x inner x outputs matrix product that moves the
    fewest ciphertext bytes.  Raises E_MATRIX_SHAPE / E_QK_REVERSE64_SHAPE."""
    out = MatrixPackingT()
    check(lib().praghip_matrix_packing(batch, inner, outputs, int(bool(qk_reverse64)), ctypes.byref(out)))
    return MatrixPacking(int(out.reduction), int(out.columns), int(out.returns), int(out.inputs))


class Matrix:
    """`input`: [blocks][2][len(q)][2^log_n] ciphertexts in coefficient form
    (canonical), kept on the device in NTT form.  evaluate(ring) with ring
    [blocks][2^log_n] ring-2^59 words returns the coefficient-form product
    [2][len(q)][2^log_n]; evaluate_selective keeps only the target
    coefficients of c0 (1..512 strictly increasing indices)."""

    def __init__(self, q, log_n: int, input, device: int = 0):
        self.q = [int(x) for x in q]
        self.log_n = log_n
        a = host_u64(input)
        n = 1 << log_n
        if a.size % (2 * len(self.q) * n):
            raise ValueError("MATRIX_GPU_SHAPE")
        self.blocks = a.size // (2 * len(self.q) * n)
        qa = np.asarray(self.q, dtype=np.uint64)
        h = ctypes.c_void_p()
        check(lib().praghip_matrix_plan_create(device, qa.ctypes.data, len(self.q), log_n, a.ctypes.data, self.blocks,
                                               ctypes.byref(h)))
        self._h = h

    def _out(self):
        return np.empty((2, len(self.q), 1 << self.log_n), dtype=np.uint64)

    def evaluate(self, ring) -> np.ndarray:
        r = host_u64(ring)
        out = self._out()
        check(lib().praghip_matrix_evaluate(self._h, r.ctypes.data, out.ctypes.data, None, 0))
        return out

    def evaluate_selective(self, ring, targets) -> np.ndarray:
        r = host_u64(ring)
        t = np.ascontiguousarray(targets, dtype=np.uint64)
        out = self._out()
        check(lib().praghip_matrix_evaluate(self._h, r.ctypes.data, out.ctypes.data, t.ctypes.data, t.size))
        return out

    def evaluate_device(self, ring, out, stream=None):
        """ring: GPU [blocks][2^log_n] words below 2^59 (not checked); out: GPU [2][P][2^log_n]."""
        check(lib().praghip_matrix_evaluate_device(self._h, dev_ptr(ring, u64_dtypes()), dev_ptr(out, u64_dtypes()),
                                                   stream_handle(stream)))
        return out

    def reserve(self, groups: int):
        """Allocates the scratch of evaluate_device_batch for up to `groups` evaluations (once)."""
        check(lib().praghip_matrix_reserve(self._h, groups))

    def evaluate_device_batch(self, rings, out, targets=None, selected=None, stream=None):
        """rings: GPU [groups][blocks][2^log_n] words below 2^59 (not checked);
        out: GPU [groups][2][P][2^log_n].  With `targets` (host, 1..512
        strictly increasing coefficient indices) the selective form on the
        device: c0 zero outside the targets, and `selected` (GPU
        [groups][P][len(targets)] or None) receives the target coefficients of
        c0 (gather_c0, matrix.cu:41-44)."""
        n = 1 << self.log_n
        groups = rings.numel() // (self.blocks * n)
        if groups * self.blocks * n != rings.numel() or out.numel() != groups * 2 * len(self.q) * n:
            raise shape_error("MATRIX_GPU_SHAPE")
        if targets is None:
            check(lib().praghip_matrix_evaluate_device_batch(self._h, dev_ptr(rings, u64_dtypes()),
                                                             dev_ptr(out, u64_dtypes()), groups,
                                                             stream_handle(stream)))
            return out
        t = np.ascontiguousarray(targets, dtype=np.uint64)
        if selected is not None and selected.numel() != groups * len(self.q) * t.size:
            raise shape_error("MATRIX_GPU_SHAPE")
        sp = None if selected is None else dev_ptr(selected, u64_dtypes())
        check(lib().praghip_matrix_evaluate_device_batch_selective(self._h, dev_ptr(rings, u64_dtypes()),
                                                                   dev_ptr(out, u64_dtypes()), groups,
                                                                   t.ctypes.data, t.size, sp,
                                                                   stream_handle(stream)))
        return out

    def device_bytes(self) -> int:
        return int(lib().praghip_matrix_device_bytes(self._h))

    def close(self) -> Cleanup:
        c = Cleanup()
        check(lib().praghip_matrix_close(self._h, ctypes.byref(c)))
        return c

    def __del__(self):
        h = getattr(self, "_h", None)
        if h is not None:
            try:
                lib().praghip_matrix_destroy(h)
            except Exception:
                pass
            self._h = None


class PublicZero:
    """Mirror of prag::enc0_gpu::PublicZero (enc0.hpp:15-25): the public key
    pk [2][K][N] (NTT form, K = data primes + 1) stays on the device;
    evaluate(samples [3][K][N]) -> ModDown(INTT(NTT(u) * pk) + e) [2][K-1][N]."""

    def __init__(self, q, log_n: int, pk, device: int = 0):
        self.q = [int(x) for x in q]
        self.log_n = log_n
        a = host_u64(pk)
        qa = np.asarray(self.q, dtype=np.uint64)
        h = ctypes.c_void_p()
        check(lib().praghip_enc0_plan_create(device, qa.ctypes.data, len(self.q) - 1, log_n, a.ctypes.data,
                                             ctypes.byref(h)))
        self._h = h

    def evaluate(self, samples) -> np.ndarray:
        s = host_u64(samples)
        out = np.empty((2, len(self.q) - 1, 1 << self.log_n), dtype=np.uint64)
        check(lib().praghip_enc0_evaluate(self._h, s.ctypes.data, out.ctypes.data))
        return out

    def evaluate_device(self, samples, out, stream=None):
        check(lib().praghip_enc0_evaluate_device(self._h, dev_ptr(samples, u64_dtypes()), dev_ptr(out, u64_dtypes()),
                                                 stream_handle(stream)))
        return out

    def reserve(self, count: int):
        """Allocates the scratch of evaluate_device_batch for up to `count` encryptions (once)."""
        check(lib().praghip_enc0_reserve(self._h, count))

    def evaluate_device_batch(self, samples, out, stream=None):
        """samples: GPU [count][3][K][N] (not checked); out: GPU [count][2][K-1][N]."""
        K, n = len(self.q), 1 << self.log_n
        count = samples.numel() // (3 * K * n)
        if count * 3 * K * n != samples.numel() or out.numel() != count * 2 * (K - 1) * n:
            raise shape_error("E_SWITCH_SHAPE")
        check(lib().praghip_enc0_evaluate_device_batch(self._h, dev_ptr(samples, u64_dtypes()),
                                                       dev_ptr(out, u64_dtypes()), count, stream_handle(stream)))
        return out

    def close(self) -> Cleanup:
        c = Cleanup()
        check(lib().praghip_enc0_close(self._h, ctypes.byref(c)))
        return c

    def __del__(self):
        h = getattr(self, "_h", None)
        if h is not None:
            try:
                lib().praghip_enc0_destroy(h)
            except Exception:
                pass
            self._h = None
