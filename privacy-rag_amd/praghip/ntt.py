"""NttBatch: batched negacyclic NTT/INTT over RNS primes (ntt.hpp:22-40, ntt.cu:99-199)."""
from __future__ import annotations

import ctypes

import numpy as np

from ._lib import Cleanup, Timing, check, lib, shape_error
from ._util import dev_ptr, host_ptr, host_u64, stream_handle, u64_dtypes


def ntt_tables(q: int, log_n: int):
    """SEAL NTTTables of one prime as exported by seal_tables.cpp:22-33:
    (forward [N][2], inverse [N][2], invn [2], psi)."""
    n = 1 << log_n
    fwd = np.zeros((n, 2), dtype=np.uint64)
    inv = np.zeros((n, 2), dtype=np.uint64)
    invn = np.zeros(2, dtype=np.uint64)
    psi = ctypes.c_uint64(0)
    check(lib().praghip_ntt_tables(q, log_n, host_ptr(fwd), host_ptr(inv), host_ptr(invn), ctypes.byref(psi)))
    return fwd, inv, invn, psi.value


class NttBatch:
    """Plan over a prime list; limb l of a [limbs][N] buffer uses prime l % len(q).

    forward: natural -> SEAL bit-reversed order; inverse: bit-reversed -> natural.
    ``batches`` sizes the plan's own buffer used by the host-array calls
    (``transform``/``client_phase``), whose arrays are [batches][primes][N].
    """

    def __init__(self, q, log_n: int, batches: int = 0, device: int = 0, tables=None):
        self.q = [int(x) for x in q]
        self.log_n = log_n
        self.batches = batches
        qa = np.asarray(self.q, dtype=np.uint64)
        f = i = n = None
        if tables is not None:
            f, i, n = (host_u64(x) for x in tables)
        h = ctypes.c_void_p()
        check(lib().praghip_ntt_plan_create(device, host_ptr(qa), len(self.q), log_n,
                                            None if f is None else host_ptr(f), None if i is None else host_ptr(i),
                                            None if n is None else host_ptr(n), batches, ctypes.byref(h)))
        self._h = h

    # device tensors, in place, asynchronous on `stream` (default: torch's current stream)
    def _limbs(self, data, limbs):
        have = data.numel() >> self.log_n
        if data.numel() != have << self.log_n or (limbs is not None and not 0 <= limbs <= have):
            raise shape_error("E_NTT_SHAPE")
        return have if limbs is None else limbs

    def forward(self, data, limbs: int | None = None, stream=None):
        limbs = self._limbs(data, limbs)
        check(lib().praghip_ntt_forward(self._h, dev_ptr(data, u64_dtypes()), limbs, stream_handle(stream)))
        return data

    def inverse(self, data, limbs: int | None = None, stream=None):
        limbs = self._limbs(data, limbs)
        check(lib().praghip_ntt_inverse(self._h, dev_ptr(data, u64_dtypes()), limbs, stream_handle(stream)))
        return data

    # host arrays [batches][primes][N], synchronous, canonical-input check (ntt.cu:145-168)
    @property
    def words(self) -> int:
        return self.batches * len(self.q) << self.log_n

    def transform(self, data, inverse: bool = False) -> np.ndarray:
        src = host_u64(data)
        if src.size != self.words or not self.words:
            raise shape_error("E_NTT_SHAPE")
        out = np.empty_like(src)
        check(lib().praghip_ntt_transform(self._h, host_ptr(src), host_ptr(out), int(inverse)))
        return out

    def bind_client_key(self, key) -> None:
        k = host_u64(key)
        if k.size != len(self.q) << self.log_n:
            raise shape_error("E_CLIENT_KEY_SHAPE")
        check(lib().praghip_ntt_bind_client_key(self._h, host_ptr(k)))

    def client_phase(self, data) -> np.ndarray:
        src = host_u64(data)
        if src.size != self.words or not self.words:
            raise shape_error("E_NTT_SHAPE")
        out = np.empty_like(src)
        check(lib().praghip_ntt_client_phase(self._h, host_ptr(src), host_ptr(out)))
        return out

    def sync(self) -> None:
        check(lib().praghip_ntt_sync(self._h))

    def timing(self) -> Timing:
        t = Timing()
        check(lib().praghip_ntt_timing(self._h, ctypes.byref(t)))
        return t

    def close(self) -> Cleanup:
        c = Cleanup()
        check(lib().praghip_ntt_close(self._h, ctypes.byref(c)))
        return c

    def __del__(self):
        h = getattr(self, "_h", None)
        if h:
            lib().praghip_ntt_destroy(h)
            self._h = None
