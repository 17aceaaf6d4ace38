"""Switch: BFV keyswitch with Galois automorphism (switch.hpp:12-28, switch.cu:113-125)."""
from __future__ import annotations

import ctypes

import numpy as np

from ._lib import Cleanup, SwitchPhases, Timing, check, lib, shape_error
from ._util import dev_ptr, host_ptr, host_u64, stream_handle, u64_dtypes


class Switch:
    """Keyswitch plan over q = data primes + [special prime].

    ``key``: host [dnum][2][L+1][N] NTT-form switching key for ``element`` (or
    None when keys are passed per call).  dnum = L is the reference's one prime
    per digit; dnum < L uses fast base conversion.

    ``tables``: optional dict of the SEAL arrays ``Switch::initialize(q, f, r,
    ni, invp, keys)`` takes (switch.hpp:24, keyswitch/seal_adapter.cpp:24-41):
    ``fwd`` / ``inv`` [L+1][N][2], ``invn`` [L+1][2], ``invp`` [L][2]
    (inv_q_last_mod_q).  Each given array is checked against the one derived
    from q (E_NTT_CONTEXT on a mismatch).
    """

    def __init__(self, q, log_n: int, dnum: int, key=None, element: int = 1, max_batch: int = 1, device: int = 0,
                 tables=None):
        self.q = [int(x) for x in q]
        self.L = len(self.q) - 1
        self.log_n = log_n
        self.dnum = dnum
        self.element = element
        qa = np.asarray(self.q, dtype=np.uint64)
        k = None if key is None else host_u64(key)
        if k is not None and k.size != dnum * 2 * (self.L + 1) << log_n:
            raise shape_error("E_SWITCH_KEY_SHAPE")
        tables = tables or {}
        K, n = self.L + 1, 1 << log_n
        sizes = {"fwd": K * n * 2, "inv": K * n * 2, "invn": K * 2, "invp": self.L * 2}
        unknown = set(tables) - set(sizes)
        if unknown:
            raise ValueError(f"unknown table names {sorted(unknown)}")
        arrs = {}
        for name, size in sizes.items():
            t = tables.get(name)
            if t is None:
                continue
            arrs[name] = host_u64(t)
            if arrs[name].size != size:
                raise shape_error("E_NTT_CONTEXT")
        tp = [host_ptr(arrs[nm]) if nm in arrs else None for nm in ("fwd", "inv", "invn", "invp")]
        h = ctypes.c_void_p()
        check(lib().praghip_switch_plan_create(device, host_ptr(qa), self.L, log_n, dnum, *tp,
                                               None if k is None else host_ptr(k), element, max_batch,
                                               ctypes.byref(h)))
        self._h = h

    @property
    def key_words(self) -> int:
        return self.dnum * 2 * (self.L + 1) << self.log_n

    def apply(self, ct) -> np.ndarray:
        """Switch::apply on a host [2][L][N] coefficient-form ciphertext."""
        src = host_u64(ct)
        if src.size != (2 * self.L) << self.log_n:
            raise shape_error("E_SWITCH_SHAPE")
        out = np.empty_like(src)
        check(lib().praghip_switch_apply(self._h, host_ptr(src), host_ptr(out)))
        return out

    def evaluate(self, ct) -> np.ndarray:
        """Switch::evaluate (switch.cu:113-125): keyswitch only, on a host [2][L][N]
        ciphertext already permuted by the plan's element (the reference's
        apply permutes on the CPU first, keyswitch/seal_adapter.cpp:49-51)."""
        src = host_u64(ct)
        if src.size != (2 * self.L) << self.log_n:
            raise shape_error("E_SWITCH_SHAPE")
        out = np.empty_like(src)
        check(lib().praghip_switch_evaluate(self._h, host_ptr(src), host_ptr(out)))
        return out

    def keyswitch(self, ct, out, batch: int | None = None, keys=None, key_stride: int = 0, galois: int = 1,
                  stream=None):
        """Device [batch][2][L][N] -> [batch][2][L][N]; keys device tensor or None (plan key)."""
        ct_words = (2 * self.L) << self.log_n
        have = ct.numel() // ct_words
        batch = have if batch is None else batch
        if not 0 <= batch <= have or out.numel() < batch * ct_words:
            raise shape_error("E_SWITCH_SHAPE")
        if keys is not None and batch and keys.numel() < (batch - 1) * key_stride + self.key_words:
            raise shape_error("E_SWITCH_KEY_SHAPE")
        kp = None if keys is None else dev_ptr(keys, u64_dtypes())
        check(lib().praghip_keyswitch(self._h, dev_ptr(ct, u64_dtypes()), dev_ptr(out, u64_dtypes()), batch, kp,
                                      key_stride, galois, stream_handle(stream)))
        return out

    def sync(self) -> None:
        check(lib().praghip_switch_sync(self._h))

    def timing(self) -> Timing:
        t = Timing()
        check(lib().praghip_switch_timing(self._h, ctypes.byref(t)))
        return t

    def phase_timing(self) -> SwitchPhases:
        """Switch::timing (switch.hpp:10): phases of the last apply / evaluate."""
        t = SwitchPhases()
        check(lib().praghip_switch_phase_timing(self._h, ctypes.byref(t)))
        return t

    def close(self) -> Cleanup:
        c = Cleanup()
        check(lib().praghip_switch_close(self._h, ctypes.byref(c)))
        return c

    def __del__(self):
        h = getattr(self, "_h", None)
        if h:
            lib().praghip_switch_destroy(h)
            self._h = None
