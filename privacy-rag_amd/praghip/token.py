"""Token-resident path and acyclic packing tree: mirrors of
prag::experimental::resident::TokenWeights (resident.hpp:20-45) and
prag::experimental_full_switch::Packing (bfv_gpu_packing.hpp:10-45) over
praghip_token_* and praghip_pack_*."""
from __future__ import annotations

import ctypes
from dataclasses import dataclass

import numpy as np

from ._lib import Cleanup, Timing, TokenPhases, check, lib, shape_error
from ._util import dev_ptr, host_u64, stream_handle, u64_dtypes


@dataclass(frozen=True)
class DeviceCipherBatch:
    """A borrowed device view (resident.hpp:16-19): `data` is the device
    address of `words` u64 words, valid until the producer's next call."""
    data: int
    words: int
    owner: object


class TokenWeights:
    """`inputs` [blocks][slots][2][len(q)][2^log_n]: coefficient-form
    ciphertexts (the adapter's flat order, resident/seal_adapter.cpp:27-33),
    transformed to NTT form on the device.  The reference fixes 6 primes,
    19 blocks of width 8192 and at most 4 slots; here they are parameters."""

    def __init__(self, q, log_n: int, inputs, block_width: int, levels: int = 9, device: int = 0):
        self.q = [int(x) for x in q]
        self.log_n = log_n
        a = host_u64(inputs)
        if a.ndim != 5 or a.shape[2:] != (2, len(self.q), 1 << log_n):
            raise shape_error("E_GPU_TOKEN_CONTEXT_LAYOUT")
        self.blocks, self.slots = int(a.shape[0]), int(a.shape[1])
        self.block_width, self.levels = block_width, levels
        qa = np.asarray(self.q, dtype=np.uint64)
        h = ctypes.c_void_p()
        check(lib().praghip_token_plan_create(device, qa.ctypes.data, len(self.q), log_n, self.slots, self.blocks,
                                              block_width, levels, a.ctypes.data, ctypes.byref(h)))
        self._h = h

    @property
    def ct_words(self) -> int:
        return 2 * len(self.q) << self.log_n

    def _ring(self, ring):
        r = host_u64(ring)
        return r, r.size

    def evaluate(self, ring) -> np.ndarray:
        """[slots][2][P][N] NTT-form sum of products (resident.cu:135-151)."""
        r, n = self._ring(ring)
        out = np.empty((self.slots, 2, len(self.q), 1 << self.log_n), dtype=np.uint64)
        check(lib().praghip_token_evaluate(self._h, r.ctypes.data, n, out.ctypes.data))
        return out

    def bind_local_shares(self, shares):
        s = host_u64(shares)
        check(lib().praghip_token_bind_local_shares(self._h, s.ctypes.data, s.size))

    def _batch(self, view) -> DeviceCipherBatch:
        return DeviceCipherBatch(int(view.value), self.slots * self.ct_words, self)

    def evaluate_finished(self, ring, local) -> DeviceCipherBatch:
        r, n = self._ring(ring)
        m = host_u64(local)
        if m.size != self.slots:
            raise shape_error("E_GPU_TOKEN_CONTEXT_LAYOUT")
        v = ctypes.c_void_p()
        check(lib().praghip_token_evaluate_finished(self._h, r.ctypes.data, n, m.ctypes.data, ctypes.byref(v)))
        return self._batch(v)

    def evaluate_local_finished(self, ring) -> DeviceCipherBatch:
        r, n = self._ring(ring)
        v = ctypes.c_void_p()
        check(lib().praghip_token_evaluate_local_finished(self._h, r.ctypes.data, n, ctypes.byref(v)))
        return self._batch(v)

    def evaluate_device(self, ring, out, residues=None, stream=None):
        """ring: GPU [blocks][width]; residues: GPU [slots][P] or None (bound
        shares); out: GPU [slots][2][P][N]."""
        rp = None if residues is None else dev_ptr(residues, u64_dtypes())
        check(lib().praghip_token_evaluate_device(self._h, dev_ptr(ring, u64_dtypes()), rp,
                                                  dev_ptr(out, u64_dtypes()), stream_handle(stream)))
        return out

    def reserve(self, coords: int):
        """Allocates the scratch of evaluate_device_batch for up to `coords` columns (once)."""
        check(lib().praghip_token_reserve(self._h, coords))

    def evaluate_device_batch(self, rings, out, residues=None, stream=None):
        """rings: GPU [coords][blocks][width]; residues: GPU [coords][slots][P]
        or None (bound shares); out: GPU [coords][slots][2][P][N]."""
        coords = rings.numel() // (self.blocks * self.block_width)
        if coords * self.blocks * self.block_width != rings.numel() or out.numel() != coords * self.slots * self.ct_words:
            raise shape_error("E_RESIDENT_BATCH")
        rp = None if residues is None else dev_ptr(residues, u64_dtypes())
        check(lib().praghip_token_evaluate_device_batch(self._h, dev_ptr(rings, u64_dtypes()), rp,
                                                        dev_ptr(out, u64_dtypes()), coords, stream_handle(stream)))
        return out

    def slot_view(self, batch: DeviceCipherBatch, slot: int) -> DeviceCipherBatch:
        return DeviceCipherBatch(batch.data + slot * self.ct_words * 8, self.ct_words, batch.owner)

    def stack_store(self, slot: int, level: int, view, stream=None, ready=None):
        """view: a DeviceCipherBatch of one ciphertext or a GPU tensor of 2 P N
        words, produced on `stream` (default: torch's current stream); with
        `ready` (a torch.cuda.Event recorded after the producer's writes) the
        plan's own stream waits on that event instead (resident.cu:176-179)."""
        if isinstance(view, DeviceCipherBatch):
            words, ptr = view.words, view.data
        else:
            words, ptr = view.numel(), dev_ptr(view, u64_dtypes())
        if words != self.ct_words:
            raise shape_error("E_DEVICE_STACK_VIEW")
        if ready is not None:
            check(lib().praghip_token_stack_store_ready(self._h, slot, level, ptr, ready.cuda_event))
            return
        check(lib().praghip_token_stack_store(self._h, slot, level, ptr, stream_handle(stream)))

    def stack_view(self, slot: int, level: int) -> DeviceCipherBatch:
        v = ctypes.c_void_p()
        check(lib().praghip_token_stack_view(self._h, slot, level, ctypes.byref(v)))
        return DeviceCipherBatch(int(v.value), self.ct_words, self)

    def download(self, view: DeviceCipherBatch, ready=None) -> np.ndarray:
        """Host copy of a view; with `ready` (torch.cuda.Event) the copy waits on it."""
        if view.words != self.ct_words:
            raise shape_error("E_DEVICE_DOWNLOAD_VIEW")
        out = np.empty((2, len(self.q), 1 << self.log_n), dtype=np.uint64)
        if ready is not None:
            check(lib().praghip_token_download_ready(self._h, view.data, ready.cuda_event, out.ctypes.data))
        else:
            check(lib().praghip_token_download(self._h, view.data, out.ctypes.data))
        return out

    def timing(self) -> Timing:
        t = Timing()
        check(lib().praghip_token_timing(self._h, ctypes.byref(t)))
        return t

    def phase_timing(self) -> TokenPhases:
        """TokenWeights::timing (resident.hpp:11-12): phases of the last host-buffer evaluation."""
        t = TokenPhases()
        check(lib().praghip_token_phase_timing(self._h, ctypes.byref(t)))
        return t

    def close(self) -> Cleanup:
        c = Cleanup()
        check(lib().praghip_token_close(self._h, ctypes.byref(c)))
        return c

    def __del__(self):
        h = getattr(self, "_h", None)
        if h is not None:
            try:
                lib().praghip_token_destroy(h)
            except Exception:
                pass
            self._h = None


def packed_target(coordinate: int, levels: int = 9, log_n: int = 14) -> int:
    """Coefficient that coordinate lands on after the packing tree
    (bfv_acyclic_pack.hpp:53-56, praghip_packed_target): its low `levels`
    bits reversed, times N >> levels (32 for the reference's 9 levels at
    N = 16384)."""
    out = ctypes.c_uint64()
    check(lib().praghip_packed_target(int(coordinate), int(levels), int(log_n), ctypes.byref(out)))
    return int(out.value)


class Packing:
    """`keys` [levels][2][dnum][2][len(q)][N] NTT form; q has the data primes
    and the special prime last.  pair(left, right, level) on host ciphertexts
    [2][L][N]; pair_device on `count` device pairs; tree_device reduces
    [leaves][slots] device ciphertexts to the roots in place."""

    def __init__(self, q, log_n: int, keys, dnum: int | None = None, max_pairs: int = 64, device: int = 0):
        self.q = [int(x) for x in q]
        self.log_n = log_n
        k = host_u64(keys)
        K, n = len(self.q), 1 << log_n
        self.dnum = dnum if dnum is not None else K - 1
        per_level = 2 * self.dnum * 2 * K * n
        if k.size == 0 or k.size % per_level:
            raise shape_error("E_PACK_KEY_LEVELS")
        self.levels = k.size // per_level
        qa = np.asarray(self.q, dtype=np.uint64)
        h = ctypes.c_void_p()
        check(lib().praghip_pack_plan_create(device, qa.ctypes.data, K - 1, log_n, self.dnum, self.levels,
                                             k.ctypes.data, max_pairs, ctypes.byref(h)))
        self._h = h

    @property
    def ct_words(self) -> int:
        return 2 * (len(self.q) - 1) << self.log_n

    def pair(self, left, right, level: int) -> np.ndarray:
        a, b = host_u64(left), host_u64(right)
        if a.size != self.ct_words or b.size != self.ct_words:
            raise shape_error("E_PACK_CIPHERTEXT")
        out = np.empty((2, len(self.q) - 1, 1 << self.log_n), dtype=np.uint64)
        check(lib().praghip_pack_pair(self._h, a.ctypes.data, b.ctypes.data, level, out.ctypes.data))
        return out

    def pair_device(self, left, right, level: int, out=None, stream=None):
        """left, right: GPU [count][2][L][N] tensors or DeviceCipherBatch
        views; out: GPU tensor (allocated when None); returns out."""
        import torch
        words = [v.words if isinstance(v, DeviceCipherBatch) else v.numel() for v in (left, right)]
        count = words[0] // self.ct_words
        if count == 0 or words[0] != words[1] or words[0] != count * self.ct_words:
            raise shape_error("E_PACK_DEVICE_VIEW")
        if out is None:
            out = torch.empty(words[0], dtype=torch.int64, device="cuda")
        ptr = [v.data if isinstance(v, DeviceCipherBatch) else dev_ptr(v, u64_dtypes()) for v in (left, right)]
        check(lib().praghip_pack_pair_device(self._h, ptr[0], ptr[1], count, level, dev_ptr(out, u64_dtypes()),
                                             stream_handle(stream)))
        return out

    def tree_device(self, nodes, slots: int = 1, stream=None):
        """nodes: GPU [leaves][slots][2][L][N], reduced in place; returns the
        roots nodes[0] ([slots][2][L][N])."""
        leaves = nodes.numel() // (slots * self.ct_words)
        if nodes.numel() != leaves * slots * self.ct_words:
            raise shape_error("E_PACK_LEVEL")
        check(lib().praghip_pack_tree_device(self._h, dev_ptr(nodes, u64_dtypes()), leaves, slots,
                                             stream_handle(stream)))
        return nodes.view(leaves, slots, -1)[0]

    def merges(self) -> int:
        m = ctypes.c_uint64()
        check(lib().praghip_pack_merges(self._h, ctypes.byref(m)))
        return int(m.value)

    def timing(self) -> Timing:
        t = Timing()
        check(lib().praghip_pack_timing(self._h, ctypes.byref(t)))
        return t

    def close(self) -> Cleanup:
        c = Cleanup()
        check(lib().praghip_pack_close(self._h, ctypes.byref(c)))
        return c

    def __del__(self):
        h = getattr(self, "_h", None)
        if h is not None:
            try:
                lib().praghip_pack_destroy(h)
            except Exception:
                pass
            self._h = None
