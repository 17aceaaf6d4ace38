"""praghip: MI355X (gfx950) backend for the BFV polynomial engine and the
party-local Z_2^64 share GEMM of HaoR265/privacy-rag.

Python mirror of the reference's GPU backend classes over the C ABI of
libpraghip.so:

* :class:`NttBatch`  - prag::experimental::ntt::NttBatch (ntt.hpp:22-40)
* :class:`Switch`    - prag::experimental_full_switch::Switch (switch.hpp:12-28)
* :func:`share_gemm` - the party-local share GEMM (bfv_matrix.inc:101-105),
  offered as a LocalShares operation (local_shares.hpp:22-32)
* :class:`LocalShares` and the ring ops, :func:`lift59`, :func:`dyadic_mac`,
  :func:`local_dot_scale` - compute/local_shares.cu, resident.cu, matrix.cu
* :class:`MappedWeights` - the int32 .npy weight reader (artifacts.hpp:31-49)
* :class:`Matrix` - the HE matrix product on resident ciphertexts
  (matrix_gpu::Matrix, matrix.hpp:9-24)
* :class:`PublicZero` - the public-key encryption of zero (enc0.hpp:15-25)
* :class:`TokenWeights` and :class:`Packing` - the token-resident path
  (resident.hpp:20-45) and the acyclic packing tree (bfv_gpu_packing.hpp:10-45)
* :class:`Qwen3LocalGemms` - the local products of a Qwen3 forward
  (model.hpp:66-126) as one batched call

Device data is handed over as torch tensors on the GPU (int64 or uint64 with
u64 bit patterns); torch is used only for memory and streams.
"""
from __future__ import annotations

from ._lib import Cleanup, PraghipError, Timing, check, lib  # noqa: F401
from .ntt import NttBatch, ntt_tables  # noqa: F401
from .keyswitch import Switch  # noqa: F401
from .shares import (LocalShares, ShareStorage, bfv_delta, dyadic_mac, lift59, local_dot_scale,  # noqa: F401
                     local_dot_scale_noalloc, ring_add, ring_layout, ring_scale, ring_sum_rows, share_gemm,
                     share_gemm_valu, split_weights)
from .weights import MappedWeights  # noqa: F401
from .qwen3 import QWEN3_0_6B, Qwen3LocalGemms, Qwen3Shape  # noqa: F401
from .matrix import Matrix, MatrixPacking, PublicZero, matrix_packing  # noqa: F401
from .token import DeviceCipherBatch, Packing, TokenWeights, packed_target  # noqa: F401
from . import frames, synth  # noqa: F401


def device_count() -> int:
    return int(lib().praghip_device_count())


def device_identity(device: int = 0) -> tuple[str, str]:
    """(uuid, pci) of a gfx950 device: the two strings a binding compares
    ("GPU-..." from hipDeviceProp_t.uuid, the PCI bus id)."""
    import ctypes
    uuid, pci = ctypes.create_string_buffer(64), ctypes.create_string_buffer(64)
    check(lib().praghip_device_identity(int(device), uuid, 64, pci, 64))
    return uuid.value.decode(), pci.value.decode()


def bind_device(uuid: str | None = None, pci: str | None = None, *, uuid_var: str = "PRAG_ENC0_GPU_UUID",
                pci_var: str = "PRAG_ENC0_GPU_PCI") -> int:
    """Index of the gfx950 device with this UUID and PCI bus id (ntt.cu:86-90).
    With uuid and pci both None the pair is read from the environment variables
    `uuid_var` / `pci_var`; an unset variable raises E_PHASE_DEVICE_BINDING and
    no matching device E_GFX950_REQUIRED."""
    import ctypes
    out = ctypes.c_int(-1)
    if uuid is None and pci is None:
        check(lib().praghip_device_bind_env(uuid_var.encode(), pci_var.encode(), ctypes.byref(out)))
    else:
        check(lib().praghip_device_bind(None if uuid is None else uuid.encode(),
                                        None if pci is None else pci.encode(), ctypes.byref(out)))
    return out.value
