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
