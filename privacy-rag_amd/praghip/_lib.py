"""ctypes binding of libpraghip.so (include/praghip.h).

The library is built in-tree by ``praghip._build.build()``.  There is no
fallback: importing the package without the built library raises.
"""
from __future__ import annotations

import ctypes
import os

_PKG = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(_PKG, "libpraghip.so")

OK, E_SHAPE, E_CANONICAL, E_CONTEXT, E_CLOSED, E_DEVICE, E_ARGUMENT, E_STATE = range(8)


class PraghipError(RuntimeError):
    def __init__(self, code: int, text: str):
        super().__init__(f"{text} (status {code})")
        self.code = code
        self.text = text


class Cleanup(ctypes.Structure):
    """Cleanup{first_cuda_error, wipe_synchronized_bytes, freed_bytes, closed} (ntt.hpp:15-19)."""
    _fields_ = [("first_hip_error", ctypes.c_int32), ("closed", ctypes.c_int32),
                ("wipe_synchronized_bytes", ctypes.c_uint64), ("freed_bytes", ctypes.c_uint64)]


class Timing(ctypes.Structure):
    _fields_ = [("upload_ms", ctypes.c_double), ("kernel_ms", ctypes.c_double), ("download_ms", ctypes.c_double),
                ("device_bytes", ctypes.c_uint64), ("sensitive_bytes", ctypes.c_uint64)]


class SwitchPhases(ctypes.Structure):
    """Switch::Timing (switch.hpp:10): praghip_switch_phases."""
    _fields_ = [(n, ctypes.c_double) for n in ("setup_upload_ms", "upload_ms", "rns_ntt_ms", "product_ms",
                                               "inverse_ms", "moddown_ms", "download_ms")] + \
               [("device_bytes", ctypes.c_uint64), ("sensitive_bytes", ctypes.c_uint64)]


class TokenPhases(ctypes.Structure):
    """TokenWeights::Timing (resident.hpp:11-12): praghip_token_phases."""
    _fields_ = [(n, ctypes.c_double) for n in ("initial_input_upload_ms", "weight_upload_ms", "lift_ms", "ntt_ms",
                                               "dyadic_ms", "download_ms", "finish_ms")] + \
               [(n, ctypes.c_uint64) for n in ("input_bytes", "ring_weight_bytes", "ntt_weight_bytes",
                                                "output_bytes", "device_bytes")]


vp, sz, u32, u64, i32 = ctypes.c_void_p, ctypes.c_size_t, ctypes.c_uint32, ctypes.c_uint64, ctypes.c_int


class GemmDesc(ctypes.Structure):
    """praghip_gemm_desc (include/praghip.h)."""
    _fields_ = [("x", ctypes.c_void_p), ("w", ctypes.c_void_p), ("shifts", ctypes.c_void_p), ("y", ctypes.c_void_p),
                ("m", ctypes.c_size_t), ("k", ctypes.c_size_t), ("n", ctypes.c_size_t),
                ("w_bits", ctypes.c_int), ("mask_bits", ctypes.c_int)]


class MatrixPackingT(ctypes.Structure):
    """praghip_matrix_packing_t (prag::MatrixPacking, bfv_layout.hpp:8)."""
    _fields_ = [("reduction", ctypes.c_uint64), ("columns", ctypes.c_uint64), ("returns", ctypes.c_uint64),
                ("inputs", ctypes.c_uint64)]


class FrameHeaderT(ctypes.Structure):
    """praghip_frame_header (the fields of channel.cpp:126-134)."""
    _fields_ = [("session", ctypes.c_uint8 * 16), ("config", ctypes.c_uint8 * 32), ("sequence", ctypes.c_uint64),
                ("size", ctypes.c_uint64), ("stage", ctypes.c_uint64), ("operation", ctypes.c_uint64)]


pp = ctypes.POINTER(ctypes.c_void_p)

SIGNATURES = {
    "praghip_last_error": (ctypes.c_char_p, []),
    "praghip_version": (i32, []),
    "praghip_device_count": (i32, []),
    "praghip_device_identity": (i32, [i32, ctypes.c_char_p, sz, ctypes.c_char_p, sz]),
    "praghip_device_bind": (i32, [ctypes.c_char_p, ctypes.c_char_p, ctypes.POINTER(ctypes.c_int)]),
    "praghip_device_bind_env": (i32, [ctypes.c_char_p, ctypes.c_char_p, ctypes.POINTER(ctypes.c_int)]),
    "praghip_ntt_tables": (i32, [u64, u32, vp, vp, vp, vp]),
    "praghip_ntt_plan_create": (i32, [i32, vp, sz, u32, vp, vp, vp, sz, pp]),
    "praghip_ntt_forward": (i32, [vp, vp, sz, vp]),
    "praghip_ntt_inverse": (i32, [vp, vp, sz, vp]),
    "praghip_ntt_transform": (i32, [vp, vp, vp, i32]),
    "praghip_ntt_bind_client_key": (i32, [vp, vp]),
    "praghip_ntt_client_phase": (i32, [vp, vp, vp]),
    "praghip_ntt_sync": (i32, [vp]),
    "praghip_ntt_timing": (i32, [vp, ctypes.POINTER(Timing)]),
    "praghip_ntt_close": (i32, [vp, ctypes.POINTER(Cleanup)]),
    "praghip_ntt_destroy": (None, [vp]),
    "praghip_switch_plan_create": (i32, [i32, vp, sz, u32, sz, vp, vp, vp, vp, vp, u32, sz, pp]),
    "praghip_switch_apply": (i32, [vp, vp, vp]),
    "praghip_switch_evaluate": (i32, [vp, vp, vp]),
    "praghip_keyswitch": (i32, [vp, vp, vp, sz, vp, sz, u32, vp]),
    "praghip_switch_sync": (i32, [vp]),
    "praghip_switch_timing": (i32, [vp, ctypes.POINTER(Timing)]),
    "praghip_switch_phase_timing": (i32, [vp, ctypes.POINTER(SwitchPhases)]),
    "praghip_switch_close": (i32, [vp, ctypes.POINTER(Cleanup)]),
    "praghip_switch_destroy": (None, [vp]),
    "praghip_share_gemm": (i32, [i32, vp, vp, i32, vp, vp, sz, sz, sz, i32, vp]),
    "praghip_share_gemm_valu": (i32, [i32, vp, vp, vp, vp, sz, sz, sz, i32, vp]),
    "praghip_weights_split": (i32, [i32, vp, vp, sz, vp]),
    "praghip_ring_add": (i32, [i32, vp, vp, vp, sz, i32, vp]),
    "praghip_ring_scale": (i32, [i32, vp, u64, vp, sz, i32, vp]),
    "praghip_ring_layout": (i32, [i32, vp, sz, vp, vp, sz, vp]),
    "praghip_ring_sum_rows": (i32, [i32, vp, vp, sz, sz, i32, vp]),
    "praghip_storage_allocate": (i32, [i32, sz, pp]),
    "praghip_storage_write": (i32, [vp, sz, vp, sz]),
    "praghip_storage_read": (i32, [vp, sz, sz, vp]),
    "praghip_storage_data": (i32, [vp, ctypes.POINTER(ctypes.c_void_p), ctypes.POINTER(ctypes.c_size_t)]),
    "praghip_storage_stats": (i32, [vp, ctypes.POINTER(ctypes.c_uint64), ctypes.POINTER(ctypes.c_uint64)]),
    "praghip_storage_clear": (i32, [vp, ctypes.POINTER(Cleanup)]),
    "praghip_storage_destroy": (None, [vp]),
    "praghip_lift59": (i32, [i32, vp, vp, sz, u32, sz, vp, sz, vp]),
    "praghip_dyadic_mac": (i32, [i32, vp, vp, vp, sz, sz, u32, sz, vp, sz, vp]),
    "praghip_local_dot_workspace_words": (sz, [sz]),
    "praghip_local_dot_scale": (i32, [i32, vp, vp, sz, sz, vp, u64, vp, sz, vp, vp, vp]),
    "praghip_local_dot_scale_noalloc": (i32, [i32, vp, vp, sz, sz, vp, u64, vp, sz, vp, vp]),
    "praghip_matrix_plan_create": (i32, [i32, vp, sz, u32, vp, sz, pp]),
    "praghip_matrix_evaluate": (i32, [vp, vp, vp, vp, sz]),
    "praghip_matrix_evaluate_device": (i32, [vp, vp, vp, vp]),
    "praghip_matrix_reserve": (i32, [vp, sz]),
    "praghip_matrix_evaluate_device_batch": (i32, [vp, vp, vp, sz, vp]),
    "praghip_matrix_evaluate_device_batch_selective": (i32, [vp, vp, vp, sz, vp, sz, vp, vp]),
    "praghip_matrix_packing": (i32, [sz, sz, sz, i32, ctypes.POINTER(MatrixPackingT)]),
    "praghip_matrix_device_bytes": (sz, [vp]),
    "praghip_matrix_close": (i32, [vp, ctypes.POINTER(Cleanup)]),
    "praghip_matrix_destroy": (None, [vp]),
    "praghip_enc0_plan_create": (i32, [i32, vp, sz, u32, vp, pp]),
    "praghip_enc0_evaluate": (i32, [vp, vp, vp]),
    "praghip_enc0_evaluate_device": (i32, [vp, vp, vp, vp]),
    "praghip_enc0_reserve": (i32, [vp, sz]),
    "praghip_enc0_evaluate_device_batch": (i32, [vp, vp, vp, sz, vp]),
    "praghip_enc0_close": (i32, [vp, ctypes.POINTER(Cleanup)]),
    "praghip_enc0_destroy": (None, [vp]),
    "praghip_token_plan_create": (i32, [i32, vp, sz, u32, sz, sz, sz, sz, vp, pp]),
    "praghip_token_evaluate": (i32, [vp, vp, sz, vp]),
    "praghip_token_bind_local_shares": (i32, [vp, vp, sz]),
    "praghip_token_evaluate_finished": (i32, [vp, vp, sz, vp, pp]),
    "praghip_token_evaluate_local_finished": (i32, [vp, vp, sz, pp]),
    "praghip_token_evaluate_device": (i32, [vp, vp, vp, vp, vp]),
    "praghip_token_reserve": (i32, [vp, sz]),
    "praghip_token_evaluate_device_batch": (i32, [vp, vp, vp, vp, sz, vp]),
    "praghip_token_stack_store": (i32, [vp, sz, ctypes.c_uint, vp, vp]),
    "praghip_token_stack_view": (i32, [vp, sz, ctypes.c_uint, pp]),
    "praghip_token_download": (i32, [vp, vp, vp]),
    "praghip_token_stack_store_ready": (i32, [vp, sz, ctypes.c_uint, vp, vp]),
    "praghip_token_download_ready": (i32, [vp, vp, vp, vp]),
    "praghip_token_timing": (i32, [vp, ctypes.POINTER(Timing)]),
    "praghip_token_phase_timing": (i32, [vp, ctypes.POINTER(TokenPhases)]),
    "praghip_token_close": (i32, [vp, ctypes.POINTER(Cleanup)]),
    "praghip_token_destroy": (None, [vp]),
    "praghip_pack_plan_create": (i32, [i32, vp, sz, u32, sz, sz, vp, sz, pp]),
    "praghip_pack_pair": (i32, [vp, vp, vp, ctypes.c_uint, vp]),
    "praghip_pack_pair_device": (i32, [vp, vp, vp, sz, ctypes.c_uint, vp, vp]),
    "praghip_pack_tree_device": (i32, [vp, vp, sz, sz, vp]),
    "praghip_pack_merges": (i32, [vp, ctypes.POINTER(u64)]),
    "praghip_packed_target": (i32, [sz, ctypes.c_uint, u32, ctypes.POINTER(ctypes.c_uint64)]),
    "praghip_pack_timing": (i32, [vp, ctypes.POINTER(Timing)]),
    "praghip_pack_close": (i32, [vp, ctypes.POINTER(Cleanup)]),
    "praghip_pack_destroy": (None, [vp]),
    "praghip_weights_open": (i32, [ctypes.c_char_p, sz, sz, i32, pp]),
    "praghip_weights_shape": (i32, [vp, ctypes.POINTER(sz), ctypes.POINTER(sz)]),
    "praghip_weights_data": (vp, [vp]),
    "praghip_weights_at": (i32, [vp, sz, sz, ctypes.POINTER(u64)]),
    "praghip_weights_max_abs": (i32, [vp, ctypes.POINTER(u64)]),
    "praghip_weights_upload": (i32, [vp, i32, vp, vp]),
    "praghip_weights_upload_split": (i32, [vp, i32, vp, vp]),
    "praghip_weights_close": (None, [vp]),
    "praghip_frame_encode": (i32, [ctypes.POINTER(FrameHeaderT), vp]),
    "praghip_frame_decode": (i32, [vp, ctypes.POINTER(FrameHeaderT)]),
    "praghip_frame_check": (i32, [vp, ctypes.POINTER(FrameHeaderT)]),
    "praghip_fill_residues": (i32, [i32, vp, sz, u32, vp, sz, u64, vp]),
    "praghip_fill_u64": (i32, [i32, vp, sz, u64, vp]),
    "praghip_fill_i8": (i32, [i32, vp, sz, u64, vp]),
    "praghip_fill_shift": (i32, [i32, vp, sz, u64, vp]),
    "praghip_share_gemm_batch": (i32, [i32, vp, sz, vp]),
}

_lib = None


def lib() -> ctypes.CDLL:
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            raise ImportError(f"{LIB_PATH} is not built; run __graft_entry__.build() (hipcc, gfx950)")
        L = ctypes.CDLL(LIB_PATH)
        for name, (res, args) in SIGNATURES.items():
            f = getattr(L, name)
            f.restype = res
            f.argtypes = args
        _lib = L
    return _lib


def shape_error(text: str) -> PraghipError:
    return PraghipError(E_SHAPE, text)


def check(rc: int) -> None:
    if rc != OK:
        raise PraghipError(rc, lib().praghip_last_error().decode())
