"""The 96-byte PRGCF001 frame header of the reference's Channel
(native/src/channel.cpp:122-150) over praghip_frame_*, and ciphertext frames
whose payload is the [component][prime][N] little-endian u64 layout."""
from __future__ import annotations

import ctypes

import numpy as np

from ._lib import FrameHeaderT, check, lib, shape_error

HEADER_BYTES = 96


def _header(session: bytes, config: bytes, sequence: int, size: int, stage: int, operation: int) -> FrameHeaderT:
    if len(session) != 16 or len(config) != 32:
        raise shape_error("E_FRAME_BINDING")
    h = FrameHeaderT()
    ctypes.memmove(h.session, session, 16)
    ctypes.memmove(h.config, config, 32)
    h.sequence, h.size, h.stage, h.operation = sequence, size, stage, operation
    return h


def encode_header(session: bytes, config: bytes, sequence: int, size: int, stage: int = 1,
                  operation: int = 0) -> bytes:
    """Channel::send_data's header for a `size`-byte payload."""
    out = (ctypes.c_uint8 * HEADER_BYTES)()
    check(lib().praghip_frame_encode(ctypes.byref(_header(session, config, sequence, size, stage, operation)), out))
    return bytes(out)


def decode_header(frame: bytes) -> dict:
    """Fields of a header (E_FRAME_BINDING for a wrong magic or version)."""
    if len(frame) < HEADER_BYTES:
        raise shape_error("E_FRAME_BINDING")
    buf = (ctypes.c_uint8 * HEADER_BYTES).from_buffer_copy(frame[:HEADER_BYTES])
    h = FrameHeaderT()
    check(lib().praghip_frame_decode(buf, ctypes.byref(h)))
    return {"session": bytes(h.session), "config": bytes(h.config), "sequence": h.sequence, "size": h.size,
            "stage": h.stage, "operation": h.operation}


def check_header(frame: bytes, session: bytes, config: bytes, sequence: int, size: int, stage: int = 1,
                 operation: int = 0) -> None:
    """Channel::recv_data's binding check (E_FRAME_BINDING on any mismatch)."""
    if len(frame) < HEADER_BYTES:
        raise shape_error("E_FRAME_BINDING")
    buf = (ctypes.c_uint8 * HEADER_BYTES).from_buffer_copy(frame[:HEADER_BYTES])
    check(lib().praghip_frame_check(buf, ctypes.byref(_header(session, config, sequence, size, stage, operation))))


def frame_ciphertext(ct, session: bytes, config: bytes, sequence: int, stage: int = 1, operation: int = 0) -> bytes:
    """Header + payload of a host ciphertext [2][L][N] (u64, little-endian)."""
    payload = np.ascontiguousarray(ct, dtype="<u8").tobytes()
    return encode_header(session, config, sequence, len(payload), stage, operation) + payload


def unframe_ciphertext(frame: bytes, shape, session: bytes, config: bytes, sequence: int, stage: int = 1,
                       operation: int = 0) -> np.ndarray:
    """Checks the header against the expected binding and returns the payload as u64 `shape`."""
    words = int(np.prod(shape))
    check_header(frame, session, config, sequence, words * 8, stage, operation)
    if len(frame) != HEADER_BYTES + words * 8:
        raise shape_error("E_FRAME_BINDING")
    return np.frombuffer(frame, dtype="<u8", offset=HEADER_BYTES, count=words).astype(np.uint64).reshape(shape)
