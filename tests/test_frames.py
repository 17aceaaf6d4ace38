"""The PRGCF001 frame header (channel.cpp:122-150) through the C ABI, on the
CPU: a known-answer header assembled field by field with Python's struct
(big-endian u64s), decode/encode round trips, every binding mismatch and a
ciphertext frame whose payload is the ciphertext layout."""
import struct

import numpy as np
import pytest

import oracle
import praghip
from praghip import frames

SESSION = bytes(range(16))
CONFIG = bytes(range(100, 132))


def test_header_known_answer():
    got = frames.encode_header(SESSION, CONFIG, sequence=7, size=1572864, stage=3, operation=0x0102030405060708)
    want = b"PRGCF001" + SESSION + CONFIG + struct.pack(">5Q", 7, 1572864, 3, 0x0102030405060708, 1)
    assert len(got) == 96 and got == want


def test_decode_and_binding_checks():
    h = frames.encode_header(SESSION, CONFIG, 11, 64, 2, 5)
    assert frames.decode_header(h) == {"session": SESSION, "config": CONFIG, "sequence": 11, "size": 64, "stage": 2,
                                       "operation": 5}
    frames.check_header(h, SESSION, CONFIG, 11, 64, 2, 5)
    for kw in [dict(session=bytes(16)), dict(config=bytes(32)), dict(sequence=12), dict(size=65), dict(stage=1),
               dict(operation=4)]:
        args = dict(session=SESSION, config=CONFIG, sequence=11, size=64, stage=2, operation=5)
        args.update(kw)
        with pytest.raises(praghip.PraghipError, match="E_FRAME_BINDING"):
            frames.check_header(h, **args)
    for bad in [b"PRGCF002" + h[8:], h[:88] + struct.pack(">Q", 2)]:
        with pytest.raises(praghip.PraghipError, match="E_FRAME_BINDING"):
            frames.decode_header(bad)


def test_ciphertext_frame_round_trip():
    q = [1152921504599080961, 1152921504600260609]
    ct = oracle.fill_residues(2 * 2, 64, q, 5).reshape(2, 2, 64)
    f = frames.frame_ciphertext(ct, SESSION, CONFIG, sequence=3)
    assert len(f) == 96 + ct.size * 8
    assert f[96:104] == int(ct[0, 0, 0]).to_bytes(8, "little")
    np.testing.assert_array_equal(frames.unframe_ciphertext(f, ct.shape, SESSION, CONFIG, 3), ct)
    with pytest.raises(praghip.PraghipError, match="E_FRAME_BINDING"):
        frames.unframe_ciphertext(f, ct.shape, SESSION, CONFIG, 4)
    with pytest.raises(praghip.PraghipError, match="E_FRAME_BINDING"):
        frames.unframe_ciphertext(f[:-8], ct.shape, SESSION, CONFIG, 3)
