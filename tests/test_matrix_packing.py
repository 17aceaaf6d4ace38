"""prag::matrix_packing / matrix_packing_qk_reverse64 (bfv_layout.hpp:8-27)
through the C ABI, on the CPU.

The expected packing is found by brute force: for every power-of-two
reduction width the outputs are cut into explicit groups of 512/b columns,
each group into returned ciphertexts of at most `cap` columns, the inner
dimension into explicit chunks, and the bytes are those of the ciphertext
frames moved (a full [2][6][16384] ciphertext or one component, each with the
96-byte frame header).  The C function must pick the cheapest width (the
smallest on a tie), and its answer must satisfy what a packing has to:
it fits the 8192 slots, covers every inner term and every output column."""
import itertools

import pytest

import praghip

N, PRIMES, FRAME_HEADER = 16384, 6, 96
INPUT_BYTES = 2 * PRIMES * N * 8 + FRAME_HEADER   # one input ciphertext
RETURN_BYTES = PRIMES * N * 8 + FRAME_HEADER      # one returned component


def brute_force(b, k, o):
    per_group = 512 // b
    groups = [min(per_group, o - s) for s in range(0, o, per_group)]
    best = None
    d = 16
    while d <= 8192 // b:
        cap = min(per_group, 8192 // (b * d))
        returns = 0
        for size in groups:
            left = size
            while left > 0:
                returns += 1
                left -= cap
        inputs = len(range(0, k, d))
        cost = inputs * INPUT_BYTES + returns * RETURN_BYTES
        if best is None or cost < best[0]:
            best = (cost, (d, cap, returns, inputs))
        d *= 2
    return best[1]


def test_frame_constants():
    # the reference's cost constants are these frame sizes
    assert (INPUT_BYTES, RETURN_BYTES) == (1572960, 786528)


@pytest.mark.parametrize("b,k,o", list(itertools.product([1, 2, 3, 4, 7, 16], [1, 64, 1000, 1024, 3072, 8192],
                                                          [1, 511, 512, 3072, 4096, 155648])))
def test_packing_matches_brute_force(b, k, o):
    got = praghip.matrix_packing(b, k, o)
    assert tuple(got) == brute_force(b, k, o)
    d, cap, returns, inputs = got
    assert d & (d - 1) == 0 and 16 <= d <= 8192 // b
    assert b * d * cap <= 8192                           # one returned ciphertext fits its slots
    assert inputs * d >= k > (inputs - 1) * d            # every inner term, no empty chunk
    assert returns * cap >= o                            # every output column


def test_known_answer():
    # b = 1, K = 1024, 3072 outputs (the Qwen3 gate/up shape): widths 16, 32, 64,
    # 128 cost 105.4, 59.8, 44.0 and 50.3 MB; 64 wins with 128 columns per return
    assert tuple(praghip.matrix_packing(1, 1024, 3072)) == (64, 128, 24, 16)


def test_qk_reverse64_and_shape_errors():
    assert tuple(praghip.matrix_packing(64, 0, 0, qk_reverse64=True)) == (128, 1, 1, 1)
    assert tuple(praghip.matrix_packing(1, 5, 5, qk_reverse64=True)) == (128, 1, 1, 1)
    for args in [(0, 5, 5, True), (65, 5, 5, True)]:
        with pytest.raises(praghip.PraghipError, match="E_QK_REVERSE64_SHAPE"):
            praghip.matrix_packing(*args)
    for b, k, o in [(0, 5, 5), (17, 5, 5), (1, 0, 5), (1, 8193, 5), (1, 5, 0), (1, 5, 155649)]:
        with pytest.raises(praghip.PraghipError, match="E_MATRIX_SHAPE"):
            praghip.matrix_packing(b, k, o)
