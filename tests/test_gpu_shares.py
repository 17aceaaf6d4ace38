"""GPU parity of the ring ops, the lift, the dyadic MAC and the local dot with
Delta scaling (compute/local_shares.cu, resident.cu, matrix.cu) against the
oracle, plus the LocalShares host mirror and the weight reader feeding the GEMM."""
import numpy as np
import pytest

import oracle
import praghip
from conftest import from_dev, to_dev
from golden import closed_form as cf

pytestmark = pytest.mark.gpu

T59 = (1 << 59) - 1


def _sync():
    import torch
    torch.cuda.synchronize()


@pytest.mark.parametrize("n", [1, 2, 7, 4096, 100003])
@pytest.mark.parametrize("bits", [59, 64])
def test_ring_add_scale(gpu, n, bits):
    print(f"[ring] add/scale n={n} bits={bits}", flush=True)
    a = oracle.fill_u64(n, 100 + n) & np.uint64((1 << bits) - 1)
    b = oracle.fill_u64(n, 200 + n) & np.uint64((1 << bits) - 1)
    a[0] = (1 << bits) - 1
    b[0] = (1 << bits) - 1
    ta, tb = to_dev(a), to_dev(b)
    got = from_dev(praghip.ring_add(ta, tb, mask_bits=bits))
    np.testing.assert_array_equal(got, oracle.ring_add(a, b, bits))
    k = (1 << 58) + 12345
    got = from_dev(praghip.ring_scale(ta, k, mask_bits=bits))
    np.testing.assert_array_equal(got, oracle.ring_scale(a, k, bits))


@pytest.mark.parametrize("rows,cols", [(1, 1), (3, 5), (17, 64), (1000, 129), (4, 155648)])
def test_ring_sum_rows(gpu, rows, cols):
    print(f"[ring] sum_rows {rows}x{cols}", flush=True)
    a = oracle.fill_u64(rows * cols, rows + 7 * cols) & np.uint64(T59)
    got = from_dev(praghip.ring_sum_rows(to_dev(a), cols))
    np.testing.assert_array_equal(got, oracle.ring_sum_rows(a, cols))


def test_ring_layout(gpu):
    a = oracle.fill_u64(1000, 5) & np.uint64(T59)
    idx = (oracle.fill_u64(5000, 6) % np.uint64(1000)).astype(np.uint64)
    idx[:3] = [999, 0, 123456789]  # the last one is out of range: the device gather writes 0
    got = from_dev(praghip.ring_layout(to_dev(a), to_dev(idx)))
    np.testing.assert_array_equal(got, oracle.ring_layout(a, idx))


def test_local_shares_mirror(gpu):
    """Host-vector LocalShares: results and the reference's errors."""
    ls = praghip.LocalShares()
    a = oracle.fill_u64(300, 1) & np.uint64(T59)
    b = oracle.fill_u64(300, 2) & np.uint64(T59)
    np.testing.assert_array_equal(ls.add(a, b), oracle.ring_add(a, b))
    np.testing.assert_array_equal(ls.scale(a, 12345), oracle.ring_scale(a, 12345))
    np.testing.assert_array_equal(ls.sum_rows(a, 30), oracle.ring_sum_rows(a, 30))
    idx = np.array([3, 1, 299, 0], dtype=np.uint64)
    np.testing.assert_array_equal(ls.layout(a, idx), oracle.ring_layout(a, idx))
    with pytest.raises(praghip.PraghipError, match="E_CUDA_PUBLIC_MAP"):
        ls.layout(a, [300])
    with pytest.raises(praghip.PraghipError, match="E_CUDA_WORD"):
        ls.add(np.array([1 << 59], dtype=np.uint64), np.array([0], dtype=np.uint64))
    with pytest.raises(praghip.PraghipError, match="E_CUDA_SHAPE"):
        ls.add(a, b[:10])
    with pytest.raises(praghip.PraghipError, match="E_CUDA_SHAPE"):
        ls.sum_rows(a, 7)
    x = oracle.fill_u64(4 * 96, 9) & np.uint64(T59)
    w = (oracle.fill_u64(5 * 96, 10) % np.uint64(1 << 21)).astype(np.int64) - (1 << 20)
    got = ls.matmul(x, w.astype(np.int32), 4, 96, 5)
    np.testing.assert_array_equal(got, oracle.share_gemm(x.reshape(4, 96), w.astype(np.int32).reshape(5, 96),
                                                         mask_bits=59))
    assert ls.stats()["kernels"] == 5


@pytest.mark.parametrize("width", [0, 1, 100, 4096])
def test_lift59(gpu, width):
    print(f"[lift] width={width}", flush=True)
    log_n, n = 12, 4096
    q = cf.LOCKED_PRIMES[:6] + cf.primes_below(50, 2 * n, 2)
    per = width if width else n
    ring = oracle.fill_u64(3 * per, 40 + width) & np.uint64(T59)
    ring[:4] = [(1 << 58) - 1, 1 << 58, T59, 0][:min(4, ring.size)]
    got = from_dev(praghip.lift59(to_dev(ring), q, log_n, width=width))
    np.testing.assert_array_equal(got, oracle.lift59_blocks(ring, q, n, width))


@pytest.mark.parametrize("blocks,limbs,wl", [(1, 1, 1), (19, 12, 6), (7, 6, 1), (64, 6, 6)])
def test_dyadic_mac(gpu, blocks, limbs, wl):
    """Extreme residues (q - 1) in block 0 so a dropped reduction shows."""
    print(f"[mac] blocks={blocks} limbs={limbs} wl={wl}", flush=True)
    n = 1024
    q = cf.LOCKED_PRIMES[:6] if limbs % 6 == 0 else cf.primes_below(50, 2 * n, 1)
    P = len(q)
    a = oracle.fill_residues(blocks * limbs, n, q, 50 + blocks).reshape(blocks, limbs, n)
    # w limb j serves limbs l = j mod wl: residues below every prime it meets
    wq = q if wl % P == 0 else [min(q)]
    w = oracle.fill_residues(blocks * wl, n, wq, 60 + blocks).reshape(blocks, wl, n)
    for l in range(limbs):
        a[0, l, :3] = q[l % P] - 1
        w[0, l % wl, :3] = wq[(l % wl) % len(wq)] - 1
    got = from_dev(praghip.dyadic_mac(to_dev(a), to_dev(w), q))
    np.testing.assert_array_equal(got, oracle.dyadic_mac(a, w, q))


@pytest.mark.parametrize("slots,words", [(1, 1), (2, 1000), (4, 155648), (3, 1 << 20)])
@pytest.mark.parametrize("primes", ["locked", "50bit"])
def test_local_dot_scale(gpu, slots, words, primes):
    print(f"[local] slots={slots} words={words} {primes}", flush=True)
    q = cf.LOCKED_PRIMES[:6] if primes == "locked" else cf.primes_below(50, 1 << 15, 6)
    delta, r = praghip.bfv_delta(q)
    shares = oracle.fill_u64(slots * words, 70 + slots) & np.uint64(T59)
    w = oracle.fill_u64(words, 71 + slots) & np.uint64(T59)
    got = from_dev(praghip.local_dot_scale(to_dev(shares.reshape(slots, words)), to_dev(w), q, delta, r))
    np.testing.assert_array_equal(got, oracle.local_dot_scale(shares.reshape(slots, words), w, delta, r, q))


def test_weights_upload_feeds_gemm(gpu, tmp_path):
    import torch
    rows, cols, m = 96, 256, 33
    w = (oracle.fill_u64(rows * cols, 80) % np.uint64(1 << 21)).astype(np.int64) - (1 << 20)
    w = w.astype("<i4").reshape(rows, cols)
    path = tmp_path / "model.layers.0.mlp.up_proj.weight.npy"
    np.save(path, w)
    x = oracle.fill_u64(m * cols, 81).reshape(m, cols) & np.uint64(T59)
    with praghip.MappedWeights(str(path), rows, cols) as mw:
        assert mw.max_abs() <= 1 << 20
        dw = torch.empty(rows * cols, dtype=torch.int32, device="cuda")
        mw.upload(dw)
    y = praghip.share_gemm(to_dev(x), dw.view(rows, cols), mask_bits=59)
    _sync()
    np.testing.assert_array_equal(from_dev(y), oracle.share_gemm(x, w, mask_bits=59))


def test_share_storage_round_trip_and_clear(gpu):
    """LocalShares::allocate / ShareStorage (local_shares.hpp:12-17,29): zero
    on allocation, write/read round trip at offsets, range and word checks,
    the device words usable by a ring op, clear wipes and frees, the
    LocalShareStats live/peak bytes."""
    import torch
    ls = praghip.LocalShares()
    st = ls.allocate(1000)
    assert ls.stats()["live_bytes"] == 8000 == ls.stats()["peak_bytes"]
    np.testing.assert_array_equal(st.read(0, 1000), np.zeros(1000, dtype=np.uint64))
    a = oracle.fill_u64(600, 90) & np.uint64(T59)
    st.write(100, a)
    np.testing.assert_array_equal(st.read(100, 600), a)
    np.testing.assert_array_equal(st.read(0, 100), np.zeros(100, dtype=np.uint64))
    np.testing.assert_array_equal(st.read(700, 300), np.zeros(300, dtype=np.uint64))
    assert st.stats() == {"uploaded_bytes": 4800, "downloaded_bytes": 8000 + 4800 + 800 + 2400}
    for bad in [lambda: st.write(900, a[:101]), lambda: st.read(1001, 0), lambda: st.read(500, 501)]:
        with pytest.raises(praghip.PraghipError, match="E_CUDA_SHAPE"):
            bad()
    with pytest.raises(praghip.PraghipError, match="E_CUDA_WORD"):
        st.write(0, np.array([1 << 59], dtype=np.uint64))
    # the device words feed the device-pointer ring ops: double words 100..163 in place
    lib = praghip.lib()
    assert lib.praghip_ring_add(0, st.data_ptr + 800, st.data_ptr + 800, st.data_ptr + 800, 64, 59, None) == 0
    torch.cuda.synchronize()
    np.testing.assert_array_equal(st.read(100, 64), (a[:64] * np.uint64(2)) & np.uint64(T59))
    c = st.clear()
    assert c.closed and c.wipe_synchronized_bytes == c.freed_bytes == 8000
    assert st.clear().closed  # idempotent
    assert ls.stats()["live_bytes"] == 0 and ls.stats()["peak_bytes"] == 8000
    with pytest.raises(praghip.PraghipError, match="E_CUDA_STORAGE_CLOSED"):
        st.read(0, 1)
    with pytest.raises(praghip.PraghipError, match="E_CUDA_SHAPE"):
        ls.allocate(0)
