"""GPU parity of the HE matrix product (matrix_gpu::Matrix, matrix.cu:48-81) and of
the public-key encryption of zero (PublicZero, enc0.cu:99-114) against the oracle
(pinned by the schoolbook negacyclic product and the big-integer ModDown closed
form): full and selective evaluation, the device entry points, the reference's
errors and the cleanup counts."""
import numpy as np
import pytest

import closed_form as cf
import oracle
import praghip
from conftest import from_dev, to_dev

pytestmark = pytest.mark.gpu

T59 = (1 << 59) - 1


@pytest.mark.parametrize("log_n,blocks,primes", [(14, 3, "locked"), (12, 5, "50bit"), (14, 1, "50bit")])
def test_matrix_evaluate(gpu, log_n, blocks, primes):
    print(f"[matrix] log_n={log_n} blocks={blocks} {primes}", flush=True)
    n = 1 << log_n
    q = cf.LOCKED_PRIMES[:6] if primes == "locked" else cf.primes_below(50, 2 * n, 6)
    ct = oracle.fill_residues(blocks * 2 * 6, n, q, 300 + blocks).reshape(blocks, 2, 6, n)
    ring = oracle.fill_u64(blocks * n, 301 + blocks).reshape(blocks, n) & np.uint64(T59)
    ring[0, :4] = [T59, 1 << 58, 0, (1 << 58) - 1]
    want = oracle.matrix_product(ct, ring, q, log_n)
    m = praghip.Matrix(q, log_n, ct)
    np.testing.assert_array_equal(m.evaluate(ring), want)
    # a second evaluation on the same plan with other weights
    ring2 = oracle.fill_u64(blocks * n, 302 + blocks).reshape(blocks, n) & np.uint64(T59)
    np.testing.assert_array_equal(m.evaluate(ring2), oracle.matrix_product(ct, ring2, q, log_n))
    # selective: c0 only at the targets, c1 complete
    targets = np.array([0, 7, 100, n - 1], dtype=np.uint64)
    sel = m.evaluate_selective(ring, targets)
    mask = np.zeros(n, dtype=bool)
    mask[targets.astype(np.int64)] = True
    np.testing.assert_array_equal(sel[1], want[1])
    np.testing.assert_array_equal(sel[0][:, mask], want[0][:, mask])
    assert not sel[0][:, ~mask].any()
    # device entry point
    out = to_dev(np.zeros((2, 6, n), dtype=np.uint64))
    m.evaluate_device(to_dev(ring), out)
    import torch
    torch.cuda.synchronize()
    np.testing.assert_array_equal(from_dev(out), want)
    c = m.close()
    assert c.closed and c.wipe_synchronized_bytes == c.freed_bytes > 0


def test_matrix_errors(gpu):
    n, q = 1 << 12, cf.primes_below(50, 1 << 13, 6)
    ct = oracle.fill_residues(2 * 6, n, q, 5).reshape(1, 2, 6, n)
    m = praghip.Matrix(q, 12, ct)
    ring = np.zeros((1, n), dtype=np.uint64)
    for bad, code in [(np.array([], dtype=np.uint64), "MATRIX_GPU_TARGET_COUNT"),
                      (np.arange(513, dtype=np.uint64), "MATRIX_GPU_TARGET_COUNT"),
                      (np.array([5, 5], dtype=np.uint64), "MATRIX_GPU_TARGET_INDEX"),
                      (np.array([n], dtype=np.uint64), "MATRIX_GPU_TARGET_INDEX")]:
        with pytest.raises(praghip.PraghipError, match=code):
            m.evaluate_selective(ring, bad)
    ring[0, 3] = 1 << 59
    with pytest.raises(praghip.PraghipError, match="MATRIX_GPU_RING"):
        m.evaluate(ring)
    bad_ct = ct.copy()
    bad_ct[0, 0, 0, 0] = q[0]
    with pytest.raises(praghip.PraghipError, match="E_NTT_CANONICAL_REQUIRED"):
        praghip.Matrix(q, 12, bad_ct)
    m.close()
    with pytest.raises(praghip.PraghipError, match="MATRIX_GPU_CLOSED"):
        m.evaluate(np.zeros((1, n), dtype=np.uint64))


def _enc0_samples(q, n, seed):
    u = ((oracle.fill_u64(n, seed) % np.uint64(3)).astype(np.int64) - 1)
    e = [(oracle.fill_u64(n, seed + 1 + c) % np.uint64(41)).astype(np.int64) - 20 for c in range(2)]
    return np.array([[np.mod(vec, m).astype(np.uint64) for m in q] for vec in [u] + e], dtype=np.uint64)


@pytest.mark.parametrize("primes", ["locked", "50bit"])
def test_enc0(gpu, primes):
    """PublicZero::evaluate (enc0.cu:99-114) against the oracle (pinned by the big-integer closed form)."""
    print(f"[enc0] {primes}", flush=True)
    log_n, n = 14, 1 << 14
    q = cf.LOCKED_PRIMES if primes == "locked" else cf.primes_below(50, 2 * n, 6) + cf.primes_below(60, 2 * n, 1)
    pk = oracle.fill_residues(2 * len(q), n, q, 400).reshape(2, len(q), n)
    z = praghip.PublicZero(q, log_n, pk)
    for seed in (410, 420):
        samples = _enc0_samples(q, n, seed)
        np.testing.assert_array_equal(z.evaluate(samples), oracle.enc0(samples, pk, q, log_n))
    out = to_dev(np.zeros((2, len(q) - 1, n), dtype=np.uint64))
    z.evaluate_device(to_dev(samples), out)
    import torch
    torch.cuda.synchronize()
    np.testing.assert_array_equal(from_dev(out), oracle.enc0(samples, pk, q, log_n))
    bad = samples.copy()
    bad[1, 0, 5] = q[0]
    with pytest.raises(praghip.PraghipError, match="E_ENC0_SAMPLE_CANONICAL"):
        z.evaluate(bad)
    c = z.close()
    assert c.closed and c.wipe_synchronized_bytes == c.freed_bytes > 0
    with pytest.raises(praghip.PraghipError, match="E_SWITCH_CLOSED"):
        z.evaluate(samples)


@pytest.mark.parametrize("log_n,blocks,groups,primes",
                         [(14, 3, 5, "locked"), (12, 2, 9, "50bit"), (12, 5, 4, "50bit"), (12, 5, 6, "62bit")])
def test_matrix_batch(gpu, log_n, blocks, groups, primes):
    """evaluate_device_batch: `groups` evaluations in one call against the
    per-evaluation entry point and the oracle (ragged last group of the
    4-column product tiles).  Every prime below 2^60: the column product's
    lazy sums (five blocks: a reduction by 8q after the fourth); primes up to
    2^62: a reduction per product."""
    import torch
    print(f"[matrix-batch] log_n={log_n} blocks={blocks} groups={groups} {primes}", flush=True)
    n = 1 << log_n
    q = {"locked": cf.LOCKED_PRIMES[:6], "50bit": cf.primes_below(50, 2 * n, 6),
         "62bit": cf.primes_below(62, 2 * n, 6)}[primes]
    ct = oracle.fill_residues(blocks * 2 * 6, n, q, 500 + blocks).reshape(blocks, 2, 6, n)
    rings = oracle.fill_u64(groups * blocks * n, 501).reshape(groups, blocks, n) & np.uint64(T59)
    rings[-1, 0, :3] = [T59, 0, 1 << 58]
    m = praghip.Matrix(q, log_n, ct)
    m.reserve(groups)
    out = to_dev(np.zeros((groups, 2, 6, n), dtype=np.uint64))
    m.evaluate_device_batch(to_dev(rings), out)
    one = to_dev(np.zeros((2, 6, n), dtype=np.uint64))
    torch.cuda.synchronize()
    got = from_dev(out)
    for g in range(groups):
        m.evaluate_device(to_dev(rings[g]), one)
        torch.cuda.synchronize()
        np.testing.assert_array_equal(got[g], from_dev(one), err_msg=f"group {g}")
    for g in (0, groups - 1):
        np.testing.assert_array_equal(got[g], oracle.matrix_product(ct, rings[g], q, log_n), err_msg=f"oracle {g}")
    # a smaller batch on the same scratch, then the limits
    m.evaluate_device_batch(to_dev(rings[:2]), out[:2])
    torch.cuda.synchronize()
    np.testing.assert_array_equal(from_dev(out[:2]), got[:2])
    with pytest.raises(praghip.PraghipError, match="MATRIX_GPU_BATCH"):
        m.evaluate_device_batch(to_dev(np.concatenate([rings, rings[:1]])), to_dev(np.zeros((groups + 1, 2, 6, n),
                                                                                                 dtype=np.uint64)))
    with pytest.raises(praghip.PraghipError, match="MATRIX_GPU_BATCH_RESERVED"):
        m.reserve(groups + 1)
    m.reserve(1)  # within the reserved count: no change
    m.close()


@pytest.mark.parametrize("targets", ["edges", "max512", "one"])
def test_matrix_batch_selective(gpu, targets):
    """The device-side selective batch (evaluate_selective + gather_c0,
    matrix.cu:41-44,65-81): every group's c0 is the full batch's c0 at the
    targets and zero elsewhere, c1 is the full batch's, `selected` holds the
    target coefficients, and group 0 equals the host evaluate_selective."""
    import torch
    log_n, blocks, groups, n = 14, 2, 5, 16384
    print(f"[matrix-selective] targets={targets}", flush=True)
    q = cf.LOCKED_PRIMES[:6]
    idx = {"edges": np.array([0, 1, 2, 777, n - 2, n - 1], dtype=np.uint64),
           "max512": np.arange(512, dtype=np.uint64) * np.uint64(31) + np.uint64(5),
           "one": np.array([4096], dtype=np.uint64)}[targets]
    ct = oracle.fill_residues(blocks * 2 * 6, n, q, 600).reshape(blocks, 2, 6, n)
    rings = oracle.fill_u64(groups * blocks * n, 601).reshape(groups, blocks, n) & np.uint64(T59)
    m = praghip.Matrix(q, log_n, ct)
    m.reserve(groups)
    full = to_dev(np.zeros((groups, 2, 6, n), dtype=np.uint64))
    m.evaluate_device_batch(to_dev(rings), full)
    sel_out = to_dev(np.zeros((groups, 2, 6, n), dtype=np.uint64))
    selected = to_dev(np.zeros((groups, 6, idx.size), dtype=np.uint64))
    m.evaluate_device_batch(to_dev(rings), sel_out, targets=idx, selected=selected)
    torch.cuda.synchronize()
    f, got, gs = from_dev(full), from_dev(sel_out), from_dev(selected)
    want = f.copy()
    keep = np.zeros(n, dtype=bool)
    keep[idx.astype(np.int64)] = True
    want[:, 0, :, ~keep] = 0
    np.testing.assert_array_equal(got, want)
    np.testing.assert_array_equal(gs, f[:, 0][:, :, idx.astype(np.int64)])
    np.testing.assert_array_equal(got[0], m.evaluate_selective(rings[0], idx))
    # without `selected`, and the host-side target checks
    m.evaluate_device_batch(to_dev(rings), sel_out, targets=idx)
    torch.cuda.synchronize()
    np.testing.assert_array_equal(from_dev(sel_out), want)
    for bad, code in [(np.array([], dtype=np.uint64), "MATRIX_GPU_TARGET_COUNT"),
                      (np.arange(513, dtype=np.uint64), "MATRIX_GPU_TARGET_COUNT"),
                      (np.array([5, 5], dtype=np.uint64), "MATRIX_GPU_TARGET_INDEX"),
                      (np.array([n], dtype=np.uint64), "MATRIX_GPU_TARGET_INDEX")]:
        with pytest.raises(praghip.PraghipError, match=code):
            m.evaluate_device_batch(to_dev(rings), sel_out, targets=bad)
    m.close()


def test_enc0_batch(gpu):
    """evaluate_device_batch: several encryptions in one call against the
    per-encryption entry point and the oracle."""
    import torch
    print("[enc0-batch]", flush=True)
    log_n, n, count = 14, 1 << 14, 6
    q = cf.primes_below(50, 2 * n, 6) + cf.primes_below(60, 2 * n, 1)
    pk = oracle.fill_residues(2 * len(q), n, q, 600).reshape(2, len(q), n)
    z = praghip.PublicZero(q, log_n, pk)
    z.reserve(count)
    samples = np.stack([_enc0_samples(q, n, 610 + 10 * e) for e in range(count)])
    out = to_dev(np.zeros((count, 2, len(q) - 1, n), dtype=np.uint64))
    z.evaluate_device_batch(to_dev(samples), out)
    torch.cuda.synchronize()
    got = from_dev(out)
    one = to_dev(np.zeros((2, len(q) - 1, n), dtype=np.uint64))
    for e in range(count):
        z.evaluate_device(to_dev(samples[e]), one)
        torch.cuda.synchronize()
        np.testing.assert_array_equal(got[e], from_dev(one), err_msg=f"encryption {e}")
    for e in (0, count - 1):
        np.testing.assert_array_equal(got[e], oracle.enc0(samples[e], pk, q, log_n), err_msg=f"oracle {e}")
    with pytest.raises(praghip.PraghipError, match="E_ENC0_BATCH"):
        z.evaluate_device_batch(to_dev(np.concatenate([samples, samples[:1]])),
                                to_dev(np.zeros((count + 1, 2, len(q) - 1, n), dtype=np.uint64)))
    with pytest.raises(praghip.PraghipError, match="E_ENC0_BATCH_RESERVED"):
        z.reserve(count + 1)
    c = z.close()
    assert c.closed and c.wipe_synchronized_bytes == c.freed_bytes > 0
