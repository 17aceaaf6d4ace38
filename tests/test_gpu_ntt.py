"""GPU parity of the batched NTT/INTT against the oracle and the golden fixtures."""
import json
import os

import numpy as np
import pytest

import closed_form as cf
import oracle
import praghip
from conftest import from_dev, to_dev

pytestmark = pytest.mark.gpu

P4096_54 = cf.primes_below(54, 4096, 2)
P16384_50 = cf.primes_below(50, 16384, 6)


def _roundtrip_case(q, log_n, limbs, seed, gpu, patterns=True):
    n = 1 << log_n
    print(f"[ntt] log_n={log_n} primes={len(q)} limbs={limbs} seed={seed:#x}", flush=True)
    a = oracle.fill_residues(limbs, n, q, seed)
    if patterns:  # check_resident.cpp:35 boundary pattern on the first limb
        qq = np.uint64(q[0])
        j = np.arange(n)
        a[0, j % 13 == 0] = 0
        a[0, j % 13 == 1] = qq - np.uint64(1)
        a[0, j % 13 == 2] = 1
        # the largest growth of the lazy float path: every word q - 1, and
        # q - 1 / 0 alternating (limb l uses prime l % len(q))
        if limbs > 2:
            a[1, :] = np.uint64(q[1 % len(q)]) - np.uint64(1)
            a[2, :] = np.where(j % 2 == 0, np.uint64(q[2 % len(q)]) - np.uint64(1), np.uint64(0))
    tab = oracle.Tables(q, log_n)
    plan = praghip.NttBatch(q, log_n, device=0)
    t = to_dev(a)
    plan.forward(t)
    got = from_dev(t)
    want = oracle.ntt(a, tab)
    np.testing.assert_array_equal(got, want)
    plan.inverse(t)
    np.testing.assert_array_equal(from_dev(t), a)
    # inverse on arbitrary (non-transform) input against the oracle inverse
    b = oracle.fill_residues(limbs, n, q, seed + 1)
    tb = to_dev(b)
    plan.inverse(tb)
    np.testing.assert_array_equal(from_dev(tb), oracle.ntt(b, tab, inverse=True))


def test_ntt_locked_primes(gpu):
    _roundtrip_case(cf.LOCKED_PRIMES, 14, 14, 0x5052414700000101, gpu)


def test_ntt_c2_primes_f64_path(gpu):
    _roundtrip_case(P16384_50, 14, 24, 0x5052414700000102, gpu)


def test_ntt_c1_config(gpu):
    # N=4096, 2 primes ~54 bits, 16 polynomials x 2 limbs
    _roundtrip_case(P4096_54, 12, 32, 0x5052414700000001, gpu)


@pytest.mark.parametrize("log_n", [4, 5, 6, 7, 9, 11, 13])
def test_ntt_all_sizes(gpu, log_n):
    n = 1 << log_n
    q = [cf.primes_below(60, n, 1)[0], cf.primes_below(50, n, 1)[0], cf.primes_below(62, n, 1)[0]]
    _roundtrip_case(q, log_n, 6, 0x77 + log_n, gpu, patterns=False)


@pytest.mark.parametrize("log_n,limbs", [(11, 4096), (12, 3072), (13, 1536)])
def test_ntt_many_limbs_per_workgroup(gpu, log_n, limbs):
    """More limbs than resident workgroups, so that each workgroup runs the
    persistent loop several times (the next limb's loads issued before the
    current limb's last pass or stores): the first and last limbs against the
    oracle, forward and inverse, and the round trip on every limb."""
    import torch
    n = 1 << log_n
    q = [cf.primes_below(50, n, 1)[0], cf.primes_below(49, n, 1)[0], cf.primes_below(60, n, 1)[0]]
    print(f"[ntt] log_n={log_n} limbs={limbs} (persistent loop)", flush=True)
    a = oracle.fill_residues(limbs, n, q, 0x5052414700000300 + log_n)
    tab = oracle.Tables(q, log_n)
    plan = praghip.NttBatch(q, log_n)
    t = to_dev(a)
    plan.forward(t)
    fwd = from_dev(t)
    # the oracle takes limb l of its input to prime l % P: slices start at a
    # multiple of P
    tail = (limbs - 48) // len(q) * len(q)
    np.testing.assert_array_equal(fwd[:48], oracle.ntt(a[:48], tab))
    np.testing.assert_array_equal(fwd[tail:], oracle.ntt(a[tail:], tab))
    plan.inverse(t)
    assert torch.equal(t, to_dev(a))
    b = oracle.fill_residues(limbs, n, q, 0x5052414700000310 + log_n)
    tb = to_dev(b)
    plan.inverse(tb)
    inv = from_dev(tb)
    np.testing.assert_array_equal(inv[:48], oracle.ntt(b[:48], tab, inverse=True))
    np.testing.assert_array_equal(inv[tail:], oracle.ntt(b[tail:], tab, inverse=True))


def test_ntt_golden_small(gpu, golden_dir):
    data = np.load(os.path.join(golden_dir, "ntt_small.npz"))
    names = sorted({k.rsplit("_", 1)[0] for k in data.files})
    done = 0
    for name in names:
        a = data[name + "_in"]
        if a.size < 16:
            continue  # the GPU plans start at N=16
        q = int(data[name + "_q"][0])
        plan = praghip.NttBatch([q], a.size.bit_length() - 1)
        t = to_dev(a[None])
        plan.forward(t)
        np.testing.assert_array_equal(from_dev(t)[0], data[name + "_out"], err_msg=name)
        done += 1
    assert done >= 8


def test_ntt_golden_sampled_full_size(gpu, golden_dir):
    with open(os.path.join(golden_dir, "ntt_sampled.json")) as f:
        cases = json.load(f)
    for case in cases:
        q, log_n, seed = int(case["q"]), case["log_n"], int(case["seed"])
        a = oracle.fill_residues(1, 1 << log_n, [q], seed)
        plan = praghip.NttBatch([q], log_n)
        t = to_dev(a)
        plan.forward(t)
        out = from_dev(t)[0]
        for k, e in zip(case["k"], case["expected"]):
            assert int(out[k]) == int(e), (case["set"], q, k)


def test_ntt_c2_full_batch_properties(gpu):
    """P16384_50 at full size: 256 ciphertexts x 2 x 6 primes = 3072 limbs.  Bit-exact
    forward against the oracle on a slice, round trip and linearity on all."""
    import torch
    n, limbs = 16384, 3072
    q = P16384_50
    plan = praghip.NttBatch(q, 14)
    a = oracle.fill_residues(limbs, n, q, 0x5052414700000002)
    t = to_dev(a)
    plan.forward(t)
    fwd = from_dev(t)
    tab = oracle.Tables(q, 14)
    np.testing.assert_array_equal(fwd[:96], oracle.ntt(a[:96], tab))
    np.testing.assert_array_equal(fwd[-60:], oracle.ntt(a[-60:], tab))
    plan.inverse(t)
    assert torch.equal(t, to_dev(a))
    # linearity: NTT(a + b) = NTT(a) + NTT(b) mod q
    b = oracle.fill_residues(limbs, n, q, 0x5052414700000003)
    qcol = np.array([q[l % 6] for l in range(limbs)], dtype=np.uint64)[:, None]
    s = (a + b) % qcol
    ts, tb = to_dev(s), to_dev(b)
    plan.forward(ts)
    plan.forward(tb)
    np.testing.assert_array_equal(from_dev(ts), (fwd + from_dev(tb)) % qcol)


def test_ntt_host_api_and_errors(gpu):
    q = cf.LOCKED_PRIMES[:6]
    plan = praghip.NttBatch(q, 14, batches=2)
    a = oracle.fill_residues(12, 16384, q, 99)
    out = plan.transform(a)
    np.testing.assert_array_equal(out, oracle.ntt(a, oracle.Tables(q, 14)))
    np.testing.assert_array_equal(plan.transform(out, inverse=True), a)
    bad = a.copy()
    bad[3, 7] = np.uint64(q[3])
    with pytest.raises(praghip.PraghipError) as e:
        plan.transform(bad)
    assert "E_NTT_CANONICAL_REQUIRED" in e.value.text
    with pytest.raises(praghip.PraghipError):
        plan.transform(a[:6])
    # client phase: NTT -> (.) key -> INTT (ntt.cu:181-199) = negacyclic product with the key
    key = oracle.fill_residues(6, 16384, q, 5)
    plan.bind_client_key(key)
    got = plan.client_phase(a)
    tab = oracle.Tables(q, 14)
    prod = np.empty_like(a)
    fa = oracle.ntt(a, tab)
    for l in range(12):
        qq = q[l % 6]
        prod[l] = [(int(x) * int(y)) % qq for x, y in zip(fa[l], key[l % 6])]
    np.testing.assert_array_equal(got, oracle.ntt(prod, tab, inverse=True))
    t = plan.timing()
    assert t.kernel_ms > 0 and t.sensitive_bytes == 12 * 16384 * 8 + 6 * 16384 * 16
    c = plan.close()
    assert c.closed and c.first_hip_error == 0
    assert c.wipe_synchronized_bytes == c.freed_bytes == t.sensitive_bytes
    c2 = plan.close()
    assert c2.freed_bytes == t.sensitive_bytes  # idempotent
    with pytest.raises(praghip.PraghipError) as e:
        plan.transform(a)
    assert "E_NTT_CLOSED" in e.value.text


def test_ntt_rejects_misaligned_device_buffer(gpu):
    import torch
    plan = praghip.NttBatch(P16384_50, 14)
    buf = torch.zeros(16384 + 1, dtype=torch.int64, device="cuda")
    with pytest.raises(praghip.PraghipError) as e:
        plan.forward(buf[1:])  # 8-byte aligned view
    assert "E_NTT_ALIGNMENT" in e.value.text
    assert torch.count_nonzero(buf) == 0  # nothing was launched


def test_device_binding_by_uuid_and_pci(gpu, monkeypatch):
    """ntt.cu:86-90: the plan's device chosen by the UUID + PCI bus id pair
    from the environment; the bound index runs a transform."""
    uuid, pci = praghip.device_identity(0)
    print(f"[bind] device 0 uuid={uuid} pci={pci}", flush=True)
    assert uuid.startswith("GPU-") and len(uuid) > 4 and len(pci) >= 7
    assert praghip.bind_device(uuid, pci) == 0
    assert praghip.bind_device(uuid.upper(), pci.upper()) == 0
    monkeypatch.setenv("PRAG_ENC0_GPU_UUID", uuid)
    monkeypatch.setenv("PRAG_ENC0_GPU_PCI", pci)
    device = praghip.bind_device()
    assert device == 0
    with pytest.raises(praghip.PraghipError) as e:
        praghip.bind_device(uuid, "ffff:ff:1f.7")
    assert e.value.text.startswith("E_GFX950_REQUIRED")
    q = P16384_50[:1]
    a = oracle.fill_residues(1, 1 << 10, q, 0x51)
    plan = praghip.NttBatch(q, 10, device=device)
    t = to_dev(a)
    plan.forward(t)
    np.testing.assert_array_equal(from_dev(t), oracle.ntt(a, oracle.Tables(q, 10)))
