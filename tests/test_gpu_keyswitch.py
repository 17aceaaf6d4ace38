"""GPU parity of the batched keyswitch against the oracle and the closed-form fixtures."""
import os

import numpy as np
import pytest

import closed_form as cf
import oracle
import praghip
from conftest import from_dev, to_dev

pytestmark = pytest.mark.gpu

P16384_SWITCH = cf.primes_below(50, 16384, 6) + cf.primes_below(60, 16384, 1)


def test_keyswitch_golden_fixtures(gpu, golden_dir):
    data = np.load(os.path.join(golden_dir, "keyswitch_small.npz"))
    tags = sorted({k.rsplit("_", 1)[0] for k in data.files})
    for tag in tags:
        q = [int(x) for x in data[tag + "_q"]]
        dnum, g, n = (int(v) for v in data[tag + "_meta"])
        print(f"[ks-golden] {tag}", flush=True)
        sw = praghip.Switch(q, n.bit_length() - 1, dnum, key=data[tag + "_key"], element=g)
        np.testing.assert_array_equal(sw.apply(data[tag + "_ct"]), data[tag + "_out"], err_msg=tag)


@pytest.mark.parametrize("element", [1, 3, (1 << 10) + 1, 2 * 16384 - 1])
def test_keyswitch_locked_reference_dnum6(gpu, element):
    """The reference configuration: 7 locked 60-bit primes, one digit per data prime."""
    q, n, L, dnum, batch = cf.LOCKED_PRIMES, 16384, 6, 6, 2
    print(f"[ks] locked dnum=6 element={element}", flush=True)
    ct = oracle.fill_residues(batch * 2 * L, n, q[:L], 0x5052414700000203).reshape(batch, 2, L, n)
    key = oracle.fill_residues(dnum * 2 * (L + 1), n, q, 0x5052414700010203).reshape(dnum, 2, L + 1, n)
    want = oracle.keyswitch(ct, key, q, dnum, 14, element)
    sw = praghip.Switch(q, 14, dnum, key=key, element=element, max_batch=batch)
    tin, tout = to_dev(ct), to_dev(np.zeros_like(ct))
    sw.keyswitch(tin, tout, galois=element)
    np.testing.assert_array_equal(from_dev(tout), want)
    # host Switch::apply path (upload, Galois(element), keyswitch, download)
    np.testing.assert_array_equal(sw.apply(ct[1]), want[1])


@pytest.mark.parametrize("dnum", [3, 2, 6])
def test_keyswitch_c3_modup_per_ciphertext_keys(gpu, dnum):
    """P16384_SWITCH shape: 6 data primes ~50 bits + 60-bit special prime, dnum digits, one key per ciphertext."""
    q, n, L, batch = P16384_SWITCH, 16384, 6, 3
    print(f"[ks] c3 dnum={dnum}", flush=True)
    ct = oracle.fill_residues(batch * 2 * L, n, q[:L], 0x5052414700000303).reshape(batch, 2, L, n)
    keys = oracle.fill_residues(batch * dnum * 2 * (L + 1), n, q, 0x5052414700010303).reshape(
        batch, dnum, 2, L + 1, n)
    want = oracle.keyswitch(ct, keys, q, dnum, 14, 5, per_ct_keys=True)
    sw = praghip.Switch(q, 14, dnum, max_batch=2)  # batch 3 runs as two chunks
    tin, tout, tk = to_dev(ct), to_dev(np.zeros_like(ct)), to_dev(keys)
    sw.keyswitch(tin, tout, keys=tk, key_stride=sw.key_words, galois=5)
    np.testing.assert_array_equal(from_dev(tout), want)
    # shared key (key_stride 0) on the same inputs
    want0 = oracle.keyswitch(ct, keys[0], q, dnum, 14, 1)
    sw.keyswitch(tin, tout, keys=tk, key_stride=0, galois=1)
    np.testing.assert_array_equal(from_dev(tout), want0)


def test_keyswitch_edge_inputs(gpu):
    """Zero ciphertext, all q-1, and the check_switch.cpp:20 patterns in c1."""
    q, n, L, dnum = P16384_SWITCH, 16384, 6, 3
    key = oracle.fill_residues(dnum * 2 * (L + 1), n, q, 77).reshape(dnum, 2, L + 1, n)
    sw = praghip.Switch(q, 14, dnum, key=key, element=3)
    qs = np.array(q[:L], dtype=np.uint64)[:, None]
    cases = {
        "zero": np.zeros((2, L, n), dtype=np.uint64),
        "max": np.broadcast_to(qs - np.uint64(1), (2, L, n)).copy(),
        "pattern": np.stack([np.zeros((L, n), dtype=np.uint64),
                             (((np.arange(n, dtype=np.uint64) * np.uint64(7919) + np.uint64(123456))
                               & np.uint64((1 << 59) - 1))[None, :] % qs)]),
    }
    for name, ct in cases.items():
        want = oracle.keyswitch(ct[None], key, q, dnum, 14, 3)[0]
        np.testing.assert_array_equal(sw.apply(ct), want, err_msg=name)


@pytest.mark.parametrize("dnum", [3, 6])
def test_keyswitch_max_key_words(gpu, dnum):
    """Every key word q_t - 1 and every ciphertext word q_i - 1: the largest key
    products, whose sums over the digits the float items add without
    re-centring (dnum = 6: six one-prime digits, re-centred after the fourth)."""
    q, n, L = P16384_SWITCH, 16384, 6
    print(f"[ks] max key words dnum={dnum}", flush=True)
    qk = np.array(q, dtype=np.uint64)[None, None, :, None]
    key = np.broadcast_to(qk - np.uint64(1), (dnum, 2, L + 1, n)).copy()
    sw = praghip.Switch(q, 14, dnum, key=key)
    qs = np.array(q[:L], dtype=np.uint64)[:, None]
    ct = np.broadcast_to(qs - np.uint64(1), (2, L, n)).copy()
    want = oracle.keyswitch(ct[None], key, q, dnum, 14, 1)[0]
    np.testing.assert_array_equal(sw.apply(ct), want)


def test_switch_errors_and_cleanup(gpu):
    q, n, L, dnum = cf.LOCKED_PRIMES, 16384, 6, 6
    key = oracle.fill_residues(dnum * 2 * (L + 1), n, q, 1).reshape(dnum, 2, L + 1, n)
    sw = praghip.Switch(q, 14, dnum, key=key, element=1)
    ct = oracle.fill_residues(2 * L, n, q[:L], 2).reshape(2, L, n)
    bad = ct.copy()
    bad[1, 2, 5] = np.uint64(q[2])
    with pytest.raises(praghip.PraghipError) as e:
        sw.apply(bad)
    assert "E_SWITCH_CIPHERTEXT" in e.value.text
    tin, tout = to_dev(ct), to_dev(np.zeros_like(ct))
    with pytest.raises(praghip.PraghipError) as e:
        sw.keyswitch(tin, tout, galois=2)
    assert "E_SWITCH_ELEMENT" in e.value.text
    # keys are read in 16-byte pairs: an 8-byte offset or an odd stride is refused
    tk = to_dev(np.concatenate([np.zeros(2, dtype=np.uint64), key.reshape(-1)]))
    for keys, stride in [(tk[1:1 + key.size], 0), (tk[2:], 1)]:
        with pytest.raises(praghip.PraghipError) as e:
            sw.keyswitch(tin, tout, keys=keys, key_stride=stride)
        assert "E_SWITCH_ALIGNMENT" in e.value.text
    sw.keyswitch(tin, tout, keys=tk[2:], key_stride=0)
    import torch
    torch.cuda.synchronize()
    np.testing.assert_array_equal(from_dev(tout), sw.apply(ct))
    t = sw.timing()
    # sensitive: key [6][2][7][N], products [2][7][N], expanded digits [6][7][N],
    # staging in and out [2][6][N] each; no fused-kernel scratch at N = 16384
    assert t.sensitive_bytes == (6 * 2 * 7 + 2 * 7 + 6 * 7 + 2 * 12) * n * 8
    # public: twiddle tables 7 x N x 48 B (5.25 MiB) and constants
    assert 7 * n * 48 <= t.device_bytes - t.sensitive_bytes < 7 * n * 48 + (64 << 10)
    c = sw.close()
    assert c.closed and c.first_hip_error == 0
    assert c.wipe_synchronized_bytes == c.freed_bytes == t.sensitive_bytes > 0
    assert sw.close().freed_bytes == t.sensitive_bytes
    with pytest.raises(praghip.PraghipError) as e:
        sw.apply(ct)
    assert "E_SWITCH_CLOSED" in e.value.text
    bad_key = key.copy()
    bad_key[0, 0, 6, 0] = np.uint64(q[6])
    with pytest.raises(praghip.PraghipError) as e:
        praghip.Switch(q, 14, dnum, key=bad_key)
    assert "E_SWITCH_KEY_CANONICAL" in e.value.text


def test_keyswitch_rows_chunks(gpu):
    """A batch of 67 at N=16384 runs as two internal chunks of the three-phase
    path (64 + 3, the second starting at ciphertext 64) with per-ciphertext
    keys and a Galois element; spot-checked against the oracle."""
    import torch
    q, n, L, dnum, batch = P16384_SWITCH, 16384, 6, 3, 67
    print("[ks] rows chunks batch=67", flush=True)
    sw = praghip.Switch(q, 14, dnum, max_batch=batch)
    ct = oracle.fill_residues(batch * 2 * L, n, q[:L], 0x5052414700000903).reshape(batch, 2, L, n)
    keys = oracle.fill_residues(batch * dnum * 2 * (L + 1), n, q, 0x5052414700010903).reshape(
        batch, dnum, 2, L + 1, n)
    tin, tout = to_dev(ct), to_dev(np.zeros_like(ct))
    sw.keyswitch(tin, tout, keys=to_dev(keys), key_stride=sw.key_words, galois=3)
    torch.cuda.synchronize()
    got = from_dev(tout)
    for b in (0, 63, 64, 66):
        np.testing.assert_array_equal(got[b], oracle.keyswitch(ct[b:b + 1], keys[b], q, dnum, 14, 3)[0],
                                      err_msg=f"ciphertext {b}")


@pytest.mark.parametrize("L,dnum", [(3, 3), (4, 2), (5, 5), (2, 1)])
def test_keyswitch_rows_shapes(gpu, L, dnum):
    """Other (L, dnum) at N=16384 through the three-phase kernels (equal
    digits of 1 or 2 primes, fewer float targets than one column thread
    holds)."""
    import torch
    print(f"[ks] rows L={L} dnum={dnum}", flush=True)
    n, batch = 16384, 5
    q = cf.primes_below(50, 2 * n, L) + cf.primes_below(60, 2 * n, 1)
    ct = oracle.fill_residues(batch * 2 * L, n, q[:L], 0x50524147000A0000 + L).reshape(batch, 2, L, n)
    keys = oracle.fill_residues(batch * dnum * 2 * (L + 1), n, q, 0x50524147000B0000 + dnum).reshape(
        batch, dnum, 2, L + 1, n)
    sw = praghip.Switch(q, 14, dnum, max_batch=batch)
    tin, tout = to_dev(ct), to_dev(np.zeros_like(ct))
    sw.keyswitch(tin, tout, keys=to_dev(keys), key_stride=sw.key_words, galois=2 * n - 1)
    torch.cuda.synchronize()
    np.testing.assert_array_equal(from_dev(tout), oracle.keyswitch(ct, keys, q, dnum, 14, 2 * n - 1,
                                                                    per_ct_keys=True))


@pytest.mark.parametrize("log_n,element", [(14, 3), (14, (1 << 9) + 1), (12, 3), (12, (1 << 9) + 1)])
def test_switch_evaluate_after_cpu_galois(gpu, log_n, element):
    """The reference's calling convention (keyswitch/seal_adapter.cpp:44-52):
    apply() permutes both components on the CPU, then Switch::evaluate
    keyswitches.  The oracle's permutation fed through praghip_switch_evaluate
    must equal the oracle's keyswitch with the element, and praghip_switch_apply
    on the un-permuted input.  Elements 3 and 2^9 + 1 are packing levels 0 and
    8 (bfv_acyclic_pack.hpp:44-52).  N = 16384 runs the three-phase kernels,
    N = 4096 the fused one."""
    q, L, dnum = cf.LOCKED_PRIMES, 6, 6
    n = 1 << log_n
    print(f"[ks] evaluate after CPU Galois log_n={log_n} element={element}", flush=True)
    ct = oracle.fill_residues(2 * L, n, q[:L], 0x5052414700000C03 + log_n).reshape(2, L, n)
    key = oracle.fill_residues(dnum * 2 * (L + 1), n, q, 0x5052414700010C03 + element).reshape(dnum, 2, L + 1, n)
    permuted = np.stack([np.stack([oracle.galois(ct[c, i], q[i], log_n, element) for i in range(L)])
                         for c in range(2)])
    want = oracle.keyswitch(ct[None], key, q, dnum, log_n, element)[0]
    sw = praghip.Switch(q, log_n, dnum, key=key, element=element)
    np.testing.assert_array_equal(sw.evaluate(permuted), want)
    np.testing.assert_array_equal(sw.apply(ct), want)
    # element 1: evaluate and apply coincide
    sw1 = praghip.Switch(q, log_n, dnum, key=key, element=1)
    np.testing.assert_array_equal(sw1.evaluate(ct), sw1.apply(ct))


@pytest.mark.parametrize("dnum", [2, 3])
def test_keyswitch_locked_primes_multi_prime_digits(gpu, dnum):
    """The seven locked 60-bit primes with digits of 3 or 2 primes: every
    prime on the integer path, ModUp by fast base conversion in 64-bit
    Shoup arithmetic (the column-forward kernel's ArU64 instance with D > 1)."""
    q, n, L, batch = cf.LOCKED_PRIMES, 16384, 6, 2
    print(f"[ks] locked primes dnum={dnum}", flush=True)
    ct = oracle.fill_residues(batch * 2 * L, n, q[:L], 0x5052414700000D03 + dnum).reshape(batch, 2, L, n)
    keys = oracle.fill_residues(batch * dnum * 2 * (L + 1), n, q, 0x5052414700010D03 + dnum).reshape(
        batch, dnum, 2, L + 1, n)
    want = oracle.keyswitch(ct, keys, q, dnum, 14, 5, per_ct_keys=True)
    sw = praghip.Switch(q, 14, dnum, max_batch=batch)
    tin, tout = to_dev(ct), to_dev(np.zeros_like(ct))
    sw.keyswitch(tin, tout, keys=to_dev(keys), key_stride=sw.key_words, galois=5)
    np.testing.assert_array_equal(from_dev(tout), want)


def test_keyswitch_data_prime_below_2_32(gpu):
    """A data prime below 2^32 keeps the data primes on the float path but
    rules out the FP64 ModDown (it needs every data prime in (2^32, 2^50)):
    the inverse columns then finish with the generic integer ModDown."""
    n, L, dnum, batch = 16384, 6, 3, 2
    q = cf.primes_below(31, n, 1) + cf.primes_below(50, n, L - 1) + cf.primes_below(60, n, 1)
    assert q[0] < 1 << 32
    print("[ks] data prime below 2^32", flush=True)
    ct = oracle.fill_residues(batch * 2 * L, n, q[:L], 0x5052414700000E03).reshape(batch, 2, L, n)
    keys = oracle.fill_residues(batch * dnum * 2 * (L + 1), n, q, 0x5052414700010E03).reshape(
        batch, dnum, 2, L + 1, n)
    want = oracle.keyswitch(ct, keys, q, dnum, 14, 3, per_ct_keys=True)
    sw = praghip.Switch(q, 14, dnum, max_batch=batch)
    tin, tout = to_dev(ct), to_dev(np.zeros_like(ct))
    sw.keyswitch(tin, tout, keys=to_dev(keys), key_stride=sw.key_words, galois=3)
    np.testing.assert_array_equal(from_dev(tout), want)


def test_keyswitch_with_seal_tables_and_phase_timing(gpu):
    """Switch::initialize(q, f, r, ni, invp, keys) with the SEAL tables passed
    in (switch.hpp:24): the plan accepts them and switches exactly as the
    oracle; the per-phase times of Switch::Timing (switch.hpp:10) sum to the
    kernel time."""
    from test_abi import seal_switch_tables
    q, n, L, dnum = cf.LOCKED_PRIMES, 16384, 6, 6
    print("[ks] seal tables dnum=6", flush=True)
    ct = oracle.fill_residues(2 * L, n, q[:L], 0x5052414700000903).reshape(1, 2, L, n)
    key = oracle.fill_residues(dnum * 2 * (L + 1), n, q, 0x5052414700010903).reshape(dnum, 2, L + 1, n)
    sw = praghip.Switch(q, 14, dnum, key=key, element=3, tables=seal_switch_tables(q, 14))
    np.testing.assert_array_equal(sw.apply(ct[0]), oracle.keyswitch(ct, key, q, dnum, 14, 3)[0])
    ph, t = sw.phase_timing(), sw.timing()
    parts = [ph.rns_ntt_ms, ph.product_ms, ph.inverse_ms, ph.moddown_ms]
    assert all(x > 0 for x in parts) and ph.setup_upload_ms > 0 and ph.upload_ms > 0 and ph.download_ms > 0
    assert abs(sum(parts) - t.kernel_ms) <= 0.05 * t.kernel_ms
    assert ph.device_bytes == t.device_bytes and ph.sensitive_bytes == t.sensitive_bytes


@pytest.mark.parametrize("bits,dnum", [(61, 1), (62, 2), (62, 3)])
def test_keyswitch_wide_special_prime_three_phase(gpu, bits, dnum):
    """A special prime of 61 or 62 bits (the API takes primes up to 2^62): the
    three-phase path at N = 16384 then runs the per-stage Harvey transforms
    and Shoup key products (no key prime below 2^60 for the lazy form)."""
    q = cf.primes_below(50, 16384, 6) + cf.primes_below(bits, 16384, 1)
    n, L, batch = 16384, 6, 2
    print(f"[ks] special prime {bits} bits dnum={dnum}", flush=True)
    ct = oracle.fill_residues(batch * 2 * L, n, q[:L], 0x5052414700000a03 + bits).reshape(batch, 2, L, n)
    keys = oracle.fill_residues(batch * dnum * 2 * (L + 1), n, q, 0x5052414700010a03 + dnum).reshape(
        batch, dnum, 2, L + 1, n)
    want = oracle.keyswitch(ct, keys, q, dnum, 14, 3, per_ct_keys=True)
    sw = praghip.Switch(q, 14, dnum, max_batch=batch)
    tin, tout, tk = to_dev(ct), to_dev(np.zeros_like(ct)), to_dev(keys)
    sw.keyswitch(tin, tout, keys=tk, key_stride=sw.key_words, galois=3)
    np.testing.assert_array_equal(from_dev(tout), want)
