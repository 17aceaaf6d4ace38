"""Pins the CPU oracle (oracle/oracle.c) against closed forms and fixtures.

Nothing here retypes the oracle's butterfly or limb formulas: the checks are
direct evaluation of the transform, big-integer CRT arithmetic, decryption
invariants and the committed fixtures written from tests/golden/closed_form.py.
"""
import json
import os
import random

import numpy as np
import pytest

import closed_form as cf
import oracle

MASK64 = (1 << 64) - 1


@pytest.fixture(scope="module")
def primes(golden_dir):
    with open(os.path.join(golden_dir, "primes.json")) as f:
        return json.load(f)


def test_locked_primes_and_q(primes):
    locked = [int(x) for x in primes["locked_primes"]]
    assert locked == cf.LOCKED_PRIMES
    # SEAL CoeffModulus::Create(16384, {60 x7}) rule (bfv.cpp:94-95)
    assert oracle.gen_primes(60, 16384, 7) == locked
    Qk = 1
    for q in locked:
        assert cf.is_prime(q) and q % 32768 == 1
        Qk *= q
    assert Qk == int(primes["Q_key_level"])
    assert Qk // locked[6] == int(primes["Q_data_level"])
    for name, vals in primes["sets"].items():
        bits = {"locked_16384": 60, "c1_54bit_4096": 54, "c2_50bit_16384": 50, "c3_special_60bit_16384": 60}[name]
        n = 4096 if "4096" in name else 16384
        want = [int(v) for v in vals]
        assert oracle.gen_primes(bits, n, len(want)) == want


def test_minimal_root_matches_closed_form(primes):
    psis = [int(x) for x in primes["psi_16384"]]
    # values independently listed for the 7 locked primes
    assert psis[:3] == [92056553354496, 27543819356734, 52069629205452]
    for q, psi in zip(cf.LOCKED_PRIMES, psis):
        assert oracle.minimal_root(q, 16384) == psi
        assert pow(psi, 16384, q) == q - 1
    for n in (2, 8, 64, 1024):
        q = cf.primes_below(50, n, 1)[0]
        assert oracle.minimal_root(q, n) == cf.minimal_psi(q, n)


@pytest.mark.parametrize("log_n", [3, 6, 10, 14])
def test_tables_closed_form(log_n):
    n = 1 << log_n
    for q in (cf.LOCKED_PRIMES[0], cf.LOCKED_PRIMES[6], cf.primes_below(50, max(n, 2), 1)[0]):
        fwd, inv, invn = oracle.ntt_tables(q, log_n)
        psi = oracle.minimal_root(q, n)
        rng = random.Random(log_n)
        for i in [1, 2, n - 1] + [rng.randrange(1, n) for _ in range(20)]:
            if i >= n:
                continue
            assert int(fwd[cf.bitrev(i, log_n), 0]) == pow(psi, i, q)
            assert int(inv[cf.bitrev(i - 1, log_n) + 1, 0]) == pow(psi, -i, q)
        assert int(fwd[0, 0]) == 1 and int(inv[0, 0]) == 1
        assert int(invn[0]) * n % q == 1
        for tab in (fwd, inv):
            for i in (0, 1, n // 2, n - 1):
                w, wq = int(tab[i, 0]), int(tab[i, 1])
                assert wq == (w << 64) // q


def test_ntt_small_fixture(golden_dir):
    data = np.load(os.path.join(golden_dir, "ntt_small.npz"))
    names = sorted({k.rsplit("_", 1)[0] for k in data.files})
    assert len(names) >= 12
    for name in names:
        q = int(data[name + "_q"][0])
        a, want = data[name + "_in"], data[name + "_out"]
        log_n = a.size.bit_length() - 1
        t = oracle.Tables([q], log_n)
        got = oracle.ntt(a[None, :], t)[0]
        np.testing.assert_array_equal(got, want, err_msg=name)
        back = oracle.ntt(got[None, :], t, inverse=True)[0]
        np.testing.assert_array_equal(back, a, err_msg=name)


def test_ntt_sampled_full_size(golden_dir):
    with open(os.path.join(golden_dir, "ntt_sampled.json")) as f:
        cases = json.load(f)
    assert len(cases) == 15
    import hashlib
    for case in cases:
        q, log_n, seed = int(case["q"]), case["log_n"], int(case["seed"])
        n = 1 << log_n
        a = oracle.fill_residues(1, n, [q], seed)
        assert hashlib.sha256(a.tobytes()).hexdigest() == case["input_sha256"]
        t = oracle.Tables([q], log_n)
        out = oracle.ntt(a, t)[0]
        for k, e in zip(case["k"], case["expected"]):
            assert int(out[k]) == int(e), (case["set"], q, k)
        assert np.array_equal(oracle.ntt(out[None], t, inverse=True)[0], a[0])


def test_generator_matches_closed_form():
    q = [cf.LOCKED_PRIMES[1], cf.LOCKED_PRIMES[4]]
    got = oracle.fill_residues(3, 16, q, 12345)
    want = cf.residues(12345, 3, 16, q)
    assert got.tolist() == want
    assert oracle.fill_u64(5, 7).tolist() == [cf.splitmix64(7, i) for i in range(5)]
    i8 = oracle.fill_i8(1000, 99)
    assert i8.min() >= -127 and i8.max() <= 127
    assert i8.tolist()[:4] == [((cf.splitmix64(99, i) * 255) >> 64) - 127 for i in range(4)]


def test_negacyclic_convolution_via_ntt():
    log_n = 6
    n = 1 << log_n
    for q in (cf.LOCKED_PRIMES[2], cf.primes_below(50, n, 1)[0]):
        t = oracle.Tables([q], log_n)
        a = oracle.fill_residues(1, n, [q], 1)
        b = oracle.fill_residues(1, n, [q], 2)
        fa, fb = oracle.ntt(a, t)[0], oracle.ntt(b, t)[0]
        prod = np.array([int(x) * int(y) % q for x, y in zip(fa, fb)], dtype=np.uint64)
        c = oracle.ntt(prod[None], t, inverse=True)[0]
        assert c.tolist() == cf.negacyclic(a[0].tolist(), b[0].tolist(), q)


def test_modmul_primitives():
    rng = random.Random(5)
    for q in cf.LOCKED_PRIMES + cf.primes_below(50, 16384, 2) + [(1 << 62) - 57]:
        vals = [0, 1, q - 1, q // 2] + [rng.randrange(q) for _ in range(200)]
        for a in vals[:40]:
            for b in vals[::13]:
                assert oracle.lib().orc_mul_barrett(a, b, q) == a * b % q
                wq = (b << 64) // q
                assert oracle.lib().orc_mul_shoup(a, b, wq, q) == a * b % q


def test_galois_and_monomial_shift():
    log_n = 5
    n = 1 << log_n
    q = cf.LOCKED_PRIMES[3]
    a = oracle.fill_residues(1, n, [q], 3)[0]
    for g in (1, 3, 5, 17, 2 * n - 1):
        assert oracle.galois(a, q, log_n, g).tolist() == cf.galois(a.tolist(), g, q)
    for e in (0, 1, 7, n, n + 3, 2 * n - 1):
        mono = [0] * n
        if e % (2 * n) < n:
            mono[e % (2 * n)] = 1
        else:
            mono[e % (2 * n) - n] = q - 1
        assert oracle.monomial_shift(a, q, log_n, e).tolist() == cf.negacyclic(a.tolist(), mono, q)


def test_keyswitch_fixture(golden_dir):
    data = np.load(os.path.join(golden_dir, "keyswitch_small.npz"))
    tags = sorted({k.rsplit("_", 1)[0] for k in data.files})
    assert len(tags) == 20
    for tag in tags:
        q = data[tag + "_q"]
        dnum, g, n = (int(v) for v in data[tag + "_meta"])
        got = oracle.keyswitch(data[tag + "_ct"][None], data[tag + "_key"], q, dnum, n.bit_length() - 1, g)
        np.testing.assert_array_equal(got[0], data[tag + "_out"], err_msg=tag)


def _ternary(rng, n):
    return [rng.choice((-1, 0, 1)) for _ in range(n)]


def _bfv_keyswitch_roundtrip(q, dnum, g, log_n, seed):
    """Encrypt under s_old, keyswitch with a key built for (sigma_g(s_old) -> s_new),
    decrypt under s_new: must give sigma_g(m)."""
    rng = random.Random(seed)
    n = 1 << log_n
    L = len(q) - 1
    t = 1 << 59
    s_old, s_new = _ternary(rng, n), _ternary(rng, n)
    key = cf.switch_key(rng, q, dnum, cf.signed_galois(s_old, g), s_new)
    m = [rng.randrange(t) for _ in range(n)]
    ct = np.array(cf.encrypt(rng, m, s_old, q[:L], t), dtype=np.uint64)
    out = oracle.keyswitch(ct[None], np.array(key, dtype=np.uint64), q, dnum, log_n, g)[0]
    assert cf.decrypt(out, s_new, q[:L], t) == cf.galois(m, g, t)


@pytest.mark.parametrize("dnum,g", [(6, 1), (6, 3), (3, 1), (3, 2 * 32 - 1), (2, 5)])
def test_keyswitch_decrypts(dnum, g):
    log_n = 5
    n = 1 << log_n
    if dnum == 6:
        q = cf.LOCKED_PRIMES
    else:
        q = cf.primes_below(50, n, 6) + cf.primes_below(60, n, 1)
    _bfv_keyswitch_roundtrip(q, dnum, g, log_n, seed=dnum * 100 + g)


def test_share_gemm_fixture(golden_dir):
    data = np.load(os.path.join(golden_dir, "gemm_small.npz"))
    for name in ("i8_a", "i8_shift59", "i32_a", "i32_shift59"):
        sh = data[name + "_shift"] if name + "_shift" in data.files else None
        got = oracle.share_gemm(data[name + "_x"], data[name + "_w"], sh, int(data[name + "_mask"][0]))
        np.testing.assert_array_equal(got, data[name + "_y"], err_msg=name)
    yc = oracle.share_gemm(data["probe_client"], data["probe_weight"], None, 59)
    ys = oracle.share_gemm(data["probe_server"], data["probe_weight"], None, 59)
    recon = (yc + ys) & np.uint64((1 << 59) - 1)
    np.testing.assert_array_equal(recon, data["probe_plain"])


def test_share_gemm_numpy_wraps():
    x = oracle.fill_u64(7 * 300, 11).reshape(7, 300)
    w = oracle.fill_i8(5 * 300, 12).reshape(5, 300)
    want = x @ w.astype(np.int64).astype(np.uint64).T  # numpy integer matmul wraps mod 2^64
    np.testing.assert_array_equal(oracle.share_gemm(x, w), want)


def test_lift_and_local_scale():
    t = 1 << 59
    for q in cf.LOCKED_PRIMES[:6]:
        for v in (0, 1, (1 << 58) - 1, 1 << 58, t - 1, t - 5):
            signed = v - t if v >= (1 << 58) else v
            assert oracle.lift59(v, q) == signed % q
    q = cf.LOCKED_PRIMES[:6]
    Q = 1
    for x in q:
        Q *= x
    delta = [(Q // t) % x for x in q]
    r = Q % t
    shares = oracle.fill_u64(2 * 50, 3).reshape(2, 50) & np.uint64(t - 1)
    w = oracle.fill_u64(50, 4) & np.uint64(t - 1)
    got = oracle.local_dot_scale(shares, w, delta, r, q)
    for s in range(2):
        m = sum(int(a) * int(b) for a, b in zip(shares[s], w)) % t
        want = [((Q * m + t // 2) // t) % x for x in q]  # round(Q*m/t) mod q_k
        assert got[s].tolist() == want


def test_dyadic_mac_closed_form():
    """out[l][z] = sum_b a[b][l][z] * w[b][l % wl][z] mod q[l % P], by Python integers,
    with extreme residues (q-1) in block 0 so a dropped reduction shows."""
    q = [cf.LOCKED_PRIMES[0], cf.LOCKED_PRIMES[5], cf.primes_below(50, 64, 1)[0]]
    blocks, limbs, n = 5, 6, 32
    a = oracle.fill_residues(blocks * limbs, n, q, 21).reshape(blocks, limbs, n)
    w = oracle.fill_residues(blocks * 3, n, q, 22).reshape(blocks, 3, n)
    for l in range(limbs):
        a[0, l, :4] = q[l % 3] - 1
        w[0, l % 3, :4] = q[l % 3] - 1
    got = oracle.dyadic_mac(a, w, q)
    for l in range(limbs):
        ql = q[l % 3]
        want = [sum(int(a[b, l, z]) * int(w[b, l % 3, z]) for b in range(blocks)) % ql for z in range(n)]
        assert got[l].tolist() == want, l


def test_ring_ops_closed_form():
    """LocalShares ring ops against Python integers mod 2^59 (and 2^64), including
    words at the mask edge, so a missing mask or a wrong width shows."""
    t59 = (1 << 59) - 1
    a = oracle.fill_u64(37, 31) & np.uint64(t59)
    b = oracle.fill_u64(37, 32) & np.uint64(t59)
    a[:3] = [t59, t59, 0]
    b[:3] = [t59, 1, 0]
    for bits in (59, 64):
        m = (1 << bits) - 1
        assert oracle.ring_add(a, b, bits).tolist() == [(int(x) + int(y)) & m for x, y in zip(a, b)]
        k = (1 << 58) + 3
        assert oracle.ring_scale(a, k, bits).tolist() == [(int(x) * k) & m for x in a]
        rows = oracle.ring_sum_rows(a[:36], 9, bits)
        assert rows.tolist() == [sum(int(x) for x in a[9 * r:9 * r + 9]) & m for r in range(4)]
    idx = np.array([5, 0, 36, 36, 2, 40], dtype=np.uint64)
    assert oracle.ring_layout(a, idx).tolist() == [int(a[5]), int(a[0]), int(a[36]), int(a[36]), int(a[2]), 0]


def test_lift_blocks_layouts():
    """Block lift: width 0 is the element-wise lift per prime (matrix.cu); width > 0
    reverses each block of `width` words and pads with zeros (resident.cu)."""
    q = [cf.LOCKED_PRIMES[0], cf.primes_below(50, 64, 1)[0]]
    t = 1 << 59
    ring = oracle.fill_u64(3 * 16, 41) & np.uint64(t - 1)
    ring[:4] = [(1 << 58) - 1, 1 << 58, t - 1, 0]
    out = oracle.lift59_blocks(ring, q, 16)
    for b in range(3):
        for k, qk in enumerate(q):
            for z in range(16):
                v = int(ring[b * 16 + z])
                assert int(out[b, k, z]) == (v - t if v >> 58 else v) % qk
    ring5 = ring[:10]
    out = oracle.lift59_blocks(ring5, q, 16, width=5)
    for b in range(2):
        for k, qk in enumerate(q):
            for z in range(16):
                v = int(ring5[b * 5 + 4 - z]) if z < 5 else None
                want = 0 if v is None else (v - t if v >> 58 else v) % qk
                assert int(out[b, k, z]) == want


def test_matrix_product_closed_form():
    """The HE matrix product equals sum_b ct_b(X) * m_b(X) mod (X^N + 1, q) with m_b the
    lifted ring block (schoolbook negacyclic products in Python integers)."""
    log_n, n = 5, 32
    q = cf.primes_below(50, 2 * n, 2)
    blocks = 3
    ct = oracle.fill_residues(blocks * 2 * 2, n, q, 91).reshape(blocks, 2, 2, n)
    ring = oracle.fill_u64(blocks * n, 92).reshape(blocks, n) & np.uint64((1 << 59) - 1)
    ring[0, :3] = [(1 << 59) - 1, 1 << 58, 5]
    got = oracle.matrix_product(ct, ring, q, log_n)
    t = 1 << 59
    for c in range(2):
        for k, qk in enumerate(q):
            want = [0] * n
            for b in range(blocks):
                m = [(int(v) - t if int(v) >> 58 else int(v)) for v in ring[b]]
                a = [int(v) for v in ct[b, c, k]]
                for i in range(n):
                    for j in range(n):
                        s = a[i] * m[j]
                        if i + j < n:
                            want[i + j] += s
                        else:
                            want[i + j - n] -= s
            assert got[c, k].tolist() == [v % qk for v in want], (c, k)


@pytest.mark.parametrize("primes", ["locked", "small"])
def test_enc0_closed_form(primes):
    """PublicZero: ModDown(INTT(NTT(u) * pk) + e) equals floor((u*PK + e + floor(p/2)) / p) mod q_i
    in big integers, with ternary u and small signed noise as residues."""
    log_n, n = 4, 16
    q = cf.LOCKED_PRIMES if primes == "locked" else cf.primes_below(50, 2 * n, 3) + cf.primes_below(60, 2 * n, 1)
    K = len(q)
    u = [(int(v) % 3) - 1 for v in oracle.fill_u64(n, 51)]
    e = [[(int(v) % 41) - 20 for v in oracle.fill_u64(n, 52 + c)] for c in range(2)]
    samples = np.array([[[x % m for x in vec] for m in q] for vec in [u] + e], dtype=np.uint64)
    pk = oracle.fill_residues(2 * K, n, q, 53).reshape(2, K, n)
    got = oracle.enc0(samples, pk, q, log_n)
    want = cf.enc0(samples.tolist(), pk.tolist(), q)
    assert got.tolist() == want


def _signed_ring(rng, count):
    """Ring-2^59 words of signed weights |w| <= 2^20, boundary values included
    (check_resident.cpp:48)."""
    edge = [0, 1, -1, 1 << 20, -(1 << 20), (1 << 20) - 1, -((1 << 20) - 1)]
    vals = [edge[i] if i < len(edge) else rng.randint(-(1 << 20), 1 << 20) for i in range(count)]
    rng.shuffle(vals)
    return vals, np.array([v & ((1 << 59) - 1) for v in vals], dtype=np.uint64)


@pytest.mark.parametrize("bits,width", [(60, 8), (60, 32), (50, 8), (50, 1)])
def test_token_closed_form(bits, width):
    """finished[s][c] = sum_b (sum_j w_b[j] X^-j) ct_b[s][c] + [c = 0] round(Q m_s / 2^59):
    the resident path's reverse-lift, product, add_shift chain against the
    direct negacyclic statement; evaluate() against the product with the
    reversed weights; the scaled term against the exact rounded division."""
    log_n, P, blocks, slots = 5, 2, 3, 2
    n = 1 << log_n
    q = cf.LOCKED_PRIMES[:P] if bits == 60 else cf.primes_below(50, n, P)
    rng = random.Random(bits * 100 + width)
    ct = np.array([[[[[rng.randrange(x) for _ in range(n)] for x in q] for _ in range(2)] for _ in range(slots)]
                   for _ in range(blocks)], dtype=np.uint64)
    signed, ring = _signed_ring(rng, blocks * width)
    local = [rng.randrange(1 << 59) for _ in range(slots - 1)] + [(1 << 59) - 1]
    Q = q[0] * q[1]
    scaled = oracle.token_scaled(local, q)
    for s, m in enumerate(local):
        assert [int(v) for v in scaled[s]] == [((2 * Q * m + (1 << 59)) // (1 << 60)) % x for x in q]
    got = oracle.token_finished(ct, ring, scaled, q, log_n, width)
    ev = oracle.ntt(oracle.token_evaluate(ct, ring, q, log_n, width).reshape(-1, n), oracle.Tables(q, log_n),
                    inverse=True).reshape(slots, 2, P, n)
    for s in range(slots):
        for c in range(2):
            for k, x in enumerate(q):
                want, want_ev = [0] * n, [0] * n
                for b in range(blocks):
                    w = signed[b * width:(b + 1) * width]
                    inv = [0] * n            # sum_j w[j] X^-j, X^-j = -X^(n-j)
                    rev = [0] * n            # sum_j w[j] X^(width-1-j)
                    for j, v in enumerate(w):
                        if j == 0:
                            inv[0] += v
                        else:
                            inv[n - j] -= v
                        rev[width - 1 - j] += v
                    a = [int(v) for v in ct[b, s, c, k]]
                    want = [(u + v) % x for u, v in zip(want, cf.negacyclic(a, inv, x))]
                    want_ev = [(u + v) % x for u, v in zip(want_ev, cf.negacyclic(a, rev, x))]
                if c == 0:
                    want[0] = (want[0] + int(scaled[s, k])) % x
                assert [int(v) for v in got[s, c, k]] == want, (s, c, k)
                assert [int(v) for v in ev[s, c, k]] == want_ev, (s, c, k)


@pytest.mark.parametrize("dnum", [6, 3])
def test_pack_pair_and_tree_decrypt(dnum):
    """Packing invariant with the acyclic key chain s_0 -> s_1 -> s_2 (level l's
    keys switch s_l and sigma_g(s_l) to s_(l+1), bfv_acyclic_pack.hpp:23-42):
    pair(L, R, l) decrypts under s_(l+1) to m_L + X^s m_R + sigma_g(m_L - X^s m_R),
    and a tree over four leaves per slot decrypts under s_2 to that map applied
    level by level."""
    log_n, levels = 5, 2
    n = 1 << log_n
    q = cf.LOCKED_PRIMES
    L = len(q) - 1
    t = 1 << 59
    rng = random.Random(dnum)
    sec = [_ternary(rng, n) for _ in range(levels + 1)]
    keys = []
    for lv in range(levels):
        g = (2 << lv) + 1
        keys.append([cf.switch_key(rng, q, dnum, sec[lv], sec[lv + 1]),
                     cf.switch_key(rng, q, dnum, cf.signed_galois(sec[lv], g), sec[lv + 1])])
    keys = np.array(keys, dtype=np.uint64)
    slots = 2
    ms = [[[rng.randrange(t) for _ in range(n)] for _ in range(slots)] for _ in range(4)]
    cts = np.array([[cf.encrypt(rng, m, sec[0], q[:L], t) for m in row] for row in ms], dtype=np.uint64)
    out = oracle.pack_pair(cts[0, 0], cts[1, 0], 0, keys, q, dnum, log_n)
    assert cf.decrypt(out, sec[1], q[:L], t) == cf.pack_plain(ms[0][0], ms[1][0], 0, t)
    roots = oracle.pack_tree(cts, keys, q, dnum, log_n)
    for s in range(slots):
        want = cf.pack_plain(cf.pack_plain(ms[0][s], ms[1][s], 0, t), cf.pack_plain(ms[2][s], ms[3][s], 0, t), 1, t)
        assert cf.decrypt(roots[s], sec[2], q[:L], t) == want
