"""Closed-form definitions of the BFV path, in plain Python integers.

These are the mathematical statements the oracle (oracle/oracle.c) and the HIP
kernels must agree with.  They share no code with either: the NTT here is the
direct evaluation of the transform at the roots, the keyswitch is big-integer
polynomial arithmetic followed by CRT and an exact rounded division, the GEMM is
an integer dot product reduced mod 2^64.  Used by gen_golden.py to write the
committed fixtures and by the CPU tests for small on-the-fly cases.
"""
from __future__ import annotations

MASK64 = (1 << 64) - 1
GOLDEN = 0x9E3779B97F4A7C15

# The locked reference primes (implementation_v1/artifacts/bfv_context.json,
# chain_index 6, key level); the last one is the special prime.
LOCKED_PRIMES = [
    1152921504599080961, 1152921504600260609, 1152921504604979201, 1152921504605962241,
    1152921504606584833, 1152921504606683137, 1152921504606748673,
]


# ------------------------------------------------------------------ generator
def splitmix64(seed: int, index: int) -> int:
    z = (seed + (index + 1) * GOLDEN) & MASK64
    z = ((z ^ (z >> 30)) * 0xBF58476D1CE4E5B9) & MASK64
    z = ((z ^ (z >> 27)) * 0x94D049BB133111EB) & MASK64
    return z ^ (z >> 31)


def residues(seed: int, limbs: int, n: int, q: list[int]) -> list[list[int]]:
    """[limbs][n], limb l uniform mod q[l % len(q)] (Lemire mulhi)."""
    return [[(splitmix64(seed, l * n + k) * q[l % len(q)]) >> 64 for k in range(n)] for l in range(limbs)]


# --------------------------------------------------------------- number theory
def is_prime(n: int) -> bool:
    if n < 2:
        return False
    small = [2, 3, 5, 7, 11, 13, 17, 19, 23, 29, 31, 37]
    for p in small:
        if n % p == 0:
            return n == p
    d, s = n - 1, 0
    while d % 2 == 0:
        d //= 2
        s += 1
    for a in small:
        x = pow(a, d, n)
        if x in (1, n - 1):
            continue
        for _ in range(s - 1):
            x = x * x % n
            if x == n - 1:
                break
        else:
            return False
    return True


def primes_below(bits: int, n: int, count: int) -> list[int]:
    """Largest `count` primes < 2^bits with p == 1 mod 2n, ascending."""
    out = []
    v = (1 << bits) - 2 * n + 1
    while len(out) < count:
        if is_prime(v):
            out.append(v)
        v -= 2 * n
    return sorted(out)


def minimal_psi(q: int, n: int) -> int:
    """Smallest primitive 2n-th root of unity mod q (brute force over odd powers)."""
    assert (q - 1) % (2 * n) == 0
    for x in range(2, q):
        g = pow(x, (q - 1) // (2 * n), q)
        if pow(g, n, q) == q - 1:
            break
    return min(pow(g, k, q) for k in range(1, 2 * n, 2))


def bitrev(x: int, bits: int) -> int:
    return int(format(x, f"0{bits}b")[::-1], 2) if bits else 0


# ------------------------------------------------------------------------ NTT
def ntt_point(a: list[int], q: int, psi: int, k: int, log_n: int) -> int:
    """Output k of the SEAL-order negacyclic NTT: a evaluated at psi^(2*bitrev(k)+1)."""
    w = pow(psi, 2 * bitrev(k, log_n) + 1, q)
    acc = 0
    for c in reversed(a):
        acc = (acc * w + c) % q
    return acc


def ntt(a: list[int], q: int, psi: int) -> list[int]:
    n = len(a)
    log_n = n.bit_length() - 1
    return [ntt_point(a, q, psi, k, log_n) for k in range(n)]


def intt(ah: list[int], q: int, psi: int) -> list[int]:
    """Inverse of ntt(): a_j = n^-1 * sum_k ah_k * psi^-(2*bitrev(k)+1)*j."""
    n = len(ah)
    log_n = n.bit_length() - 1
    ninv = pow(n, -1, q)
    pinv = pow(psi, -1, q)
    roots = [pow(pinv, 2 * bitrev(k, log_n) + 1, q) for k in range(n)]
    return [ninv * sum(ah[k] * pow(roots[k], j, q) for k in range(n)) % q for j in range(n)]


def negacyclic(a: list[int], b: list[int], mod: int | None = None) -> list[int]:
    n = len(a)
    out = [0] * n
    for i, x in enumerate(a):
        if not x:
            continue
        for j, y in enumerate(b):
            if i + j < n:
                out[i + j] += x * y
            else:
                out[i + j - n] -= x * y
    return [v % mod for v in out] if mod else out


def galois(a: list[int], g: int, q: int) -> list[int]:
    """a(X) -> a(X^g) mod (X^n + 1, q)."""
    n = len(a)
    out = [0] * n
    for i, v in enumerate(a):
        e = (i * g) % (2 * n)
        if e < n:
            out[e] = (out[e] + v) % q
        else:
            out[e - n] = (out[e - n] - v) % q
    return out


def crt(residues_: list[int], moduli: list[int]) -> int:
    M = 1
    for m in moduli:
        M *= m
    x = 0
    for r, m in zip(residues_, moduli):
        Mi = M // m
        x += r * Mi * pow(Mi % m, -1, m)
    return x % M


# ------------------------------------------------------------------ keyswitch
def digit_primes(L: int, dnum: int, j: int) -> range:
    """Data primes of digit j: a balanced split, the first L % dnum digits hold one extra."""
    base, extra = divmod(L, dnum)
    lo = j * base + min(j, extra)
    return range(lo, lo + base + (1 if j < extra else 0))


def keyswitch(ct, key_ntt, q: list[int], dnum: int, g: int = 1):
    """Big-integer statement of the keyswitch.

    ct: [2][L][n] coefficient residues over q[0..L-1]; key_ntt: [dnum][2][L+1][n]
    NTT-form residues over q[0..L] (q[L] = special prime p).  Returns [2][L][n].

      perm   = ct(X^g)
      D_j    = sum_{i in digit j (digit_primes)} [c1_i * (Q_j/q_i)^-1]_{q_i} * (Q_j/q_i)   (integers)
      X_c    = sum_j D_j * K_{j,c}  mod (X^n+1, Q*p),   K = CRT of the key's coefficients
      out_c  = [c==0]*perm0 + floor((X_c + floor(p/2)) / p)   mod q_i
    """
    L = len(q) - 1
    n = len(ct[0][0])
    p = q[L]
    QP = 1
    for m in q:
        QP *= m
    psis = [minimal_psi(m, n) for m in q]
    perm = [[galois(ct[c][i], g, q[i]) for i in range(L)] for c in range(2)]
    digits = []
    for j in range(dnum):
        idx = list(digit_primes(L, dnum, j))
        Qj = 1
        for i in idx:
            Qj *= q[i]
        D = [0] * n
        for i in idx:
            hat = Qj // q[i]
            inv_hat = pow(hat % q[i], -1, q[i])
            for k in range(n):
                D[k] += (perm[1][i][k] * inv_hat % q[i]) * hat
        digits.append(D)
    out = [[None] * L for _ in range(2)]
    for c in range(2):
        X = [0] * n
        for j in range(dnum):
            Kc = [intt(key_ntt[j][c][t], q[t], psis[t]) for t in range(L + 1)]
            K = [crt([Kc[t][k] for t in range(L + 1)], q) for k in range(n)]
            prod = negacyclic(digits[j], K)
            X = [x + y for x, y in zip(X, prod)]
        X = [x % QP for x in X]
        rounded = [(x + p // 2) // p for x in X]
        for i in range(L):
            out[c][i] = [((perm[0][i][k] if c == 0 else 0) + rounded[k]) % q[i] for k in range(n)]
    return out


# ----------------------------------------------------------------------- GEMM
def share_gemm(x, w, shifts=None, mask_bits: int = 64):
    """Y[b][o] = (sum_j x[b][j] * w[o][j]) << s_o  mod 2^mask_bits (w signed)."""
    mask = (1 << mask_bits) - 1
    out = []
    for row in x:
        r = []
        for o, wr in enumerate(w):
            acc = sum(a * b for a, b in zip(row, wr))
            if shifts is not None:
                acc <<= int(shifts[o])
            r.append(acc & mask)
        out.append(r)
    return out


def enc0(samples, pk_ntt, q: list[int]):
    """Big-integer statement of the public-key encryption of zero with ModDown.

    samples: [3][K][n] residues of u, e0, e1 over q[0..K-1] (q[K-1] = p);
    pk_ntt: [2][K][n] NTT-form residues.  Returns [2][K-1][n]:
      X_c   = CRT(u) * CRT(pk_c) + CRT(e_c)  mod (X^n+1, Q*p)
      out_c = floor((X_c + floor(p/2)) / p)  mod q_i
    """
    K = len(q)
    n = len(samples[0][0])
    p = q[K - 1]
    QP = 1
    for m in q:
        QP *= m
    psis = [minimal_psi(m, n) for m in q]
    u = [crt([samples[0][t][k] for t in range(K)], q) for k in range(n)]
    out = []
    for c in range(2):
        pc = [intt(pk_ntt[c][t], q[t], psis[t]) for t in range(K)]
        P = [crt([pc[t][k] for t in range(K)], q) for k in range(n)]
        e = [crt([samples[c + 1][t][k] for t in range(K)], q) for k in range(n)]
        X = [(a + b) % QP for a, b in zip(negacyclic(u, P), e)]
        out.append([[((x + p // 2) // p) % q[i] for x in X] for i in range(K - 1)])
    return out


# --------------------------------------------- BFV encryption for invariants
def signed_galois(a: list[int], g: int) -> list[int]:
    """a(X) -> a(X^g) mod X^n + 1 over the integers (small signed coefficients)."""
    big = 1 << 200
    return [v - big if v > big // 2 else v for v in galois([v % big for v in a], g, big)]


def switch_key(rng, q: list[int], dnum: int, s_src: list[int], s_dst: list[int]) -> list:
    """NTT-form key [dnum][2][L+1][N] switching s_src to s_dst: digit j holds
    (b, a) with b = -a s_dst + e + [p]_{q_t} s_src on the digit's primes
    (the structure of acyclic_keys, bfv_acyclic_pack.hpp:31-40)."""
    n = len(s_dst)
    L = len(q) - 1
    p = q[L]
    psis = [minimal_psi(x, n) for x in q]
    key = []
    for j in range(dnum):
        digit = digit_primes(L, dnum, j)
        comp = [[], []]
        e = [rng.randrange(-3, 4) for _ in range(n)]  # one integer error polynomial for all primes
        for ti, qt in enumerate(q):
            a = [rng.randrange(qt) for _ in range(n)]
            b = [(x + y) % qt for x, y in zip(negacyclic([-v for v in a], s_dst, qt), e)]
            if ti in digit:
                b = [(x + (p % qt) * v) % qt for x, v in zip(b, s_src)]
            comp[0].append(ntt(b, qt, psis[ti]))
            comp[1].append(ntt(a, qt, psis[ti]))
        key.append(comp)
    return key


def encrypt(rng, m: list[int], s: list[int], q: list[int], t: int) -> list:
    """Symmetric BFV encryption of m mod t under s: [2][len(q)][n] residues."""
    n = len(m)
    Q = 1
    for x in q:
        Q *= x
    a = [rng.randrange(Q) for _ in range(n)]
    e = [rng.randrange(-3, 4) for _ in range(n)]
    c0 = [(x + y + (Q // t) * z) % Q for x, y, z in zip(negacyclic([-v for v in a], s, Q), e, m)]
    return [[[v % qi for v in c0] for qi in q], [[v % qi for v in a] for qi in q]]


def decrypt(ct, s: list[int], q: list[int], t: int) -> list[int]:
    """round(t (c0 + c1 s) / Q) mod t, c0 and c1 rebuilt by CRT."""
    n = len(s)
    Q = 1
    for x in q:
        Q *= x
    d0 = [crt([int(ct[0][i][k]) for i in range(len(q))], q) for k in range(n)]
    d1 = [crt([int(ct[1][i][k]) for i in range(len(q))], q) for k in range(n)]
    phase = [(x + y) % Q for x, y in zip(d0, negacyclic(d1, s, Q))]
    return [((t * v + Q // 2) // Q) % t for v in phase]


def monomial(a: list[int], e: int, mod: int) -> list[int]:
    """X^e a(X) mod (X^n + 1, mod)."""
    n = len(a)
    x = [0] * n
    e %= 2 * n
    if e < n:
        x[e] = 1
    else:
        x[e - n] = mod - 1
    return negacyclic(a, x, mod)


def pack_plain(ml: list[int], mr: list[int], level: int, t: int) -> list[int]:
    """Plaintext of a packing pair: m_L + X^s m_R + sigma_g(m_L - X^s m_R),
    s = n >> (level+1), g = 2^(level+1) + 1 (bfv_acyclic_pack.hpp:44-52)."""
    n = len(ml)
    sh = monomial(mr, n >> (level + 1), t)
    g = (2 << level) + 1
    d = galois([(x - y) % t for x, y in zip(ml, sh)], g, t)
    return [(x + y + z) % t for x, y, z in zip(ml, sh, d)]
