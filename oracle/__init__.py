"""CPU oracle for the BFV NTT / keyswitch / share-GEMM path (ctypes over liboracle.so).

TEST INFRASTRUCTURE ONLY: imported by tests/, by ``__graft_entry__.smoke()`` and
by the cpu_baseline leg of ``bench.py``, and there only to check results.  The
product package never imports it.

The C restatement lives in ``oracle.c`` (each function cites the reference
file:line it follows).  ``build()`` compiles it with the committed Makefile.
"""
from __future__ import annotations

import ctypes
import os
import subprocess

import numpy as np

_HERE = os.path.dirname(os.path.abspath(__file__))
_LIB_PATH = os.path.join(_HERE, "liboracle.so")
_lib = None

u64p = ctypes.POINTER(ctypes.c_uint64)


def build() -> str:
    subprocess.run(["make", "-s", "-C", _HERE], check=True)
    return _LIB_PATH


def lib():
    global _lib
    if _lib is None:
        if not os.path.exists(_LIB_PATH):
            build()
        L = ctypes.CDLL(_LIB_PATH)
        vp, sz, u64, i32, u32 = ctypes.c_void_p, ctypes.c_size_t, ctypes.c_uint64, ctypes.c_int, ctypes.c_uint32
        sig = {
            "orc_splitmix64": (u64, [u64, u64]),
            "orc_fill_residues": (None, [vp, sz, sz, vp, sz, u64]),
            "orc_fill_u64": (None, [vp, sz, u64]),
            "orc_fill_i8": (None, [vp, sz, u64]),
            "orc_fill_shift": (None, [vp, sz, u64]),
            "orc_mulmod": (u64, [u64, u64, u64]),
            "orc_powmod": (u64, [u64, u64, u64]),
            "orc_invmod": (u64, [u64, u64]),
            "orc_is_prime": (i32, [u64]),
            "orc_gen_primes": (sz, [i32, u64, sz, vp]),
            "orc_minimal_root": (u64, [u64, u64]),
            "orc_shoup_quotient": (u64, [u64, u64]),
            "orc_ntt_tables": (i32, [u64, ctypes.c_uint, vp, vp, vp]),
            "orc_mul_shoup": (u64, [u64, u64, u64, u64]),
            "orc_mul_barrett": (u64, [u64, u64, u64]),
            "orc_ntt_forward": (None, [vp, ctypes.c_uint, u64, vp]),
            "orc_ntt_inverse": (None, [vp, ctypes.c_uint, u64, vp, vp]),
            "orc_ntt_batch": (None, [vp, sz, ctypes.c_uint, sz, vp, vp, vp, vp, i32, i32]),
            "orc_galois": (None, [vp, vp, ctypes.c_uint, u64, u32]),
            "orc_monomial_shift": (None, [vp, vp, ctypes.c_uint, u64, sz]),
            "orc_keyswitch": (i32, [vp, vp, vp, sz, sz, vp, sz, sz, ctypes.c_uint, u32, vp, vp, vp, i32]),
            "orc_share_gemm": (i32, [vp, vp, i32, vp, vp, sz, sz, sz, i32, i32]),
            "orc_lift59": (u64, [u64, u64]),
            "orc_dyadic_mac": (None, [vp, vp, vp, sz, sz, sz, sz, vp, sz]),
            "orc_local_dot_scale": (None, [vp, vp, sz, sz, vp, u64, vp, sz, vp]),
            "orc_lift59_blocks": (None, [vp, vp, sz, sz, sz, vp, sz]),
            "orc_enc0": (i32, [vp, vp, vp, vp, sz, ctypes.c_uint, vp, vp, vp, i32]),
            "orc_ring_add": (None, [vp, vp, vp, sz, i32]),
            "orc_ring_scale": (None, [vp, u64, vp, sz, i32]),
            "orc_ring_layout": (None, [vp, sz, vp, vp, sz]),
            "orc_ring_sum_rows": (None, [vp, vp, sz, sz, i32]),
        }
        for name, (res, args) in sig.items():
            f = getattr(L, name)
            f.restype = res
            f.argtypes = args
        _lib = L
    return _lib


def _p(a: np.ndarray | None):
    if a is None:
        return None
    assert a.flags["C_CONTIGUOUS"]
    return a.ctypes.data


def _u64(a) -> np.ndarray:
    return np.ascontiguousarray(np.asarray(a, dtype=np.uint64))


# ---------------------------------------------------------------- generators
def fill_residues(limbs: int, n: int, q, seed: int) -> np.ndarray:
    q = _u64(q)
    out = np.empty((limbs, n), dtype=np.uint64)
    lib().orc_fill_residues(_p(out), limbs, n, _p(q), len(q), seed)
    return out


def fill_u64(count: int, seed: int) -> np.ndarray:
    out = np.empty(count, dtype=np.uint64)
    lib().orc_fill_u64(_p(out), count, seed)
    return out


def fill_i8(count: int, seed: int) -> np.ndarray:
    out = np.empty(count, dtype=np.int8)
    lib().orc_fill_i8(_p(out), count, seed)
    return out


def fill_shift(count: int, seed: int) -> np.ndarray:
    out = np.empty(count, dtype=np.int8)
    lib().orc_fill_shift(_p(out), count, seed)
    return out


# ------------------------------------------------------------- number theory
def gen_primes(bits: int, n: int, count: int) -> list[int]:
    """Largest primes below 2^bits congruent to 1 mod 2n, ascending (SEAL order)."""
    out = np.zeros(count, dtype=np.uint64)
    found = lib().orc_gen_primes(bits, 2 * n, count, _p(out))
    assert found == count
    return sorted(int(v) for v in out)


def minimal_root(q: int, n: int) -> int:
    return int(lib().orc_minimal_root(q, 2 * n))


def ntt_tables(q: int, log_n: int):
    n = 1 << log_n
    fwd = np.zeros((n, 2), dtype=np.uint64)
    inv = np.zeros((n, 2), dtype=np.uint64)
    invn = np.zeros(2, dtype=np.uint64)
    rc = lib().orc_ntt_tables(q, log_n, _p(fwd), _p(inv), _p(invn))
    if rc:
        raise ValueError("q is not 1 mod 2N")
    return fwd, inv, invn


class Tables:
    """Stacked [primes][N][2] tables for a prime list."""

    def __init__(self, q, log_n: int):
        self.q = _u64(q)
        self.log_n = log_n
        f, i, n = zip(*(ntt_tables(int(x), log_n) for x in self.q))
        self.fwd = np.ascontiguousarray(np.stack(f))
        self.inv = np.ascontiguousarray(np.stack(i))
        self.invn = np.ascontiguousarray(np.stack(n))


# ----------------------------------------------------------------------- NTT
def ntt(data: np.ndarray, tables: Tables, inverse: bool = False, threads: int = 0) -> np.ndarray:
    """Batched transform of a [..][N] buffer whose limb l uses prime l % P (copy)."""
    n = 1 << tables.log_n
    out = np.array(data, dtype=np.uint64, copy=True, order="C")
    limbs = out.size // n
    lib().orc_ntt_batch(_p(out), limbs, tables.log_n, len(tables.q), _p(tables.q), _p(tables.fwd),
                        _p(tables.inv), _p(tables.invn), int(inverse), threads)
    return out


def galois(poly: np.ndarray, q: int, log_n: int, g: int) -> np.ndarray:
    src = _u64(poly)
    out = np.empty_like(src)
    lib().orc_galois(_p(src), _p(out), log_n, q, g)
    return out


def monomial_shift(poly: np.ndarray, q: int, log_n: int, e: int) -> np.ndarray:
    src = _u64(poly)
    out = np.empty_like(src)
    lib().orc_monomial_shift(_p(src), _p(out), log_n, q, e)
    return out


# ----------------------------------------------------------------- keyswitch
def keyswitch(ct: np.ndarray, key: np.ndarray, q, dnum: int, log_n: int, galois_elt: int = 1,
              tables: Tables | None = None, per_ct_keys: bool = False, threads: int = 0) -> np.ndarray:
    """ct [batch][2][L][N] coefficient form; key [dnum][2][L+1][N] (or
    [batch][dnum][2][L+1][N] with per_ct_keys) NTT form; q has L+1 primes."""
    q = _u64(q)
    L = len(q) - 1
    n = 1 << log_n
    ct = _u64(ct)
    key = _u64(key)
    batch = ct.size // (2 * L * n)
    if tables is None:
        tables = Tables(q, log_n)
    out = np.empty_like(ct)
    stride = dnum * 2 * (L + 1) * n if per_ct_keys else 0
    rc = lib().orc_keyswitch(_p(ct), _p(out), _p(key), stride, batch, _p(q), L, dnum, log_n, galois_elt,
                             _p(tables.fwd), _p(tables.inv), _p(tables.invn), threads)
    if rc:
        raise ValueError(f"orc_keyswitch failed ({rc})")
    return out


# ---------------------------------------------------------------------- GEMM
def share_gemm(x: np.ndarray, w: np.ndarray, shifts: np.ndarray | None = None, mask_bits: int = 64,
               threads: int = 0) -> np.ndarray:
    x = _u64(x)
    w = np.ascontiguousarray(w)
    assert w.dtype in (np.int8, np.int32)
    m, k = x.shape
    n, k2 = w.shape
    assert k == k2
    y = np.empty((m, n), dtype=np.uint64)
    sh = None if shifts is None else np.ascontiguousarray(shifts, dtype=np.int8)
    rc = lib().orc_share_gemm(_p(x), _p(w), 8 if w.dtype == np.int8 else 32, _p(sh), _p(y), m, k, n,
                              mask_bits, threads)
    assert rc == 0
    return y


def lift59(v: int, q: int) -> int:
    return int(lib().orc_lift59(v, q))


def local_dot_scale(shares: np.ndarray, weights: np.ndarray, delta, r: int, q) -> np.ndarray:
    shares = _u64(shares)
    weights = _u64(weights)
    slots, words = shares.shape
    q = _u64(q)
    delta = _u64(delta)
    out = np.empty((slots, len(q)), dtype=np.uint64)
    lib().orc_local_dot_scale(_p(shares), _p(weights), words, slots, _p(delta), r, _p(q), len(q), _p(out))
    return out


def dyadic_mac(a: np.ndarray, w: np.ndarray, q) -> np.ndarray:
    """a [blocks][limbs][N], w [blocks][wl][N] (limb l uses w limb l % wl, prime l % P)."""
    a = _u64(a)
    w = _u64(w)
    q = _u64(q)
    blocks, limbs, n = a.shape
    wl = w.shape[1]
    out = np.empty((limbs, n), dtype=np.uint64)
    lib().orc_dyadic_mac(_p(a), _p(w), _p(out), blocks, limbs, n, len(q), _p(q), wl)
    return out


def lift59_blocks(ring: np.ndarray, q, n: int, width: int = 0) -> np.ndarray:
    """[blocks][len(q)][n] lifted residues; ring is [blocks][n] (width 0) or [blocks][width]."""
    ring = _u64(ring)
    q = _u64(q)
    per = width if width else n
    blocks = ring.size // per
    out = np.empty((blocks, len(q), n), dtype=np.uint64)
    lib().orc_lift59_blocks(_p(ring), _p(out), blocks, n, width, _p(q), len(q))
    return out


def ring_add(a, b, bits: int = 59) -> np.ndarray:
    a, b = _u64(a), _u64(b)
    out = np.empty_like(a)
    lib().orc_ring_add(_p(a), _p(b), _p(out), a.size, bits)
    return out


def ring_scale(a, k: int, bits: int = 59) -> np.ndarray:
    a = _u64(a)
    out = np.empty_like(a)
    lib().orc_ring_scale(_p(a), int(k) & (2**64 - 1), _p(out), a.size, bits)
    return out


def ring_layout(a, index_map) -> np.ndarray:
    a, m = _u64(a), _u64(index_map)
    out = np.empty(m.size, dtype=np.uint64)
    lib().orc_ring_layout(_p(a), a.size, _p(m), _p(out), m.size)
    return out


def ring_sum_rows(a, cols: int, bits: int = 59) -> np.ndarray:
    a = _u64(a)
    rows = a.size // cols
    out = np.empty(rows, dtype=np.uint64)
    lib().orc_ring_sum_rows(_p(a), _p(out), rows, cols, bits)
    return out


def matrix_product(ct: np.ndarray, ring: np.ndarray, q, log_n: int, threads: int = 0) -> np.ndarray:
    """matrix_gpu::Matrix::evaluate (matrix.cu:56-70): ct [blocks][2][P][N] coefficient form,
    ring [blocks][N] ring-2^59 words -> INTT(sum_b NTT(ct_b) (.) NTT(lift(ring_b))) [2][P][N]."""
    n = 1 << log_n
    P = len(q)
    t = Tables(q, log_n)
    ct = _u64(ct).reshape(-1, 2 * P, n)
    blocks = ct.shape[0]
    w = lift59_blocks(_u64(ring).reshape(blocks, n), q, n)           # [blocks][P][N]
    wf = ntt(w.reshape(blocks * P, n), t, threads=threads).reshape(blocks, P, n)
    cf_ = ntt(ct.reshape(blocks * 2 * P, n), t, threads=threads).reshape(blocks, 2 * P, n)
    acc = dyadic_mac(cf_, wf, q)                                       # [2P][N]
    return ntt(acc, t, inverse=True, threads=threads).reshape(2, P, n)


def enc0(samples: np.ndarray, pk: np.ndarray, q, log_n: int, threads: int = 0) -> np.ndarray:
    """PublicZero::evaluate (enc0.cu:99-114): samples [3][K][N] (u, e0, e1 residues), pk [2][K][N]
    NTT form -> ModDown(INTT(NTT(u) * pk_c) + e_c) [2][K-1][N]."""
    q = _u64(q)
    K = len(q)
    n = 1 << log_n
    t = Tables(q, log_n)
    s = _u64(samples)
    k = _u64(pk)
    out = np.empty((2, K - 1, n), dtype=np.uint64)
    rc = lib().orc_enc0(_p(s), _p(k), _p(out), _p(q), K - 1, log_n, _p(t.fwd), _p(t.inv), _p(t.invn), threads)
    assert rc == 0
    return out


# ------------------------------------------------- token-resident path, packing
def _monomial_shift_limbs(a: np.ndarray, q, log_n: int, e: int) -> np.ndarray:
    """x^e times every [..][P][N] limb (limb l over q[l % P])."""
    n = 1 << log_n
    q = _u64(q)
    flat = _u64(a).reshape(-1, n)
    out = np.empty_like(flat)
    for l in range(flat.shape[0]):
        lib().orc_monomial_shift(_p(flat[l]), _p(out[l]), log_n, int(q[l % len(q)]), e)
    return out.reshape(np.shape(a))


def token_inputs(ct: np.ndarray, q, log_n: int, threads: int = 0) -> np.ndarray:
    """The resident form of TokenWeights' inputs (resident/seal_adapter.cpp:29-33):
    ct [blocks][slots][2][P][N] coefficient form -> [blocks][slots*2*P][N] NTT form."""
    n = 1 << log_n
    ct = _u64(ct)
    blocks = ct.shape[0]
    return ntt(ct.reshape(-1, n), Tables(q, log_n), threads=threads).reshape(blocks, -1, n)


def token_product(resident: np.ndarray, ring: np.ndarray, q, log_n: int, width: int, threads: int = 0) -> np.ndarray:
    """sum_b resident_b (.) NTT(lift of ring_b reversed into coefficients
    width-1..0) over NTT-form inputs [blocks][limbs][N] -> [limbs][N]
    (resident.cu:143-145: lift, forward stages, accumulate)."""
    n = 1 << log_n
    P = len(q)
    ring = _u64(ring)
    blocks = ring.size // width
    w = lift59_blocks(ring.reshape(blocks, width), q, n, width)            # [blocks][P][N]
    wf = ntt(w.reshape(blocks * P, n), Tables(q, log_n), threads=threads).reshape(blocks, P, n)
    return dyadic_mac(_u64(resident), wf, q)


def token_evaluate(ct: np.ndarray, ring: np.ndarray, q, log_n: int, width: int, threads: int = 0) -> np.ndarray:
    """TokenWeights::evaluate (resident.cu:135-151; the CPU sequence of
    check_resident.cpp:51-59): ct [blocks][slots][2][P][N] coefficient form,
    ring [blocks][width] -> [slots][2][P][N] NTT form,
    sum_b NTT(ct_b) (.) NTT(lift of ring_b reversed into coefficients width-1..0)."""
    n = 1 << log_n
    P = len(q)
    acc = token_product(token_inputs(ct, q, log_n, threads), ring, q, log_n, width, threads)
    return acc.reshape(-1, 2, P, n)


def token_scaled(local, q, t_bits: int = 59) -> np.ndarray:
    """Delta-scaled local terms [slots][P] (resident/seal_adapter.cpp:43-53):
    Delta_k m + floor((r m + t/2) / t) mod q_k, Delta_k = floor(Q/t) mod q_k,
    r = Q mod t, Q = prod q."""
    Q = 1
    for x in q:
        Q *= int(x)
    t = 1 << t_bits
    r = Q % t
    out = np.empty((len(local), len(q)), dtype=np.uint64)
    for s, m in enumerate(local):
        m = int(m)
        fix = (r * m + t // 2) // t
        for k, x in enumerate(q):
            out[s, k] = (m * ((Q // t) % int(x)) + fix) % int(x)
    return out


def token_finished(ct: np.ndarray, ring: np.ndarray, scaled: np.ndarray, q, log_n: int, width: int,
                   threads: int = 0, resident: np.ndarray | None = None) -> np.ndarray:
    """TokenWeights::evaluate_device (resident.cu:152-173): INTT of the
    evaluate() product, scaled[slot][k] added at coefficient width-1 of c0,
    then the negacyclic shift by x^-(width-1) (add_shift, resident.cu:54-59).
    `resident` (token_inputs of ct) skips the inputs' transform."""
    n = 1 << log_n
    P = len(q)
    if resident is None:
        resident = token_inputs(ct, q, log_n, threads)
    acc = token_product(resident, ring, q, log_n, width, threads).reshape(-1, 2, P, n)
    slots = acc.shape[0]
    coeff = ntt(acc.reshape(-1, n), Tables(q, log_n), inverse=True, threads=threads).reshape(slots, 2, P, n)
    qa = _u64(q)
    sc = _u64(scaled).reshape(slots, P)
    coeff[:, 0, :, width - 1] = (coeff[:, 0, :, width - 1] + sc) % qa
    return _monomial_shift_limbs(coeff, q, log_n, 2 * n - (width - 1))


def pack_pair(left: np.ndarray, right: np.ndarray, level: int, keys: np.ndarray, q, dnum: int, log_n: int,
              tables: Tables | None = None, threads: int = 0) -> np.ndarray:
    """Acyclic packing merge (pack_pair, bfv_acyclic_pack.hpp:44-52; GPU
    sequence switch.cu:157-185): right times x^(N >> (level+1)); the sum is
    switched with key [level][0] (element 1), the difference with key
    [level][1] (element 2^(level+1)+1, Galois applied first); results added.
    left/right [2][L][N] coefficient form, keys [levels][2][dnum][2][L+1][N]."""
    q = _u64(q)
    L = len(q) - 1
    n = 1 << log_n
    dq = q[:L]
    shifted = _monomial_shift_limbs(_u64(right).reshape(2, L, n), dq, log_n, n >> (level + 1))
    lft = _u64(left).reshape(2, L, n)
    qcol = dq.reshape(1, L, 1)
    total = (lft + shifted) % qcol
    diff = (lft + qcol - shifted) % qcol
    k = _u64(keys)
    kl = k.reshape(-1, 2, dnum * 2 * (L + 1) * n)[level]
    if tables is None:
        tables = Tables(q, log_n)
    a = keyswitch(total[None], kl[0], q, dnum, log_n, 1, tables=tables, threads=threads)[0]
    b = keyswitch(diff[None], kl[1], q, dnum, log_n, (2 << level) + 1, tables=tables, threads=threads)[0]
    return (a + b) % qcol


def pack_tree(leaves: np.ndarray, keys: np.ndarray, q, dnum: int, log_n: int, threads: int = 0) -> np.ndarray:
    """The stack merge of bfv_token_batch.inc:194-206 over [leaves][slots][2][L][N]
    coordinates in arrival order (leaf count a power of two): every arrival
    merges with the stack entries below it, left = the older entry.  Returns
    the roots [slots][2][L][N]."""
    q = _u64(q)
    lv = _u64(leaves)
    m, slots = lv.shape[0], lv.shape[1]
    tables = Tables(q, log_n)
    roots = []
    for s in range(slots):
        stack = {}
        for c in range(m):
            cur, level = lv[c, s], 0
            while level in stack:
                cur = pack_pair(stack.pop(level), cur, level, keys, q, dnum, log_n, tables, threads)
                level += 1
            stack[level] = cur
        assert list(stack) == [m.bit_length() - 1]
        roots.append(stack[m.bit_length() - 1])
    return np.stack(roots)
