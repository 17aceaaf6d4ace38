"""BFV parameter sets of the hot path.

LOCKED_PRIMES are the reference's locked key-level primes
(implementation_v1/artifacts/bfv_context.json; bfv.cpp:91-105): six data primes
and the special prime last.  ``primes_below`` is SEAL's CoeffModulus::Create
rule (the largest primes < 2^bits congruent to 1 mod 2N), used for the
50/54-bit benchmark sets.
"""
from __future__ import annotations

LOCKED_PRIMES = (
    1152921504599080961, 1152921504600260609, 1152921504604979201, 1152921504605962241,
    1152921504606584833, 1152921504606683137, 1152921504606748673,
)
PLAIN_MODULUS = 1 << 59  # bfv.cpp:96, secure_ops.hpp:10


def _is_prime(n: int) -> bool:
    if n < 2:
        return False
    bases = (2, 3, 5, 7, 11, 13, 17, 19, 23, 29, 31, 37)
    for p in bases:
        if n % p == 0:
            return n == p
    d, s = n - 1, 0
    while not d & 1:
        d >>= 1
        s += 1
    for a in bases:
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
    """The `count` largest primes below 2^bits with q == 1 mod 2n, ascending."""
    out, v = [], (1 << bits) - 2 * n + 1
    while len(out) < count and v > 2 * n:
        if _is_prime(v):
            out.append(v)
        v -= 2 * n
    return sorted(out)


def primes_n4096_54bit() -> list[int]:
    """N=4096, two ~54-bit primes."""
    return primes_below(54, 4096, 2)


def primes_n16384_50bit() -> list[int]:
    """N=16384, six ~50-bit primes."""
    return primes_below(50, 16384, 6)


def primes_n16384_switch() -> list[int]:
    """N=16384: six ~50-bit data primes + one ~60-bit special prime (last)."""
    return primes_below(50, 16384, 6) + primes_below(60, 16384, 1)
