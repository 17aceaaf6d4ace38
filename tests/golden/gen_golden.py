"""Writes the committed golden fixtures of tests/golden/ from closed_form.py.

Run from the repository root:  python tests/golden/gen_golden.py
Every expected value here comes from the closed forms (direct NTT evaluation,
big-integer keyswitch, integer GEMM), never from the oracle or the HIP library.
The only reference-derived data are the locked primes and Q values of
implementation_v1/artifacts/bfv_context.json, restated as constants.
"""
from __future__ import annotations

import hashlib
import json
import os
import sys

import numpy as np

sys.path.insert(0, os.path.dirname(os.path.abspath(__file__)))
import closed_form as cf  # noqa: E402

OUT = os.path.dirname(os.path.abspath(__file__))

# bfv_context.json: Q at the key level (chain_index 6, 7 primes) and data level (chain_index 5).
Q_KEY = 2707685248123455388423494518824985952592310062380342907551585901899183014955553421723044638653468080151073037037004040661303297
Q_DATA = 2348542582738122206855069782186871985803490093435884473355019481976564023197476749942235793077603734285221889

SEED_BASE = 0x5052414700000000


def seed(config: int, tag: int = 0) -> int:
    return SEED_BASE | (tag << 8) | config


def input_digest(rows) -> str:
    return hashlib.sha256(np.asarray(rows, dtype=np.uint64).tobytes()).hexdigest()


def primes_fixture():
    n = 16384
    psis = [cf.minimal_psi(q, n) for q in cf.LOCKED_PRIMES]
    sets = {
        "locked_16384": cf.LOCKED_PRIMES,
        "c1_54bit_4096": cf.primes_below(54, 4096, 2),
        "c2_50bit_16384": cf.primes_below(50, 16384, 6),
        "c3_special_60bit_16384": cf.primes_below(60, 16384, 1),
    }
    return {
        "locked_primes": [str(q) for q in cf.LOCKED_PRIMES],
        "Q_key_level": str(Q_KEY),
        "Q_data_level": str(Q_DATA),
        "psi_16384": [str(p) for p in psis],
        "sets": {k: [str(q) for q in v] for k, v in sets.items()},
    }


def ntt_small_fixture():
    arrays = {}
    primes = [cf.LOCKED_PRIMES[0], cf.LOCKED_PRIMES[6], cf.primes_below(54, 64, 1)[0], cf.primes_below(50, 64, 1)[0]]
    for log_n in (1, 2, 3, 4, 6):
        n = 1 << log_n
        for pi, q in enumerate(primes):
            if (q - 1) % (2 * n):
                continue
            psi = cf.minimal_psi(q, n)
            a = cf.residues(seed(0, 16 + log_n * 4 + pi), 1, n, [q])[0]
            arrays[f"n{n}_p{pi}_q"] = np.array([q], dtype=np.uint64)
            arrays[f"n{n}_p{pi}_in"] = np.array(a, dtype=np.uint64)
            arrays[f"n{n}_p{pi}_out"] = np.array(cf.ntt(a, q, psi), dtype=np.uint64)
    return arrays


def ntt_sampled_fixture():
    cases = []
    plan = [
        ("locked_16384", 14, cf.LOCKED_PRIMES),
        ("c2_50bit_16384", 14, cf.primes_below(50, 16384, 6)),
        ("c1_54bit_4096", 12, cf.primes_below(54, 4096, 2)),
    ]
    for name, log_n, primes in plan:
        n = 1 << log_n
        for pi, q in enumerate(primes):
            psi = cf.minimal_psi(q, n)
            s = seed(1, 64 + len(cases))
            a = cf.residues(s, 1, n, [q])[0]
            ks = [0, 1, 2, 3, n // 2, n // 2 + 1, n - 2, n - 1]
            ks += [(cf.splitmix64(s ^ 0xABCDEF, i) % n) for i in range(8)]
            cases.append({
                "set": name, "log_n": log_n, "q": str(q), "seed": str(s),
                "input_sha256": input_digest(a),
                "k": ks, "expected": [str(cf.ntt_point(a, q, psi, k, log_n)) for k in ks],
            })
    return cases


def keyswitch_fixture():
    arrays = {}
    n = 16
    c50 = cf.primes_below(50, n, 6)
    c60 = cf.primes_below(60, n, 1)
    setups = [
        ("locked_d6", cf.LOCKED_PRIMES, 6),
        ("c3_d3", c50 + c60, 3),
        ("c3_d2", c50 + c60, 2),
        ("c3_d6", c50 + c60, 6),
        ("c3_d4", c50 + c60, 4),  # digits of 2, 2, 1, 1 primes
    ]
    for si, (name, q, dnum) in enumerate(setups):
        L = len(q) - 1
        for gi, g in enumerate((1, 3, 5, 2 * n - 1)):
            s = seed(2, 16 * si + gi)
            ct = cf.residues(s, 2 * L, n, q[:L])
            ct = [ct[:L], ct[L:]]
            key = cf.residues(s + 1, dnum * 2 * (L + 1), n, q)
            key = [[key[(j * 2 + c) * (L + 1):(j * 2 + c + 1) * (L + 1)] for c in range(2)] for j in range(dnum)]
            out = cf.keyswitch(ct, key, q, dnum, g)
            tag = f"{name}_g{g}"
            arrays[tag + "_q"] = np.array(q, dtype=np.uint64)
            arrays[tag + "_meta"] = np.array([dnum, g, n], dtype=np.uint64)
            arrays[tag + "_ct"] = np.array(ct, dtype=np.uint64)
            arrays[tag + "_key"] = np.array(key, dtype=np.uint64)
            arrays[tag + "_out"] = np.array(out, dtype=np.uint64)
    return arrays


def gemm_fixture():
    arrays = {}
    cases = [("i8_a", 3, 17, 5, 8, False, 64), ("i8_shift59", 4, 40, 6, 8, True, 59),
             ("i32_a", 5, 33, 7, 32, False, 64), ("i32_shift59", 2, 70, 9, 32, True, 59)]
    for ci, (name, m, k, n, wb, with_shift, mask) in enumerate(cases):
        s = seed(4, ci)
        x = [[cf.splitmix64(s, b * k + j) for j in range(k)] for b in range(m)]
        if wb == 8:
            w = [[((cf.splitmix64(s + 1, o * k + j) * 255) >> 64) - 127 for j in range(k)] for o in range(n)]
        else:  # reference f12 domain |w| <= 2^20 (numeric_profile.hpp:14)
            w = [[((cf.splitmix64(s + 1, o * k + j) * ((1 << 21) + 1)) >> 64) - (1 << 20) for j in range(k)]
                 for o in range(n)]
            w[0][0], w[0][1], w[1][0] = 1 << 20, -(1 << 20), -1
        sh = [(cf.splitmix64(s + 2, o) * 8) >> 64 for o in range(n)] if with_shift else None
        y = cf.share_gemm(x, w, sh, mask)
        arrays[name + "_x"] = np.array(x, dtype=np.uint64)
        arrays[name + "_w"] = np.array(w, dtype=np.int8 if wb == 8 else np.int32)
        if sh is not None:
            arrays[name + "_shift"] = np.array(sh, dtype=np.int8)
        arrays[name + "_mask"] = np.array([mask], dtype=np.uint64)
        arrays[name + "_y"] = np.array(y, dtype=np.uint64)
    # dev_matrix_probe.cpp:12-20,31-32 synthetic shares: the two parties' local
    # GEMMs must sum to the plaintext product mod 2^59.
    MASK = (1 << 59) - 1
    batch, inner, outputs = 3, 40, 6
    whole = [[(((j * 13 + b * 19 + 7) % 255) - 127) & MASK for j in range(inner)] for b in range(batch)]
    weight = [[0 if o == 1 else ((j * 7 + o * 11 + 3) % 63) - 31 for j in range(inner)] for o in range(outputs)]
    client = [[(0x21fedcba987654 + b * 797 + j * 125939) & MASK for j in range(inner)] for b in range(batch)]
    server = [[(whole[b][j] - client[b][j]) & MASK for j in range(inner)] for b in range(batch)]
    plain = cf.share_gemm(whole, weight, None, 59)
    arrays["probe_client"] = np.array(client, dtype=np.uint64)
    arrays["probe_server"] = np.array(server, dtype=np.uint64)
    arrays["probe_weight"] = np.array(weight, dtype=np.int8)
    arrays["probe_plain"] = np.array(plain, dtype=np.uint64)
    return arrays


def main():
    with open(os.path.join(OUT, "primes.json"), "w") as f:
        json.dump(primes_fixture(), f, indent=1)
    np.savez_compressed(os.path.join(OUT, "ntt_small.npz"), **ntt_small_fixture())
    with open(os.path.join(OUT, "ntt_sampled.json"), "w") as f:
        json.dump(ntt_sampled_fixture(), f, indent=1)
    np.savez_compressed(os.path.join(OUT, "keyswitch_small.npz"), **keyswitch_fixture())
    np.savez_compressed(os.path.join(OUT, "gemm_small.npz"), **gemm_fixture())
    print("fixtures written to", OUT)


if __name__ == "__main__":
    main()
