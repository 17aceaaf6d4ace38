"""Host-side check of the float-path NTT arithmetic (q < 2^50): the device
code's mul_f64_hq / reduce_f64 and re-centring schedule, run stage by stage on
the CPU, keep every intermediate an exact integer congruent to the true
residue, every product factor within 4q and every value below 2^53, and the
outputs equal the oracle's transform (which is pinned by the closed form)."""
import os
import shutil
import subprocess
import tempfile

import numpy as np
import pytest

import closed_form as cf
import oracle

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HIPCC = shutil.which("hipcc") or "/opt/rocm/bin/hipcc"


def _inputs(q, n, seed):
    rnd = oracle.fill_residues(1, n, [q], seed)[0]
    top = np.full(n, q - 1, dtype=np.uint64)
    alt = np.where(np.arange(n) % 2 == 0, np.uint64(q - 1), np.uint64(0)).astype(np.uint64)
    half = np.full(n, q // 2 + 1, dtype=np.uint64)
    return [rnd, top, alt, half]


@pytest.mark.skipif(not os.path.exists(HIPCC), reason="no hipcc")
def test_float_path_exact_and_bounded():
    cases = [(q, 14) for q in cf.primes_below(50, 16384, 6)]
    cases += [(cf.primes_below(50, 1 << lg, 1)[0], lg) for lg in (4, 5, 6, 7, 10, 12, 13)]
    with tempfile.TemporaryDirectory() as d:
        exe = os.path.join(d, "f64_check")
        subprocess.run([HIPCC, "-O2", "-std=c++17", "-x", "hip", "--offload-arch=gfx950",
                        "-ffp-contract=off", "-I", os.path.join(ROOT, "privacy-rag_amd", "csrc"),
                        os.path.join(ROOT, "tests", "cpp", "f64_ntt_check.cpp"), "-o", exe],
                       check=True, capture_output=True)
        for q, lg in cases:
            n = 1 << lg
            t = oracle.Tables([q], lg)
            ins = _inputs(q, n, q % 1000)
            path = os.path.join(d, "case.bin")
            with open(path, "wb") as f:
                np.array([q, lg, len(ins)], dtype=np.uint64).tofile(f)
                t.fwd[0].tofile(f)
                t.inv[0].tofile(f)
                t.invn[0].tofile(f)
                for a in ins:
                    a.astype(np.uint64).tofile(f)
                    oracle.ntt(a[None], t)[0].tofile(f)
            r = subprocess.run([exe, path], capture_output=True, text=True)
            assert r.returncode == 0 and "ALL OK" in r.stdout, (q, lg, r.stdout, r.stderr)


@pytest.mark.skipif(not os.path.exists(HIPCC), reason="no hipcc")
def test_integer_helpers_exact():
    """shoup_quotient, mul_shoup, mul_barrett, mul_mont and mul_f64_hq of modarith.hpp against
    128-bit host arithmetic (and the float product against its bound)."""
    with tempfile.TemporaryDirectory() as d:
        exe = os.path.join(d, "modarith_check")
        subprocess.run([HIPCC, "-O2", "-std=c++17", "-x", "hip", "--offload-arch=gfx950", "-ffp-contract=off",
                        "-I", os.path.join(ROOT, "privacy-rag_amd", "csrc"),
                        os.path.join(ROOT, "tests", "cpp", "modarith_check.cpp"), "-o", exe],
                       check=True, capture_output=True)
        r = subprocess.run([exe], capture_output=True, text=True)
        assert r.returncode == 0 and "ALL OK" in r.stdout, r.stdout
