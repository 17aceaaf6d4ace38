"""packed_target (bfv_acyclic_pack.hpp:53-56) through the C ABI, on the CPU.

Pinned by the packing tree itself rather than by the bit-reversal formula:
every leaf c of a tree over 2^levels coordinates holds only a constant term
(c + 1, as the token finish leaves a coordinate at x^0), the leaves are merged
level by level in the stack order of bfv_token_batch.inc:194-206 with the
plaintext map of a packing pair, m_L + X^s m_R + sigma_g(m_L - X^s m_R),
s = N >> (l+1), g = 2^(l+1) + 1 (bfv_acyclic_pack.hpp:44-52), evaluated on
sparse polynomials; the root then holds 2^levels (c + 1) at exactly one
coefficient per leaf, which must be packed_target(c)."""
import pytest

import praghip


def monomial(poly, e, n):
    out = {}
    for i, v in poly.items():
        j = (i + e) % (2 * n)
        out[j % n] = out.get(j % n, 0) + (-v if j >= n else v)
    return out


def galois(poly, g, n):
    out = {}
    for i, v in poly.items():
        j = (i * g) % (2 * n)
        out[j % n] = out.get(j % n, 0) + (-v if j >= n else v)
    return out


def add(*polys, sign=None):
    out = {}
    for k, p in enumerate(polys):
        s = 1 if sign is None else sign[k]
        for i, v in p.items():
            out[i] = out.get(i, 0) + s * v
    return {i: v for i, v in out.items() if v}


def pack_plain(ml, mr, level, n):
    sh = monomial(mr, n >> (level + 1), n)
    d = galois(add(ml, sh, sign=[1, -1]), (2 << level) + 1, n)
    return add(ml, sh, d)


@pytest.mark.parametrize("levels,log_n", [(9, 14), (4, 6), (3, 3), (1, 4)])
def test_packed_target_matches_tree(levels, log_n):
    n = 1 << log_n
    nodes = [{0: c + 1} for c in range(1 << levels)]
    for level in range(levels):
        nodes = [pack_plain(nodes[2 * a], nodes[2 * a + 1], level, n) for a in range(len(nodes) // 2)]
    root = nodes[0]
    assert len(root) == 1 << levels
    where = {v >> levels: i for i, v in root.items()}
    assert all(v % (1 << levels) == 0 for v in root.values())
    for c in range(1 << levels):
        assert praghip.packed_target(c, levels, log_n) == where[c + 1], c


def test_packed_target_reference_values_and_errors():
    # 9 levels at N = 16384: coordinate 1 lands half-way, spacing 32
    assert praghip.packed_target(0) == 0
    assert praghip.packed_target(1) == 8192
    assert praghip.packed_target(2) == 4096
    assert praghip.packed_target(511) == 511 * 32
    assert praghip.packed_target(512 + 3) == praghip.packed_target(3)  # low 9 bits, as the reference
    for levels, log_n in [(0, 14), (15, 14), (5, 4), (1, 15)]:
        with pytest.raises(praghip.PraghipError, match="E_PACK_KEY_LEVELS"):
            praghip.packed_target(1, levels, log_n)
