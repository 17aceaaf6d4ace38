"""The allocation-free local dot (praghip_local_dot_scale_noalloc) against the
entry point it varies (praghip_local_dot_scale with a caller workspace) and
the oracle, through the C ABI: two calls in a row on the same device scratch,
the second with fewer slots and words, then the slot limit."""
import numpy as np
import pytest

import closed_form as cf
import oracle
import praghip
from conftest import from_dev, to_dev

pytestmark = pytest.mark.gpu
T59 = (1 << 59) - 1


def _case(slots, words, q, seed):
    shares = (oracle.fill_u64(slots * words, seed) & np.uint64(T59)).reshape(slots, words)
    w = oracle.fill_u64(words, seed + 1) & np.uint64(T59)
    return shares, w


def test_local_dot_noalloc_matches_workspace_entry(gpu):
    import torch
    q = cf.LOCKED_PRIMES[:6]
    delta, r = praghip.bfv_delta(q)
    # first call at the limit (64 slots fill the whole scratch), second smaller
    for slots, words, seed in [(64, 155648, 0x5052414700000F01), (3, 1000, 0x5052414700000F02)]:
        print(f"[noalloc] slots={slots} words={words}", flush=True)
        shares, w = _case(slots, words, q, seed)
        ds, dw = to_dev(shares), to_dev(w)
        out = torch.zeros(slots * len(q), dtype=torch.int64, device=gpu)
        praghip.local_dot_scale_noalloc(ds, dw, q, delta, r, out)
        ref = praghip.local_dot_scale(ds, dw, q, delta, r)
        torch.cuda.synchronize()
        got = from_dev(out).reshape(slots, len(q))
        np.testing.assert_array_equal(got, from_dev(ref))
        np.testing.assert_array_equal(got, oracle.local_dot_scale(shares, w, delta, r, q))


def test_local_dot_noalloc_50bit_primes_and_limit(gpu):
    import torch
    q = cf.primes_below(50, 1 << 15, 6)
    delta, r = praghip.bfv_delta(q)
    shares, w = _case(5, 4097, q, 0x5052414700000F03)
    ds, dw = to_dev(shares), to_dev(w)
    out = torch.zeros(5 * len(q), dtype=torch.int64, device=gpu)
    praghip.local_dot_scale_noalloc(ds, dw, q, delta, r, out)
    torch.cuda.synchronize()
    np.testing.assert_array_equal(from_dev(out).reshape(5, len(q)), oracle.local_dot_scale(shares, w, delta, r, q))
    # above the scratch's 64 slots: refused on the host before any launch
    big = torch.zeros((65, 8), dtype=torch.int64, device=gpu)
    with pytest.raises(praghip.PraghipError) as e:
        praghip.local_dot_scale_noalloc(big, dw[:8], q, delta, r,
                                        torch.zeros(65 * len(q), dtype=torch.int64, device=gpu))
    assert "E_LOCAL_NOALLOC_SLOTS" in e.value.text
