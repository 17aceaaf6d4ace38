"""The device entry points under HIP graph capture: a forward+inverse NTT, a
batched keyswitch (whose work-queue counters the kernel itself zeroes at the
end of every launch), a split-K share GEMM (output cleared by a kernel, not a
memset) and a packing-tree level are captured once with torch's graph API and
replayed several times, with eager work and synchronisations between the
replays; every replay must reproduce the eager results bit for bit."""
import numpy as np
import pytest

import closed_form as cf
import oracle
import praghip
from conftest import from_dev, to_dev

pytestmark = pytest.mark.gpu


def test_graph_replays_match_eager(gpu):
    import torch
    print("[graph] capture and replay", flush=True)
    log_n, n, L, dnum, batch = 14, 1 << 14, 6, 3, 16
    q = cf.primes_below(50, 2 * n, 6) + cf.primes_below(60, 2 * n, 1)
    ntt = praghip.NttBatch(q[:L], log_n)
    sw = praghip.Switch(q, log_n, dnum, max_batch=batch)
    ct = to_dev(oracle.fill_residues(batch * 2 * L, n, q[:L], 11))
    keys = to_dev(oracle.fill_residues(batch * dnum * 2 * (L + 1), n, q, 12))
    limbs = to_dev(oracle.fill_residues(96, n, q[:L], 13))
    x = to_dev(oracle.fill_u64(512 * 3072, 14).reshape(512, 3072))
    w = torch.from_numpy(oracle.fill_i8(1024 * 3072, 15).reshape(1024, 3072)).to("cuda")
    pq = q[:2] + q[-1:]  # two data primes and the special prime, N = 1024
    pk_keys = oracle.fill_residues(2 * 2 * 2 * 2 * 3, n >> 4, pq, 16)  # [2 levels][2][dnum 2][2][3][N]
    pk = praghip.Packing(pq, 10, pk_keys, dnum=2)
    pairs = to_dev(oracle.fill_residues(4 * 2 * 2, n >> 4, q[:2], 17).reshape(4, -1))  # 4 ciphertexts

    def work(ks_out, lim, y, pk_out):
        ntt.forward(lim)
        ntt.inverse(lim)
        sw.keyswitch(ct, ks_out, keys=keys, key_stride=sw.key_words)
        praghip.share_gemm(x, w, y=y, mask_bits=59)
        pk.pair_device(pairs[:2], pairs[2:], 1, out=pk_out)

    # eager reference
    e_ks, e_lim, e_y, e_pk = torch.empty_like(ct), limbs.clone(), torch.empty((512, 1024), dtype=torch.int64,
                                                                              device="cuda"), torch.empty_like(pairs[:2])
    work(e_ks, e_lim, e_y, e_pk)
    torch.cuda.synchronize()
    # graph
    g_ks, g_lim, g_y, g_pk = torch.empty_like(ct), limbs.clone(), torch.empty_like(e_y), torch.empty_like(e_pk)
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):  # warm-up on the capture stream
        work(g_ks, g_lim, g_y, g_pk)
    torch.cuda.current_stream().wait_stream(side)
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        work(g_ks, g_lim, g_y, g_pk)
    for rep in range(4):
        g_ks.zero_()
        g_y.zero_()
        g_pk.zero_()
        g_lim.copy_(limbs)
        ntt.forward(e_lim)  # eager work between replays
        ntt.inverse(e_lim)
        torch.cuda.synchronize()
        graph.replay()
        torch.cuda.synchronize()
        assert torch.equal(g_ks, e_ks), f"keyswitch replay {rep}"
        assert torch.equal(g_lim, limbs), f"NTT round trip replay {rep}"
        assert torch.equal(g_y, e_y), f"GEMM replay {rep}"
        assert torch.equal(g_pk, e_pk), f"packing replay {rep}"
    np.testing.assert_array_equal(from_dev(e_y)[:4], oracle.share_gemm(from_dev(x)[:4], from_dev(w), None, 59))
