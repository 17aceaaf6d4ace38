"""GPU parity of the token-resident path (TokenWeights, resident.cu:104-195) and
of the acyclic packing tree (Packing, bfv_gpu_packing.hpp:10-45) against the
oracle (pinned by the negacyclic closed form of the resident chain and by the
packing decryption invariant): evaluate, finished with host and bound local
terms, the device entry points, the stack, pair / pair_device / tree_device,
the reference's token loop (bfv_token_batch.inc:194-206) end to end, the
reference's errors and the cleanup counts."""
import numpy as np
import pytest

import closed_form as cf
import oracle
import praghip
from conftest import from_dev, to_dev

pytestmark = pytest.mark.gpu

MASK59 = (1 << 59) - 1


def _ring(blocks, width, seed, boundary=False):
    """Ring words of signed weights |w| <= 2^20; `boundary` gives the
    reference's seventh column case (check_resident.cpp:48)."""
    count = blocks * width
    if boundary:
        edge = np.array([0, 1, -1, 1 << 20, -(1 << 20), (1 << 20) - 1, -((1 << 20) - 1)], dtype=np.int64)
        v = edge[np.arange(count) % 7]
    else:
        v = (oracle.fill_u64(count, seed) % np.uint64(2 * (1 << 20) + 1)).astype(np.int64) - (1 << 20)
    return (v.astype(np.uint64) & np.uint64(MASK59)).reshape(blocks, width)


def _inputs(q, n, blocks, slots, seed):
    """[blocks][slots][2][P][N] coefficient-form residues with the reference's
    0 / q-1 / 1 pattern every 13 coefficients (check_resident.cpp:35)."""
    P = len(q)
    ct = oracle.fill_residues(blocks * slots * 2 * P, n, q, seed).reshape(blocks, slots, 2, P, n)
    qa = np.array(q, dtype=np.uint64).reshape(1, 1, 1, P, 1)
    j = np.arange(n) % 13
    ct[..., j == 0] = 0
    ct[..., j == 1] = np.broadcast_to(qa - np.uint64(1), ct[..., j == 1].shape)
    ct[..., j == 2] = 1
    return ct


def _delta(q):
    Q = 1
    for x in q:
        Q *= int(x)
    return [(Q >> 59) % int(x) for x in q], Q & MASK59


@pytest.mark.parametrize("slots", [1, 4])
def test_token_reference_size(gpu, slots):
    """The reference's shape: N = 16384, the six locked primes, 19 blocks of 8192."""
    print(f"[token] reference size slots={slots}", flush=True)
    log_n, blocks, width = 14, 19, 8192
    n = 1 << log_n
    q = cf.LOCKED_PRIMES[:6]
    ct = _inputs(q, n, blocks, slots, 700 + slots)
    tw = praghip.TokenWeights(q, log_n, ct, width)
    for case in range(2):
        ring = _ring(blocks, width, 710 + case, boundary=case == 1)
        np.testing.assert_array_equal(tw.evaluate(ring), oracle.token_evaluate(ct, ring, q, log_n, width),
                                      err_msg=f"evaluate case {case}")
    ring = _ring(blocks, width, 720)
    local = [int(v) & MASK59 for v in oracle.fill_u64(slots, 721)]
    local[0] = MASK59
    want = oracle.token_finished(ct, ring, oracle.token_scaled(local, q), q, log_n, width)
    batch = tw.evaluate_finished(ring, local)
    for s in range(slots):
        np.testing.assert_array_equal(tw.download(tw.slot_view(batch, s)), want[s], err_msg=f"finished slot {s}")
    # the stack keeps copies: store slot views at two levels and read them back
    tw.stack_store(0, 0, tw.slot_view(batch, slots - 1))
    tw.stack_store(slots - 1, 9, tw.slot_view(batch, 0))
    np.testing.assert_array_equal(tw.download(tw.stack_view(0, 0)), want[slots - 1])
    np.testing.assert_array_equal(tw.download(tw.stack_view(slots - 1, 9)), want[0])
    # bound local shares: m = (shares . ring mod 2^64) & (2^59 - 1) on the device
    shares = (oracle.fill_u64(slots * blocks * width, 722) & np.uint64(MASK59)).reshape(slots, -1)
    tw.bind_local_shares(shares)
    delta, r = _delta(q)
    scaled = oracle.local_dot_scale(shares, ring.reshape(-1), delta, r, q)
    want_local = oracle.token_finished(ct, ring, scaled, q, log_n, width)
    batch = tw.evaluate_local_finished(ring)
    for s in range(slots):
        np.testing.assert_array_equal(tw.download(tw.slot_view(batch, s)), want_local[s], err_msg=f"local slot {s}")
    # TokenWeights::Timing (resident.hpp:11-12) of that call: the lift is in
    # the transform's loads on the locked primes, the phases sum to the kernel time
    ph, t = tw.phase_timing(), tw.timing()
    assert ph.ntt_ms > 0 and ph.dyadic_ms > 0 and ph.finish_ms > 0 and ph.lift_ms == 0
    assert abs(ph.lift_ms + ph.ntt_ms + ph.dyadic_ms + ph.finish_ms - t.kernel_ms) <= 0.05 * t.kernel_ms
    assert ph.initial_input_upload_ms > 0 and ph.ntt_weight_bytes == blocks * 6 * n * 8
    # device entry point, explicit residues and bound shares
    import torch
    out = to_dev(np.zeros((slots, 2, 6, n), dtype=np.uint64))
    tw.evaluate_device(to_dev(ring), out, residues=to_dev(oracle.token_scaled(local, q)))
    torch.cuda.synchronize()
    np.testing.assert_array_equal(from_dev(out), want)
    tw.evaluate_device(to_dev(ring), out)
    torch.cuda.synchronize()
    np.testing.assert_array_equal(from_dev(out), want_local)
    t = tw.timing()
    assert t.device_bytes >= t.sensitive_bytes > 0
    c = tw.close()
    assert c.closed and c.first_hip_error == 0 and c.wipe_synchronized_bytes == c.freed_bytes > 0
    assert tw.close().freed_bytes == c.freed_bytes
    with pytest.raises(praghip.PraghipError, match="E_RESIDENT_CLOSED"):
        tw.evaluate(ring)


@pytest.mark.parametrize("log_n,P,blocks,slots,width", [(12, 3, 2, 3, 4096), (12, 2, 3, 2, 1), (13, 4, 5, 1, 100)])
def test_token_shapes(gpu, log_n, P, blocks, slots, width):
    """Other primes (50-bit), full and single-coefficient widths, odd widths."""
    print(f"[token] log_n={log_n} P={P} blocks={blocks} slots={slots} width={width}", flush=True)
    n = 1 << log_n
    q = cf.primes_below(50, 2 * n, P)
    ct = _inputs(q, n, blocks, slots, 730 + width)
    tw = praghip.TokenWeights(q, log_n, ct, width, levels=3)
    ring = _ring(blocks, width, 731)
    np.testing.assert_array_equal(tw.evaluate(ring), oracle.token_evaluate(ct, ring, q, log_n, width))
    local = [int(v) & MASK59 for v in oracle.fill_u64(slots, 732)]
    want = oracle.token_finished(ct, ring, oracle.token_scaled(local, q), q, log_n, width)
    batch = tw.evaluate_finished(ring, local)
    for s in range(slots):
        np.testing.assert_array_equal(tw.download(tw.slot_view(batch, s)), want[s])
    # 50-bit primes: the lift is a kernel of its own, timed apart
    ph, t = tw.phase_timing(), tw.timing()
    assert ph.lift_ms > 0 and ph.ntt_ms > 0 and ph.dyadic_ms > 0 and ph.finish_ms > 0
    assert abs(ph.lift_ms + ph.ntt_ms + ph.dyadic_ms + ph.finish_ms - t.kernel_ms) <= 0.05 * t.kernel_ms
    tw.close()


def test_token_ready_event_views(gpu):
    """Device views handed over with a ready event (DeviceCipherBatch::ready,
    resident.hpp:17-20): evaluate_device runs on a side stream, an event is
    recorded there, and stack_store / download wait on that event on the
    plan's own stream (resident.cu:176-179,187-189)."""
    import torch
    log_n, P, blocks, slots, width = 12, 3, 2, 2, 64
    n = 1 << log_n
    print("[token] ready-event views", flush=True)
    q = cf.primes_below(50, 2 * n, P)
    ct = _inputs(q, n, blocks, slots, 760)
    tw = praghip.TokenWeights(q, log_n, ct, width, levels=2)
    ring = _ring(blocks, width, 761)
    local = [int(v) & MASK59 for v in oracle.fill_u64(slots, 762)]
    want = oracle.token_finished(ct, ring, oracle.token_scaled(local, q), q, log_n, width)
    side = torch.cuda.Stream()
    dring, dres = to_dev(ring), to_dev(oracle.token_scaled(local, q))
    out = to_dev(np.zeros((slots, 2, P, n), dtype=np.uint64))
    torch.cuda.synchronize()
    with torch.cuda.stream(side):
        tw.evaluate_device(dring, out, residues=dres, stream=side)
        ready = torch.cuda.Event()
        ready.record(side)
    tw.stack_store(0, 2, out[1], ready=ready)
    tw.stack_store(1, 0, out[0], ready=ready)
    np.testing.assert_array_equal(tw.download(tw.stack_view(0, 2), ready=ready), want[1])
    np.testing.assert_array_equal(tw.download(tw.stack_view(1, 0), ready=ready), want[0])
    lib = praghip.lib()
    assert lib.praghip_token_stack_store_ready(tw._h, 0, 0, out.data_ptr(), None) == praghip._lib.E_ARGUMENT
    assert b"E_DEVICE_STACK_VIEW" in lib.praghip_last_error()
    dl = np.empty((2, P, n), dtype=np.uint64)
    view = tw.stack_view(0, 0)
    assert lib.praghip_token_download_ready(tw._h, view.data, None, dl.ctypes.data) == praghip._lib.E_ARGUMENT
    assert b"E_DEVICE_DOWNLOAD_VIEW" in lib.praghip_last_error()
    tw.close()


def test_token_errors(gpu):
    log_n, blocks, width, slots = 12, 2, 64, 2
    n = 1 << log_n
    q = cf.LOCKED_PRIMES[:6]
    ct = _inputs(q, n, blocks, slots, 740)
    tw = praghip.TokenWeights(q, log_n, ct, width, levels=2)
    ok = _ring(blocks, width, 741)
    for v in [1 << 59, (1 << 20) + 1, (1 << 59) - (1 << 20) - 1]:
        bad = ok.copy()
        bad[0, 0] = v
        with pytest.raises(praghip.PraghipError, match="E_RESIDENT_WEIGHT_BOUND"):
            tw.evaluate(bad)
    with pytest.raises(praghip.PraghipError, match="E_RESIDENT_WEIGHT_SHAPE"):
        tw.evaluate(ok.reshape(-1)[:-1])
    with pytest.raises(praghip.PraghipError, match="E_RESIDENT_LOCAL_SHAPE"):
        tw.evaluate_local_finished(ok)
    with pytest.raises(praghip.PraghipError, match="E_GPU_TOKEN_CONTEXT_LAYOUT"):
        tw.evaluate_finished(ok, [1 << 59, 0])
    with pytest.raises(praghip.PraghipError, match="E_DEVICE_STACK_INDEX"):
        tw.stack_view(0, 3)
    with pytest.raises(praghip.PraghipError, match="E_DEVICE_STACK_INDEX"):
        tw.stack_view(slots, 0)
    with pytest.raises(praghip.PraghipError, match="E_DEVICE_STACK_VIEW"):
        tw.stack_store(0, 3, tw.stack_view(0, 0))
    bad_shares = np.zeros((slots, blocks * width), dtype=np.uint64)
    bad_shares[1, 5] = 1 << 59
    with pytest.raises(praghip.PraghipError, match="E_LOCAL_BINDING"):
        tw.bind_local_shares(bad_shares)
    tw.bind_local_shares(np.zeros((slots, blocks * width), dtype=np.uint64))
    with pytest.raises(praghip.PraghipError, match="E_LOCAL_BINDING"):
        tw.bind_local_shares(np.zeros((slots, blocks * width), dtype=np.uint64))
    bad_ct = ct.copy()
    bad_ct[1, 1, 1, 5, 7] = q[5]
    with pytest.raises(praghip.PraghipError, match="E_GPU_TOKEN_CONTEXT_LAYOUT"):
        praghip.TokenWeights(q, log_n, bad_ct, width)
    tw.close()


def _pack_keys(q, n, dnum, levels, seed):
    K = len(q)
    return oracle.fill_residues(levels * 2 * dnum * 2 * K, n, q, seed).reshape(levels, 2, dnum, 2, K, n)


@pytest.mark.parametrize("primes,dnum", [("locked", 6), ("50bit", 3)])
def test_pack_pair(gpu, primes, dnum):
    """pair at the first and last of nine levels, pair_device over several
    pairs, at N = 16384."""
    print(f"[pack] pair {primes} dnum={dnum}", flush=True)
    log_n, levels = 14, 9
    n = 1 << log_n
    q = cf.LOCKED_PRIMES if primes == "locked" else cf.primes_below(50, 2 * n, 6) + cf.primes_below(60, 2 * n, 1)
    L = len(q) - 1
    keys = _pack_keys(q, n, dnum, levels, 750 + dnum)
    cts = oracle.fill_residues(6 * 2 * L, n, q[:L], 751).reshape(6, 2, L, n)
    pk = praghip.Packing(q, log_n, keys, dnum=dnum, max_pairs=2)
    for level in (0, levels - 1):
        np.testing.assert_array_equal(pk.pair(cts[0], cts[1], level),
                                      oracle.pack_pair(cts[0], cts[1], level, keys, q, dnum, log_n),
                                      err_msg=f"level {level}")
    import torch
    left, right = to_dev(cts[:3]), to_dev(cts[3:])
    out = pk.pair_device(left, right, 4)   # three pairs, chunks of two
    torch.cuda.synchronize()
    got = from_dev(out).reshape(3, 2, L, n)
    for i in range(3):
        np.testing.assert_array_equal(got[i], oracle.pack_pair(cts[i], cts[3 + i], 4, keys, q, dnum, log_n),
                                      err_msg=f"pair_device {i}")
    assert pk.merges() == 2 + 3
    c = pk.close()
    assert c.closed and c.first_hip_error == 0 and c.wipe_synchronized_bytes == c.freed_bytes > 0
    with pytest.raises(praghip.PraghipError, match="E_PACK_CLOSED"):
        pk.pair(cts[0], cts[1], 0)


@pytest.mark.parametrize("max_pairs", [64, 3])
def test_pack_tree(gpu, max_pairs):
    """tree_device over 8 leaves x 2 slots equals the oracle's stack merge;
    max_pairs 3 splits every level into chunks (in-place reduction)."""
    print(f"[pack] tree max_pairs={max_pairs}", flush=True)
    log_n, levels, dnum, slots, leaves = 13, 4, 3, 2, 8
    n = 1 << log_n
    q = cf.primes_below(50, 2 * n, 6) + cf.primes_below(60, 2 * n, 1)
    L = len(q) - 1
    keys = _pack_keys(q, n, dnum, levels, 760)
    lv = oracle.fill_residues(leaves * slots * 2 * L, n, q[:L], 761).reshape(leaves, slots, 2, L, n)
    pk = praghip.Packing(q, log_n, keys, dnum=dnum, max_pairs=max_pairs)
    import torch
    nodes = to_dev(lv)
    roots = pk.tree_device(nodes, slots=slots)
    torch.cuda.synchronize()
    want = oracle.pack_tree(lv, keys, q, dnum, log_n)
    np.testing.assert_array_equal(from_dev(roots).reshape(slots, 2, L, n), want)
    assert pk.merges() == (leaves - 1) * slots
    pk.close()


def test_pack_errors(gpu):
    log_n, dnum, levels = 12, 2, 3
    n = 1 << log_n
    q = cf.primes_below(50, 2 * n, 4) + cf.primes_below(60, 2 * n, 1)
    L = len(q) - 1
    keys = _pack_keys(q, n, dnum, levels, 770)
    pk = praghip.Packing(q, log_n, keys, dnum=dnum)
    ct = oracle.fill_residues(2 * L, n, q[:L], 771).reshape(2, L, n)
    with pytest.raises(praghip.PraghipError, match="E_PACK_LEVEL"):
        pk.pair(ct, ct, levels)
    bad = ct.copy()
    bad[1, 2, 3] = q[2]
    with pytest.raises(praghip.PraghipError, match="E_PACK_CIPHERTEXT"):
        pk.pair(ct, bad, 0)
    import torch
    d = to_dev(np.stack([ct, ct]))
    with pytest.raises(praghip.PraghipError, match="E_PACK_DEVICE_LEVEL"):
        pk.pair_device(d[0], d[1], levels)
    with pytest.raises(praghip.PraghipError, match="E_PACK_DEVICE_VIEW"):
        pk.pair_device(d[0], d[1], 0, out=d[1])
    with pytest.raises(praghip.PraghipError, match="E_PACK_LEVEL"):
        pk.tree_device(torch.zeros(3 * 2 * L * n, dtype=torch.int64, device="cuda"))
    bad_keys = keys.copy()
    bad_keys[0, 1, 0, 0, L, 5] = q[L]
    with pytest.raises(praghip.PraghipError, match="E_SWITCH_KEY_CANONICAL"):
        praghip.Packing(q, log_n, bad_keys, dnum=dnum)
    with pytest.raises(praghip.PraghipError, match="E_PACK_KEY_LEVELS"):
        praghip.Packing(q, log_n, keys[:1].repeat(13, axis=0), dnum=dnum)
    pk.close()


def test_token_loop_end_to_end(gpu):
    """The reference's server loop (bfv_token_batch.inc:186-206): every
    coordinate's finished batch merged through the per-slot stack with
    pair_device, against tree_device over the same coordinates and against
    the oracle's finished batches packed by the oracle's stack merge."""
    print("[token] end-to-end loop", flush=True)
    import torch
    log_n, P, blocks, width, slots, coords = 12, 3, 3, 1024, 2, 8
    n = 1 << log_n
    q = cf.primes_below(50, 2 * n, P) + cf.primes_below(60, 2 * n, 1)
    levels = coords.bit_length() - 1
    ct = _inputs(q[:P], n, blocks, slots, 780)
    keys = _pack_keys(q, n, P, levels, 781)
    tw = praghip.TokenWeights(q[:P], log_n, ct, width, levels=levels)
    pk = praghip.Packing(q, log_n, keys, dnum=P)
    rings = [_ring(blocks, width, 790 + c) for c in range(coords)]
    locals_ = [[int(v) & MASK59 for v in oracle.fill_u64(slots, 800 + c)] for c in range(coords)]
    used = [[False] * (levels + 1) for _ in range(slots)]
    finished = []
    for c in range(coords):
        batch = tw.evaluate_finished(rings[c], locals_[c])
        finished.append(np.stack([tw.download(tw.slot_view(batch, s)) for s in range(slots)]))
        for s in range(slots):
            current, level = tw.slot_view(batch, s), 0
            while used[s][level]:
                current = pk.pair_device(tw.stack_view(s, level), current, level)
                used[s][level] = False
                level += 1
            tw.stack_store(s, level, current)
            used[s][level] = True
    stack_roots = np.stack([tw.download(tw.stack_view(s, levels)) for s in range(slots)])
    nodes = to_dev(np.stack(finished))
    tree_roots = from_dev(pk.tree_device(nodes, slots=slots)).reshape(slots, 2, P, n)
    np.testing.assert_array_equal(tree_roots, stack_roots)
    want_leaves = np.stack([oracle.token_finished(ct, rings[c], oracle.token_scaled(locals_[c], q[:P]), q[:P], log_n,
                                                  width) for c in range(coords)])
    np.testing.assert_array_equal(np.stack(finished), want_leaves)
    np.testing.assert_array_equal(stack_roots, oracle.pack_tree(want_leaves, keys, q, P, log_n))
    torch.cuda.synchronize()
    tw.close()
    pk.close()


@pytest.mark.parametrize("log_n,P,blocks,slots,width,coords,locked", [(12, 3, 3, 2, 512, 6, False),
                                                                       (14, 6, 19, 4, 8192, 5, True)])
def test_token_batch(gpu, log_n, P, blocks, slots, width, coords, locked):
    """evaluate_device_batch equals evaluate_device column by column (explicit
    residues and bound shares), and the oracle on the first and last column."""
    print(f"[token] batch log_n={log_n} coords={coords} slots={slots}", flush=True)
    import torch
    n = 1 << log_n
    q = cf.LOCKED_PRIMES[:P] if locked else cf.primes_below(50, 2 * n, P)
    ct = _inputs(q, n, blocks, slots, 900 + coords)
    tw = praghip.TokenWeights(q, log_n, ct, width, levels=2)
    tw.reserve(coords)
    tw.reserve(coords - 1)          # a smaller request keeps the reservation
    with pytest.raises(praghip.PraghipError, match="E_RESIDENT_BATCH_RESERVED"):
        tw.reserve(coords + 1)
    rings = np.stack([_ring(blocks, width, 910 + c, boundary=c == 1) for c in range(coords)])
    locals_ = [[int(v) & MASK59 for v in oracle.fill_u64(slots, 930 + c)] for c in range(coords)]
    res = np.stack([oracle.token_scaled(m, q) for m in locals_])
    d_rings, d_res = to_dev(rings), to_dev(res)
    out = torch.zeros(coords * slots * 2 * P * n, dtype=torch.int64, device="cuda")
    tw.evaluate_device_batch(d_rings, out, residues=d_res)
    one = torch.zeros(slots * 2 * P * n, dtype=torch.int64, device="cuda")
    got = from_dev(out).reshape(coords, slots, 2, P, n)
    for c in range(coords):
        tw.evaluate_device(d_rings[c], one, residues=d_res[c])
        torch.cuda.synchronize()
        np.testing.assert_array_equal(got[c], from_dev(one).reshape(slots, 2, P, n), err_msg=f"column {c}")
    for c in (0, coords - 1):
        np.testing.assert_array_equal(got[c], oracle.token_finished(ct, rings[c], res[c], q, log_n, width))
    shares = (oracle.fill_u64(slots * blocks * width, 940) & np.uint64(MASK59)).reshape(slots, -1)
    tw.bind_local_shares(shares)
    tw.evaluate_device_batch(d_rings, out)
    got = from_dev(out).reshape(coords, slots, 2, P, n)
    for c in range(coords):
        tw.evaluate_device(d_rings[c], one)
        torch.cuda.synchronize()
        np.testing.assert_array_equal(got[c], from_dev(one).reshape(slots, 2, P, n), err_msg=f"bound column {c}")
    with pytest.raises(praghip.PraghipError, match="E_RESIDENT_BATCH"):
        tw.evaluate_device_batch(to_dev(np.concatenate([rings, rings[:1]])),
                                 torch.zeros((coords + 1) * slots * 2 * P * n, dtype=torch.int64, device="cuda"))
    tw.close()
