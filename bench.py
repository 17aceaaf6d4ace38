"""Benchmark of the BFV hot path on one MI355X.

Primary line: batched forward + inverse negacyclic NTT at N=16384 over six
~50-bit primes, 256 ciphertexts x 2 polynomials = 3072 limbs (one step = one
forward and one inverse launch over all limbs).  Also reported in the same
JSON line: the keyswitch at N=16384, L=6 + 1 special prime (dnum=3, 64
ciphertexts, 64 independent keys) and the share GEMM (512x1024x3072,
int8 weights, mod 2^64).  Inputs are generated on the GPU and are resident in
HBM before timing; every timed result is checked afterwards (round trip,
re-run equality) and a slice is compared with the oracle.

The cpu_baseline legs time the C oracle (oracle/, the same algorithms in
scalar C, OpenMP over limbs/ciphertexts/rows) on bounded samples of the same
workloads.
"""
from __future__ import annotations

import argparse
import json
import os
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
for _p in (ROOT, os.path.join(ROOT, "privacy-rag_amd")):
    if _p not in sys.path:
        sys.path.insert(0, _p)

METRIC = "keyswitch/s and NTT/s at N=16384 L=6; share-GEMM TOPS; % HBM/MFMA roofline"
HBM_PEAK_GBS = 8000.0
I8_PEAK_TOPS = 5000.0  # dense int8 MFMA, MI355X
N = 16384
LOG_N = 14


# Committed rocprofv3 summaries behind each leg's `traffic`: the summary under
# profiles/, a pattern for the kernels of one timed step, and the launches the
# step's bytes are divided over (None: the average over the matching kernels'
# dispatches, for a leg whose step launches the same kernel on many shapes).
TRAFFIC_SOURCES = {
    "ntt": ("ntt_n16384_3072limbs.md", r"ntt_kernel<14,", 2),
    "keyswitch": ("keyswitch_n16384_L6_dnum3_batch64.md", r"ks_", 1),
    "keyswitch_rotation": ("keyswitch_n16384_L6_dnum3_rotation_batch64.md", r"ks_", 1),
    "keyswitch_reference": ("keyswitch_n16384_locked_dnum6_batch64.md", r"ks_", 1),
    "gemm": ("share_gemm_512x1024x3072_i8.md", r"share_gemm_dma_kernel", 1),
    "gemm_f12": ("share_gemm_512x1024x3072_f12.md", r"share_gemm_dma_kernel|gemm_clear_kernel", 1),
    "qwen3": ("qwen3_0.6b_local_gemms_28_layers.md", r"share_gemm_dma_kernel", None),
}


def profile_counters(name: str):
    """{kernel: {counter: (average per dispatch, dispatches)}} from the
    'Counters (average per dispatch)' table of a committed summary."""
    path = os.path.join(ROOT, "profiles", name)
    if not os.path.exists(path):
        return None
    out = {}
    with open(path) as f:
        for line in f:
            cells = [c.strip().strip("`") for c in line.strip().strip("|").split("|")]
            if len(cells) == 4 and cells[1].isupper() and cells[3].isdigit():
                try:
                    out.setdefault(cells[0], {})[cells[1]] = (float(cells[2]), int(cells[3]))
                except ValueError:
                    continue
    return out


def copy_calibration():
    """FETCH_SIZE and WRITE_SIZE scale factors from the 384 MiB device copy
    (profiles/copy_384MiB_calibration.md): true KiB / counted KiB."""
    c = profile_counters("copy_384MiB_calibration.md")
    if not c or "__amd_rocclr_copyBuffer" not in c:
        return None
    k = c["__amd_rocclr_copyBuffer"]
    true_kib = 3072 * N * 8 / 1024
    return round(true_kib / k["FETCH_SIZE"][0], 2), round(true_kib / k["WRITE_SIZE"][0], 2)


def measured_traffic(workload: str):
    """HBM bytes per launch (per step for multi-kernel legs) from the FETCH_SIZE
    and WRITE_SIZE rows of the workload's committed rocprofv3 summary, scaled
    by the copy calibration; None without a summary."""
    src, cal = TRAFFIC_SOURCES.get(workload), copy_calibration()
    if not src or not cal:
        return None
    name, pattern, launches = src
    c = profile_counters(name)
    if not c:
        return None
    import re
    per = {k: (cal[0] * v["FETCH_SIZE"][0] + cal[1] * v["WRITE_SIZE"][0]) * 1024
           for k, v in c.items() if re.match(pattern, k) and "FETCH_SIZE" in v and "WRITE_SIZE" in v}
    if not per:
        return None
    if launches is None:  # average over the matching dispatches
        d = {k: c[k]["FETCH_SIZE"][1] for k in per}
        return int(sum(per[k] * d[k] for k in per) / sum(d.values()))
    return int(sum(per.values()) / launches)


def log(msg: str) -> None:
    print(f"[bench] {msg}", file=sys.stderr, flush=True)


class Timer:
    """HIP events on the stream the kernels are launched on (torch's current stream)."""

    def __init__(self, torch):
        self.torch = torch

    def run(self, fn, steps: int, warmup: int) -> float:
        torch = self.torch
        for _ in range(warmup):
            fn()
        torch.cuda.synchronize()
        start, end = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        start.record()
        for _ in range(steps):
            fn()
        end.record()
        torch.cuda.synchronize()
        return start.elapsed_time(end) / steps  # ms per step


def bench_ntt(torch, praghip, steps, warmup):
    from praghip import params, synth
    q = params.primes_n16384_50bit()
    limbs = 256 * 2 * 6
    data = torch.empty(limbs * N, dtype=torch.int64, device="cuda")
    synth.fill_residues(data, q, LOG_N, 0x5052414700000002)
    ref = data.clone()
    plan = praghip.NttBatch(q, LOG_N)

    def step():
        plan.forward(data)
        plan.inverse(data)

    ms = Timer(torch).run(step, steps, warmup)
    assert torch.equal(data, ref), "NTT round trip changed the data"
    launch_ms = ms / 2
    bytes_per_launch = limbs * 2 * N * 8
    gbs = bytes_per_launch / (launch_ms * 1e-3) / 1e9
    return {
        "limbs": limbs, "q": q, "ms_per_step": ms, "launch_ms": launch_ms,
        "ntt_per_s": 2 * limbs / (ms * 1e-3), "poly_ntt_per_s": 2 * limbs / 6 / (ms * 1e-3),
        "roofline": {"bound": "hbm", "achieved": round(gbs, 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                     "frac": round(gbs / HBM_PEAK_GBS, 4), "traffic": measured_traffic("ntt"),
                     "kernel": "ntt_kernel<14> (forward and inverse launches)",
                     "algorithmic_bytes_per_launch": bytes_per_launch},
    }


def bench_keyswitch(torch, praghip, steps, warmup, reference=False, galois=1):
    """64 keyswitches with their own keys at N=16384, L=6: dnum=3 over six
    ~50-bit data primes + a 60-bit special prime, or (reference=True) the
    reference's own shape, dnum=6 over the seven locked 60-bit primes.
    galois: 1 is relinearization; an odd element (3: the rotation by one
    slot's generator) gathers c1 through the automorphism inside the ModUp
    reads and c0 inside the ModDown."""
    from praghip import params, synth
    q = list(params.LOCKED_PRIMES) if reference else params.primes_n16384_switch()
    L, dnum, batch = 6, (6 if reference else 3), 64
    sw = praghip.Switch(q, LOG_N, dnum, max_batch=batch)
    ct = torch.empty(batch * 2 * L * N, dtype=torch.int64, device="cuda")
    out = torch.empty_like(ct)
    keys = torch.empty(batch * sw.key_words, dtype=torch.int64, device="cuda")
    synth.fill_residues(ct, q[:L], LOG_N, 0x5052414700000003)
    synth.fill_residues(keys, q, LOG_N, 0x5052414700000103)

    def step():
        sw.keyswitch(ct, out, keys=keys, key_stride=sw.key_words, galois=galois)

    ms = Timer(torch).run(step, steps, warmup)
    first = out.clone()
    step()
    torch.cuda.synchronize()
    assert torch.equal(first, out), "keyswitch not deterministic"
    bytes_per_ks = 8 * N * (2 * L + 2 * L + dnum * 2 * (L + 1))
    gbs = batch * bytes_per_ks / (ms * 1e-3) / 1e9
    return {
        "batch": batch, "dnum": dnum, "galois": galois, "ms_per_step": ms, "keyswitch_per_s": batch / (ms * 1e-3),
        "roofline": {"bound": "hbm", "achieved": round(gbs, 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                     "frac": round(gbs / HBM_PEAK_GBS, 4),
                     "traffic": measured_traffic("keyswitch_reference" if reference else
                                                 ("keyswitch" if galois == 1 else "keyswitch_rotation")),
                     "kernel": "whole keyswitch batch (all its launches); traffic is per batch",
                     "algorithmic_bytes_per_batch": batch * bytes_per_ks,
                     "algorithmic_bytes_per_keyswitch": bytes_per_ks},
        "_tensors": (ct, keys, out, q),
    }


def bench_gemm(torch, praghip, steps, warmup):
    from praghip import synth
    m, k, n = 512, 1024, 3072
    x = torch.empty(m * k, dtype=torch.int64, device="cuda").view(m, k)
    w = torch.empty(n * k, dtype=torch.int8, device="cuda").view(n, k)
    y = torch.empty((m, n), dtype=torch.int64, device="cuda")
    synth.fill_u64(x, 0x5052414700000004)
    synth.fill_i8(w, 0x5052414700000104)

    def step():
        praghip.share_gemm(x, w, y=y)

    ms = Timer(torch).run(step, steps, warmup)
    tops = 2 * m * k * n / (ms * 1e-3) / 1e12
    mfma_tops = 8 * tops  # eight i8 digit products per u64 x i8 product
    # the same product on VALU dot products (v_dot4_i32_i8 on the same digit
    # planes): the alternative the MFMA kernel is measured against
    y_valu = torch.empty_like(y)
    ms_valu = Timer(torch).run(lambda: praghip.share_gemm_valu(x, w, y=y_valu), max(1, steps // 2), 2)
    assert torch.equal(y_valu, y), "VALU and MFMA share GEMMs differ"
    return {
        "shape": [m, k, n], "ms_per_step": ms, "tops": tops,
        "valu_form": {"ms_per_step": ms_valu, "tops": 2 * m * k * n / (ms_valu * 1e-3) / 1e12,
                      "kernel": "share_gemm_valu_kernel (v_dot4_i32_i8, same digit planes)",
                      "mfma_speedup": ms_valu / ms},
        "roofline": {"bound": "mfma", "achieved": round(mfma_tops, 2), "peak": I8_PEAK_TOPS, "unit": "TFLOP/s",
                     "frac": round(mfma_tops / I8_PEAK_TOPS, 4), "traffic": measured_traffic("gemm"),
                     "kernel": "share_gemm_dma_kernel (i8 MFMA ops executed)"},
        "_tensors": (x, w, y),
    }


def bench_gemm_f12(torch, praghip, steps, warmup):
    """C4's shape with the reference's own weights: int32 f12, |w| <= 2^20
    (quantize_weights.py:91,102), split once into three signed-byte planes
    (the split is outside the timed region, as weights are static); one launch
    of the i8-MFMA kernel covers the three planes."""
    from praghip import synth
    m, k, n = 512, 1024, 3072
    x = torch.empty(m * k, dtype=torch.int64, device="cuda").view(m, k)
    raw = torch.empty(n * k, dtype=torch.int64, device="cuda")
    y = torch.empty((m, n), dtype=torch.int64, device="cuda")
    synth.fill_u64(x, 0x5052414700000014)
    synth.fill_u64(raw, 0x5052414700000114)
    w = ((raw.view(n, k) & ((1 << 21) - 1)) - (1 << 20)).to(torch.int32)  # in [-2^20, 2^20)
    planes = praghip.split_weights(w)

    def step():
        praghip.share_gemm(x, planes, y=y)

    ms = Timer(torch).run(step, steps, warmup)
    tops = 2 * m * k * n / (ms * 1e-3) / 1e12
    mfma_tops = 24 * tops  # eight share digits x three weight planes per u64 x f12 product
    return {
        "shape": [m, k, n], "weights": "int32 f12, |w| <= 2^20, pre-split into 3 int8 planes",
        "ms_per_step": ms, "tops": tops,
        "roofline": {"bound": "mfma", "achieved": round(mfma_tops, 2), "peak": I8_PEAK_TOPS, "unit": "TFLOP/s",
                     "frac": round(mfma_tops / I8_PEAK_TOPS, 4), "traffic": measured_traffic("gemm_f12"),
                     "kernel": "share_gemm_dma_kernel, 3 weight planes (i8 MFMA ops executed)"},
        "_tensors": (x, w, y),
    }


def bench_qwen3(torch, praghip, steps, warmup):
    """Every local share GEMM of a Qwen3-0.6B forward over 512 tokens: 28 layers x
    {joint q|k|v 1024->4096, o 2048->1024, joint gate|up 1024->6144, down 3072->1024},
    int8 weights with per-channel shifts, one batched call per forward."""
    m = praghip.Qwen3LocalGemms(rows=512)
    ms = Timer(torch).run(m.forward, steps, warmup)
    tops = m.ops / (ms * 1e-3) / 1e12
    return {"layers": m.shape.layers, "rows": m.rows, "ms_per_forward": ms, "ms_per_step": ms,
            "layers_per_s": m.shape.layers / (ms * 1e-3), "tops": tops,
            "ops_per_forward": m.ops,
            "roofline": {"bound": "mfma", "achieved": round(8 * tops, 2), "peak": I8_PEAK_TOPS, "unit": "TFLOP/s",
                         "frac": round(8 * tops / I8_PEAK_TOPS, 4), "traffic": measured_traffic("qwen3"),
                         "kernel": "share_gemm_dma_kernel over the 112 products (i8 MFMA ops executed); "
                                   "traffic is the average per product"},
            "_model": m}


def bench_token(torch, praghip, steps, warmup, slots=4):
    """One 512-coordinate tile of the token-resident path at the reference's
    shape (bfv_token_batch.inc:176-215 with the locked context: N=16384, six
    60-bit primes + special, 19 blocks of 8192 per slot, 4 slots, bound local
    shares): every coordinate's weight column evaluated to a finished batch
    (lift, NTT, 19-block product, INTT, Delta term, shift; 64 columns per
    batched call), then the 9-level
    acyclic packing tree over the tile (511 merges per slot, 2 keyswitches each,
    dnum=6), level by level in batched launches."""
    from praghip import params, synth
    q = list(params.LOCKED_PRIMES)
    P, blocks, width, coords, levels = 6, 19, 8192, 512, 9
    ct_words = 2 * P * N
    inputs = torch.empty(blocks * slots * ct_words, dtype=torch.int64, device="cuda")
    synth.fill_residues(inputs, q[:P], LOG_N, 0x5052414700000006)
    host_ct = inputs.cpu().numpy().reshape(blocks, slots, 2, P, N)
    tw = praghip.TokenWeights(q[:P], LOG_N, host_ct, width, levels)
    del inputs
    shares = torch.empty(slots * blocks * width, dtype=torch.int64, device="cuda")
    synth.fill_u64(shares, 0x5052414700000106)
    host_shares = (shares & ((1 << 59) - 1)).cpu().numpy()
    tw.bind_local_shares(host_shares)
    del shares
    keys = torch.empty(levels * 2 * P * 2 * (P + 1) * N, dtype=torch.int64, device="cuda")
    synth.fill_residues(keys, q, LOG_N, 0x5052414700000206)
    host_keys = keys.cpu().numpy()
    pk = praghip.Packing(q, LOG_N, host_keys, dnum=P, max_pairs=512)
    del keys
    rings = torch.empty(coords * blocks * width, dtype=torch.int64, device="cuda")
    synth.fill_u64(rings, 0x5052414700000306)
    rings = ((rings & ((1 << 21) - 1)) - (1 << 20)) & ((1 << 59) - 1)  # signed |w| <= 2^20 as ring words
    rings = rings.view(coords, blocks * width)
    nodes = torch.empty((coords, slots * ct_words), dtype=torch.int64, device="cuda")
    chunk = 64  # 64 x 114 limbs per transform: 28.5 rounds of one limb per CU, a small tail
    tw.reserve(chunk)

    def evaluate_all():
        for c in range(0, coords, chunk):
            tw.evaluate_device_batch(rings[c:c + chunk], nodes[c:c + chunk])

    def step():
        evaluate_all()
        pk.tree_device(nodes, slots=slots)

    ms = Timer(torch).run(step, steps, warmup)
    ms_eval = Timer(torch).run(evaluate_all, steps, 1)
    merges = (coords - 1) * slots
    # samples for the CPU leg's parity: the finished batches of coordinates 0
    # and 1, and their level-0 merge in slot 0
    evaluate_all()
    fin = nodes[:2].clone()
    pair = pk.pair_device(fin[0, :ct_words], fin[1, :ct_words], 0)
    torch.cuda.synchronize()
    sample = {"q": q, "ct": host_ct, "shares": host_shares.reshape(slots, -1), "keys": host_keys,
              "rings": rings[:2].cpu().numpy(), "finished": fin.cpu().numpy(), "pair": pair.cpu().numpy()}
    return {"slots": slots, "coordinates": coords, "blocks": blocks, "block_width": width, "levels": levels,
            "ms_per_step": ms, "ms_per_tile": ms, "coordinates_per_s": coords / (ms * 1e-3),
            "evaluate_ms_per_tile": ms_eval, "pack_ms_per_tile": ms - ms_eval,
            "merges_per_tile": merges, "pack_keyswitch_per_s": 2 * merges / ((ms - ms_eval) * 1e-3),
            "device_bytes": int(tw.timing().device_bytes + pk.timing().device_bytes),
            "_plans": (tw, pk, rings, nodes), "_sample": sample}


def bench_matrix(torch, praghip, steps, warmup, blocks=3, groups=64):
    """The HE matrix product at the reference shape (matrix.cu:48-81: N=16384,
    six 60-bit primes): `blocks` resident ciphertext blocks, one evaluation
    per output group (weight ring [blocks][N]), 64 groups in one batched call
    (the per-evaluation entry point, one call per group, is timed beside it)."""
    from praghip import params, synth
    q = list(params.LOCKED_PRIMES[:6])
    P = 6
    ct = torch.empty(blocks * 2 * P * N, dtype=torch.int64, device="cuda")
    synth.fill_residues(ct, q, LOG_N, 0x5052414700000007)
    host_ct = ct.cpu().numpy().reshape(blocks, 2, P, N)
    m = praghip.Matrix(q, LOG_N, host_ct)
    rings = torch.empty(groups * blocks * N, dtype=torch.int64, device="cuda")
    synth.fill_u64(rings, 0x5052414700000107)
    rings = (rings & ((1 << 59) - 1)).view(groups, blocks * N)
    out = torch.empty((groups, 2 * P * N), dtype=torch.int64, device="cuda")
    m.reserve(groups)

    def single():
        for g in range(groups):
            m.evaluate_device(rings[g], out[g])

    ms_single = Timer(torch).run(single, max(1, steps // 2), warmup)
    ms = Timer(torch).run(lambda: m.evaluate_device_batch(rings, out), steps, warmup)
    torch.cuda.synchronize()
    return {"blocks": blocks, "groups_per_step": groups, "ms_per_step": ms,
            "evaluations_per_s": groups / (ms * 1e-3), "us_per_evaluation": ms * 1e3 / groups,
            "us_per_evaluation_one_per_call": ms_single * 1e3 / groups,
            "_sample": {"q": q, "ct": host_ct, "ring": rings[0].cpu().numpy(), "out": out[0].cpu().numpy()},
            "_keep": (m,)}


def bench_enc0(torch, praghip, steps, warmup, count=64):
    """Public-key encryption of zero at the reference shape (enc0.cu:99-114:
    N=16384, six 60-bit data primes + the special prime): `count`
    encryptions in one batched call, each from its own samples [3][7][N] (the
    per-encryption entry point, one call each, is timed beside it)."""
    from praghip import params, synth
    q = list(params.LOCKED_PRIMES)
    K = 7
    pk = torch.empty(2 * K * N, dtype=torch.int64, device="cuda")
    synth.fill_residues(pk, q, LOG_N, 0x5052414700000008)
    host_pk = pk.cpu().numpy().reshape(2, K, N)
    z = praghip.PublicZero(q, LOG_N, host_pk)
    samples = torch.empty((count, 3 * K * N), dtype=torch.int64, device="cuda")
    synth.fill_residues(samples, q, LOG_N, 0x5052414700000108)
    out = torch.empty((count, 2 * (K - 1) * N), dtype=torch.int64, device="cuda")
    z.reserve(count)

    def single():
        for i in range(count):
            z.evaluate_device(samples[i], out[i])

    ms_single = Timer(torch).run(single, max(1, steps // 2), warmup)
    ms = Timer(torch).run(lambda: z.evaluate_device_batch(samples, out), steps, warmup)
    torch.cuda.synchronize()
    return {"encryptions_per_step": count, "ms_per_step": ms, "encryptions_per_s": count / (ms * 1e-3),
            "us_per_encryption": ms * 1e3 / count, "us_per_encryption_one_per_call": ms_single * 1e3 / count,
            "_sample": {"q": q, "pk": host_pk, "samples": samples[0].cpu().numpy(), "out": out[0].cpu().numpy()},
            "_keep": (z,)}


def bench_copy(torch, steps, warmup):
    """Plain device copy of 384 MiB (the bytes one NTT launch reads, and again writes):
    the reference point for scaling rocprofv3 FETCH_SIZE / WRITE_SIZE to bytes."""
    src = torch.empty(3072 * N, dtype=torch.int64, device="cuda")
    dst = torch.empty_like(src)
    src.fill_(1)
    ms = Timer(torch).run(lambda: dst.copy_(src), steps, warmup)
    nbytes = src.numel() * 8
    return {"bytes_each_way": nbytes, "ms_per_step": ms, "gbs": 2 * nbytes / (ms * 1e-3) / 1e9}


def cpu_model() -> str:
    """The host CPU's model name (/proc/cpuinfo)."""
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                if line.startswith("model name"):
                    return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return "unknown"


def cpu_baselines(torch, res, budget_s: float):
    """Oracle timings on bounded samples (rank 0, N=1 only).  Every leg runs
    twice: on all host threads (OpenMP over limbs / ciphertexts / rows; its
    output checked against the GPU's for the same inputs), and on one thread
    over a smaller part of the same sample, as the reference's CPU path runs
    (one limb at a time on one core, bfv.cpp:499-517; the scalar GEMM loop
    bfv_matrix.inc:177-182)."""
    import numpy as np

    import oracle
    threads = len(os.sched_getaffinity(0))
    model = cpu_model()
    out = {}

    def leg(name, rate, unit, sample, one_core_rate, one_core_sample):
        out[name] = {"value": rate, "unit": unit, "cores": threads, "kind": "port", "sample": sample,
                     "value_1core": one_core_rate, "sample_1core": one_core_sample, "cpu_model": model}

    def timed(fn):
        t0 = time.perf_counter()
        r = fn()
        return r, time.perf_counter() - t0

    # NTT: sample of the 3072-limb batch
    q = res["ntt"]["q"]
    tab = oracle.Tables(q, LOG_N)
    limbs = 384
    a = oracle.fill_residues(limbs, N, q, 0x5052414700000002)
    _, dt = timed(lambda: oracle.ntt(oracle.ntt(a, tab, threads=threads), tab, inverse=True, threads=threads))
    reps = max(1, int(budget_s / 3 / max(dt, 1e-3)))
    _, dt = timed(lambda: [oracle.ntt(oracle.ntt(a, tab, threads=threads), tab, inverse=True, threads=threads)
                           for _ in range(reps)])
    dt /= reps
    a1 = a[:24]
    back, dt1 = timed(lambda: oracle.ntt(oracle.ntt(a1, tab, threads=1), tab, inverse=True, threads=1))
    assert np.array_equal(back, a1), "oracle NTT round trip"
    leg("ntt", 2 * limbs / dt, "limb-NTT/s", f"{limbs} limbs of the 3072-limb N=16384 batch, forward+inverse, x{reps}",
        2 * 24 / dt1, "24 limbs of the same batch, forward+inverse, one thread")
    # keyswitch (dnum = 3): a few of the 64 ciphertexts with their keys
    ct_t, keys_t, out_t, q3 = res["keyswitch"]["_tensors"]
    nb = min(2 * threads if threads <= 8 else threads, 64)
    ct = ct_t[: nb * 2 * 6 * N].cpu().numpy().view(np.uint64).reshape(nb, 2, 6, N)
    kw = 3 * 2 * 7 * N
    keys = keys_t[: nb * kw].cpu().numpy().view(np.uint64).reshape(nb, 3, 2, 7, N)
    gpu_slice = out_t[: nb * 2 * 6 * N].cpu().numpy().view(np.uint64).reshape(nb, 2, 6, N)
    tab3 = oracle.Tables(q3, LOG_N)
    got, dt = timed(lambda: oracle.keyswitch(ct, keys, q3, 3, LOG_N, 1, tables=tab3, per_ct_keys=True,
                                             threads=threads))
    got1, dt1 = timed(lambda: oracle.keyswitch(ct[:1], keys[:1], q3, 3, LOG_N, 1, tables=tab3, per_ct_keys=True,
                                               threads=1))
    out["keyswitch_parity"] = bool(np.array_equal(got, gpu_slice) and np.array_equal(got1, gpu_slice[:1]))
    leg("keyswitch", nb / dt, "keyswitch/s", f"{nb} of the 64 N=16384 ciphertexts (dnum=3) with their own keys",
        1 / dt1, "one of those ciphertexts, one thread")
    # the rotation (Galois element 3) and the reference shape (dnum = 6, the
    # locked 60-bit primes): the sampled ciphertexts with their keys
    for name, dnum, g, what in (("keyswitch_rotation", 3, 3, "dnum=3, Galois element 3"),
                                ("keyswitch_reference", 6, 1, "dnum=6, locked primes")):
        if name not in res or "_sample" not in res[name]:
            continue
        sm = res[name]["_sample"]
        nb = sm["ct"].shape[0]
        tb = oracle.Tables(sm["q"], LOG_N)
        got, dt = timed(lambda: oracle.keyswitch(sm["ct"], sm["keys"], sm["q"], dnum, LOG_N, g, tables=tb,
                                                 per_ct_keys=True, threads=threads))
        got1, dt1 = timed(lambda: oracle.keyswitch(sm["ct"][:1], sm["keys"][:1], sm["q"], dnum, LOG_N, g, tables=tb,
                                                   per_ct_keys=True, threads=1))
        out[name + "_parity"] = bool(np.array_equal(got, sm["out"]) and np.array_equal(got1, sm["out"][:1]))
        leg(name, nb / dt, "keyswitch/s", f"{nb} of the 64 N=16384 ciphertexts ({what}) with their own keys",
            1 / dt1, "one of those ciphertexts, one thread")
    # GEMM: 64 rows of the 512x1024 activations against all 3072 weight rows
    x_t, w_t, y_t = res["gemm"]["_tensors"]
    rows = 64
    x = x_t[:rows].cpu().numpy().view(np.uint64)
    w = w_t.cpu().numpy()
    yg = y_t[:rows].cpu().numpy().view(np.uint64)
    y, dt = timed(lambda: oracle.share_gemm(x, w, threads=threads))
    y1, dt1 = timed(lambda: oracle.share_gemm(x[:4], w, threads=1))
    out["gemm_parity"] = bool(np.array_equal(y, yg) and np.array_equal(y1, yg[:4]))
    leg("gemm", 2 * rows * 1024 * 3072 / dt / 1e12, "TOPS", f"{rows} of 512 activation rows x 1024 x 3072",
        2 * 4 * 1024 * 3072 / dt1 / 1e12, "4 of those rows, one thread")
    # f12 GEMM: 16 activation rows against the int32 weights, parity with the
    # pre-split GPU product
    if "gemm_f12" in res and "_tensors" in res["gemm_f12"]:
        x_t, w_t, y_t = res["gemm_f12"]["_tensors"]
        rows = 16
        x = x_t[:rows].cpu().numpy().view(np.uint64)
        w = w_t.cpu().numpy()
        yg = y_t[:rows].cpu().numpy().view(np.uint64)
        y, dt = timed(lambda: oracle.share_gemm(x, w, threads=threads))
        y1, dt1 = timed(lambda: oracle.share_gemm(x[:2], w, threads=1))
        out["gemm_f12_parity"] = bool(np.array_equal(y, yg) and np.array_equal(y1, yg[:2]))
        leg("gemm_f12", 2 * rows * 1024 * 3072 / dt / 1e12, "TOPS",
            f"{rows} of 512 activation rows x 1024 x 3072, int32 weights",
            2 * 2 * 1024 * 3072 / dt1 / 1e12, "2 of those rows, one thread")
    # token tile: two coordinates' columns (resident inputs transformed once,
    # as the GPU plan does at creation) and one level-0 merge, scaled to the
    # tile's 512 columns and 2,044 merges
    if "token" in res and "_sample" in res["token"]:
        sm = res["token"]["_sample"]
        qd, P, width = sm["q"][:6], 6, res["token"]["block_width"]
        slots = sm["shares"].shape[0]
        resident = oracle.token_inputs(sm["ct"], qd, LOG_N, threads)
        Q = 1
        for x in qd:
            Q *= int(x)
        delta, r = [(Q >> 59) % int(x) for x in qd], Q & ((1 << 59) - 1)

        def column(c, nthreads):
            ring = sm["rings"][c].view(np.uint64)
            scaled = oracle.local_dot_scale(sm["shares"], ring, delta, r, qd)
            return oracle.token_finished(None, ring, scaled, qd, LOG_N, width, nthreads, resident=resident)

        fins, t2 = timed(lambda: [column(c, threads) for c in range(2)])
        t_eval = t2 / 2
        ok = all(np.array_equal(fins[c].reshape(-1), sm["finished"][c].view(np.uint64)) for c in range(2))
        tk = oracle.Tables(sm["q"], LOG_N)

        def merge(nthreads):
            return oracle.pack_pair(fins[0][0], fins[1][0], 0, sm["keys"].view(np.uint64), sm["q"], P, LOG_N,
                                    tables=tk, threads=nthreads)

        merge(threads)  # first call outside the timing (thread pool start-up)
        pr, t_pair = timed(lambda: merge(threads))
        ok &= bool(np.array_equal(pr.reshape(-1), sm["pair"].view(np.uint64)))
        f1, t_eval1 = timed(lambda: column(0, 1))
        pr1, t_pair1 = timed(lambda: merge(1))
        ok &= bool(np.array_equal(f1, fins[0]) and np.array_equal(pr1, pr))
        coords, merges = res["token"]["coordinates"], res["token"]["merges_per_tile"]
        out["token_parity"] = ok
        leg("token", coords / (coords * t_eval + merges * t_pair), "coordinates/s",
            f"2 of 512 columns ({slots} slots, {t_eval * 1e3:.0f} ms each) and one level-0 merge "
            f"({t_pair * 1e3:.0f} ms), scaled to 512 columns + {merges} merges",
            coords / (coords * t_eval1 + merges * t_pair1),
            f"one column ({t_eval1 * 1e3:.0f} ms) and one merge ({t_pair1 * 1e3:.0f} ms), one thread, scaled the same")
    # HE matrix product and encryption of zero: one evaluation each, with parity
    if "matrix" in res and "_sample" in res["matrix"]:
        sm = res["matrix"]["_sample"]
        ring = sm["ring"].view(np.uint64)
        want, dt = timed(lambda: oracle.matrix_product(sm["ct"], ring, sm["q"], LOG_N, threads=threads))
        want1, dt1 = timed(lambda: oracle.matrix_product(sm["ct"], ring, sm["q"], LOG_N, threads=1))
        out["matrix_parity"] = bool(np.array_equal(want.reshape(-1), sm["out"].view(np.uint64))
                                    and np.array_equal(want1, want))
        leg("matrix", 1 / dt, "evaluations/s",
            f"one evaluation ({res['matrix']['blocks']} blocks, N=16384, 6 primes), inputs transformed inside the "
            "sample", 1 / dt1, "the same evaluation, one thread")
    if "enc0" in res and "_sample" in res["enc0"]:
        sm = res["enc0"]["_sample"]
        smp = sm["samples"].view(np.uint64).reshape(3, 7, N)
        want, dt = timed(lambda: oracle.enc0(smp, sm["pk"].view(np.uint64), sm["q"], LOG_N, threads=threads))
        want1, dt1 = timed(lambda: oracle.enc0(smp, sm["pk"].view(np.uint64), sm["q"], LOG_N, threads=1))
        out["enc0_parity"] = bool(np.array_equal(want.reshape(-1), sm["out"].view(np.uint64))
                                  and np.array_equal(want1, want))
        leg("enc0", 1 / dt, "encryptions/s", "one encryption of zero (N=16384, 6 + 1 primes)",
            1 / dt1, "the same encryption, one thread")
    # Qwen3: the four products of layer 0 on 16 of the 512 token rows
    if "qwen3" in res and "_sample" in res["qwen3"]:
        ok, ops, ops1, dt, dt1 = True, 0, 0, 0.0, 0.0
        for x_t, w_t, sh_t, y_t in res["qwen3"]["_sample"]:
            x = x_t.numpy().view(np.uint64)
            w = w_t.numpy()
            sh = None if sh_t is None else sh_t.numpy()
            yg = y_t.numpy().view(np.uint64)
            y, t = timed(lambda: oracle.share_gemm(x, w, sh, mask_bits=64, threads=threads))
            y1, t1 = timed(lambda: oracle.share_gemm(x[:2], w, sh, mask_bits=64, threads=1))
            dt, dt1 = dt + t, dt1 + t1
            ops += 2 * x.shape[0] * x.shape[1] * w.shape[0]
            ops1 += 2 * 2 * x.shape[1] * w.shape[0]
            ok &= bool(np.array_equal(y, yg) and np.array_equal(y1, yg[:2]))
        out["qwen3_parity"] = ok
        leg("qwen3", ops / dt / 1e12, "TOPS",
            "layer 0, 16 of 512 token rows, all four products (q|k|v, o, gate|up, down)",
            ops1 / dt1 / 1e12, "2 of those rows, one thread")
    return out


def main() -> int:
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=50)
    ap.add_argument("--warmup", type=int, default=20)
    ap.add_argument("--only", choices=["all", "ntt", "keyswitch", "keyswitch_dnum3", "keyswitch_rotation",
                                       "keyswitch_dnum6", "gemm",
                                       "gemm_f12", "qwen3", "token", "matrix", "enc0", "copy"],
                    default="all")
    ap.add_argument("--no-cpu", action="store_true", help="skip the oracle CPU baselines")
    ap.add_argument("--cpu-budget", type=float, default=12.0, help="seconds of oracle NTT timing")
    args = ap.parse_args()
    if args.gpus != 1:
        print(f"bench.py measures one GPU: praghip has no multi-GPU path (asked for --gpus {args.gpus})",
              file=sys.stderr)
        return 2
    import numpy as np
    import torch

    import praghip
    assert torch.cuda.is_available() and praghip.device_count() >= 1, "needs an MI355X"
    res = {}
    if args.only == "copy":
        r = bench_copy(torch, args.steps, args.warmup)
        log(f"copy {r['bytes_each_way']} B each way: {r['gbs']:.1f} GB/s")
        print(json.dumps({"metric": "device copy (calibration)", "value": r["gbs"], "unit": "GB/s", "n_gpus": 1,
                          "steps": args.steps, "warmup": args.warmup, "ms_per_step": r["ms_per_step"],
                          "higher_is_better": True, "bytes_each_way": r["bytes_each_way"]}), flush=True)
        return 0
    if args.only in ("all", "ntt"):
        log("NTT N=16384, 3072 limbs ...")
        res["ntt"] = bench_ntt(torch, praghip, args.steps, args.warmup)
        log(f"NTT {res['ntt']['ntt_per_s']:.4g} limb-NTT/s, {res['ntt']['roofline']['achieved']} GB/s")
    if args.only in ("all", "keyswitch", "keyswitch_dnum3"):
        log("keyswitch N=16384 dnum=3, 64 ciphertexts ...")
        res["keyswitch"] = bench_keyswitch(torch, praghip, args.steps, args.warmup)
        log(f"keyswitch {res['keyswitch']['keyswitch_per_s']:.4g}/s")
    if args.only in ("all", "keyswitch", "keyswitch_rotation"):
        log("keyswitch N=16384 dnum=3, Galois element 3 (rotation), 64 ciphertexts ...")
        res["keyswitch_rotation"] = bench_keyswitch(torch, praghip, args.steps, args.warmup, galois=3)
        ct_t, keys_t, out_t, q3 = res["keyswitch_rotation"].pop("_tensors")
        if not args.no_cpu and args.only == "all":
            nb, cw, kw = 16, 2 * 6 * N, 3 * 2 * 7 * N
            host = lambda t, w: t[: nb * w].cpu().numpy().view(np.uint64).copy()  # noqa: E731
            res["keyswitch_rotation"]["_sample"] = {"ct": host(ct_t, cw).reshape(nb, 2, 6, N),
                                                    "keys": host(keys_t, kw).reshape(nb, 3, 2, 7, N),
                                                    "out": host(out_t, cw).reshape(nb, 2, 6, N), "q": q3}
        del ct_t, keys_t, out_t
        log(f"keyswitch (rotation) {res['keyswitch_rotation']['keyswitch_per_s']:.4g}/s")
    if args.only in ("all", "keyswitch", "keyswitch_dnum6"):
        log("keyswitch N=16384 dnum=6, locked 60-bit primes (the reference shape), 64 ciphertexts ...")
        res["keyswitch_reference"] = bench_keyswitch(torch, praghip, args.steps, args.warmup, reference=True)
        ct_t, keys_t, out_t, qr = res["keyswitch_reference"].pop("_tensors")
        if not args.no_cpu and args.only == "all":
            # a few ciphertexts with their keys, on the host, for the CPU leg
            nb, cw, kw = 8, 2 * 6 * N, 6 * 2 * 7 * N
            host = lambda t, w: t[: nb * w].cpu().numpy().view(np.uint64).copy()  # noqa: E731
            res["keyswitch_reference"]["_sample"] = {"ct": host(ct_t, cw).reshape(nb, 2, 6, N),
                                                     "keys": host(keys_t, kw).reshape(nb, 6, 2, 7, N),
                                                     "out": host(out_t, cw).reshape(nb, 2, 6, N), "q": qr}
        del ct_t, keys_t, out_t
        log(f"keyswitch (reference shape) {res['keyswitch_reference']['keyswitch_per_s']:.4g}/s")
    if args.only in ("all", "gemm"):
        log("share GEMM 512x1024x3072 ...")
        res["gemm"] = bench_gemm(torch, praghip, args.steps, args.warmup)
        log(f"GEMM {res['gemm']['tops']:.4g} TOPS")
    if args.only in ("all", "gemm_f12"):
        log("share GEMM 512x1024x3072, f12 weights pre-split into 3 planes ...")
        res["gemm_f12"] = bench_gemm_f12(torch, praghip, args.steps, args.warmup)
        log(f"GEMM f12 {res['gemm_f12']['tops']:.4g} TOPS")
    if args.only in ("all", "qwen3"):
        log("Qwen3-0.6B local share GEMMs, 28 layers x 4 products, 512 tokens ...")
        res["qwen3"] = bench_qwen3(torch, praghip, args.steps, args.warmup)
        log(f"Qwen3 forward {res['qwen3']['ms_per_forward']:.3f} ms, {res['qwen3']['tops']:.4g} TOPS")
        if args.only == "all":
            # keep 16 rows of layer 0 on the host for the CPU leg, free the 2.7 GB model
            m = res["qwen3"].pop("_model")
            sample = []
            for name, _, _ in m.shape.products():
                x, w, sh, y = m.product(0, name)
                sample.append((x[:16].cpu(), w.cpu(), None if sh is None else sh.cpu(), y[:16].cpu()))
            res["qwen3"]["_sample"] = sample
            del m
    if args.only in ("all", "token"):
        log("token-resident tile: 512 coordinates x 4 slots, 9-level packing tree ...")
        tsteps = max(1, min(args.steps, 3))
        res["token"] = bench_token(torch, praghip, tsteps, 1)
        log(f"token tile {res['token']['ms_per_tile']:.1f} ms ({res['token']['coordinates_per_s']:.4g} coordinates/s, "
            f"evaluate {res['token']['evaluate_ms_per_tile']:.1f} ms)")
        res["token"]["steps"] = tsteps
        res["token"].pop("_plans")
        if args.no_cpu or args.only != "all":
            res["token"].pop("_sample")
    for name, fn, unit in (("matrix", bench_matrix, "evaluations_per_s"), ("enc0", bench_enc0, "encryptions_per_s")):
        if args.only in ("all", name):
            log(f"{name} ...")
            res[name] = fn(torch, praghip, max(1, min(args.steps, 10)), 2)
            res[name].pop("_keep")
            log(f"{name} {res[name][unit]:.4g}/s")
            if args.no_cpu or args.only != "all":
                res[name].pop("_sample")
    cpu = {}
    if not args.no_cpu and args.only == "all":
        log("oracle CPU baselines ...")
        cpu = cpu_baselines(torch, res, args.cpu_budget)
        log(f"cpu: {json.dumps(cpu)}")

    def clean(d):
        return {k: v for k, v in d.items() if not k.startswith("_")}

    key = next(k for k in ("ntt", "keyswitch", "keyswitch_rotation", "keyswitch_reference", "gemm", "gemm_f12",
                           "qwen3", "token", "matrix", "enc0") if k in res)
    primary = res[key]
    value = {"ntt": lambda r: r["ntt_per_s"], "keyswitch": lambda r: r["keyswitch_per_s"],
             "keyswitch_reference": lambda r: r["keyswitch_per_s"],
             "keyswitch_rotation": lambda r: r["keyswitch_per_s"],
             "gemm": lambda r: r["tops"], "gemm_f12": lambda r: r["tops"], "qwen3": lambda r: r["tops"],
             "token": lambda r: r["coordinates_per_s"], "matrix": lambda r: r["evaluations_per_s"],
             "enc0": lambda r: r["encryptions_per_s"]}[key](primary)
    unit = {"ntt": "limb-NTT/s", "keyswitch": "keyswitch/s", "keyswitch_reference": "keyswitch/s",
            "keyswitch_rotation": "keyswitch/s", "gemm": "TOPS",
            "gemm_f12": "TOPS", "qwen3": "TOPS",
            "token": "coordinates/s", "matrix": "evaluations/s", "enc0": "encryptions/s"}[key]
    line = {
        "metric": METRIC,
        "value": value,
        "unit": unit,
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": primary["ms_per_step"],
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": {"gemm": "i8", "gemm_f12": "i8", "qwen3": "i8"}.get(key, "u64"),
        "data": "synthetic (seeded splitmix64 on the GPU)",
        "config": {"workload": {
            "ntt": "batched forward+inverse negacyclic NTT, N=16384, 6 primes ~50 bit, "
                   "256 ciphertexts x 2 polynomials = 3072 limbs",
            "keyswitch": "keyswitch N=16384 L=6 (+1 special prime), dnum=3, 64 ciphertexts, 64 keys",
            "keyswitch_reference": "keyswitch N=16384, six locked 60-bit primes + special, dnum=6, 64 ciphertexts, "
                                   "64 keys",
            "keyswitch_rotation": "keyswitch N=16384 L=6 (+1 special prime), dnum=3, Galois element 3, "
                                  "64 ciphertexts, 64 keys",
            "gemm": "share GEMM u64[512x1024] x int8[3072x1024]^T mod 2^64",
            "gemm_f12": "share GEMM u64[512x1024] x int32 f12[3072x1024]^T mod 2^64 (pre-split weights)",
            "qwen3": "Qwen3-0.6B local share GEMMs, 28 layers x 4 products, 512 tokens",
            "token": "token-resident tile, 512 coordinates x 4 slots, 19 blocks of 8192, 9-level packing",
            "matrix": "HE matrix product, N=16384, 6 primes, 3 blocks, 64 output groups",
            "enc0": "public-key encryption of zero, N=16384, 6 + 1 primes, 64 encryptions"}[key],
            "N": N, "parallelism": "single GPU",
            "arithmetic": "exact integers mod q: primes below 2^50 are held as exact integers in FP64 registers "
                          "(error-free products by FMA), larger primes in 64-bit integer arithmetic; share GEMMs "
                          "exact mod 2^64 from i8 digit products"},
        "roofline": primary.get("roofline"),
        "cpu_baseline": cpu.get(key),
        "extra": {k: clean(v) for k, v in res.items() if k != key or len(res) == 1},
    }
    if cpu:
        line["extra"]["cpu_baselines"] = {k: v for k, v in cpu.items() if k != key}
    print(json.dumps(line), flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
