"""GPU parity of the party-local share GEMM against the oracle and fixtures."""
import os

import numpy as np
import pytest

import oracle
import praghip
from conftest import from_dev, to_dev

pytestmark = pytest.mark.gpu


def _run(x, w, shifts=None, mask_bits=64, split=False):
    """split: int32 weights pre-split on the GPU into three signed-byte planes (w_bits 24)."""
    import torch
    tx = to_dev(x)
    tw = torch.from_numpy(np.ascontiguousarray(w)).cuda()
    if split:
        tw = praghip.split_weights(tw)
    ts = None if shifts is None else torch.from_numpy(np.ascontiguousarray(shifts, dtype=np.int8)).cuda()
    y = praghip.share_gemm(tx, tw, shifts=ts, mask_bits=mask_bits)
    torch.cuda.synchronize()
    return from_dev(y)


def test_gemm_golden(gpu, golden_dir):
    data = np.load(os.path.join(golden_dir, "gemm_small.npz"))
    for name in ("i8_a", "i8_shift59", "i32_a", "i32_shift59"):
        sh = data[name + "_shift"] if name + "_shift" in data.files else None
        got = _run(data[name + "_x"], data[name + "_w"], sh, int(data[name + "_mask"][0]))
        np.testing.assert_array_equal(got, data[name + "_y"], err_msg=name)
    yc = _run(data["probe_client"], data["probe_weight"], None, 59)
    ys = _run(data["probe_server"], data["probe_weight"], None, 59)
    np.testing.assert_array_equal((yc + ys) & np.uint64((1 << 59) - 1), data["probe_plain"])


@pytest.mark.parametrize("m,k,n", [(1, 1, 1), (5, 7, 3), (33, 65, 129), (64, 128, 256), (100, 1000, 300),
                                   (31, 2048, 127), (512, 64, 128)])
@pytest.mark.parametrize("wdt", ["i8", "i32", "i32split"])
def test_gemm_ragged_vs_oracle(gpu, m, k, n, wdt):
    print(f"[gemm] m={m} k={k} n={n} {wdt}", flush=True)
    x = oracle.fill_u64(m * k, 1000 + m).reshape(m, k)
    if wdt == "i8":
        w = oracle.fill_i8(n * k, 2000 + n).reshape(n, k)
    else:
        w = (oracle.fill_u64(n * k, 3000 + n) % np.uint64(1 << 21)).astype(np.int64) - (1 << 20)
        w = w.astype(np.int32).reshape(n, k)
    sh = oracle.fill_shift(n, 4000 + k)
    for shifts, mask in ((None, 64), (sh, 59)):
        want = oracle.share_gemm(x, w, shifts, mask)
        np.testing.assert_array_equal(_run(x, w, shifts, mask, split=wdt == "i32split"), want)


def test_gemm_extreme_values(gpu):
    m, k, n = 40, 256, 160
    x = np.full((m, k), np.uint64((1 << 64) - 1))
    x[1] = 0
    x[2] = np.uint64(1 << 63)
    x[3] = np.uint64(0x8080808080808080)
    w = np.full((n, k), -127, dtype=np.int8)
    w[1] = 127
    w[2] = -128
    w[3] = 0
    np.testing.assert_array_equal(_run(x, w), oracle.share_gemm(x, w))
    w32 = np.full((n, k), -(1 << 20), dtype=np.int32)
    w32[1] = 1 << 20
    w32[2] = 0x7F7F7F  # largest weight with three balanced signed bytes
    w32[3] = -0x808080  # smallest
    np.testing.assert_array_equal(_run(x, w32), oracle.share_gemm(x, w32))
    np.testing.assert_array_equal(_run(x, w32, split=True), oracle.share_gemm(x, w32))


def test_gemm_c4_full_shape(gpu):
    """Qwen3 up/gate shape: activation shares u64 [512 x 1024] times int8 [3072 x 1024] -> [512 x 3072] mod 2^64."""
    m, k, n = 512, 1024, 3072
    x = oracle.fill_u64(m * k, 0x5052414700000004).reshape(m, k)
    w = oracle.fill_i8(n * k, 0x5052414700000104).reshape(n, k)
    np.testing.assert_array_equal(_run(x, w), oracle.share_gemm(x, w))


@pytest.mark.parametrize("m,k,n", [(512, 2048, 1024), (512, 3072, 1024), (96, 4096, 256)])
def test_gemm_split_k_shapes(gpu, m, k, n):
    """Shapes whose tiles leave most workgroup slots empty run split-K (64-bit
    atomic accumulation into a zeroed y, then the 59-bit mask): the Qwen3 o
    and down products, and a long-K thin case."""
    print(f"[gemm] split-K m={m} k={k} n={n}", flush=True)
    x = oracle.fill_u64(m * k, 5000 + k).reshape(m, k)
    w = oracle.fill_i8(n * k, 6000 + k).reshape(n, k)
    sh = oracle.fill_shift(n, 7000 + k)
    for shifts, mask in ((None, 64), (sh, 59)):
        np.testing.assert_array_equal(_run(x, w, shifts, mask), oracle.share_gemm(x, w, shifts, mask))


@pytest.mark.parametrize("m,k,n", [(512, 1024, 3072), (500, 1024, 3000), (481, 640, 2900)])
def test_gemm_wide_tiles(gpu, m, k, n):
    """Shapes whose 128-column grid would load the CUs unevenly run 192-column
    tiles with one workgroup per CU (the pipelined kernel): ragged rows and
    columns, shifts and the 59-bit ring included."""
    print(f"[gemm] wide tiles m={m} k={k} n={n}", flush=True)
    x = oracle.fill_u64(m * k, 9000 + n).reshape(m, k)
    w = oracle.fill_i8(n * k, 9100 + n).reshape(n, k)
    sh = oracle.fill_shift(n, 9200 + n)
    for shifts, mask in ((None, 64), (sh, 59)):
        np.testing.assert_array_equal(_run(x, w, shifts, mask), oracle.share_gemm(x, w, shifts, mask))


def test_gemm_c4_f12_presplit(gpu, tmp_path):
    """C4's shape with the reference's weight domain (int32 f12, |w| <= 2^20,
    quantize_weights.py:91,102) pre-split into three signed-byte planes: once
    on the GPU (split_weights) and once on the host at upload
    (MappedWeights.upload_split), both identical and bit-exact against the
    oracle's int32 product, shifts and the 59-bit ring included."""
    import torch
    m, k, n = 512, 1024, 3072
    x = oracle.fill_u64(m * k, 0x5052414700000014).reshape(m, k)
    w = ((oracle.fill_u64(n * k, 0x5052414700000114) % np.uint64((1 << 21) + 1)).astype(np.int64)
         - (1 << 20)).astype("<i4").reshape(n, k)
    w[0, :4] = [1 << 20, -(1 << 20), 0x7F7F7F, -0x808080]
    sh = oracle.fill_shift(n, 0x5052414700000214)
    planes = praghip.split_weights(torch.from_numpy(w).cuda())
    path = tmp_path / "model.layers.0.mlp.up_proj.weight.npy"
    np.save(path, w)
    host_planes = torch.empty((3, n, k), dtype=torch.int8, device="cuda")
    with praghip.MappedWeights(str(path), n, k) as mw:
        mw.upload_split(host_planes)
    torch.cuda.synchronize()
    assert torch.equal(planes, host_planes)
    tx, ts = to_dev(x), torch.from_numpy(sh).cuda()
    for shifts, mask in ((None, 64), (ts, 59)):
        y = praghip.share_gemm(tx, planes, shifts=shifts, mask_bits=mask)
        torch.cuda.synchronize()
        np.testing.assert_array_equal(from_dev(y), oracle.share_gemm(x, w, None if shifts is None else sh, mask))


@pytest.mark.parametrize("m,k,n", [(512, 1024, 3072), (33, 100, 129), (1, 64, 1)])
def test_gemm_valu_form(gpu, m, k, n):
    """The VALU dot-product form (the measured alternative to the MFMA
    kernels) gives the oracle's results, shifts and the 59-bit ring included."""
    import torch
    print(f"[gemm-valu] m={m} k={k} n={n}", flush=True)
    x = oracle.fill_u64(m * k, 8000 + k).reshape(m, k)
    w = oracle.fill_i8(n * k, 8100 + n).reshape(n, k)
    sh = oracle.fill_shift(n, 8200 + m)
    for shifts, mask in ((None, 64), (sh, 59)):
        ts = None if shifts is None else torch.from_numpy(shifts).cuda()
        y = praghip.share_gemm_valu(to_dev(x), torch.from_numpy(w).cuda(), shifts=ts, mask_bits=mask)
        torch.cuda.synchronize()
        np.testing.assert_array_equal(from_dev(y), oracle.share_gemm(x, w, shifts, mask))


def _batch(descs):
    import ctypes

    import torch
    from praghip import _lib
    arr = (_lib.GemmDesc * len(descs))(*[
        _lib.GemmDesc(x.data_ptr(), w.data_ptr(), 0 if s is None else s.data_ptr(), y.data_ptr(), x.shape[0],
                      x.shape[1], w.shape[0], 8, mask) for x, w, s, y, mask in descs])
    _lib.check(_lib.lib().praghip_share_gemm_batch(0, ctypes.cast(arr, ctypes.c_void_p), len(descs), None))
    torch.cuda.synchronize()


def test_gemm_batch_split_k_outputs_cleared_together(gpu):
    """praghip_share_gemm_batch zeroes the outputs of its split-K products in
    one launch before the first product (the Qwen3 o and down shapes here,
    with and without the 59-bit mask), and falls back to a clear per product
    when such an output is also an earlier product's input: product 1 reads
    buffer B as its shares, then product 2 (split K) writes B."""
    import torch
    specs = [(512, 2048, 1024, None, 64), (512, 3072, 1024, 7001, 59), (64, 1024, 512, None, 64),
             (512, 2048, 1024, 7002, 64)]
    descs, want = [], []
    for i, (m, k, n, shseed, mask) in enumerate(specs):
        x = oracle.fill_u64(m * k, 8000 + i).reshape(m, k)
        w = oracle.fill_i8(n * k, 8100 + i).reshape(n, k)
        sh = None if shseed is None else oracle.fill_shift(n, shseed)
        want.append(oracle.share_gemm(x, w, sh, mask))
        ts = None if sh is None else torch.from_numpy(sh.astype(np.int8)).cuda()
        y = to_dev(np.full((m, n), 0x1234, dtype=np.uint64))  # stale values the clear must remove
        descs.append((to_dev(x), torch.from_numpy(w).cuda(), ts, y, mask))
    print("[gemm] batch, outputs cleared together", flush=True)
    _batch(descs)
    for i, d in enumerate(descs):
        np.testing.assert_array_equal(from_dev(d[3]), want[i], err_msg=f"product {i}")
    # overlap: product 1's shares are B, product 2 (split K, [512 x 1024]) writes B
    m, k, n = 512, 1024, 1024
    xb = oracle.fill_u64(m * k, 8200).reshape(m, k)
    w1 = oracle.fill_i8(512 * k, 8201).reshape(512, k)
    x2 = oracle.fill_u64(m * 2048, 8202).reshape(m, 2048)
    w2 = oracle.fill_i8(n * 2048, 8203).reshape(n, 2048)
    B = to_dev(xb)
    y1 = to_dev(np.zeros((m, 512), dtype=np.uint64))
    y0 = to_dev(np.zeros((m, n), dtype=np.uint64))
    tw1, tw2, tx2 = torch.from_numpy(w1).cuda(), torch.from_numpy(w2).cuda(), to_dev(x2)
    print("[gemm] batch, split-K output overlapping an earlier input", flush=True)
    _batch([(tx2, tw2, None, y0, 64), (B, tw1, None, y1, 64), (tx2, tw2, None, B, 64)])
    np.testing.assert_array_equal(from_dev(y1), oracle.share_gemm(xb, w1))
    np.testing.assert_array_equal(from_dev(B), oracle.share_gemm(x2, w2))
    np.testing.assert_array_equal(from_dev(y0), oracle.share_gemm(x2, w2))
