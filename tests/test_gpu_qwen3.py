"""The local share GEMMs of a Qwen3-0.6B forward (28 layers x {q|k|v, o, gate|up,
down}, 512 tokens, int8 weights with per-channel shifts): one full layer
bit-exact against the oracle, every product of all 28 layers checked by
Freivalds' identity y.r = x.(W^T (r << s)) mod 2^64 on the host."""
import numpy as np
import pytest

import oracle
import praghip
from conftest import from_dev

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def model(gpu):
    import torch
    m = praghip.Qwen3LocalGemms(rows=512)
    m.forward()
    torch.cuda.synchronize()
    return m


def _host(t):
    import torch
    return from_dev(t) if t.dtype == torch.int64 else t.cpu().numpy()


def test_shapes_and_ops(model):
    s = praghip.QWEN3_0_6B
    assert [p[1:] for p in s.products()] == [(1024, 4096), (2048, 1024), (1024, 6144), (3072, 1024)]
    assert s.ops_per_layer(512) == 2 * 512 * 15728640  # 16.1 G ops per layer
    assert model.ops == 28 * 2 * 512 * 15728640


@pytest.mark.parametrize("layer", [0, 27])
def test_layer_bit_exact(model, layer):
    print(f"[qwen3] layer {layer} vs oracle", flush=True)
    for name, _, _ in praghip.QWEN3_0_6B.products():
        x, w, sh, y = model.product(layer, name)
        want = oracle.share_gemm(_host(x), _host(w), _host(sh), mask_bits=64, threads=0)
        np.testing.assert_array_equal(_host(y), want, err_msg=f"layer {layer} {name}")


def test_all_layers_freivalds(model):
    rng = np.random.default_rng(7)
    for layer in range(28):
        for name, _, _ in praghip.QWEN3_0_6B.products():
            x, w, sh, y = (_host(t) for t in model.product(layer, name))
            n = w.shape[0]
            for _ in range(2):
                r = rng.integers(0, 2**63, size=n, dtype=np.uint64) * np.uint64(2) + np.uint64(1)
                rs = r << sh.astype(np.uint64)  # (a << s) r = a (r << s) mod 2^64
                wr = w.astype(np.int64).astype(np.uint64).T @ rs  # wraps mod 2^64
                assert np.array_equal(y @ r, x @ wr), f"layer {layer} {name}"
