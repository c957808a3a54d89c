"""GPU parity of the router (fp32 matvec + top-k softmax), the glue kernels and the Q8_1
quantizer.  Integer results (top-k indices, quantized bytes) must be exact."""
import numpy as np
import pytest
import torch

from oracle import oracle_np as onp
from tests.conftest import rel_l2
from tests.gpu_util import case, dev, host

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("rows,cols", [(128, 4096), (1, 64), (7, 300), (130, 1024)])
def test_matvec_f32(gpu, oracle, rows, cols):
    rng = np.random.default_rng(rows + cols)
    w = rng.standard_normal((rows, cols)).astype(np.float32)
    x = rng.standard_normal(cols).astype(np.float32)
    y = torch.zeros(rows, device="cuda")
    case(f"matvec_f32 {rows}x{cols}")
    gpu.ops.matvec_f32(dev(w), dev(x), y, rows, cols)
    assert rel_l2(host(y), oracle.matvec_f32(w, x, rows, cols)) < 1e-6


@pytest.mark.parametrize("n,k", [(128, 8), (128, 1), (128, 16), (60, 8), (1024, 8), (5, 8)])
def test_topk_exact(gpu, oracle, n, k):
    rng = np.random.default_rng(n * k)
    for trial in range(20):
        s = rng.standard_normal(n).astype(np.float32)
        if trial % 4 == 1 and n > 20:
            s[rng.integers(0, n, 12)] = s[5]  # ties resolved by lower index
        idx, w = torch.zeros(k, dtype=torch.int32, device="cuda"), torch.zeros(k, device="cuda")
        case(f"topk n={n} k={k} trial={trial}")
        gpu.ops.topk_softmax(dev(s), idx, w, n, k)
        ridx, rw = oracle.topk_softmax(s, k)
        assert np.array_equal(host(idx), ridx)
        np.testing.assert_allclose(host(w), rw, rtol=1e-6, atol=1e-7)


def test_router_then_topk(gpu, oracle):
    """Router logits from the GPU matvec feed top-k; an index may only differ where the
    oracle's k-th / (k+1)-th logit gap is below the matvec's accumulation error."""
    rng = np.random.default_rng(11)
    W = rng.standard_normal((128, 4096)).astype(np.float32) * 0.02
    for trial in range(10):
        x = rng.standard_normal(4096).astype(np.float32)
        logits = torch.zeros(128, device="cuda")
        idx, w = torch.zeros(8, dtype=torch.int32, device="cuda"), torch.zeros(8, device="cuda")
        case(f"router+topk trial={trial}")
        gpu.ops.matvec_f32(dev(W), dev(x), logits, 128, 4096)
        gpu.ops.topk_softmax(logits, idx, w, 128, 8)
        z = oracle.matvec_f32(W, x, 128, 4096)
        order = np.argsort(-z, kind="stable")
        got = set(host(idx).tolist())
        if got != set(order[:8].tolist()):
            assert abs(z[order[7]] - z[order[8]]) < 1e-4


def test_swiglu_and_scaled_add(gpu, oracle):
    rng = np.random.default_rng(2)
    g = (rng.standard_normal(1536) * 4).astype(np.float32)
    u = rng.standard_normal(1536).astype(np.float32)
    out = torch.zeros(1536, device="cuda")
    case("swiglu")
    gpu.ops.swiglu(dev(g), dev(u), out, 1536)
    np.testing.assert_allclose(host(out), oracle.swiglu(g, u), rtol=2e-6, atol=1e-7)
    acc0 = rng.standard_normal(4096).astype(np.float32)
    x = rng.standard_normal(4096).astype(np.float32)
    acc = dev(acc0.copy())
    case("scaled_add")
    gpu.ops.scaled_add(acc, dev(x), 0.3, 4096)
    ref = acc0.copy()
    oracle.L.mo_scaled_add(oracle._p(ref), oracle._p(x), 0.3, 4096)
    np.testing.assert_allclose(host(acc), ref, rtol=1e-6, atol=1e-6)


@pytest.mark.parametrize("N,K", [(512, 4096), (1, 4096), (3, 128), (17, 1536)])
def test_quantize_q8_1_bit_exact(gpu, oracle, N, K):
    rng = np.random.default_rng(N + K)
    x = rng.standard_normal((N, K)).astype(np.float32)
    x[0, :32] = 0.0
    if K >= 128:
        x[-1, 32:64] = np.float32(2.5) * np.sign(rng.standard_normal(32)).astype(np.float32)
    dst = torch.zeros(N * (K // 128) * 144, dtype=torch.uint8, device="cuda")
    case(f"quantize_q8_1 {N}x{K}")
    gpu.ops.quantize_q8_1(dev(x), dst, K, N)
    got = host(dst).reshape(N, K // 128, 144)
    exp = oracle.quantize_q8_1(x)
    assert np.array_equal(got, exp)
    assert np.array_equal(exp, onp.quantize_q8_1_mmq(x))
