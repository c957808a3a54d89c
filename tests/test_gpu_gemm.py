"""GPU parity of the Q4_K/Q6_K x Q8_1 GEMM.

Reference value: dequant(W) . dequant(Q8_1(x)) (the product gemm_q4k.cu:103-112 computes).
Bar: relative L2 <= 1e-3.  Small shapes against the fp64 C oracle; the BASELINE shapes
against a torch fp32 GEMM of the oracle-dequantised operands (the fp64 oracle would take
minutes there) plus size-independent properties."""
import numpy as np
import pytest
import torch

from mnemocuda_amd import synth
from oracle import oracle_np as onp
from tests.conftest import rel_l2
from tests.gpu_util import case, dev, host

pytestmark = pytest.mark.gpu
TOL = 1e-3


def _run(gpu, type_id, wd, actd, M, K, N):
    out = torch.full((N, M), float("nan"), device="cuda")
    gpu.ops.gemm(wd, type_id, actd, out, M, K, N)
    return out


@pytest.mark.parametrize("type_id,M,K,N", [(12, 256, 1024, 128), (12, 100, 512, 37), (14, 130, 768, 9),
                                           (12, 1, 256, 1), (14, 64, 1536, 200),
                                           # ragged tiles with K split 8 ways (summed with atomics)
                                           (12, 200, 4096, 100), (14, 36, 2048, 68)])
def test_gemm_vs_oracle(gpu, oracle, type_id, M, K, N):
    rng = np.random.default_rng(M * N + K)
    w = synth.weights(rng, type_id, M, K)
    act = oracle.quantize_q8_1(rng.standard_normal((N, K)).astype(np.float32))
    case(f"gemm type={type_id} M={M} K={K} N={N}")
    out = _run(gpu, type_id, dev(w), dev(act), M, K, N)
    got, ref = host(out), oracle.gemm(type_id, w, act, M, K, N)
    err = rel_l2(got, ref)
    print(f"rel_l2={err:.2e}")
    if M * N >= 64:
        assert err < TOL
    else:
        # too few outputs for a relative L2 to concentrate: check the forward error bound
        # of two f16 operand roundings, sum_k |w_k a_k| * 2 * 2^-11 (+ fp32 accumulation)
        wa = np.abs(oracle.dequant(type_id, w, M, K)).astype(np.float64)
        aa = np.abs(oracle.dequant_q8_1(act, K, N)).astype(np.float64)
        bound = (aa @ wa.T) * (2 * 2.0**-11 + K * 2.0**-24)
        assert np.all(np.abs(got - ref) <= bound)


@pytest.mark.parametrize("type_id,M,K,N", [(12, 8192, 4096, 512), (12, 1536, 4096, 512), (14, 4096, 1536, 512)])
def test_gemm_baseline_shapes(gpu, oracle, type_id, M, K, N):
    rng = np.random.default_rng(M + N)
    w = synth.weights(rng, type_id, M, K)
    x = rng.standard_normal((N, K)).astype(np.float32)
    actd = torch.zeros(N * (K // 128) * 144, dtype=torch.uint8, device="cuda")
    case(f"gemm baseline type={type_id} M={M} K={K} N={N}")
    gpu.ops.quantize_q8_1(dev(x), actd, K, N)
    out = _run(gpu, type_id, dev(w), actd, M, K, N)
    wdeq = torch.from_numpy(oracle.dequant(type_id, w, M, K)).cuda()
    adeq = torch.from_numpy(onp.dequant_q8_1_mmq(host(actd).reshape(N, K // 128, 144), K)).cuda()
    torch.backends.cuda.matmul.allow_tf32 = False
    ref = (adeq.double() @ wdeq.double().T)
    err = rel_l2(host(out), ref.cpu().numpy())
    print(f"rel_l2={err:.2e}")
    assert err < TOL
    # linearity in the activation scale: doubling every d8 doubles the output
    a2 = actd.view(N, K // 128, 144).clone()
    ds = a2[:, :, :16].contiguous().view(torch.float16).clone()
    ds[..., 0::2] *= 2
    a2[:, :, :16] = ds.view(torch.uint8).reshape(N, K // 128, 16)
    out2 = _run(gpu, type_id, dev(w), a2.reshape(-1), M, K, N)
    assert rel_l2(host(out2), 2 * host(out)) < 1e-6


@pytest.mark.parametrize("type_id", [12, 14])
def test_gemm_large_activations(gpu, oracle, type_id):
    """Activations whose Q8_1 values d8*q8 exceed the f16 range (|x| up to ~5e6; d8 itself
    still fits f16, as the Q8_1 format requires) and rows of very different magnitude."""
    M, K, N = 192, 1024, 48
    rng = np.random.default_rng(11 + type_id)
    w = synth.weights(rng, type_id, M, K)
    x = rng.standard_normal((N, K)).astype(np.float32)
    x *= np.logspace(-3, 6, N, dtype=np.float32)[:, None]
    act = oracle.quantize_q8_1(x)
    case(f"gemm large activations type={type_id}")
    out = _run(gpu, type_id, dev(w), dev(act), M, K, N)
    got, ref = host(out), oracle.gemm(type_id, w, act, M, K, N)
    assert np.all(np.isfinite(got))
    # per token row: rows span 9 decades, so compare each on its own scale
    for j in range(N):
        assert rel_l2(got[j], ref[j]) < TOL, j
