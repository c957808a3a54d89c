"""Pins tests/torch_ref.py (the GPU-side restatement used at the benchmark's full sizes) against the
C oracle on the CPU."""
import numpy as np
import pytest
import torch

from mnemocuda_amd import synth
from tests import torch_ref as tr
from tests.conftest import rel_l2


@pytest.mark.parametrize("type_id,M,K,N", [(12, 40, 512, 7), (14, 33, 768, 5)])
def test_gemm_matches_oracle(oracle, rng, type_id, M, K, N):
    w = synth.weights(rng, type_id, M, K)
    x = rng.standard_normal((N, K)).astype(np.float32)
    x[1, 64:96] = 0.0  # a zero sub-block
    act = oracle.quantize_q8_1(x)
    got = tr.gemm(type_id, torch.from_numpy(w), torch.from_numpy(act), M, K, N).numpy()
    assert rel_l2(got, oracle.gemm(type_id, w, act, M, K, N)) < 1e-12


def test_quantize_matches_oracle(oracle, rng):
    x = rng.standard_normal((6, 1024)).astype(np.float32) * np.float32(3.0)
    x[2, :32] = 0.0
    x[3, 5] = 1e4
    got = tr.quantize_q8_1(torch.from_numpy(x)).numpy()
    assert np.array_equal(got, oracle.quantize_q8_1(x))


def test_moe_chain_matches_oracle(oracle):
    T, H, EFF, E, k, DT = 12, 512, 256, 6, 3, 14
    rng = np.random.default_rng(7)
    table = synth.expert_table(rng, E, H, EFF, DT)
    lay = synth.expert_layout(H, EFF, DT)
    idx, w = synth.zipf_routing(rng, T, E, k)
    x = rng.standard_normal((T, H)).astype(np.float32)
    ref = oracle.moe_prefill(table, *lay, DT, x, idx, w, H, EFF, E)
    got = tr.moe_prefill(torch.from_numpy(table), *lay, DT, torch.from_numpy(x), idx, w, H, EFF).numpy()
    # the two SwiGLUs use different expf implementations, which can move a requantized value
    # by one step in rare cases
    assert rel_l2(got, ref) < 1e-5
