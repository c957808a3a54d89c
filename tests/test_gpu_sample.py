"""GPU parity of cuda_sample_token (kernels.cu:2020-2174) against the C oracle.

Greedy: the same token (argmax; exact ties to the lower index).  Top-p: the same token
for every seed whose draw lies further than 1e-5 of the nucleus mass from a cumulative
boundary (the fp32 sums and exp() of two implementations may differ in the last bits,
which can only matter at a boundary; the margin comes from the numpy restatement).
Vocabulary of the lm_head (151,936) and a small one; peaked and flat logits."""
import numpy as np
import pytest
import torch

from oracle import oracle_np as onp
from tests.gpu_util import case, dev, host

pytestmark = pytest.mark.gpu


def _gpu_sample(gpu, z, T, top_p, seed):
    out = torch.full((1,), -7, dtype=torch.int32, device="cuda")
    gpu.ops.sample_token(dev(z), z.size, T, top_p, seed, out)
    return int(host(out)[0])


@pytest.mark.parametrize("V", [151936, 1000])
def test_greedy(gpu, oracle, V):
    rng = np.random.default_rng(V)
    z = (rng.standard_normal(V) * 4).astype(np.float32)
    z[[V // 3, V - 5]] = z.max() + 0.5  # tie: lower index
    case(f"sample greedy V={V}")
    assert _gpu_sample(gpu, z, 0.0, 0.9, 1) == oracle.sample_token(z, 0.0, 0.9, 1)[0] == V // 3


@pytest.mark.parametrize("V,scale,T,top_p", [(151936, 3.0, 0.7, 0.9), (151936, 1.0, 1.0, 0.95),
                                             (151936, 6.0, 0.6, 0.5), (3000, 2.0, 0.9, 0.8)])
def test_top_p(gpu, oracle, V, scale, T, top_p):
    rng = np.random.default_rng(int(V * scale))
    z = (rng.standard_normal(V) * scale).astype(np.float32)
    seeds = rng.integers(0, 2**63, 24).tolist()
    case(f"sample top-p V={V} T={T} top_p={top_p}")
    checked = 0
    for seed in seeds:
        tok, margin = onp.sample_token(z, T, top_p, seed)
        if margin < 1e-5:
            continue
        ref = oracle.sample_token(z, T, top_p, seed)[0]
        assert ref == tok
        assert _gpu_sample(gpu, z, T, top_p, seed) == ref, seed
        checked += 1
    print(f"checked {checked} seeds")
    assert checked >= 16
