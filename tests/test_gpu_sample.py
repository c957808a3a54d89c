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


def _gpu_sample_ws(gpu, z, T, top_p, seed, ws=None):
    out = torch.full((1,), -7, dtype=torch.int32, device="cuda")
    if ws is None:
        ws = torch.empty(gpu.ops.sample_workspace_bytes(), dtype=torch.uint8, device="cuda")
    gpu.ops.sample_token_ws(dev(z), z.size, T, top_p, seed, ws, out)
    return int(host(out)[0])


@pytest.mark.parametrize("V", [151936, 1000, 257, 262144])
def test_greedy_ws(gpu, oracle, V):
    """the two-launch form's argmax: ties to the lower index across class groups."""
    rng = np.random.default_rng(V + 1)
    z = (rng.standard_normal(V) * 4).astype(np.float32)
    z[[V // 3, V - 5]] = z.max() + 0.5
    case(f"sample_ws greedy V={V}")
    assert _gpu_sample_ws(gpu, z, 0.0, 0.9, 1) == oracle.sample_token(z, 0.0, 0.9, 1)[0] == V // 3


@pytest.mark.parametrize("V,scale,T,top_p,data", [(151936, 3.0, 0.7, 0.9, 12), (151936, 1.0, 1.0, 0.95, 11),
                                                  (151936, 6.0, 0.6, 0.5, 11), (3000, 2.0, 0.9, 0.8, 11),
                                                  (300, 1.0, 1.0, 0.99, 11)])
def test_top_p_ws(gpu, oracle, V, scale, T, top_p, data):
    """the same token as the oracle (and the one-launch form) for every seed away from a
    nucleus boundary; the workspace is reused across calls without clearing.  (`data` picks
    logits whose nucleus boundary is not within 1e-5 of the mass, so that most seeds count.)"""
    rng = np.random.default_rng(int(V * scale) + data)
    z = (rng.standard_normal(V) * scale).astype(np.float32)
    seeds = rng.integers(0, 2**63, 24).tolist()
    ws = torch.full((gpu.ops.sample_workspace_bytes(),), 255, dtype=torch.uint8, device="cuda")
    case(f"sample_ws top-p V={V} T={T} top_p={top_p}")
    checked = 0
    for seed in seeds:
        tok, margin = onp.sample_token(z, T, top_p, seed)
        if margin < 1e-5:
            continue
        ref = oracle.sample_token(z, T, top_p, seed)[0]
        assert ref == tok
        assert _gpu_sample_ws(gpu, z, T, top_p, seed, ws) == ref == _gpu_sample(gpu, z, T, top_p, seed), seed
        checked += 1
    print(f"checked {checked} seeds")
    assert checked >= 16


@pytest.mark.parametrize("V,step,T,top_p", [(151936, 0.5, 0.7, 0.9), (3000, 0.25, 1.0, 0.8)])
def test_top_p_ties(gpu, V, step, T, top_p):
    """logits on a coarse grid, so that most candidates share their p with others: both
    forms take equal p in increasing token id and draw the token of the numpy restatement,
    which orders them so.  (The reference orders equal p by where its selection sort's
    swaps left them, kernels.cu:2145-2166 -- the C oracle follows that -- so at a tie the
    token can differ from the reference's, while the running sums at every position agree.)"""
    rng = np.random.default_rng(V + 7)
    z = (np.round(rng.standard_normal(V) * 2.0 / step) * step).astype(np.float32)
    seeds = rng.integers(0, 2**63, 32).tolist()
    ws = torch.empty(gpu.ops.sample_workspace_bytes(), dtype=torch.uint8, device="cuda")
    case(f"sample top-p ties V={V} step={step}")
    checked = 0
    for seed in seeds:
        tok, margin = onp.sample_token(z, T, top_p, seed)
        if margin < 1e-5:
            continue
        assert _gpu_sample(gpu, z, T, top_p, seed) == tok, seed
        assert _gpu_sample_ws(gpu, z, T, top_p, seed, ws) == tok, seed
        checked += 1
    print(f"checked {checked} seeds")
    assert checked >= 16

def test_sample_ws_bad_args(gpu):
    case("sample_ws bad args")
    z = torch.zeros(300000, device="cuda")
    out = torch.zeros(1, dtype=torch.int32, device="cuda")
    ws = torch.empty(gpu.ops.sample_workspace_bytes(), dtype=torch.uint8, device="cuda")
    with pytest.raises(gpu.MnemoError):  # vocabulary above 262,144
        gpu.ops.sample_token_ws(z, 300000, 0.7, 0.9, 1, ws, out)
    with pytest.raises(gpu.MnemoError):  # workspace too small
        gpu.ops.sample_token_ws(z, 1000, 0.7, 0.9, 1, ws[:100], out)
