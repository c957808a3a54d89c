"""Golden fixtures (tests/golden/hot_path_golden.npz, written by make_golden.py): the CPU
oracle must reproduce them exactly, and the HIP path must match them to the same bars
as the oracle parity tests (bit-exact bytes/indices, 1e-3 relative L2 for sums)."""
from pathlib import Path

import numpy as np
import pytest
import torch

from tests.conftest import rel_l2

G = np.load(Path(__file__).resolve().parent / "golden" / "hot_path_golden.npz", allow_pickle=False)


def test_oracle_reproduces_golden(oracle):
    assert np.array_equal(oracle.dequant(12, G["q4k_blocks"].reshape(-1), 1, 512)[0], G["q4k_values"])
    assert np.array_equal(oracle.dequant(14, G["q6k_blocks"].reshape(-1), 1, 512)[0], G["q6k_values"])
    for name, t in (("q4k", 12), ("q6k", 14)):
        y = oracle.gemv(t, G[f"gemv_{name}_w"], G[f"gemv_{name}_x"], 64, 1024)
        assert rel_l2(y, G[f"gemv_{name}_y"]) < 1e-12
    assert np.array_equal(oracle.quantize_q8_1(G["q8_1_src"]), G["q8_1_blocks"])
    assert rel_l2(oracle.gemm(12, G["gemm_w"], G["q8_1_blocks"], 64, 512, 8), G["gemm_out"]) < 1e-12
    idx, w = oracle.topk_softmax(G["topk_logits"], 8)
    assert np.array_equal(idx, G["topk_idx"]) and np.array_equal(w, G["topk_w"])


@pytest.mark.gpu
def test_gpu_matches_golden(gpu):
    from tests.gpu_util import case, dev, host
    for name, t in (("q4k", 12), ("q6k", 14)):
        y = torch.zeros(64, device="cuda")
        case(f"golden gemv {name}")
        gpu.ops.matvec(dev(G[f"gemv_{name}_w"]), dev(G[f"gemv_{name}_x"]), y, 64, 1024, t)
        assert rel_l2(host(y), G[f"gemv_{name}_y"]) < 1e-3
    dst = torch.zeros(G["q8_1_blocks"].size, dtype=torch.uint8, device="cuda")
    case("golden q8_1")
    gpu.ops.quantize_q8_1(dev(G["q8_1_src"]), dst, 512, 8)
    assert np.array_equal(host(dst).reshape(G["q8_1_blocks"].shape), G["q8_1_blocks"])
    out = torch.zeros(8, 64, device="cuda")
    case("golden gemm")
    gpu.ops.gemm(dev(G["gemm_w"]), 12, dst, out, 64, 512, 8)
    assert rel_l2(host(out), G["gemm_out"]) < 1e-3
    idx, w = torch.zeros(8, dtype=torch.int32, device="cuda"), torch.zeros(8, device="cuda")
    case("golden topk")
    gpu.ops.topk_softmax(dev(G["topk_logits"]), idx, w, 128, 8)
    assert np.array_equal(host(idx), G["topk_idx"])
    np.testing.assert_allclose(host(w), G["topk_w"], rtol=1e-6, atol=1e-7)
