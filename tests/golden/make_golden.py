#!/usr/bin/env python3
"""Writes the golden fixtures of the quantized-matmul path (tests/golden/*.npz).

The reference ships no golden vectors or kernel known-answer tests for this path (its
tests/ hold engine, heat-map and server tests only), so these fixtures are produced by
the C oracle (oracle/mnemo_oracle.c) and cross-checked here against the independent
numpy restatement (oracle/oracle_np.py) before they are written; they then pin both
restatements against regressions.  Inputs use the benchmark configs' value distributions.

Run:  python tests/golden/make_golden.py
"""
import sys
from pathlib import Path

import numpy as np

ROOT = Path(__file__).resolve().parents[2]
sys.path.insert(0, str(ROOT))

import oracle  # noqa: E402
from oracle import oracle_np as onp  # noqa: E402
from mnemocuda_amd import synth  # noqa: E402

OUT = Path(__file__).resolve().parent


def main():
    o = oracle.load()
    rng = np.random.default_rng(20261201)
    fx = {}
    # two super-blocks per format with their decoded values
    q4 = synth.q4k_blocks(rng, 2)
    q6 = synth.q6k_blocks(rng, 2)
    fx["q4k_blocks"] = q4
    fx["q4k_values"] = o.dequant(12, q4.reshape(-1), 1, 512)[0]
    fx["q6k_blocks"] = q6
    fx["q6k_values"] = o.dequant(14, q6.reshape(-1), 1, 512)[0]
    assert np.array_equal(fx["q4k_values"], onp.dequant_matrix(q4.reshape(-1), 12, 1, 512)[0])
    assert np.array_equal(fx["q6k_values"], onp.dequant_matrix(q6.reshape(-1), 14, 1, 512)[0])
    # a 64 x 1024 GEMV of each type
    for t, name in ((12, "q4k"), (14, "q6k")):
        w = synth.weights(rng, t, 64, 1024)
        x = rng.standard_normal(1024).astype(np.float32)
        y = o.gemv(t, w, x, 64, 1024)
        ref = onp.dequant_matrix(w, t, 64, 1024).astype(np.float64) @ x.astype(np.float64)
        assert np.max(np.abs(y - ref)) <= 1e-9 * np.max(np.abs(ref))
        fx[f"gemv_{name}_w"], fx[f"gemv_{name}_x"], fx[f"gemv_{name}_y"] = w, x, y
    # Q8_1 quantization of a 4 x 512 activation block and a 64 x 256 x 512 GEMM
    a = rng.standard_normal((8, 512)).astype(np.float32)
    aq = o.quantize_q8_1(a)
    assert np.array_equal(aq, onp.quantize_q8_1_mmq(a))
    fx["q8_1_src"], fx["q8_1_blocks"] = a, aq
    wg = synth.weights(rng, 12, 64, 512)
    fx["gemm_w"], fx["gemm_out"] = wg, o.gemm(12, wg, aq, 64, 512, 8)
    ref = onp.gemm_q8_1(12, wg, aq, 64, 512, 8)
    assert np.max(np.abs(fx["gemm_out"] - ref)) <= 1e-9 * np.max(np.abs(ref))
    # a 128-logit top-8 case (with a tie) and the router matvec
    logits = rng.standard_normal(128).astype(np.float32)
    logits[77] = logits[12]
    idx, w = o.topk_softmax(logits, 8)
    ridx, rw = onp.topk_softmax(logits, 8)
    assert np.array_equal(idx, ridx) and np.allclose(w, rw, rtol=1e-6)
    fx["topk_logits"], fx["topk_idx"], fx["topk_w"] = logits, idx, w
    np.savez_compressed(OUT / "hot_path_golden.npz", **fx)
    print("wrote", OUT / "hot_path_golden.npz", {k: v.shape for k, v in fx.items()})


if __name__ == "__main__":
    main()
