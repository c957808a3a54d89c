"""A C program calls the library the way the reference engine does (tests/c_caller/
engine_calls.c: plain C, hipMalloc'd buffers, the extern "C" entry points with the
reference's argument lists -- MnemoCUDA src/forward.c:160-173, 687-823), and its results
are checked here against the oracle on the same seeded inputs: the drop-in boundary seen
from C.  The program is built by __graft_entry__.build() next to the library."""
import subprocess

import numpy as np
import pytest

from mnemocuda_amd.build import CALLER
from tests.conftest import rel_l2
from tests.gpu_util import case

pytestmark = pytest.mark.gpu
TOL = 1e-3


def test_c_caller_matches_oracle(gpu, oracle, tmp_path):
    if not CALLER.exists():
        pytest.fail(f"{CALLER} is not built (run __graft_entry__.build())")
    out = tmp_path / "calls.bin"
    case("C caller of the C-ABI")
    r = subprocess.run([str(CALLER), str(out)], capture_output=True, text=True, timeout=120)
    assert r.returncode == 0, r.stdout + r.stderr
    buf = out.read_bytes()
    R, RK, C, E, K, NT = np.frombuffer(buf[:24], np.int32)
    off = 24

    def take(n, dtype):
        nonlocal off
        a = np.frombuffer(buf[off: off + n * np.dtype(dtype).itemsize], dtype)
        off += n * np.dtype(dtype).itemsize
        return a

    q4b, q6b = C // 256 * 144, C // 256 * 210
    wq4, wq6 = take(R * q4b, np.uint8), take(R * q6b, np.uint8)
    wk, wv = take(RK * q4b, np.uint8), take(RK * q6b, np.uint8)
    x, res, router = take(C, np.float32), take(R, np.float32), take(E * C, np.float32)
    x2, act = take(C, np.float32), take(NT * C, np.float32).reshape(NT, C)
    y4, y6, yadd, ya, yb, q = (take(R, np.float32) for _ in range(6))
    k, v, logits = take(RK, np.float32), take(RK, np.float32), take(E, np.float32)
    idx, w = take(K, np.int32), take(K, np.float32)
    q2, k2, v2 = take(R, np.float32), take(RK, np.float32), take(RK, np.float32)
    ysa, sw, ysc = take(R, np.float32), take(C, np.float32), take(R, np.float32)
    q8 = take(NT * (C // 128) * 144, np.uint8)
    gout = take(NT * R, np.float32).reshape(NT, R)
    HH, NH, NKV, HD, SEQ, VOC, VT = (int(v) for v in take(7, np.int32))
    nkv = SEQ * NKV * HD
    xin, anorm = take(HH, np.float32), take(HH, np.float32)
    qraw, kraw, vraw = take(NH * HD, np.float32), take(NKV * HD, np.float32), take(NKV * HD, np.float32)
    qw, kw = take(HD, np.float32), take(HD, np.float32)
    kc, vc, kc8, vc8 = take(nkv, np.uint16), take(nkv, np.uint16), take(nkv, np.int8), take(nkv, np.int8)
    ksc, vsc, lg = take(SEQ * NKV, np.float32), take(SEQ * NKV, np.float32), take(VOC, np.float32)
    table = take(VT * (HH // 256) * 144, np.uint8)
    normed, resid, normed2, radd = (take(HH, np.float32) for _ in range(4))
    att, att8, emb = take(NH * HD, np.float32), take(NH * HD, np.float32), take(HH, np.float32)
    qpost, kpost = take(NH * HD, np.float32), take(NKV * HD, np.float32)
    kc_o, vc_o, kc8_o, vc8_o = take(nkv, np.uint16), take(nkv, np.uint16), take(nkv, np.int8), take(nkv, np.int8)
    ksc_o, vsc_o = take(SEQ * NKV, np.float32), take(SEQ * NKV, np.float32)
    tok = int(take(1, np.int32)[0])
    qb = take(NH * HD, np.float32)
    assert off == len(buf)

    g4, g6 = oracle.gemv(12, wq4, x, R, C), oracle.gemv(14, wq6, x, R, C)
    assert rel_l2(y4, g4) < TOL and rel_l2(y6, g6) < TOL
    assert rel_l2(yadd, g4 + res) < TOL
    assert rel_l2(ya, g4) < TOL and rel_l2(yb, g4) < TOL
    assert rel_l2(q, g4) < TOL
    assert rel_l2(k, oracle.gemv(12, wk, x, RK, C)) < TOL and rel_l2(v, oracle.gemv(14, wv, x, RK, C)) < TOL
    ref_logits = oracle.matvec_f32(router, x, E, C)
    assert rel_l2(logits, ref_logits) < 1e-5
    ridx, rw = oracle.topk_softmax(logits, int(K))
    assert sorted(idx.tolist()) == sorted(ridx.tolist())
    assert np.allclose(w[np.argsort(idx)], rw[np.argsort(ridx)], rtol=1e-5, atol=1e-6)

    # cuda_matvec_q4k_qkv (all three Q4_K; V reuses the K matrix)
    gk = oracle.gemv(12, wk, x, RK, C)
    assert rel_l2(q2, g4) < TOL and rel_l2(k2, gk) < TOL and rel_l2(v2, gk) < TOL
    # cuda_matvec_q4k_scaled_add: res + 0.37 W x
    assert rel_l2(ysa - res, 0.37 * g4) < TOL
    # cuda_swiglu and cuda_scaled_add: elementwise fp32, against the oracle's restatement
    assert np.allclose(sw, oracle.swiglu(x, x2), rtol=2e-6, atol=1e-7)
    assert np.array_equal(ysc, (res + np.float32(0.5) * y4).astype(np.float32))
    # cuda_quantize_mmq_q8_1 byte-identical, cuda_gemm_q4k against the oracle GEMM
    ref_q8 = oracle.quantize_q8_1(act)
    assert np.array_equal(q8, ref_q8.reshape(-1))
    assert rel_l2(gout, oracle.gemm(12, wq4, ref_q8, R, C, NT)) < 1e-5

    # ---- the attention chain (forward.c:725-823), sampling and the embedding, from C
    pos, row = SEQ - 1, slice((SEQ - 1) * NKV * HD, SEQ * NKV * HD)
    wn, wr = oracle.rms_norm_residual(xin, anorm, 1e-6)
    np.testing.assert_allclose(normed, wn, rtol=2e-6, atol=1e-7)
    assert np.array_equal(resid, xin) and np.array_equal(resid, wr)
    np.testing.assert_allclose(normed2, oracle.rms_norm(xin, anorm, 1e-6), rtol=2e-6, atol=1e-7)
    assert np.array_equal(radd, (xin + anorm).astype(np.float32))
    rq, rk = oracle.rope(oracle.rms_norm_heads(qraw, qw, HD, 1e-6), oracle.rms_norm_heads(kraw, kw, HD, 1e-6),
                         HD, pos, 1e6)
    tol = 1e-5 * max(np.abs(rq).max(), np.abs(rk).max())
    np.testing.assert_allclose(qpost, rq, rtol=0, atol=tol)
    np.testing.assert_allclose(kpost, rk, rtol=0, atol=tol)
    # f16 stores at the new position only; attention over the stored caches
    keep = np.ones(nkv, bool)
    keep[row] = False
    assert np.array_equal(kc_o[keep], kc[keep]) and np.array_equal(vc_o[keep], vc[keep])
    assert np.array_equal(kc_o[row], kpost.astype(np.float16).view(np.uint16))
    assert np.array_equal(vc_o[row], vraw.astype(np.float16).view(np.uint16))
    scale = float(np.float32(1.0 / np.sqrt(128.0)))
    assert rel_l2(att, oracle.attention(qpost, kc_o, vc_o, NH, HD, NKV, SEQ, scale)) < 1e-5
    # int8 stores and the int8 attention
    qk, sk = oracle.kv_quant_int8(kpost, HD)
    qv, sv = oracle.kv_quant_int8(vraw, HD)
    assert np.array_equal(kc8_o[keep], kc8[keep]) and np.array_equal(vc8_o[keep], vc8[keep])
    assert np.array_equal(kc8_o[row], qk) and np.array_equal(vc8_o[row], qv)
    assert np.array_equal(ksc_o[pos * NKV:], sk) and np.array_equal(vsc_o[pos * NKV:], sv)
    assert np.array_equal(ksc_o[:pos * NKV], ksc[:pos * NKV]) and np.array_equal(vsc_o[:pos * NKV], vsc[:pos * NKV])
    ref8 = oracle.attention(qpost, kc8_o, vc8_o, NH, HD, NKV, SEQ, scale, k_scales=ksc_o, v_scales=vsc_o)
    assert rel_l2(att8, ref8) < 1e-5
    # sampling: the oracle's token unless the draw lies within rounding of a boundary
    from oracle import oracle_np as onp
    want, margin = onp.sample_token(lg, 0.8, 0.9, 12345)
    if margin >= 1e-5:
        assert tok == want == oracle.sample_token(lg, 0.8, 0.9, 12345)[0]
    # embedding row 5 of the Q4_K table, bit-exact
    assert np.array_equal(emb, oracle.dequant(12, table, VT, HH)[5])
    np.testing.assert_allclose(qb, oracle.rms_norm_heads(qraw, qw, HD, 1e-6), rtol=2e-6, atol=1e-7)
