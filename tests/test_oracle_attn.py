"""Pins the attention-chain oracle (oracle/mnemo_oracle_attn.c) against independent checks:
closed forms, invariants of the operations (scale invariance of RMS norm, rotations that
preserve norms and compose, softmax special cases) and the independent numpy restatement
in oracle/oracle_np.py.  Reference files cited are MnemoCUDA's.
"""
import numpy as np
import pytest

from oracle import oracle_np as onp
from tests.conftest import rel_l2


# ------------------------------------------------------------------ RMS norm (kernels.cu:692-781)
def test_rms_norm_closed_form(oracle):
    # constant c: out = w * c / sqrt(c^2 + eps)
    for c, eps in ((3.0, 1e-6), (-0.25, 1e-5), (1e-3, 1e-6)):
        x = np.full(512, c, np.float32)
        w = np.linspace(-2, 2, 512).astype(np.float32)
        want = w.astype(np.float64) * c / np.sqrt(c * c + eps)
        np.testing.assert_allclose(oracle.rms_norm(x, w, eps), want, rtol=1e-6, atol=1e-12)


def test_rms_norm_scale_invariant_and_numpy(oracle, rng):
    x = rng.standard_normal(4096).astype(np.float32)
    w = rng.standard_normal(4096).astype(np.float32)
    a = oracle.rms_norm(x, w, 0.0)
    b = oracle.rms_norm(x * np.float32(8.0), w, 0.0)  # power of two: exact scaling of x
    np.testing.assert_allclose(a, b, rtol=1e-6)
    np.testing.assert_allclose(a, onp.rms_norm(x, w, 0.0), rtol=1e-6, atol=1e-7)
    np.testing.assert_allclose(oracle.rms_norm(x, w, 1e-6), onp.rms_norm(x, w, 1e-6), rtol=1e-6, atol=1e-7)


def test_rms_norm_residual_and_heads(oracle, rng):
    x = rng.standard_normal(4096).astype(np.float32)
    w = rng.standard_normal(4096).astype(np.float32)
    n, r = oracle.rms_norm_residual(x, w, 1e-6)
    assert np.array_equal(r, x)
    assert np.array_equal(n, oracle.rms_norm(x, w, 1e-6))
    q = rng.standard_normal(64 * 128).astype(np.float32)
    wh = rng.standard_normal(128).astype(np.float32)
    got = oracle.rms_norm_heads(q, wh, 128, 1e-6)
    want = onp.rms_norm(q.reshape(64, 128), wh, 1e-6).reshape(-1)
    np.testing.assert_allclose(got, want, rtol=1e-6, atol=1e-7)
    np.testing.assert_array_equal(oracle.residual_add(x, w), x + w)


# ------------------------------------------------------------------ RoPE (kernels.cu:818-852, 1256-1266)
def test_rope_identity_at_pos0(oracle, rng):
    q = rng.standard_normal(64 * 128).astype(np.float32)
    k = rng.standard_normal(4 * 128).astype(np.float32)
    q2, k2 = oracle.rope(q, k, 128, 0, 1e6)
    assert np.array_equal(q2, q) and np.array_equal(k2, k)


def test_rope_freqs_closed_form(oracle):
    # theta^(2j/hd): j = 0 gives 1, and for theta = 2^16, hd = 128 every freq is a power of two
    for j in range(64):
        assert oracle.rope_freq(j, 128, 65536.0) == np.float32(2.0) ** (-(16 * 2 * j) / 128)
    assert oracle.rope_freq(0, 128, 1e6) == 1.0


@pytest.mark.parametrize("pos", [1, 7, 1000, 40959])
def test_rope_rotation_invariants(oracle, rng, pos):
    hd = 128
    q = rng.standard_normal(8 * hd).astype(np.float32)
    k = rng.standard_normal(2 * hd).astype(np.float32)
    q2, k2 = oracle.rope(q, k, hd, pos, 1e6)
    # each (j, j + hd/2) pair keeps its length
    for v, v2 in ((q, q2), (k, k2)):
        a = v.reshape(-1, hd).astype(np.float64)
        b = v2.reshape(-1, hd).astype(np.float64)
        n0 = a[:, :64] ** 2 + a[:, 64:] ** 2
        n1 = b[:, :64] ** 2 + b[:, 64:] ** 2
        np.testing.assert_allclose(n1, n0, rtol=1e-5, atol=1e-6)
    np.testing.assert_array_equal(q2, onp.rope(q, hd, pos, 1e6))
    np.testing.assert_array_equal(k2, onp.rope(k, hd, pos, 1e6))


def test_rope_composes(oracle, rng):
    # with theta = 2^16 the angles pos * freq are exact in fp32 for small pos, so
    # R(a) R(b) = R(a + b) up to the rounding of the two rotations
    q = rng.standard_normal(4 * 128).astype(np.float32)
    k = np.zeros(128, np.float32)
    a, _ = oracle.rope(q, k, 128, 3, 65536.0)
    ab, _ = oracle.rope(a, k, 128, 5, 65536.0)
    c, _ = oracle.rope(q, k, 128, 8, 65536.0)
    np.testing.assert_allclose(ab, c, rtol=0, atol=2e-6)


# ------------------------------------------------------------------ int8 KV (kernels.cu:1339-1377)
def test_kv_quant_int8_closed_forms(oracle, rng):
    hd = 128
    x = rng.standard_normal(4 * hd).astype(np.float32)
    x[hd:2 * hd] = 0.0  # a zero head
    q, sc = oracle.kv_quant_int8(x, hd)
    assert sc[1] == 0.0 and not q[hd:2 * hd].any()
    for h in (0, 2, 3):
        seg = x[h * hd:(h + 1) * hd]
        i = np.argmax(np.abs(seg))
        assert q[h * hd + i] == (127 if seg[i] > 0 else -127)
        assert sc[h] == np.float32(np.abs(seg).max() / np.float32(127.0))
    # ties round to even: x = 0.5 * amax / 127 * odd
    y = np.zeros(hd, np.float32)
    y[0] = 127.0
    y[1:6] = np.array([0.5, 1.5, 2.5, -0.5, -2.5], np.float32)
    qy, _ = oracle.kv_quant_int8(y, hd)
    assert list(qy[:6]) == [127, 0, 2, 2, 0, -2]
    qn, sn = onp.kv_quant_int8(x, hd)
    assert np.array_equal(q, qn) and np.array_equal(sc, sn)


# ------------------------------------------------------------------ attention (kernels.cu:1382-1481, 1550-1660)
def _f16(a):
    return np.asarray(a, np.float32).astype(np.float16).view(np.uint16)


def test_attention_special_cases(oracle, rng):
    nh, hd, nkv = 8, 64, 2
    q = rng.standard_normal(nh * hd).astype(np.float32)
    k = rng.standard_normal((5, nkv, hd)).astype(np.float32)
    v = rng.standard_normal((5, nkv, hd)).astype(np.float32)
    kb, vb = _f16(k), _f16(v)
    vf = vb.view(np.float16).astype(np.float32)
    # one position: out = v_0 of the head's kv head
    o1 = oracle.attention(q, kb, vb, nh, hd, nkv, 1, 0.125).reshape(nh, hd)
    for h in range(nh):
        np.testing.assert_array_equal(o1[h], vf[0, h // (nh // nkv)])
    # q = 0: uniform weights, out = mean over positions
    o0 = oracle.attention(np.zeros_like(q), kb, vb, nh, hd, nkv, 5, 0.125).reshape(nh, hd)
    for h in range(nh):
        np.testing.assert_allclose(o0[h], vf[:, h // (nh // nkv)].mean(axis=0), rtol=1e-6, atol=1e-7)
    # a dominant score selects its position
    kd = np.zeros((5, nkv, hd), np.float32)
    kd[3] = 1.0
    qd = np.full(nh * hd, 4.0, np.float32)
    od = oracle.attention(qd, _f16(kd), vb, nh, hd, nkv, 5, 1.0).reshape(nh, hd)
    for h in range(nh):
        np.testing.assert_allclose(od[h], vf[3, h // (nh // nkv)], rtol=1e-6, atol=1e-6)


def test_attention_numpy_f16_and_int8(oracle, rng):
    nh, hd, nkv, seq = 16, 128, 4, 300
    q = rng.standard_normal(nh * hd).astype(np.float32)
    k = rng.standard_normal((seq, nkv, hd)).astype(np.float32)
    v = rng.standard_normal((seq, nkv, hd)).astype(np.float32)
    kb, vb = _f16(k), _f16(v)
    got = oracle.attention(q, kb, vb, nh, hd, nkv, seq, 1 / np.sqrt(hd))
    want = onp.attention(q, kb.view(np.float16).astype(np.float32).reshape(seq, nkv, hd),
                         vb.view(np.float16).astype(np.float32).reshape(seq, nkv, hd), nh, hd, nkv, 1 / np.sqrt(hd))
    assert rel_l2(got, want) < 1e-6
    kq, ks = onp.kv_quant_int8(k.reshape(-1), hd)
    vq, vs = onp.kv_quant_int8(v.reshape(-1), hd)
    got8 = oracle.attention(q, kq, vq, nh, hd, nkv, seq, 1 / np.sqrt(hd), ks, vs)
    kd = (kq.reshape(seq, nkv, hd).astype(np.float32) * ks.reshape(seq, nkv, 1))
    vd = (vq.reshape(seq, nkv, hd).astype(np.float32) * vs.reshape(seq, nkv, 1))
    want8 = onp.attention(q, kd, vd, nh, hd, nkv, 1 / np.sqrt(hd))
    assert rel_l2(got8, want8) < 1e-6
