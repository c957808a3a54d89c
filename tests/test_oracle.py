"""Pins the CPU oracle (oracle/mnemo_oracle.c) against independent checks.

Each block below checks one oracle routine against something other than its own formula:
hardware/library conversions, the layout text via one-hot brute force, closed forms,
linearity, the independent numpy restatement (oracle/oracle_np.py) and numpy fp64
matmuls.  Reference files cited are MnemoCUDA's.
"""
import numpy as np
import pytest
import torch

from oracle import oracle_np as onp
from mnemocuda_amd import synth
from tests.conftest import rel_l2

# ------------------------------------------------------------------ F1: f16 <-> f32


def test_f16_to_f32_exhaustive(oracle):
    bits = np.arange(65536, dtype=np.uint32).astype(np.uint16)
    ours = np.array([oracle.f16_to_f32(int(b)) for b in bits], np.float32)
    ref_np = bits.view(np.float16).astype(np.float32)
    ref_t = torch.from_numpy(bits.view(np.int16).copy()).view(torch.float16).float().numpy()
    nan = np.isnan(ref_np)
    assert np.array_equal(np.isnan(ours), nan)
    assert np.array_equal(ours[~nan].view(np.uint32), ref_np[~nan].view(np.uint32))
    assert np.array_equal(ours[~nan].view(np.uint32), ref_t[~nan].view(np.uint32))


def test_f32_to_f16_rne(oracle, rng):
    edge = np.array([0.0, -0.0, 1.0, 65504.0, 65519.99, 65520.0, 1e9, -1e9, 2.0**-24, 2.0**-25,
                     1.5 * 2.0**-25, 2.0**-14, 2.0**-14 - 2.0**-25, 1.0 + 2.0**-11, 1.0 + 3 * 2.0**-11,
                     np.inf, -np.inf, 6.1e-5, 3.0e-8], np.float32)
    bitsr = rng.integers(0, 2**32, 1 << 16, dtype=np.uint64).astype(np.uint32)
    vals = np.concatenate([edge, bitsr.view(np.float32), rng.standard_normal(1 << 14).astype(np.float32) * 0.01])
    vals = vals[~np.isnan(vals)]
    ours = np.array([oracle.f32_to_f16(float(v)) for v in vals], np.uint16)
    with np.errstate(over="ignore"):
        ref = vals.astype(np.float16).view(np.uint16)
    assert np.array_equal(ours, ref)


# ------------------------------------------------------------------ F2: 6-bit scales


def test_scale_min_k4_round_trip(oracle, rng):
    sc = rng.integers(0, 64, (4000, 8), dtype=np.uint8)
    m = rng.integers(0, 64, (4000, 8), dtype=np.uint8)
    packed = onp.pack_scale_min_k4(sc, m)
    # packing is a bijection of 96 bits: every byte pattern is reachable
    assert len({bytes(r) for r in packed}) == 4000
    for r in range(0, 4000, 97):
        for j in range(8):
            assert oracle.scale_min_k4(j, packed[r]) == (sc[r, j], m[r, j])
    s2, m2 = onp.scale_min_k4_all(packed)
    assert np.array_equal(s2, sc) and np.array_equal(m2, m)


def test_scale_min_packed_int_form(rng):
    """gemm_q4k.cu:53-56 (four 6-bit values per uint32) agrees with kernels.cu:45-53."""
    raw = rng.integers(0, 256, (2000, 12), dtype=np.uint8)
    sc, m = onp.scale_min_k4_all(raw)
    for ksc, (src, lo) in enumerate([(sc, 0), (sc, 4), (m, 0), (m, 4)]):
        v = onp.unpack_scales_q45k_int(raw, ksc)
        got = np.stack([(v >> (8 * t)) & 0xFF for t in range(4)], axis=1).astype(np.uint8)
        assert np.array_equal(got, src[:, lo:lo + 4]), ksc


# ------------------------------------------------------------------ F3: Q4_K


def _q4k_unit_block(d=1.0, dmin=0.0, sc=1, m=0):
    b = np.zeros(144, np.uint8)
    b[0:2] = np.array([d], np.float16).view(np.uint8)
    b[2:4] = np.array([dmin], np.float16).view(np.uint8)
    b[4:16] = onp.pack_scale_min_k4(np.full(8, sc, np.uint8), np.full(8, m, np.uint8))
    return b


def test_q4k_one_hot_layout(oracle):
    """Value v lives in qs[32*(v//64) + v%32], low nibble iff v%64 < 32 (llama.cpp Q4_K text)."""
    for v in range(256):
        b = _q4k_unit_block()
        byte = 16 + 32 * (v // 64) + v % 32
        b[byte] = 1 if v % 64 < 32 else 0x10
        out = oracle.dequant(12, b, 1, 256)[0]
        expect = np.zeros(256, np.float32)
        expect[v] = 1.0
        assert np.array_equal(out, expect), v


def test_q4k_closed_forms(oracle, rng):
    for _ in range(20):
        sc = rng.integers(0, 64, 8, dtype=np.uint8)
        m = rng.integers(0, 64, 8, dtype=np.uint8)
        d, dmin = np.float16(abs(rng.standard_normal()) * 0.01), np.float16(abs(rng.standard_normal()) * 0.01)
        b = np.zeros(144, np.uint8)
        b[0:2] = np.array([d]).view(np.uint8)
        b[2:4] = np.array([dmin]).view(np.uint8)
        b[4:16] = onp.pack_scale_min_k4(sc, m)
        sub = np.arange(256) // 32
        zero = oracle.dequant(12, b, 1, 256)[0]
        assert np.array_equal(zero, (-(np.float32(dmin) * m[sub].astype(np.float32))).astype(np.float32))
        b[16:] = 0xFF
        full = oracle.dequant(12, b, 1, 256)[0]
        exp = (np.float32(d) * sc[sub].astype(np.float32) * np.float32(15)
               - np.float32(dmin) * m[sub].astype(np.float32)).astype(np.float32)
        assert np.array_equal(full, exp)


def test_q4k_linear_in_d_dmin(oracle, rng):
    b = synth.q4k_blocks(rng, 1)[0]
    b[2:4] = 0  # dmin = 0 -> linear in d
    b[0:2] = np.array([np.float16(1.0)]).view(np.uint8)
    one = oracle.dequant(12, b, 1, 256)[0]
    b[0:2] = np.array([np.float16(0.5)]).view(np.uint8)
    half = oracle.dequant(12, b, 1, 256)[0]
    assert np.array_equal(half * 2, one)


def test_q4k_matches_numpy_restatement(oracle, rng):
    w = synth.weights(rng, 12, 64, 1024)
    a = oracle.dequant(12, w, 64, 1024)
    b = onp.dequant_matrix(w, 12, 64, 1024)
    assert np.array_equal(a.view(np.uint32), b.view(np.uint32))


def test_q4k_ragged_tail(oracle, rng):
    w = synth.weights(rng, 12, 3, 300)  # 2 blocks per row, last one partial
    full = onp.dequant_matrix(w, 12, 3, 512)
    got = oracle.dequant(12, w, 3, 300)
    assert np.array_equal(got, full[:, :300])


# ------------------------------------------------------------------ F4: Q6_K


def _q6k_block_all(qval: int, d=1.0, scales=None):
    """Every value = qval (0..63) through the layout text: lo4 in ql, hi2 in qh."""
    b = np.zeros(210, np.uint8)
    lo, hi = qval & 15, qval >> 4
    b[0:128] = lo | (lo << 4)
    b[128:192] = hi | (hi << 2) | (hi << 4) | (hi << 6)
    b[192:208] = (np.ones(16, np.int8) if scales is None else np.asarray(scales, np.int8)).view(np.uint8)
    b[208:210] = np.array([np.float16(d)]).view(np.uint8)
    return b


def test_q6k_one_hot_layout(oracle):
    """Value v: h=v//128, u=v%128, grp=u//32, l=u%32; lo4 in ql[64h+32(grp&1)+l] (high nibble
    iff grp>=2), hi2 in qh[32h+l] at bit 2*grp (validate_dequant.py:253-319 text)."""
    for v in range(256):
        b = _q6k_block_all(32)  # q-32 == 0 everywhere
        h, u = divmod(v, 128)
        grp, l = divmod(u, 32)
        byte = 64 * h + 32 * (grp & 1) + l
        b[byte] |= (1 << 4) if grp >= 2 else 1  # q = 33 -> value 1
        out = oracle.dequant(14, b, 1, 256)[0]
        expect = np.zeros(256, np.float32)
        expect[v] = 1.0
        assert np.array_equal(out, expect), v


def test_q6k_qh_and_scale_index(oracle, rng):
    sc = rng.integers(-128, 128, 16).astype(np.int8)
    b = _q6k_block_all(63, scales=sc)
    assert np.array_equal(oracle.dequant(14, b, 1, 256)[0], (31.0 * sc[np.arange(256) // 16]).astype(np.float32))
    b = _q6k_block_all(0, d=0.5, scales=sc)
    assert np.array_equal(oracle.dequant(14, b, 1, 256)[0], (-16.0 * sc[np.arange(256) // 16]).astype(np.float32))


def test_q6k_matches_numpy_restatement(oracle, rng):
    w = synth.weights(rng, 14, 64, 1536)
    a = oracle.dequant(14, w, 64, 1536)
    b = onp.dequant_matrix(w, 14, 64, 1536)
    assert np.array_equal(a.view(np.uint32), b.view(np.uint32))


# ------------------------------------------------------------------ G1-G7 / R1: GEMVs


@pytest.mark.parametrize("type_id,rows,cols", [(12, 96, 1024), (14, 80, 1536), (12, 5, 300)])
def test_gemv_vs_numpy_fp64(oracle, rng, type_id, rows, cols):
    w = synth.weights(rng, type_id, rows, cols)
    x = rng.standard_normal(cols).astype(np.float32)
    y = oracle.gemv(type_id, w, x, rows, cols)
    ref = onp.dequant_matrix(w, type_id, rows, cols).astype(np.float64) @ x.astype(np.float64)
    assert rel_l2(y, ref) < 1e-12


def test_gemv_f32acc_baseline_close(oracle, rng):
    w = synth.weights(rng, 12, 64, 4096)
    x = rng.standard_normal(4096).astype(np.float32)
    y = oracle.gemv_f32acc(12, w, x, 64, 4096, 2)
    assert rel_l2(y, oracle.gemv(12, w, x, 64, 4096)) < 1e-5


@pytest.mark.parametrize("type_id", [12, 14])
def test_vectorised_cpu_baseline_close(oracle, rng, type_id):
    """bench.py's CPU baseline (cpu_baseline.c: vectorised, FMA-contracted) computes the same
    product as the checker within fp32 rounding."""
    import oracle as O

    w = synth.weights(rng, type_id, 96, 4096)
    x = rng.standard_normal(4096).astype(np.float32)
    ref = oracle.gemv(type_id, w, x, 96, 4096)
    b = O.load_baseline()
    for nthreads in (1, 4):
        assert rel_l2(b.gemv(type_id, w, x, 96, 4096, nthreads), ref) < 1e-5


def test_matvec_f32(oracle, rng):
    w = rng.standard_normal((128, 512)).astype(np.float32)
    x = rng.standard_normal(512).astype(np.float32)
    assert rel_l2(oracle.matvec_f32(w, x, 128, 512), w.astype(np.float64) @ x) < 1e-12


# ------------------------------------------------------------------ R2: top-k softmax


def test_topk_softmax(oracle, rng):
    for trial in range(50):
        s = rng.standard_normal(128).astype(np.float32)
        if trial % 5 == 0:
            s[rng.integers(0, 128, 10)] = s[3]  # ties
        idx, w = oracle.topk_softmax(s, 8)
        ridx, rw = onp.topk_softmax(s, 8)
        assert np.array_equal(idx, ridx)
        assert np.allclose(w, rw, rtol=1e-6, atol=1e-7)
        assert abs(float(w.sum()) - 1.0) < 1e-6


def test_topk_edge_cases(oracle):
    idx, w = oracle.topk_softmax(np.array([1.0, -2.0, 0.5], np.float32), 5)  # k > n
    assert list(idx) == [0, 2, 1, -1, -1] and w[3] == 0 and w[4] == 0
    idx, w = oracle.topk_softmax(np.full(16, 2.0, np.float32), 4)  # all tied: lowest indices
    assert list(idx) == [0, 1, 2, 3] and np.allclose(w, 0.25)


# ------------------------------------------------------------------ Q1: Q8_1 quantizer


def test_q8_1_matches_numpy_restatement(oracle, rng):
    x = rng.standard_normal((7, 512)).astype(np.float32)
    x[2, :32] = 0.0  # all-zero sub-block
    a = oracle.quantize_q8_1(x)
    b = onp.quantize_q8_1_mmq(x)
    assert np.array_equal(a, b)


def test_q8_1_closed_forms(oracle):
    x = np.zeros((1, 128), np.float32)
    x[0, :32] = np.linspace(-127, 127, 32).astype(np.float32)  # amax = 127 -> d = 1, id = 1
    x[0, 0:4] = [2.5, 3.5, -2.5, 127.0]  # half-even ties
    x[0, 64:96] = 0.0
    x[0, 96] = -7.0  # amax 7, value maps to -127
    blk = oracle.quantize_q8_1(x)[0, 0]
    q = blk[16:].view(np.int8)
    assert list(q[0:4]) == [2, 4, -2, 127]
    assert np.all(q[64:96] == 0) and q[96] == -127
    ds = blk[:16].view(np.float16).astype(np.float32)
    assert ds[0] == 1.0 and ds[4] == 0.0 and ds[5] == 0.0
    assert ds[6] == np.float32(np.float16(7.0 / 127.0))


def test_q8_1_dequant_error_bound(oracle, rng):
    x = rng.standard_normal((4, 1024)).astype(np.float32)
    xd = oracle.dequant_q8_1(oracle.quantize_q8_1(x), 1024, 4)
    amax = np.abs(x.reshape(4, 32, 32)).max(axis=2, keepdims=True)
    err = np.abs((xd - x).reshape(4, 32, 32))
    # rounding to the grid (d/2) plus the f16 rounding of d carried by |q| <= 127
    assert np.all(err <= amax / 127 * (0.5 + 127 * 2.0**-11) * 1.001 + 1e-7)


# ------------------------------------------------------------------ G9/G10: GEMM


@pytest.mark.parametrize("type_id", [12, 14])
def test_gemm_vs_numpy(oracle, rng, type_id):
    M, K, N = 24, 512, 6
    w = synth.weights(rng, type_id, M, K)
    act = oracle.quantize_q8_1(rng.standard_normal((N, K)).astype(np.float32))
    out = oracle.gemm(type_id, w, act, M, K, N)
    assert rel_l2(out, onp.gemm_q8_1(type_id, w, act, M, K, N)) < 1e-12
    full = onp.dequant_q8_1_mmq(act, K).astype(np.float64) @ onp.dequant_matrix(w, type_id, M, K).T.astype(np.float64)
    if type_id == 14:  # no min term: the product of the dequantised operands
        assert rel_l2(out, full) < 1e-12
        return
    # Q4_K: the reference takes the min term from the block's ds field (gemm_q4k.cu:166), so
    # out - (full dequantised product) = sum_s dmin*m_s * (d8 * sum_k q8_k - ds), computed
    # here from the raw bytes alone
    b = w.reshape(M, K // 256, 144)
    dmin = b[..., 2:4].copy().view(np.float16)[..., 0].astype(np.float64)
    _, m = onp.scale_min_k4_all(b[..., 4:16].reshape(-1, 12))
    mins = (dmin[..., None] * m.reshape(M, -1, 8)).reshape(M, K // 32)
    ab = act.reshape(N, K // 128, 144)
    d8 = ab[..., :16].copy().view(np.float16)[..., 0::2].astype(np.float64).reshape(N, K // 32)
    ds = ab[..., :16].copy().view(np.float16)[..., 1::2].astype(np.float64).reshape(N, K // 32)
    qsum = ab[..., 16:].view(np.int8).reshape(N, K // 32, 32).sum(axis=2).astype(np.float64)
    diff = (d8 * qsum - ds) @ mins.T
    # (full holds the fp32-rounded dequantised weights: |error| <= 2^-24 sum_k |w_k a_k|)
    bound = 2.0**-23 * (np.abs(onp.dequant_q8_1_mmq(act, K)).astype(np.float64)
                        @ np.abs(onp.dequant_matrix(w, 12, M, K)).T.astype(np.float64))
    assert np.all(np.abs(out - full - diff) <= bound + 1e-12)
    # min term alone: d = 0 leaves -sum_s dmin * m_s * ds
    w2 = w.reshape(-1, 144).copy()
    w2[:, 0:2] = 0
    out2 = oracle.gemm(12, w2.reshape(-1), act, M, K, N)
    assert rel_l2(out2, -(ds @ mins.T)) < 1e-12


# ------------------------------------------------------------------ next-token selection
def test_xoroshiro_matches_independent_restatement(oracle):
    rng = np.random.default_rng(0)
    for seed in [0, 1, 0xDEADBEEF, 2**63 + 12345] + rng.integers(0, 2**63, 20).tolist():
        a, b = int(seed), int(seed) ^ 0xDEADBEEFCAFEBABE
        x, y = a, b
        for _ in range(6):
            v1, a, b = oracle.xoroshiro_next(a, b)
            v2, x, y = onp.xoroshiro_next(x, y)
            assert (v1, a, b) == (v2, x, y)


def test_sample_greedy_is_first_argmax(oracle):
    rng = np.random.default_rng(1)
    z = rng.standard_normal(5000).astype(np.float32)
    z[[17, 4000]] = z.max() + 1.0  # an exact tie: the lower index wins
    assert oracle.sample_token(z, 0.0, 0.9, 7)[0] == 17
    assert oracle.sample_token(z, -1.0, 0.9, 7)[0] == 17


def test_sample_tiny_top_p_is_argmax(oracle):
    rng = np.random.default_rng(2)
    z = rng.standard_normal(151936).astype(np.float32)
    for seed in range(20):
        assert oracle.sample_token(z, 0.8, 1e-9, seed)[0] == int(np.argmax(z))


@pytest.mark.parametrize("top_p", [1.0, 0.6])
def test_sample_frequencies_follow_nucleus(oracle, top_p):
    """Draw frequencies over many seeds against the renormalised nucleus distribution
    (V < 2048, so every token is a candidate): chi-square well inside its bound."""
    rng = np.random.default_rng(3)
    V, T, n = 40, 0.9, 6000
    z = rng.standard_normal(V).astype(np.float32)
    p = np.exp((z.astype(np.float64) - z.max()) / T)
    o = np.argsort(-p)
    c = np.cumsum(p[o])
    keep = o[: int(np.searchsorted(c, top_p * p.sum()) + 1)]
    q = np.zeros(V)
    q[keep] = p[keep] / p[keep].sum()
    # random 64-bit seeds (four xoroshiro steps from seed, seed ^ const do not decorrelate
    # consecutive small seeds; the draw quality itself is the reference's)
    seeds = rng.integers(0, 2**63, n).tolist()
    counts = np.bincount([oracle.sample_token(z, T, top_p, s)[0] for s in seeds], minlength=V)
    assert counts[q == 0].sum() == 0
    exp = q[q > 0] * n
    chi2 = ((counts[q > 0] - exp) ** 2 / exp).sum()
    dof = (q > 0).sum() - 1
    assert chi2 < dof + 6 * np.sqrt(2 * dof)


def test_sample_matches_numpy_restatement(oracle):
    rng = np.random.default_rng(4)
    z = (rng.standard_normal(151936) * 3).astype(np.float32)
    checked = 0
    for seed in range(40):
        tok, margin = onp.sample_token(z, 0.7, 0.9, seed)
        if margin < 1e-5:
            continue
        assert oracle.sample_token(z, 0.7, 0.9, seed)[0] == tok
        checked += 1
    assert checked >= 30
