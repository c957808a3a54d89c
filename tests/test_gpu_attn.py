"""GPU parity of the attention chain (MnemoCUDA kernels.cu:692-852, 1196-1244, 1309-1673)
against the C oracle (oracle/mnemo_oracle_attn.c).

Bars: RMS norms and residual add within fp32 rounding (rtol 2e-6 / exact); RoPE within
1e-5 of max|x| (same fp32 frequencies and angles, accurate sin/cos on both sides); f16
stores bit-exact; int8 KV bytes and scales bit-exact on the entry points (same fp32
arithmetic); attention rel-L2 <= 1e-5 against the fp64 softmax (the cache values are the
same f16 / int8 numbers on both sides).  Shapes: Qwen3-235B attention (64 query heads,
4 KV heads, head_dim 128), plus head_dim 64 and 256, one position, positions across the
1024-position tile boundary, and pos up to 40959."""
import numpy as np
import pytest
import torch

from oracle import oracle_np as onp
from tests.conftest import rel_l2
from tests.gpu_util import case, dev, host

pytestmark = pytest.mark.gpu

NH, NKV, HD = 64, 4, 128


def test_rms_norm_variants(gpu, oracle, rng):
    x = rng.standard_normal(4096).astype(np.float32)
    w = rng.standard_normal(4096).astype(np.float32)
    case("rms_norm 4096")
    out = torch.empty(4096, device="cuda")
    gpu.ops.rms_norm(dev(x), dev(w), out, 1e-6)
    np.testing.assert_allclose(host(out), oracle.rms_norm(x, w, 1e-6), rtol=2e-6, atol=1e-7)
    res = torch.zeros(4096, device="cuda")
    out2 = torch.empty(4096, device="cuda")
    gpu.ops.rms_norm(dev(x), dev(w), out2, 1e-6, residual=res)
    assert np.array_equal(host(res), x)
    assert np.array_equal(host(out2), host(out))
    # in place, n not a multiple of the block
    y = rng.standard_normal(5000).astype(np.float32)
    wy = rng.standard_normal(5000).astype(np.float32)
    t = dev(y)
    gpu.ops.rms_norm(t, dev(wy), t, 1e-5)
    np.testing.assert_allclose(host(t), oracle.rms_norm(y, wy, 1e-5), rtol=2e-6, atol=1e-7)
    a, b = dev(x), dev(w)
    s = torch.empty(4096, device="cuda")
    gpu.ops.residual_add(a, b, s)
    assert np.array_equal(host(s), x + w)


@pytest.mark.parametrize("hd", [64, 128, 256])
def test_rms_norm_heads(gpu, oracle, rng, hd):
    q = rng.standard_normal(NH * hd).astype(np.float32)
    k = rng.standard_normal(NKV * hd).astype(np.float32)
    qw = rng.standard_normal(hd).astype(np.float32)
    kw = rng.standard_normal(hd).astype(np.float32)
    case(f"rms_norm heads hd={hd}")
    out = torch.empty(NH * hd, device="cuda")
    gpu.ops.rms_norm_batched(dev(q), dev(qw), out, hd, 1e-6)
    np.testing.assert_allclose(host(out), oracle.rms_norm_heads(q, qw, hd, 1e-6), rtol=2e-6, atol=1e-7)
    tq, tk = dev(q), dev(k)
    gpu.ops.rms_norm_qk(tq, tk, dev(qw), dev(kw), hd, 1e-6)
    np.testing.assert_allclose(host(tq), oracle.rms_norm_heads(q, qw, hd, 1e-6), rtol=2e-6, atol=1e-7)
    np.testing.assert_allclose(host(tk), oracle.rms_norm_heads(k, kw, hd, 1e-6), rtol=2e-6, atol=1e-7)


@pytest.mark.parametrize("pos,theta,hd", [(0, 1e6, 128), (1, 1e6, 128), (1000, 1e6, 128), (40959, 1e6, 128),
                                          (777, 1e4, 64), (12345, 5e5, 256)])
def test_rope(gpu, oracle, rng, pos, theta, hd):
    q = rng.standard_normal(NH * hd).astype(np.float32)
    k = rng.standard_normal(NKV * hd).astype(np.float32)
    case(f"rope pos={pos} theta={theta} hd={hd}")
    tq, tk = dev(q), dev(k)
    gpu.ops.rope(tq, tk, hd, pos, theta)
    wq, wk = oracle.rope(q, k, hd, pos, theta)
    if pos == 0:
        assert np.array_equal(host(tq), q) and np.array_equal(host(tk), k)
    tol = 1e-5 * max(np.abs(q).max(), np.abs(k).max())
    np.testing.assert_allclose(host(tq), wq, rtol=0, atol=tol)
    np.testing.assert_allclose(host(tk), wk, rtol=0, atol=tol)


def test_kv_stores(gpu, oracle, rng):
    k = (rng.standard_normal(NKV * HD) * 3).astype(np.float32)
    v = (rng.standard_normal(NKV * HD) * 3).astype(np.float32)
    k[HD:2 * HD] = 0.0  # a zero head: scale 0, all-zero bytes
    case("f32_to_f16_dual / f32_to_int8_kv_dual")
    ok = torch.empty(NKV * HD, dtype=torch.float16, device="cuda")
    ov = torch.empty_like(ok)
    gpu.ops.f32_to_f16_dual(dev(k), dev(v), ok, ov)
    assert np.array_equal(host(ok).view(np.uint16), k.astype(np.float16).view(np.uint16))
    assert np.array_equal(host(ov).view(np.uint16), v.astype(np.float16).view(np.uint16))
    qk = torch.empty(NKV * HD, dtype=torch.int8, device="cuda")
    qv = torch.empty_like(qk)
    ks = torch.full((NKV,), -1.0, device="cuda")
    vs = torch.full((NKV,), -1.0, device="cuda")
    tk = dev(k)
    gpu.ops.f32_to_int8_kv_dual(tk, dev(v), qk, qv, ks, vs, HD)
    wk, wks = oracle.kv_quant_int8(k, HD)
    wv, wvs = oracle.kv_quant_int8(v, HD)
    assert np.array_equal(host(qk), wk) and np.array_equal(host(ks), wks)
    assert np.array_equal(host(qv), wv) and np.array_equal(host(vs), wvs)
    assert np.array_equal(host(tk), k)  # the input is not written


def _caches(rng, seq, nkv, hd, kind):
    k = rng.standard_normal((seq, nkv, hd)).astype(np.float32)
    v = rng.standard_normal((seq, nkv, hd)).astype(np.float32)
    if kind == "f16":
        return k.astype(np.float16).view(np.uint16), v.astype(np.float16).view(np.uint16), None, None
    kq, ks = onp.kv_quant_int8(k.reshape(-1), hd)
    vq, vs = onp.kv_quant_int8(v.reshape(-1), hd)
    return kq, vq, ks, vs


def _to_dev(a):
    if a is None:
        return None
    if a.dtype == np.uint16:
        return dev(a.view(np.float16))
    return dev(a)


@pytest.mark.parametrize("kind", ["f16", "int8"])
@pytest.mark.parametrize("seq,hd,nh,nkv", [(1, 128, NH, NKV), (5, 128, NH, NKV), (1000, 128, NH, NKV),
                                           (2500, 128, NH, NKV), (300, 64, 16, 2), (700, 256, 8, 8)])
def test_attention(gpu, oracle, rng, kind, seq, hd, nh, nkv):
    q = rng.standard_normal(nh * hd).astype(np.float32)
    kc, vc, ks, vs = _caches(rng, seq, nkv, hd, kind)
    scale = 1.0 / np.sqrt(hd)
    case(f"attention {kind} seq={seq} hd={hd} nh={nh} nkv={nkv}")
    out = torch.full((nh * hd,), np.nan, device="cuda")
    gpu.ops.attention(dev(q), _to_dev(kc), _to_dev(vc), out, nh, hd, nkv, seq, scale, _to_dev(ks), _to_dev(vs))
    want = oracle.attention(q, kc, vc, nh, hd, nkv, seq, scale, ks, vs)
    got = host(out)
    assert rel_l2(got, want) < 1e-5
    if seq == 1:
        np.testing.assert_allclose(got, want, rtol=1e-6, atol=1e-6)


@pytest.mark.parametrize("kind", ["f16", "int8"])
def test_attn_prep_and_dev_attention(gpu, oracle, rng, kind):
    """mnemo_attn_prep (QK norm + RoPE + store at *pos) then mnemo_attention over 0..*pos,
    against the oracle chain; the cache rows below pos hold earlier tokens."""
    ctx, pos, theta, eps = 64, 37, 1e6, 1e-6
    q = rng.standard_normal(NH * HD).astype(np.float32)
    k = rng.standard_normal(NKV * HD).astype(np.float32)
    v = rng.standard_normal(NKV * HD).astype(np.float32)
    qw = (1 + 0.1 * rng.standard_normal(HD)).astype(np.float32)
    kw = (1 + 0.1 * rng.standard_normal(HD)).astype(np.float32)
    kc, vc, ks, vs = _caches(rng, ctx, NKV, HD, kind)
    tkc, tvc, tks, tvs = _to_dev(kc), _to_dev(vc), _to_dev(ks), _to_dev(vs)
    tq, tk, tv = dev(q), dev(k), dev(v)
    pos_dev = torch.tensor([pos], dtype=torch.int32, device="cuda")
    case(f"attn_prep {kind} pos={pos}")
    gpu.ops.attn_prep(tq, tk, tv, dev(qw), dev(kw), HD, eps, theta, pos_dev, tkc, tvc, tks, tvs)
    wq, wk = oracle.rope(oracle.rms_norm_heads(q, qw, HD, eps), oracle.rms_norm_heads(k, kw, HD, eps), HD, pos,
                         theta)
    tol = 1e-5 * max(np.abs(wq).max(), np.abs(wk).max())
    gq, gk = host(tq), host(tk)
    np.testing.assert_allclose(gq, wq, rtol=0, atol=tol)
    np.testing.assert_allclose(gk, wk, rtol=0, atol=tol)
    # cache rows: pos holds the stored k / v; other rows untouched
    if kind == "f16":
        ck, cv = host(tkc).view(np.uint16).reshape(ctx, -1), host(tvc).view(np.uint16).reshape(ctx, -1)
        assert np.array_equal(ck[pos], gk.astype(np.float16).view(np.uint16))
        assert np.array_equal(cv[pos], v.astype(np.float16).view(np.uint16))
        rows = np.arange(ctx) != pos
        assert np.array_equal(ck[rows], kc.reshape(ctx, -1)[rows]) and np.array_equal(cv[rows], vc.reshape(ctx, -1)[rows])
    else:
        ck, cv = host(tkc).reshape(ctx, -1), host(tvc).reshape(ctx, -1)
        wkq, wks = oracle.kv_quant_int8(gk, HD)
        wvq, wvs = oracle.kv_quant_int8(v, HD)
        assert np.array_equal(ck[pos], wkq) and np.array_equal(host(tks).reshape(ctx, -1)[pos], wks)
        assert np.array_equal(cv[pos], wvq) and np.array_equal(host(tvs).reshape(ctx, -1)[pos], wvs)
    # attention over 0..pos with the length read on the device (the per-head kernel) against the
    # entry point with seq = pos + 1 (the split-chunk kernels at head_dim 128): both ~fp32
    out = torch.empty(NH * HD, device="cuda")
    out2 = torch.empty(NH * HD, device="cuda")
    gpu.ops.attention_dev(tq, tkc, tvc, out, NH, HD, NKV, pos_dev, 1 / np.sqrt(HD), tks, tvs)
    gpu.ops.attention(tq, tkc, tvc, out2, NH, HD, NKV, pos + 1, 1 / np.sqrt(HD), tks, tvs)
    assert rel_l2(host(out2), host(out)) < 1e-5
    if kind == "f16":
        kk, vv = host(tkc).view(np.uint16), host(tvc).view(np.uint16)
        want = oracle.attention(gq, kk, vv, NH, HD, NKV, pos + 1, 1 / np.sqrt(HD))
    else:
        want = oracle.attention(gq, host(tkc), host(tvc), NH, HD, NKV, pos + 1, 1 / np.sqrt(HD), host(tks),
                                host(tvs))
    assert rel_l2(host(out), want) < 1e-5


def test_attn_chain_graph_replay(gpu, rng):
    """prep + attention captured once, replayed for consecutive positions (pos in device
    memory); every replay equals the eager chain at that position."""
    ctx, theta, eps = 32, 1e6, 1e-6
    qs = rng.standard_normal((4, NH * HD)).astype(np.float32)
    ks_ = rng.standard_normal((4, NKV * HD)).astype(np.float32)
    vs_ = rng.standard_normal((4, NKV * HD)).astype(np.float32)
    qw = np.ones(HD, np.float32)
    kw = np.ones(HD, np.float32)

    def run(graph: bool):
        kc = torch.zeros(ctx * NKV * HD, dtype=torch.float16, device="cuda")
        vc = torch.zeros_like(kc)
        q = torch.empty(NH * HD, device="cuda")
        k = torch.empty(NKV * HD, device="cuda")
        v = torch.empty(NKV * HD, device="cuda")
        out = torch.empty(NH * HD, device="cuda")
        pos_dev = torch.zeros(1, dtype=torch.int32, device="cuda")
        tqw, tkw = dev(qw), dev(kw)
        s = torch.cuda.Stream()
        outs = []

        def step():
            gpu.ops.attn_prep(q, k, v, tqw, tkw, HD, eps, theta, pos_dev, kc, vc)
            gpu.ops.attention_dev(q, kc, vc, out, NH, HD, NKV, pos_dev, 1 / np.sqrt(HD))

        with torch.cuda.stream(s):
            g = None
            if graph:
                q.copy_(dev(qs[0])); k.copy_(dev(ks_[0])); v.copy_(dev(vs_[0]))
                step()  # eager once
                torch.cuda.synchronize()
                kc.zero_(); vc.zero_()
                g = torch.cuda.CUDAGraph()
                with torch.cuda.graph(g, stream=s):
                    step()
            for t in range(4):
                pos_dev.fill_(t)
                q.copy_(dev(qs[t])); k.copy_(dev(ks_[t])); v.copy_(dev(vs_[t]))
                if graph:
                    g.replay()
                else:
                    step()
                torch.cuda.synchronize()
                outs.append(out.clone())
        return outs

    case("attention chain graph replay")
    eager, replay = run(False), run(True)
    for a, b in zip(eager, replay):
        assert torch.equal(a, b)


def test_bad_args(gpu):
    case("attention bad args")
    q = torch.zeros(NH * HD, device="cuda")
    kc = torch.zeros(4 * NKV * HD, dtype=torch.float16, device="cuda")
    pos = torch.zeros(1, dtype=torch.int32, device="cuda")
    out = torch.empty_like(q)
    with pytest.raises(gpu.MnemoError):
        gpu.ops.attention_dev(q, kc, kc, out, NH, 96, NKV, pos, 0.1)  # head_dim 96 unsupported
    with pytest.raises(gpu.MnemoError):
        gpu.ops.attention_dev(q, kc, kc, out, 63, HD, NKV, pos, 0.1)  # 63 % 4
    with pytest.raises(gpu.MnemoError):
        gpu.ops.attn_prep(q, q, q, q[:HD], None, HD, 1e-6, 1e6, pos, kc, kc)  # one norm weight


# ------------------------------------------------------------------ GQA-batched decode attention
def _blocked(v, max_ctx, nkv, hd):
    """[pos][nkv][hd] -> the blocked V layout [pos/64][nkv][hd][pos%64], zero-padded."""
    nb = (max_ctx + 63) // 64
    x = np.zeros((nb * 64, nkv, hd), v.dtype)
    x[:max_ctx] = v.reshape(max_ctx, nkv, hd)
    return np.ascontiguousarray(x.reshape(nb, 64, nkv, hd).transpose(0, 2, 3, 1)).reshape(-1)


@pytest.mark.parametrize("v_layout", [0, 1])
@pytest.mark.parametrize("kind", ["f16", "int8"])
@pytest.mark.parametrize("seq,nh,nkv,max_ctx", [(1, NH, NKV, 8192), (63, NH, NKV, 8192), (64, NH, NKV, 8192),
                                                (65, NH, NKV, 8192), (1000, NH, NKV, 8192), (4097, NH, NKV, 8192),
                                                (300, 32, 4, 8192), (200, 8, 8, 8192), (1000, NH, NKV, 1000),
                                                # past 128 chunks each workgroup walks several (merged as it goes)
                                                (8193, NH, NKV, 16384), (10000, NH, NKV, 16384),
                                                (33000, NH, NKV, 40960), (20000, 8, 8, 20000)])
def test_attention_decode(gpu, oracle, rng, kind, seq, nh, nkv, max_ctx, v_layout):
    q = rng.standard_normal(nh * HD).astype(np.float32)
    kc, vc, ks, vs = _caches(rng, max_ctx, nkv, HD, kind)
    pos_dev = torch.tensor([seq - 1], dtype=torch.int32, device="cuda")
    ws = torch.empty(gpu.ops.attention_decode_workspace_bytes(nkv, max_ctx), dtype=torch.uint8, device="cuda")
    out = torch.full((nh * HD,), np.nan, device="cuda")
    scale = 1.0 / np.sqrt(HD)
    case(f"attention_decode {kind} v_layout={v_layout} seq={seq} nh={nh} nkv={nkv} max_ctx={max_ctx}")
    vdev = _to_dev(vc if v_layout == 0 else _blocked(vc, max_ctx, nkv, HD))
    if v_layout == 1:
        assert vdev.numel() * vdev.element_size() == gpu.ops.v_cache_bytes(nkv, HD, max_ctx, 0 if kind == "f16" else 1, 1)
    gpu.ops.attention_decode(dev(q), _to_dev(kc), vdev, out, nh, HD, nkv, max_ctx, pos_dev, scale, ws,
                             _to_dev(ks), _to_dev(vs), v_layout=v_layout)
    if kind == "f16":
        want = oracle.attention(q, kc[:seq], vc[:seq], nh, HD, nkv, seq, scale)
    else:
        want = oracle.attention(q, kc[:seq * nkv * HD], vc[:seq * nkv * HD], nh, HD, nkv, seq, scale,
                                ks[:seq * nkv], vs[:seq * nkv])
    assert rel_l2(host(out), want) < 1e-5


def test_attn_prep_blocked_v(gpu, rng):
    """mnemo_attn_prep with v_layout 1 stores V at its blocked position; the K rows and
    everything else in the caches are untouched."""
    ctx, pos = 200, 131
    q = dev(rng.standard_normal(NH * HD).astype(np.float32))
    k = dev(rng.standard_normal(NKV * HD).astype(np.float32))
    v = rng.standard_normal(NKV * HD).astype(np.float32)
    for kind in ("f16", "int8"):
        case(f"attn_prep blocked V {kind}")
        dt = torch.float16 if kind == "f16" else torch.int8
        kc = torch.zeros(ctx * NKV * HD, dtype=dt, device="cuda")
        nb = gpu.ops.v_cache_bytes(NKV, HD, ctx, 0 if kind == "f16" else 1, 1) // kc.element_size()
        vc = torch.zeros(nb, dtype=dt, device="cuda")
        ks = torch.zeros(ctx * NKV, device="cuda")
        vs = torch.zeros(ctx * NKV, device="cuda")
        pos_dev = torch.tensor([pos], dtype=torch.int32, device="cuda")
        gpu.ops.attn_prep(q.clone(), k.clone(), dev(v), None, None, HD, 1e-6, 1e6, pos_dev, kc, vc,
                          ks if kind == "int8" else None, vs if kind == "int8" else None, v_layout=1)
        got = host(vc)
        if kind == "f16":
            want_row = v.astype(np.float16)
            got_rows = got.reshape(-1, NKV, HD, 64)[pos // 64, :, :, pos % 64].reshape(-1)
            assert np.array_equal(got_rows.view(np.uint16), want_row.view(np.uint16))
        else:
            want_row, _ = onp.kv_quant_int8(v, HD)
            got_rows = got.reshape(-1, NKV, HD, 64)[pos // 64, :, :, pos % 64].reshape(-1)
            assert np.array_equal(got_rows, want_row)
        assert np.count_nonzero(got) == np.count_nonzero(got_rows)


def test_attention_decode_graph_replay(gpu, rng):
    """captured once; replays at growing positions equal the eager calls."""
    max_ctx = 1024
    q = dev(rng.standard_normal(NH * HD).astype(np.float32))
    kc, vc, _, _ = _caches(rng, max_ctx, NKV, HD, "f16")
    tkc, tvc = _to_dev(kc), _to_dev(vc)
    pos_dev = torch.zeros(1, dtype=torch.int32, device="cuda")
    ws = torch.empty(gpu.ops.attention_decode_workspace_bytes(NKV, max_ctx), dtype=torch.uint8, device="cuda")
    out = torch.empty(NH * HD, device="cuda")
    s = torch.cuda.Stream()
    case("attention_decode graph replay")
    positions = [0, 5, 63, 64, 500, 1023]
    eager = []
    with torch.cuda.stream(s):
        for p in positions:
            pos_dev.fill_(p)
            gpu.ops.attention_decode(q, tkc, tvc, out, NH, HD, NKV, max_ctx, pos_dev, 0.088, ws)
            torch.cuda.synchronize()
            eager.append(out.clone())
        g = torch.cuda.CUDAGraph()
        with torch.cuda.graph(g, stream=s):
            gpu.ops.attention_decode(q, tkc, tvc, out, NH, HD, NKV, max_ctx, pos_dev, 0.088, ws)
        for p, e in zip(positions, eager):
            pos_dev.fill_(p)
            g.replay()
            torch.cuda.synchronize()
            assert torch.equal(out, e), p


def test_attention_decode_bad_args(gpu):
    case("attention_decode bad args")
    q = torch.zeros(NH * HD, device="cuda")
    kc = torch.zeros(64 * NKV * HD, dtype=torch.float16, device="cuda")
    pos = torch.zeros(1, dtype=torch.int32, device="cuda")
    out = torch.empty_like(q)
    ws = torch.empty(gpu.ops.attention_decode_workspace_bytes(NKV, 64), dtype=torch.uint8, device="cuda")
    with pytest.raises(gpu.MnemoError):  # workspace too small for max_ctx
        gpu.ops.attention_decode(q, kc, kc, out, NH, HD, NKV, 4096, pos, 0.1, ws)
    with pytest.raises(gpu.MnemoError):  # gqa 32 > 16
        gpu.ops.attention_decode(q, kc, kc, out, NH, HD, 2, 64, pos, 0.1, ws)
    with pytest.raises(gpu.MnemoError):  # head_dim 64 not on this path
        gpu.ops.attention_decode(q, kc, kc, out, NH, 64, NKV, 64, pos, 0.1, ws)


# ------------------------------------------------------------------ decode attention with the prep fused
def _prep_inputs(rng, kind, max_ctx, nh, nkv, v_layout, pos):
    kc, vc, ks, vs = _caches(rng, max_ctx, nkv, HD, kind)
    if v_layout == 1:
        vc = _blocked(vc, max_ctx, nkv, HD)
    t = [_to_dev(a) for a in (kc, vc, ks, vs)]
    # the row at pos holds garbage until this token stores it (the fused path must not read it)
    if kind == "f16":
        t[0].view(-1, nkv, HD)[pos] = float("nan")
        if v_layout == 0:
            t[1].view(-1, nkv, HD)[pos] = float("nan")
        else:
            t[1].view(-1, nkv, HD, 64)[pos // 64, :, :, pos % 64] = float("nan")
    else:
        t[2].view(-1, nkv)[pos] = float("nan")
        t[3].view(-1, nkv)[pos] = float("nan")
    return t


@pytest.mark.parametrize("norm", [True, False])
@pytest.mark.parametrize("v_layout", [0, 1])
@pytest.mark.parametrize("kind", ["f16", "int8"])
@pytest.mark.parametrize("pos,nh,nkv,max_ctx", [(0, NH, NKV, 4096), (63, NH, NKV, 4096), (64, NH, NKV, 4096),
                                                (1000, NH, NKV, 4096), (130, 32, 4, 512), (77, 8, 8, 200),
                                                (199, 8, 8, 200), (9000, NH, NKV, 12000), (8191, NH, NKV, 8192)])
def test_attention_decode_prep_matches_two_step(gpu, rng, kind, v_layout, norm, pos, nh, nkv, max_ctx):
    """mnemo_attention_decode_prep == mnemo_attn_prep then mnemo_attention_decode, bit for bit:
    the output, both caches (and int8 scales); q, k, v are left unchanged."""
    q = dev(rng.standard_normal(nh * HD).astype(np.float32) * 2)
    k = dev(rng.standard_normal(nkv * HD).astype(np.float32) * 2)
    v = dev(rng.standard_normal(nkv * HD).astype(np.float32))
    qw = dev(1 + 0.2 * rng.standard_normal(HD).astype(np.float32)) if norm else None
    kw = dev(1 + 0.2 * rng.standard_normal(HD).astype(np.float32)) if norm else None
    eps, theta, scale = 1e-6, 1e6, 1.0 / np.sqrt(HD)
    st = rng.bit_generator.state
    a = _prep_inputs(rng, kind, max_ctx, nh, nkv, v_layout, pos)
    rng.bit_generator.state = st
    b = _prep_inputs(rng, kind, max_ctx, nh, nkv, v_layout, pos)
    pos_dev = torch.tensor([pos], dtype=torch.int32, device="cuda")
    ws = torch.empty(gpu.ops.attention_decode_workspace_bytes(nkv, max_ctx), dtype=torch.uint8, device="cuda")
    out_a = torch.full((nh * HD,), np.nan, device="cuda")
    out_b = torch.full((nh * HD,), np.nan, device="cuda")
    case(f"attention_decode_prep {kind} v_layout={v_layout} norm={norm} pos={pos} nh={nh} nkv={nkv}")
    qa, ka = q.clone(), k.clone()
    gpu.ops.attn_prep(qa, ka, v, qw, kw, HD, eps, theta, pos_dev, a[0], a[1], a[2], a[3], v_layout=v_layout)
    gpu.ops.attention_decode(qa, a[0], a[1], out_a, nh, HD, nkv, max_ctx, pos_dev, scale, ws, a[2], a[3],
                             v_layout=v_layout)
    q0, k0, v0 = q.clone(), k.clone(), v.clone()
    gpu.ops.attention_decode_prep(q, k, v, qw, kw, eps, theta, b[0], b[1], out_b, nh, HD, nkv, max_ctx, pos_dev,
                                  scale, ws, b[2], b[3], v_layout=v_layout)
    torch.cuda.synchronize()
    assert torch.equal(q, q0) and torch.equal(k, k0) and torch.equal(v, v0)
    assert not torch.isnan(out_b).any()
    assert torch.equal(out_a, out_b)
    for x, y in zip(a, b):
        if x is not None:
            assert torch.equal(x.view(torch.uint8) if x.dtype != torch.float32 else x,
                               y.view(torch.uint8) if y.dtype != torch.float32 else y)


def test_attention_decode_prep_token_sequence_graph(gpu, rng):
    """a captured graph replayed token after token (position in device memory) reads back the
    rows it stored at earlier replays and matches the eager two-step path at every token."""
    max_ctx, nh, nkv = 300, NH, NKV
    qw = dev(1 + 0.2 * rng.standard_normal(HD).astype(np.float32))
    kw = dev(1 + 0.2 * rng.standard_normal(HD).astype(np.float32))
    kc_a = torch.zeros(max_ctx * nkv * HD, dtype=torch.float16, device="cuda")
    vc_a = torch.zeros(gpu.ops.v_cache_bytes(nkv, HD, max_ctx, 0, 1) // 2, dtype=torch.float16, device="cuda")
    kc_b, vc_b = kc_a.clone(), vc_a.clone()
    q, k, v = (torch.empty(n * HD, device="cuda") for n in (nh, nkv, nkv))
    pos_a = torch.zeros(1, dtype=torch.int32, device="cuda")
    pos_b = torch.zeros(1, dtype=torch.int32, device="cuda")
    ws_a = torch.empty(gpu.ops.attention_decode_workspace_bytes(nkv, max_ctx), dtype=torch.uint8, device="cuda")
    ws_b = torch.empty_like(ws_a)
    out_a, out_b = torch.empty(nh * HD, device="cuda"), torch.empty(nh * HD, device="cuda")
    s = torch.cuda.Stream()
    case("attention_decode_prep graph over a token sequence")
    with torch.cuda.stream(s):
        g = torch.cuda.CUDAGraph()
        with torch.cuda.graph(g, stream=s):
            gpu.ops.attention_decode_prep(q, k, v, qw, kw, 1e-6, 1e6, kc_b, vc_b, out_b, nh, HD, nkv, max_ctx,
                                          pos_b, 0.088, ws_b, v_layout=1)
        kc_b.zero_()
        vc_b.zero_()
        for t in range(70):
            q.copy_(torch.randn(nh * HD, device="cuda"))
            k.copy_(torch.randn(nkv * HD, device="cuda"))
            v.copy_(torch.randn(nkv * HD, device="cuda"))
            qa, ka = q.clone(), k.clone()
            pos_a.fill_(t)
            gpu.ops.attn_prep(qa, ka, v, qw, kw, HD, 1e-6, 1e6, pos_a, kc_a, vc_a, v_layout=1)
            gpu.ops.attention_decode(qa, kc_a, vc_a, out_a, nh, HD, nkv, max_ctx, pos_a, 0.088, ws_a, v_layout=1)
            pos_b.fill_(t)
            g.replay()
            torch.cuda.synchronize()
            if not torch.equal(out_a, out_b):
                d = (out_a - out_b).abs()
                bad = torch.nonzero(d).flatten()
                msg = (f"token {t}: {bad.numel()} outputs differ, max {d.max().item():.3e}, first {bad[:8].tolist()}, "
                       f"k rows equal {torch.equal(kc_a, kc_b)}, v equal {torch.equal(vc_a, vc_b)}")
                ka3, kb3 = kc_a.view(max_ctx, nkv, HD).float(), kc_b.view(max_ctx, nkv, HD).float()
                dk = torch.nonzero(ka3 != kb3)
                msg += f"; k diffs (pos, head, dim) {dk[:12].tolist()} n={dk.shape[0]}"
                if dk.shape[0]:
                    p_, h_, d_ = dk[0].tolist()
                    msg += f" a={ka3[p_, h_, d_].item()} b={kb3[p_, h_, d_].item()}"
                raise AssertionError(msg)
    assert torch.equal(kc_a, kc_b) and torch.equal(vc_a, vc_b)


def test_attention_decode_prep_bad_args(gpu):
    case("attention_decode_prep bad args")
    q = torch.zeros(NH * HD, device="cuda")
    k = torch.zeros(NKV * HD, device="cuda")
    kc = torch.zeros(64 * NKV * HD, dtype=torch.float16, device="cuda")
    pos = torch.zeros(1, dtype=torch.int32, device="cuda")
    out = torch.empty_like(q)
    ws = torch.empty(gpu.ops.attention_decode_workspace_bytes(NKV, 64), dtype=torch.uint8, device="cuda")
    with pytest.raises(gpu.MnemoError):  # only one of the QK-norm weights
        gpu.ops.attention_decode_prep(q, k, k, torch.ones(HD, device="cuda"), None, 1e-6, 1e6, kc, kc, out, NH, HD,
                                      NKV, 64, pos, 0.1, ws)
    with pytest.raises(gpu.MnemoError):  # int8 caches without scales
        kc8 = torch.zeros(64 * NKV * HD, dtype=torch.int8, device="cuda")
        gpu.ops.attention_decode_prep(q, k, k, None, None, 1e-6, 1e6, kc8, kc8, out, NH, HD, NKV, 64, pos, 0.1, ws)


@pytest.mark.parametrize("kind", ["f16", "int8"])
def test_attention_entry_point_paths(gpu, oracle, rng, kind):
    """cuda_attention_* runs the split kernel on a workspace slot bound to the calling stream:
    on the current stream, on a second stream, and for a sequence longer than its workgroups
    have chunks (66,000 positions: every workgroup merges several chunks), all match the
    oracle."""
    nh, hd, nkv, scale = NH, 128, NKV, 1.0 / np.sqrt(128)
    for seq, streams in [(3000, ("current", "side")), (66000, ("current",))]:
        q = rng.standard_normal(nh * hd).astype(np.float32)
        kc, vc, ks, vs = _caches(rng, seq, nkv, hd, kind)
        want = oracle.attention(q, kc, vc, nh, hd, nkv, seq, scale, ks, vs)
        tkc, tvc, tks, tvs = _to_dev(kc), _to_dev(vc), _to_dev(ks), _to_dev(vs)
        for which in streams:
            s = torch.cuda.current_stream() if which == "current" else torch.cuda.Stream()
            out = torch.full((nh * hd,), np.nan, device="cuda")
            case(f"attention entry point {kind} seq={seq} stream={which}")
            with torch.cuda.stream(s):
                gpu.ops.attention(dev(q), tkc, tvc, out, nh, hd, nkv, seq, scale, tks, tvs)
            torch.cuda.synchronize()
            assert rel_l2(host(out), want) < 1e-5, (seq, which)


def test_attention_entry_graph_on_other_stream(gpu, rng):
    """cuda_attention_f16kv captured on stream A and replayed on stream B while eager calls
    with other inputs run on A: the captured call holds a workspace slot of its own, so both
    give exactly the serial results."""
    nh, hd, nkv, scale = NH, 128, NKV, 1.0 / np.sqrt(128)
    q1, q2 = (dev(rng.standard_normal(nh * hd).astype(np.float32)) for _ in range(2))
    c1 = [_to_dev(c) for c in _caches(rng, 3000, nkv, hd, "f16")[:2]]
    c2 = [_to_dev(c) for c in _caches(rng, 2000, nkv, hd, "f16")[:2]]
    A, B = torch.cuda.Stream(), torch.cuda.Stream()
    ref1, ref2 = torch.empty(nh * hd, device="cuda"), torch.empty(nh * hd, device="cuda")
    out_g, out_e = torch.empty(nh * hd, device="cuda"), torch.empty(nh * hd, device="cuda")
    case("attention entry point: graph from stream A replayed on B next to eager calls on A")
    with torch.cuda.stream(A):
        gpu.ops.attention(q1, c1[0], c1[1], ref1, nh, hd, nkv, 3000, scale)
        gpu.ops.attention(q2, c2[0], c2[1], ref2, nh, hd, nkv, 2000, scale)
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g, stream=A):
        gpu.ops.attention(q1, c1[0], c1[1], out_g, nh, hd, nkv, 3000, scale)
    torch.cuda.synchronize()
    for _ in range(20):
        out_g.zero_()
        out_e.zero_()
        torch.cuda.synchronize()
        with torch.cuda.stream(B):
            g.replay()
        with torch.cuda.stream(A):
            for _ in range(3):
                gpu.ops.attention(q2, c2[0], c2[1], out_e, nh, hd, nkv, 2000, scale)
        torch.cuda.synchronize()
        assert torch.equal(out_g, ref1) and torch.equal(out_e, ref2)
