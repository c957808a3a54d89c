"""The reference engine's attention-graph path from C (tests/c_caller/attn_graph.c):
build_attention_graphs captures one layer's chain, finds the RoPE, f16 KV-store and
attention nodes through cuda_get_*_kernel_ptr and patches their position, destinations and
sequence length before every replay (MnemoCUDA src/forward.c:1290-1420, 633-668).  24
tokens decoded after a 9,000-position prompt: the patched replays must equal the eager calls
bit for bit, and every step must match the oracle chain."""
import subprocess

import numpy as np
import pytest

from mnemocuda_amd.build import GRAPH_CALLER
from tests.conftest import rel_l2
from tests.gpu_util import case

pytestmark = pytest.mark.gpu
THETA, EPS = 1e6, 1e-6


def test_attention_graph_patching_matches_oracle(gpu, oracle, tmp_path):
    if not GRAPH_CALLER.exists():
        pytest.fail(f"{GRAPH_CALLER} is not built (run __graft_entry__.build())")
    out = tmp_path / "graph.bin"
    case("C attention graph, patched replays")
    r = subprocess.run([str(GRAPH_CALLER), str(out)], capture_output=True, text=True, timeout=120)
    assert r.returncode == 0, r.stdout + r.stderr
    buf = out.read_bytes()
    H, NH, NKV, HD, P0, NTOK, CTX = (int(v) for v in np.frombuffer(buf[:28], np.int32))
    off = 28

    def take(n, dtype):
        nonlocal off
        a = np.frombuffer(buf[off: off + n * np.dtype(dtype).itemsize], dtype)
        off += n * np.dtype(dtype).itemsize
        return a

    q4 = lambda cols: cols // 256 * 144  # noqa: E731
    wq, wk = take(NH * HD * q4(H), np.uint8), take(NKV * HD * q4(H), np.uint8)
    wv, wo = take(NKV * HD * q4(H), np.uint8), take(H * q4(NH * HD), np.uint8)
    anorm, qn, kn = take(H, np.float32), take(HD, np.float32), take(HD, np.float32)
    hin = take(NTOK * H, np.float32).reshape(NTOK, H)
    ncache = CTX * NKV * HD
    kc0, vc0 = take(ncache, np.uint16), take(ncache, np.uint16)
    runs = []
    for _ in range(2):  # graph, eager
        toks = []
        for _ in range(NTOK):
            toks.append(dict(q=take(NH * HD, np.float32), k=take(NKV * HD, np.float32), v=take(NKV * HD, np.float32),
                             att=take(NH * HD, np.float32), hid=take(H, np.float32)))
        runs.append(toks)
    kc, vc = take(ncache, np.uint16), take(ncache, np.uint16)
    assert off == len(buf)

    graph, eager = runs
    for t in range(NTOK):
        for key in graph[t]:
            assert np.array_equal(graph[t][key], eager[t][key]), (t, key)

    row = NKV * HD
    assert np.array_equal(kc[: P0 * row], kc0[: P0 * row]) and np.array_equal(vc[: P0 * row], vc0[: P0 * row])
    scale = float(np.float32(1.0 / np.sqrt(HD)))
    for t in range(NTOK):
        pos, g = P0 + t, graph[t]
        normed, resid = oracle.rms_norm_residual(hin[t], anorm, EPS)
        q = oracle.gemv(12, wq, normed, NH * HD, H)
        k = oracle.gemv(12, wk, normed, NKV * HD, H)
        v = oracle.gemv(12, wv, normed, NKV * HD, H)
        assert rel_l2(g["v"], v) < 1e-3, t
        rq, rk = oracle.rope(oracle.rms_norm_heads(q.astype(np.float32), qn, HD, EPS),
                             oracle.rms_norm_heads(k.astype(np.float32), kn, HD, EPS), HD, pos, THETA)
        assert rel_l2(g["q"], rq) < 1e-3 and rel_l2(g["k"], rk) < 1e-3, t
        # the patched destinations: row pos holds f16 of this token's K and V
        assert np.array_equal(kc[pos * row:(pos + 1) * row], g["k"].astype(np.float16).view(np.uint16)), t
        assert np.array_equal(vc[pos * row:(pos + 1) * row], g["v"].astype(np.float16).view(np.uint16)), t
        # the patched length: positions 0..pos
        want = oracle.attention(g["q"], kc, vc, NH, HD, NKV, pos + 1, scale)
        assert rel_l2(g["att"], want) < 1e-5, t
        assert rel_l2(g["hid"], oracle.gemv(12, wo, g["att"], H, NH * HD) + resid) < 1e-3, t
