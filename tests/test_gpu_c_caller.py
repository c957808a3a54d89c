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
    R, RK, C, E, K = np.frombuffer(buf[:20], np.int32)
    off = 20

    def take(n, dtype):
        nonlocal off
        a = np.frombuffer(buf[off: off + n * np.dtype(dtype).itemsize], dtype)
        off += n * np.dtype(dtype).itemsize
        return a

    q4b, q6b = C // 256 * 144, C // 256 * 210
    wq4, wq6 = take(R * q4b, np.uint8), take(R * q6b, np.uint8)
    wk, wv = take(RK * q4b, np.uint8), take(RK * q6b, np.uint8)
    x, res, router = take(C, np.float32), take(R, np.float32), take(E * C, np.float32)
    y4, y6, yadd, ya, yb, q = (take(R, np.float32) for _ in range(6))
    k, v, logits = take(RK, np.float32), take(RK, np.float32), take(E, np.float32)
    idx, w = take(K, np.int32), take(K, np.float32)
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
