"""GPU parity of the decode GEMV family against the CPU oracle (fp64 of fp32-dequantised
weights).  Bar: relative L2 <= 1e-3; the 16-bit x encoding (two
bytes per value) is expected to land near 1e-5, which is also recorded."""
import numpy as np
import pytest
import torch

from mnemocuda_amd import synth
from tests.conftest import rel_l2
from tests.gpu_util import case, dev, host

pytestmark = pytest.mark.gpu
TOL = 1e-3


def _mk(rng, type_id, rows, cols):
    w = synth.weights(rng, type_id, rows, cols)
    return w, dev(w)


SHAPES = [
    (12, 4096, 4096), (12, 8192, 4096), (12, 512, 4096), (12, 1536, 4096), (12, 4096, 1536),
    (12, 4096, 8192), (14, 512, 4096), (14, 4096, 1536), (14, 333, 4096),
    (12, 1, 256), (14, 3, 512), (12, 7, 300), (14, 5, 1000), (12, 2, 16384),
    # launches small enough for the split-columns kernel (1024 columns per wave), with the
    # last wave's columns partly past n: 4000 and 3332 (4 waves), 7424 and 8192 (8 waves)
    (12, 64, 4000), (14, 40, 3332), (12, 24, 7424), (14, 600, 8192), (12, 9, 4096),
    # Q6_K rows of 4096 values over several rounds: the staged kernel (rows % 16 == 0), and the
    # whole-row kernel for a row count it does not take
    (14, 20480, 4096), (14, 20482, 4096),
]


@pytest.mark.parametrize("type_id,rows,cols", SHAPES)
def test_matvec(gpu, oracle, type_id, rows, cols):
    rng = np.random.default_rng(rows * 31 + cols + type_id)
    w, wd = _mk(rng, type_id, rows, cols)
    x = rng.standard_normal(cols).astype(np.float32)
    y = torch.full((rows,), float("nan"), device="cuda")
    case(f"matvec type={type_id} {rows}x{cols}")
    (gpu.ops.matvec_q4k if type_id == 12 else gpu.ops.matvec_q6k)(wd, dev(x), y, rows, cols)
    err = rel_l2(host(y), oracle.gemv(type_id, w, x, rows, cols))
    print(f"rel_l2={err:.2e}")
    assert err < TOL


def test_dispatcher_matvec(gpu, oracle):
    rng = np.random.default_rng(7)
    for t, rows, cols in [(12, 64, 1024), (14, 64, 1024)]:
        w, wd = _mk(rng, t, rows, cols)
        x = rng.standard_normal(cols).astype(np.float32)
        y = torch.zeros(rows, device="cuda")
        case(f"mnemo_matvec type={t}")
        gpu.ops.matvec(wd, dev(x), y, rows, cols, t)
        assert rel_l2(host(y), oracle.gemv(t, w, x, rows, cols)) < TOL
    wr = rng.standard_normal((128, 4096)).astype(np.float32)
    x = rng.standard_normal(4096).astype(np.float32)
    y = torch.zeros(128, device="cuda")
    case("mnemo_matvec type=0 (router)")
    gpu.ops.matvec(dev(wr), dev(x), y, 128, 4096, 0)
    assert rel_l2(host(y), oracle.matvec_f32(wr, x, 128, 4096)) < 1e-6


@pytest.mark.parametrize("rows,cols", [(4096, 8192), (100, 4096), (33, 512)])
def test_matvec_add_residual(gpu, oracle, rows, cols):
    rng = np.random.default_rng(rows + cols)
    w, wd = _mk(rng, 12, rows, cols)
    x = rng.standard_normal(cols).astype(np.float32)
    res = rng.standard_normal(rows).astype(np.float32)
    y = torch.zeros(rows, device="cuda")
    case(f"matvec_q4k_add {rows}x{cols}")
    gpu.ops.matvec_q4k_add(wd, dev(x), dev(res), y, rows, cols)
    assert rel_l2(host(y), oracle.gemv(12, w, x, rows, cols) + res) < TOL


@pytest.mark.parametrize("q_rows,kv_rows,cols", [(8192, 512, 4096), (64, 6, 512), (40, 3, 1024)])
def test_qkv(gpu, oracle, q_rows, kv_rows, cols):
    rng = np.random.default_rng(q_rows + kv_rows)
    ws = [_mk(rng, 12, r, cols) for r in (q_rows, kv_rows, kv_rows)]
    x = rng.standard_normal(cols).astype(np.float32)
    outs = [torch.zeros(r, device="cuda") for r in (q_rows, kv_rows, kv_rows)]
    case(f"qkv {q_rows}/{kv_rows}x{cols}")
    gpu.ops.matvec_q4k_qkv(ws[0][1], ws[1][1], ws[2][1], dev(x), *outs, q_rows, kv_rows, cols)
    for (w, _), o, r in zip(ws, outs, (q_rows, kv_rows, kv_rows)):
        assert rel_l2(host(o), oracle.gemv(12, w, x, r, cols)) < TOL


@pytest.mark.parametrize("types,q_rows,kv_rows,cols", [((12, 12, 14), 8192, 512, 4096), ((14, 12, 14), 70, 9, 768),
                                                       ((12, 14, 12), 33, 64, 1000)])
def test_qkv_mixed(gpu, oracle, types, q_rows, kv_rows, cols):
    rng = np.random.default_rng(q_rows * 3 + kv_rows)
    rows = (q_rows, kv_rows, kv_rows)
    ws = [_mk(rng, t, r, cols) for t, r in zip(types, rows)]
    x = rng.standard_normal(cols).astype(np.float32)
    outs = [torch.full((r,), float("nan"), device="cuda") for r in rows]
    case(f"qkv mixed {types} {q_rows}/{kv_rows}x{cols}")
    gpu.ops.matvec_qkv(ws[0][1], types[0], ws[1][1], types[1], ws[2][1], types[2], dev(x), *outs,
                       q_rows, kv_rows, cols)
    for (w, _), t, o, r in zip(ws, types, outs, rows):
        assert rel_l2(host(o), oracle.gemv(t, w, x, r, cols)) < TOL


@pytest.mark.parametrize("types,q_rows,kv_rows,cols", [((12, 12, 14), 8192, 512, 4096), ((14, 12, 14), 70, 9, 768),
                                                       ((12, 14, 12), 33, 64, 1000), ((12, 12, 12), 256, 64, 12288)])
def test_qkv_rmsnorm(gpu, oracle, types, q_rows, kv_rows, cols):
    """The attention norm folded into the projection launch (forward.c:687-700 then :705-712):
    each projection equals the oracle GEMV of rms_norm(x) * norm_w."""
    rng = np.random.default_rng(q_rows * 5 + kv_rows)
    rows = (q_rows, kv_rows, kv_rows)
    ws = [_mk(rng, t, r, cols) for t, r in zip(types, rows)]
    x = (4.0 * rng.standard_normal(cols)).astype(np.float32)
    nw = (1.0 + 0.3 * rng.standard_normal(cols)).astype(np.float32)
    eps = 1e-6
    xn = oracle.rms_norm(x, nw, eps)
    outs = [torch.full((r,), float("nan"), device="cuda") for r in rows]
    case(f"qkv rmsnorm {types} {q_rows}/{kv_rows}x{cols}")
    gpu.ops.matvec_qkv_rmsnorm(ws[0][1], types[0], ws[1][1], types[1], ws[2][1], types[2], dev(x), dev(nw), eps,
                               *outs, q_rows, kv_rows, cols)
    for (w, _), t, o, r in zip(ws, types, outs, rows):
        assert rel_l2(host(o), oracle.gemv(t, w, xn, r, cols)) < TOL
    case("qkv rmsnorm: n_cols % 4 != 0 rejected")
    with pytest.raises(gpu.MnemoError):
        gpu.ops.matvec_qkv_rmsnorm(ws[0][1], types[0], ws[1][1], types[1], ws[2][1], types[2], dev(x), dev(nw), eps,
                                   *outs, q_rows, kv_rows, cols - 2)


@pytest.mark.parametrize("ta,tb,rows,cols", [(12, 12, 1536, 4096), (12, 14, 512, 4096), (14, 12, 77, 768),
                                             (14, 14, 64, 1536)])
def test_dual(gpu, oracle, ta, tb, rows, cols):
    rng = np.random.default_rng(ta * tb + rows)
    wa, wad = _mk(rng, ta, rows, cols)
    wb, wbd = _mk(rng, tb, rows, cols)
    x = rng.standard_normal(cols).astype(np.float32)
    ya, yb = torch.zeros(rows, device="cuda"), torch.zeros(rows, device="cuda")
    case(f"dual {ta}/{tb} {rows}x{cols}")
    if ta == tb == 12:
        gpu.ops.matvec_q4k_dual(wad, wbd, dev(x), ya, yb, rows, cols)
    else:
        gpu.ops.matvec_dual(wad, ta, wbd, tb, dev(x), ya, yb, rows, cols)
    assert rel_l2(host(ya), oracle.gemv(ta, wa, x, rows, cols)) < TOL
    assert rel_l2(host(yb), oracle.gemv(tb, wb, x, rows, cols)) < TOL


@pytest.mark.parametrize("type_id,rows,cols", [(12, 4096, 1536), (14, 4096, 1536), (14, 100, 4096)])
def test_scaled_add(gpu, oracle, type_id, rows, cols):
    rng = np.random.default_rng(rows * type_id)
    w, wd = _mk(rng, type_id, rows, cols)
    x = rng.standard_normal(cols).astype(np.float32)
    y0 = rng.standard_normal(rows).astype(np.float32)
    y = dev(y0.copy())
    s = 0.37
    case(f"scaled_add type={type_id} {rows}x{cols}")
    (gpu.ops.matvec_q4k_scaled_add if type_id == 12 else gpu.ops.matvec_q6k_scaled_add)(wd, dev(x), y, rows, cols, s)
    exp = y0 + s * oracle.gemv(type_id, w, x, rows, cols)
    assert rel_l2(host(y) - y0, exp - y0) < TOL


@pytest.mark.parametrize("type_id", [12, 14])
def test_swiglu_fused_down(gpu, oracle, type_id):
    rng = np.random.default_rng(99 + type_id)
    H, EFF = 4096, 1536
    w, wd = _mk(rng, type_id, H, EFF)
    g = rng.standard_normal(EFF).astype(np.float32)
    u = rng.standard_normal(EFF).astype(np.float32)
    y0 = rng.standard_normal(H).astype(np.float32)
    y = dev(y0.copy())
    case(f"swiglu_scaled_add type={type_id}")
    gpu.ops.matvec_swiglu_scaled_add(wd, type_id, dev(g), dev(u), y, H, EFF, 0.25)
    exp = 0.25 * oracle.gemv(type_id, w, oracle.swiglu(g, u), H, EFF)
    assert rel_l2(host(y) - y0, exp) < TOL


def test_expert_fwd_host_composition(gpu, oracle):
    """mnemo_expert_fwd (forward.c:1122-1142 composition): blob [gate][up][down Q6_K]."""
    rng = np.random.default_rng(5)
    H, EFF = 4096, 1536
    gate, up = synth.weights(rng, 12, EFF, H), synth.weights(rng, 12, EFF, H)
    down = synth.weights(rng, 14, H, EFF)
    blob = np.concatenate([gate, up, down])
    x = rng.standard_normal(H).astype(np.float32)
    acc0 = rng.standard_normal(H).astype(np.float32)
    acc = dev(acc0.copy())
    gb, ub = torch.zeros(EFF, device="cuda"), torch.zeros(EFF, device="cuda")
    case("expert_fwd")
    gpu.ops.expert_fwd(dev(blob), gate.size, up.size, H, EFF, 14, 0.6, dev(x), gb, ub, acc)
    gy = oracle.gemv(12, gate, x, EFF, H).astype(np.float32)
    uy = oracle.gemv(12, up, x, EFF, H).astype(np.float32)
    exp = 0.6 * oracle.gemv(14, down, oracle.swiglu(gy, uy), H, EFF)
    assert rel_l2(host(acc) - acc0, exp) < TOL


def test_repeat_calls_are_deterministic(gpu):
    rng = np.random.default_rng(3)
    w, wd = _mk(rng, 12, 2048, 4096)
    x = dev(rng.standard_normal(4096).astype(np.float32))
    ys = []
    for _ in range(3):
        y = torch.zeros(2048, device="cuda")
        gpu.ops.matvec_q4k(wd, x, y, 2048, 4096)
        ys.append(host(y))
    assert all(np.array_equal(ys[0], t) for t in ys[1:])


# ---------------------------------------------------------------- adversarial x
# x is carried as a 16-bit integer (two bytes) per value, scaled per 32-value block by the
# block's max |x| (step max|x| / 32767), so a block that mixes one huge value with small ones quantises the
# small ones coarsely.  These inputs stress that encoding; the bar stays relative L2 1e-3
# against the fp64 oracle of the reference's fp32-x product (kernels.cu:124-135).
def _adversarial_x(kind: str, n: int, rng) -> np.ndarray:
    x = rng.standard_normal(n)
    if kind == "outlier_per_block":  # one 1e3-times value in every 32-value block
        pos = np.arange(0, n, 32) + rng.integers(0, 32, size=(n + 31) // 32)
        pos = pos[pos < n]
        x[pos] *= 1e3
    elif kind == "student_t2":
        x = rng.standard_t(2.0, size=n)
    elif kind == "massive_channels":  # a few channels at 1e4 over N(0, 1)
        x[rng.choice(n, size=4, replace=False)] = 1e4 * rng.choice([-1.0, 1.0], size=4)
    elif kind == "zero_blocks":  # every other 32-block (and a whole 256 block) all zero
        x = x.reshape(-1, 32)
        x[::2] = 0.0
        x = x.reshape(-1)
        x[256:512] = 0.0
    else:
        raise ValueError(kind)
    return x.astype(np.float32)


ADV = ["outlier_per_block", "student_t2", "massive_channels", "zero_blocks"]


@pytest.mark.parametrize("kind", ADV)
@pytest.mark.parametrize("type_id,rows,cols", [(12, 4096, 4096), (14, 4096, 4096), (12, 1536, 4096), (14, 512, 1536)])
def test_matvec_adversarial_x(gpu, oracle, kind, type_id, rows, cols):
    rng = np.random.default_rng(abs(hash(kind)) % 1000 + rows + type_id)
    w, wd = _mk(rng, type_id, rows, cols)
    x = _adversarial_x(kind, cols, rng)
    y = torch.full((rows,), float("nan"), device="cuda")
    case(f"matvec adversarial {kind} type={type_id} {rows}x{cols}")
    (gpu.ops.matvec_q4k if type_id == 12 else gpu.ops.matvec_q6k)(wd, dev(x), y, rows, cols)
    err = rel_l2(host(y), oracle.gemv(type_id, w, x, rows, cols))
    print(f"{kind} rel_l2={err:.2e}")
    assert err < TOL


@pytest.mark.parametrize("kind", ADV)
def test_qkv_adversarial_x(gpu, oracle, kind):
    rng = np.random.default_rng(11 + ADV.index(kind))
    types, rows, cols = (12, 12, 14), (8192, 512, 512), 4096
    ws = [_mk(rng, t, r, cols) for t, r in zip(types, rows)]
    x = _adversarial_x(kind, cols, rng)
    outs = [torch.full((r,), float("nan"), device="cuda") for r in rows]
    case(f"qkv adversarial {kind}")
    gpu.ops.matvec_qkv(ws[0][1], types[0], ws[1][1], types[1], ws[2][1], types[2], dev(x), *outs, 8192, 512, cols)
    for (w, _), t, o, r in zip(ws, types, outs, rows):
        err = rel_l2(host(o), oracle.gemv(t, w, x, r, cols))
        print(f"{kind} type={t} rel_l2={err:.2e}")
        assert err < TOL


@pytest.mark.parametrize("kind", ADV)
def test_dual_adversarial_x(gpu, oracle, kind):
    rng = np.random.default_rng(23 + ADV.index(kind))
    wa, wad = _mk(rng, 12, 1536, 4096)
    wb, wbd = _mk(rng, 14, 1536, 4096)
    x = _adversarial_x(kind, 4096, rng)
    ya, yb = torch.zeros(1536, device="cuda"), torch.zeros(1536, device="cuda")
    case(f"dual adversarial {kind}")
    gpu.ops.matvec_dual(wad, 12, wbd, 14, dev(x), ya, yb, 1536, 4096)
    assert rel_l2(host(ya), oracle.gemv(12, wa, x, 1536, 4096)) < TOL
    assert rel_l2(host(yb), oracle.gemv(14, wb, x, 1536, 4096)) < TOL


@pytest.mark.parametrize("kind", ADV)
def test_qkv_rmsnorm_adversarial_x(gpu, oracle, kind):
    rng = np.random.default_rng(37 + ADV.index(kind))
    types, rows, cols = (12, 12, 14), (8192, 512, 512), 4096
    ws = [_mk(rng, t, r, cols) for t, r in zip(types, rows)]
    x = _adversarial_x(kind, cols, rng)
    nw = (1.0 + 0.3 * rng.standard_normal(cols)).astype(np.float32)
    eps = 1e-6
    xn = oracle.rms_norm(x, nw, eps)
    outs = [torch.full((r,), float("nan"), device="cuda") for r in rows]
    case(f"qkv rmsnorm adversarial {kind}")
    gpu.ops.matvec_qkv_rmsnorm(ws[0][1], types[0], ws[1][1], types[1], ws[2][1], types[2], dev(x), dev(nw), eps,
                               *outs, 8192, 512, cols)
    for (w, _), t, o, r in zip(ws, types, outs, rows):
        assert rel_l2(host(o), oracle.gemv(t, w, xn, r, cols)) < TOL


# ---------------------------------------------------------------- x encoding, value by value
def _diag_q4k(n: int) -> np.ndarray:
    """Q4_K matrix n x n with W[r][r] = 15 and every other weight 0: d = 1, dmin = 0, all
    (sc, m) = (1, 0); the nibble of value v in its block sits in qs[32(v//64) + v%32], low
    half for v%64 < 32 (kernels.cu:114-136)."""
    bpr = n // 256
    blk = np.zeros((n, bpr, 144), dtype=np.uint8)
    blk[:, :, 0:2] = np.frombuffer(np.float16(1.0).tobytes(), dtype=np.uint8)
    # packed scales: sub-blocks 0-3 sc in bytes 0-3 (m in 4-7), 4-7 in the nibbles of 8-11
    blk[:, :, 4:8] = 1
    blk[:, :, 12:16] = 1
    for r in range(n):
        b, v = divmod(r, 256)
        byte = 16 + 32 * (v // 64) + v % 32
        blk[r, b, byte] = 0x0F if v % 64 < 32 else 0xF0
    return blk.reshape(-1)


def test_x_encoding_value_by_value(gpu, oracle):
    """Each output of the one-hot diagonal Q4_K matrix is 15 * (x as the kernel encodes it),
    so every value of x is checked against the encoding's bound |xhat - x| <= u/2,
    u = amax/32767 of its 32-value block, at the byte boundaries of the 16-bit integer
    (q = +-1, +-255, +-256, -257, +-32767, 0) and for random values."""
    n = 4096
    rng = np.random.default_rng(11)
    W = _diag_q4k(n)
    # the matrix is what the oracle decodes: 15 on the diagonal
    dense = oracle.dequant(12, W, n, n)
    assert np.array_equal(np.diag(dense), np.full(n, 15.0)) and np.count_nonzero(dense) == n
    del dense
    x = np.zeros(n, dtype=np.float32)
    qs = [32767, -32767, 255, 256, -256, -257, 1, -1, 0, 127, 128, -128, -129, 16383, -16384]
    for blk in range(n // 32):
        amax = np.float32(10.0 ** rng.uniform(-3, 3))
        vals = rng.uniform(-1, 1, 32).astype(np.float32) * amax
        vals[0] = amax if blk % 2 else -amax
        for i, q in enumerate(qs):
            vals[1 + i] = np.float32(amax * (q / 32767.0))
        x[32 * blk: 32 * blk + 32] = vals
    y = torch.zeros(n, device="cuda")
    case("matvec_q4k one-hot diagonal, x at the encoding's byte boundaries")
    gpu.ops.matvec_q4k(dev(W), dev(x), y, n, n)
    xhat = host(y).astype(np.float64) / 15.0
    amax = np.abs(x.reshape(-1, 32)).max(axis=1).repeat(32).astype(np.float64)
    bound = 0.5 * amax / 32767.0 * (1 + 1e-5) + 1e-7 * np.abs(x)
    err = np.abs(xhat - x.astype(np.float64))
    worst = int(np.argmax(err / bound))
    assert (err <= bound).all(), f"x[{worst}]={x[worst]!r} decoded {xhat[worst]!r}, bound {bound[worst]:.3e}"


def test_matvec_q6k_lm_head_unaligned(gpu, oracle):
    """A Q6_K matrix of 4096-value rows over several chip rounds whose first block sits 2 bytes
    past a 16-byte boundary: the staged kernel (aligned 16-byte loads) must decline it and the
    whole-row kernel's realigned loads give the oracle's result."""
    rows, cols = 20480, 4096
    rng = np.random.default_rng(5)
    w = synth.weights(rng, 14, rows, cols)
    buf = torch.zeros(w.size + 210, dtype=torch.uint8, device="cuda")
    buf[210:] = dev(w)
    wd = buf[210:]
    assert wd.data_ptr() % 16 == 2
    x = rng.standard_normal(cols).astype(np.float32)
    y = torch.full((rows,), float("nan"), device="cuda")
    case("matvec_q6k 20480x4096 at a 2-byte-aligned address")
    gpu.ops.matvec_q6k(wd, dev(x), y, rows, cols)
    err = rel_l2(host(y), oracle.gemv(14, w, x, rows, cols))
    print(f"rel_l2={err:.2e}")
    assert err < TOL
