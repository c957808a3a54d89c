"""Independent numpy restatement of the GGUF block formats and the hot-path arithmetic.

TEST INFRASTRUCTURE ONLY.  Written from the layout descriptions (not from the C
oracle) so that the two restatements check each other:

* Q4_K (kernels.cu:20-25, 114-136; forward.c:1212-1228): 144 B = f16 d, f16 dmin,
  12 B packed 6-bit (scale, min) x 8, 128 B nibbles.  Value v of a super-block sits in
  byte qs[32*(v//64) + v%32], low nibble when v%64 < 32; sub-block v//32.
* Q6_K (kernels.cu:27-32, 455-486; tools/validate_dequant.py:253-319): 210 B = ql[128],
  qh[64], int8 scales[16], f16 d.  ql reshaped (2, 64) gives low nibbles for values
  0..63 of each 128-half and high nibbles for 64..127; qh reshaped (2, 32) shifted by
  0, 2, 4, 6 gives the top two bits of the four 32-value groups; scale v//16.
* Q8_1 MMQ (gemm_q4k.cu:26-33, 327-358): per 128 values, 4 x (half d, half d*sum)
  followed by 128 int8.

Vectorised over blocks so that whole fixtures are decoded at once.
"""
from __future__ import annotations

import numpy as np

Q4K_BYTES = 144
Q6K_BYTES = 210
Q81_BYTES = 144


def scale_min_k4_all(scales12: np.ndarray) -> tuple[np.ndarray, np.ndarray]:
    """(sc[...,8], m[...,8]) from packed scales[...,12] (kernels.cu:45-53)."""
    q = scales12.astype(np.uint16)
    sc = np.empty(q.shape[:-1] + (8,), np.uint16)
    m = np.empty_like(sc)
    sc[..., :4] = q[..., 0:4] & 63
    m[..., :4] = q[..., 4:8] & 63
    sc[..., 4:] = (q[..., 8:12] & 0x0F) | ((q[..., 0:4] >> 6) << 4)
    m[..., 4:] = (q[..., 8:12] >> 4) | ((q[..., 4:8] >> 6) << 4)
    return sc.astype(np.uint8), m.astype(np.uint8)


def pack_scale_min_k4(sc: np.ndarray, m: np.ndarray) -> np.ndarray:
    """Inverse of scale_min_k4_all: 8 six-bit scales and mins -> 12 bytes."""
    sc = sc.astype(np.uint16)
    m = m.astype(np.uint16)
    out = np.zeros(sc.shape[:-1] + (12,), np.uint16)
    out[..., 0:4] = (sc[..., 0:4] & 63) | ((sc[..., 4:8] >> 4) << 6)
    out[..., 4:8] = (m[..., 0:4] & 63) | ((m[..., 4:8] >> 4) << 6)
    out[..., 8:12] = (sc[..., 4:8] & 15) | ((m[..., 4:8] & 15) << 4)
    return out.astype(np.uint8)


def unpack_scales_q45k_int(scales12: np.ndarray, ksc: int) -> np.ndarray:
    """Packed-int form of gemm_q4k.cu:53-56: four 6-bit values as bytes of one uint32.

    ksc 0 -> sc[0..3], 1 -> sc[4..7], 2 -> m[0..3], 3 -> m[4..7]."""
    ints = scales12.reshape(-1, 12).copy().view("<u4").astype(np.uint64)  # (n, 3)
    a = ints[:, (ksc % 2) + (1 if ksc != 0 else 0)]
    b = ints[:, ksc // 2]
    sh1 = 4 * (ksc & (ksc // 2))
    sh2 = 2 * (ksc % 2)
    v = ((a >> sh1) & 0x0F0F0F0F) | ((b >> sh2) & 0x30303030)
    return v.astype(np.uint32)


def f16_bits_to_f32(bits: np.ndarray) -> np.ndarray:
    return np.asarray(bits, np.uint16).view(np.float16).astype(np.float32)


def dequant_q4k_blocks(raw: np.ndarray) -> np.ndarray:
    """raw uint8 (..., 144) -> float32 (..., 256)."""
    raw = np.asarray(raw, np.uint8)
    shp = raw.shape[:-1]
    b = raw.reshape(-1, Q4K_BYTES)
    d = f16_bits_to_f32(b[:, 0:2].copy().view("<u2")[:, 0])
    dmin = f16_bits_to_f32(b[:, 2:4].copy().view("<u2")[:, 0])
    sc, m = scale_min_k4_all(b[:, 4:16])
    qs = b[:, 16:144].reshape(-1, 4, 32)
    q = np.empty((b.shape[0], 8, 32), np.float32)
    q[:, 0::2, :] = qs & 0x0F
    q[:, 1::2, :] = qs >> 4
    ds = (d[:, None] * sc.astype(np.float32))[:, :, None]
    ms = (dmin[:, None] * m.astype(np.float32))[:, :, None]
    w = (ds * q).astype(np.float32) - ms
    return w.astype(np.float32).reshape(shp + (256,))


def dequant_q6k_blocks(raw: np.ndarray) -> np.ndarray:
    """raw uint8 (..., 210) -> float32 (..., 256)."""
    raw = np.asarray(raw, np.uint8)
    shp = raw.shape[:-1]
    b = raw.reshape(-1, Q6K_BYTES)
    ql = b[:, 0:128].reshape(-1, 2, 64)
    qh = b[:, 128:192].reshape(-1, 2, 32)
    sc = b[:, 192:208].view(np.int8).astype(np.float32)
    d = f16_bits_to_f32(b[:, 208:210].copy().view("<u2")[:, 0])
    lo = np.concatenate([ql & 0x0F, ql >> 4], axis=2)  # (n, 2, 128)
    hi = np.stack([(qh >> s) & 3 for s in (0, 2, 4, 6)], axis=2).reshape(-1, 2, 128)
    q = ((hi.astype(np.int32) << 4) | lo.astype(np.int32)) - 32
    q = q.reshape(-1, 16, 16).astype(np.float32)
    s = (d[:, None] * sc)[:, :, None]
    return (s * q).astype(np.float32).reshape(shp + (256,))


def dequant_matrix(raw: np.ndarray, type_id: int, n_rows: int, n_cols: int) -> np.ndarray:
    bpr = (n_cols + 255) // 256
    if type_id == 0:
        return np.frombuffer(np.asarray(raw, np.uint8).tobytes(), np.float32).reshape(n_rows, n_cols)
    nb = Q4K_BYTES if type_id == 12 else Q6K_BYTES
    fn = dequant_q4k_blocks if type_id == 12 else dequant_q6k_blocks
    blocks = np.asarray(raw, np.uint8).reshape(n_rows, bpr, nb)
    return fn(blocks).reshape(n_rows, bpr * 256)[:, :n_cols]


def quantize_q8_1_mmq(src: np.ndarray) -> np.ndarray:
    """fp32 (N, K) -> uint8 (N, K//128, 144), gemm_q4k.cu:327-358 semantics."""
    src = np.ascontiguousarray(src, np.float32)
    n, k = src.shape
    xb = src.reshape(n, k // 128, 4, 32)
    amax = np.max(np.abs(xb), axis=3)
    d = (amax / np.float32(127.0)).astype(np.float32)
    with np.errstate(divide="ignore"):
        idv = np.where(amax > 0, np.float32(127.0) / amax, np.float32(0.0)).astype(np.float32)
    q = np.clip(np.rint((xb * idv[..., None]).astype(np.float32)), -127, 127).astype(np.int8)
    s = np.zeros(amax.shape, np.float32)
    for i in range(32):  # sequential fp32 sum, as the reference's loop
        s = (s + xb[..., i]).astype(np.float32)
    hd = d.astype(np.float16).view(np.uint16)
    hs = (d * s).astype(np.float32).astype(np.float16).view(np.uint16)
    out = np.zeros((n, k // 128, Q81_BYTES), np.uint8)
    ds = np.stack([hd, hs], axis=-1).astype("<u2")  # (n, nsb, 4, 2)
    out[..., :16] = ds.reshape(n, k // 128, 8).view(np.uint8)
    out[..., 16:] = q.reshape(n, k // 128, 128).view(np.uint8)
    return out


def dequant_q8_1_mmq(blocks: np.ndarray, k: int) -> np.ndarray:
    b = np.asarray(blocks, np.uint8).reshape(-1, k // 128, Q81_BYTES)
    d = f16_bits_to_f32(b[..., :16].copy().view("<u2")[..., 0::2])  # (n, nsb, 4)
    q = b[..., 16:].view(np.int8).reshape(b.shape[0], k // 128, 4, 32).astype(np.float32)
    return (d[..., None] * q).reshape(b.shape[0], k)


def topk_softmax(scores: np.ndarray, k: int) -> tuple[np.ndarray, np.ndarray]:
    order = np.argsort(-scores.astype(np.float64), kind="stable")[:k]
    v = scores[order].astype(np.float64)
    e = np.exp(v - v.max())
    return order.astype(np.int32), (e / e.sum()).astype(np.float32)


# ------------------------------------------------------------------ next-token selection
def xoroshiro_next(s0: int, s1: int) -> tuple[int, int, int]:
    """xoroshiro128+ step as kernels.cu:2134-2143 writes it, in Python integers masked to 64 bits."""
    M = (1 << 64) - 1
    t = (s0 ^ (s0 << 23)) & M
    s0n = s1
    s1n = (t ^ s1 ^ (t >> 17) ^ (s1 >> 26)) & M
    return (s0n + s1n) & M, s0n, s1n


def sample_draw(seed: int) -> float:
    """The uniform draw of kernels.cu:2127-2143 for one call."""
    M = (1 << 64) - 1
    s0, s1 = seed & M, (seed ^ 0xDEADBEEFCAFEBABE) & M
    for _ in range(3):
        _, s0, s1 = xoroshiro_next(s0, s1)
    v, s0, s1 = xoroshiro_next(s0, s1)
    return float(np.float32(np.float32(v >> 11) * np.float32(1.0 / 9007199254740992.0)))


def sample_candidates(logits: np.ndarray, temperature: float):
    """The 2048 candidates of kernels.cu:2085-2104 as a set: for every residue class
    i mod 256, the 8 largest p with earlier indices winning ties (a scan that replaces its
    minimum only by a strictly larger value keeps exactly those).  Returns (p, ids) sorted
    by (p descending, id ascending), p in fp64."""
    z = logits.astype(np.float64)
    p = np.exp((z - z.max()) / temperature)
    V = p.size
    ids, ps = [], []
    for c in range(256):
        idx = np.arange(c, V, 256)
        if idx.size == 0:
            continue
        order = np.lexsort((idx, -p[idx]))[:8]
        ids.extend(idx[order].tolist())
        ps.extend(p[idx[order]].tolist())
    ids, ps = np.array(ids), np.array(ps)
    # equal p: the lower token id first.  (The reference's selection sort, kernels.cu:2145-2166,
    # orders equal p by where its swaps left them in the class-slot array; both orders give
    # the same running sums at every position, only the token drawn at a tie can differ.)
    o = np.lexsort((ids, -ps))
    return ps[o], ids[o], p.sum()


def sample_token(logits: np.ndarray, temperature: float, top_p: float, seed: int):
    """Restatement of the top-p draw in fp64; returns (token, margin) where margin is the
    distance of the draw from the nearest cumulative boundary, relative to the nucleus
    mass (fp32 rounding in the reference can only move the choice when it is tiny)."""
    if temperature <= 0:
        return int(np.argmax(logits)), 1.0
    ps, ids, total = sample_candidates(logits, temperature)
    c = np.cumsum(ps)
    n = int(np.searchsorted(c, top_p * total) + 1)
    n = min(n, ps.size)
    mass_margin = abs(c[n - 1] - top_p * total) / total if n - 1 < ps.size else 1.0
    if n >= 2:
        mass_margin = min(mass_margin, abs(c[n - 2] - top_p * total) / total)
    nsum = c[n - 1]
    target = sample_draw(seed) * nsum
    k = int(np.searchsorted(c[:n], target))
    k = min(k, n - 1)
    margin = min(abs(c[k] - target), abs(target - (c[k - 1] if k else 0.0))) / nsum
    return int(ids[k]), min(margin, mass_margin)


# ---------------------------------------------------------------- attention chain
# Written from the layout and formulas in the reference's kernels.cu (norms :692-781,
# RoPE :818-852 / :1256-1266, int8 KV :1339-1377, attention :1382-1481 / :1550-1660),
# independently of mnemo_oracle_attn.c, in float64 numpy.
def rms_norm(x: np.ndarray, w: np.ndarray, eps: float) -> np.ndarray:
    x = x.astype(np.float64)
    return (x / np.sqrt(np.mean(x * x, axis=-1, keepdims=True) + eps) * w).astype(np.float32)


def rope(v: np.ndarray, head_dim: int, pos: int, theta: float) -> np.ndarray:
    half = head_dim // 2
    j = np.arange(half, dtype=np.float32)
    e = ((2 * j) / np.float32(head_dim)).astype(np.float32)
    # powf, correctly rounded: the float64 power rounded once to float32 (numpy's float32
    # power is off by up to 2 ulp)
    p = np.power(np.float64(np.float32(theta)), e.astype(np.float64)).astype(np.float32)
    freq = (np.float32(1.0) / p).astype(np.float32)
    ang = (np.float32(pos) * freq).astype(np.float64)
    c, s = np.cos(ang), np.sin(ang)
    x = v.reshape(-1, head_dim).astype(np.float64)
    a, b = x[:, :half], x[:, half:]
    return np.concatenate([a * c - b * s, a * s + b * c], axis=1).astype(np.float32).reshape(v.shape)


def kv_quant_int8(x: np.ndarray, head_dim: int):
    h = x.reshape(-1, head_dim).astype(np.float32)
    a = np.abs(h).max(axis=1)
    with np.errstate(divide="ignore"):
        inv = np.where(a > 0, np.float32(127.0) / a, np.float32(0.0)).astype(np.float32)
        sc = np.where(a > 0, a / np.float32(127.0), np.float32(0.0)).astype(np.float32)
    q = np.clip(np.rint((h * inv[:, None]).astype(np.float32)), -127, 127).astype(np.int8)
    return q.reshape(-1), sc


def attention(q: np.ndarray, k: np.ndarray, v: np.ndarray, n_heads: int, head_dim: int, n_kv_heads: int,
              scale: float) -> np.ndarray:
    """k, v: float arrays [seq][n_kv_heads][head_dim] (already dequantised)."""
    seq = k.shape[0]
    qh = q.reshape(n_heads, head_dim).astype(np.float64)
    kv = np.arange(n_heads) // (n_heads // n_kv_heads)
    out = np.zeros((n_heads, head_dim))
    for h in range(n_heads):
        s = (k[:, kv[h], :].astype(np.float64) @ qh[h]) * scale
        p = np.exp(s - s.max())
        out[h] = (p / p.sum()) @ v[:, kv[h], :].astype(np.float64)
    return out.astype(np.float32).reshape(-1)


def q8_1_ds(blocks: np.ndarray, k: int) -> np.ndarray:
    """The second half of each (d8, ds) pair: (N, k // 32) float32."""
    b = np.asarray(blocks, np.uint8).reshape(-1, k // 128, Q81_BYTES)
    return f16_bits_to_f32(b[..., :16].copy().view("<u2")[..., 1::2]).reshape(b.shape[0], k // 32)


def q4k_split(raw: np.ndarray, n_rows: int, n_cols: int):
    """Q4_K rows -> (main, mins): main (n_rows, n_cols) = d * sc * q and mins
    (n_rows, n_cols // 32) = dmin * m per 32-value sub-block, both exact in float64."""
    b = np.asarray(raw, np.uint8).reshape(n_rows, n_cols // 256, Q4K_BYTES)
    d = f16_bits_to_f32(b[..., 0:2].copy().view("<u2")[..., 0]).astype(np.float64)
    dmin = f16_bits_to_f32(b[..., 2:4].copy().view("<u2")[..., 0]).astype(np.float64)
    sc, m = scale_min_k4_all(b[..., 4:16].reshape(-1, 12))
    sc = sc.reshape(n_rows, -1, 8).astype(np.float64)
    m = m.reshape(n_rows, -1, 8).astype(np.float64)
    qs = b[..., 16:].reshape(n_rows, -1, 4, 32)
    q = np.empty(qs.shape[:2] + (8, 32), np.float64)
    q[:, :, 0::2] = qs & 0x0F
    q[:, :, 1::2] = qs >> 4
    main = (d[..., None, None] * sc[..., None]) * q
    mins = dmin[..., None] * m
    return main.reshape(n_rows, n_cols), mins.reshape(n_rows, n_cols // 32)


def gemm_q8_1(type_id: int, raw: np.ndarray, blocks: np.ndarray, M: int, K: int, N: int) -> np.ndarray:
    """fp64 (N, M): Q4_K as main . deq(Q8_1)^T - ds . mins^T (gemm_q4k.cu:164-166, the min term
    taken from the activation block's ds field); Q6_K as deq(W) . deq(Q8_1)^T."""
    a = dequant_q8_1_mmq(blocks, K).astype(np.float64)
    if type_id == 12:
        main, mins = q4k_split(raw, M, K)
        return a @ main.T - q8_1_ds(blocks, K).astype(np.float64) @ mins.T
    return a @ dequant_matrix(raw, type_id, M, K).astype(np.float64).T
