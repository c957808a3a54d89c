"""Torch restatement of the GEMM semantics and of the MoE prefill chain, for parity tests at
sizes where the C oracle would take minutes (test infrastructure only).

The GEMM semantics are oracle/mnemo_oracle.c's mo_gemm_q8_1 (gemm_q4k.cu:103-112, 164-166):
Q4_K rows split into main = d*sc*q and mins = dmin*m per 32 values, the product
main . deq(Q8_1)^T - ds . mins^T in fp64; Q6_K as deq(W) . deq(Q8_1)^T.  The decoding
here is written from the block layouts with torch tensor ops so it runs on the GPU;
tests/test_torch_ref.py pins it against the oracle on the CPU."""
import torch

Q4K, Q6K, Q81 = 144, 210, 144


def _f16(b: torch.Tensor) -> torch.Tensor:
    """(..., 2) uint8 little-endian f16 bits -> float64 (...)."""
    return b.contiguous().view(torch.float16)[..., 0].double()


def _scale_min(s12: torch.Tensor):
    """(..., 12) uint8 -> sc, m (..., 8) int64 (get_scale_min_k4, kernels.cu:45-53)."""
    s = s12.long()
    sc = torch.empty(s.shape[:-1] + (8,), dtype=torch.long, device=s.device)
    m = torch.empty_like(sc)
    sc[..., :4] = s[..., 0:4] & 63
    m[..., :4] = s[..., 4:8] & 63
    sc[..., 4:] = (s[..., 8:12] & 15) | ((s[..., 0:4] >> 6) << 4)
    m[..., 4:] = (s[..., 8:12] >> 4) | ((s[..., 4:8] >> 6) << 4)
    return sc, m


def q4k_split(raw: torch.Tensor, M: int, K: int):
    """Q4_K rows -> main (M, K) = d*sc*q and mins (M, K/32) = dmin*m, float64."""
    b = raw.reshape(M, K // 256, Q4K)
    d, dmin = _f16(b[..., 0:2]), _f16(b[..., 2:4])
    sc, m = _scale_min(b[..., 4:16])
    qs = b[..., 16:].reshape(M, K // 256, 4, 32).long()
    q = torch.stack([qs & 15, qs >> 4], dim=3).reshape(M, K // 256, 8, 32).double()
    main = d[..., None, None] * sc.double()[..., None] * q
    return main.reshape(M, K), (dmin[..., None] * m.double()).reshape(M, K // 32)


def q6k_dequant(raw: torch.Tensor, M: int, K: int) -> torch.Tensor:
    """Q6_K rows -> (M, K) float64: d * sc[v/16] * (q - 32) (tools/validate_dequant.py:253-319)."""
    b = raw.reshape(M, K // 256, Q6K)
    ql = b[..., 0:128].reshape(M, -1, 2, 64).long()
    qh = b[..., 128:192].reshape(M, -1, 2, 32).long()
    sc = b[..., 192:208].contiguous().view(torch.int8).double()
    d = _f16(b[..., 208:210])
    lo = torch.cat([ql & 15, ql >> 4], dim=3)                                    # (.., 2, 128)
    hi = torch.stack([(qh >> s) & 3 for s in (0, 2, 4, 6)], dim=3).reshape(M, -1, 2, 128)
    q = ((hi << 4) | lo).double() - 32.0
    w = (d[..., None] * sc).reshape(M, -1, 16, 1) * q.reshape(M, -1, 16, 16)
    return w.reshape(M, K)


def q8_1_parts(blocks: torch.Tensor, N: int, K: int):
    """Q8_1 MMQ rows -> values d8*q8 (N, K) and ds (N, K/32), float64."""
    b = blocks.reshape(N, K // 128, Q81)
    hdr = b[..., :16].reshape(N, K // 128, 4, 2, 2)
    d8, ds = _f16(hdr[..., 0, :]), _f16(hdr[..., 1, :])                           # (N, nb, 4)
    q = b[..., 16:].contiguous().view(torch.int8).double().reshape(N, K // 128, 4, 32)
    return (d8[..., None] * q).reshape(N, K), ds.reshape(N, K // 32)


def gemm(type_id: int, raw: torch.Tensor, blocks: torch.Tensor, M: int, K: int, N: int) -> torch.Tensor:
    """(N, M) float64, the product mo_gemm_q8_1 defines."""
    a, ds = q8_1_parts(blocks, N, K)
    if type_id == 12:
        main, mins = q4k_split(raw, M, K)
        return a @ main.T - ds @ mins.T
    return a @ q6k_dequant(raw, M, K).T


def quantize_q8_1(x: torch.Tensor) -> torch.Tensor:
    """fp32 (N, K) -> Q8_1 MMQ bytes (N, K/128, 144), gemm_q4k.cu:327-358 (the sum of each
    32 values taken sequentially in fp32, d*sum rounded to fp32 then to f16)."""
    N, K = x.shape
    xb = x.float().reshape(N, K // 128, 4, 32)
    amax = xb.abs().amax(dim=3)
    d = amax / 127.0
    idv = torch.where(amax > 0, 127.0 / amax, torch.zeros_like(amax))
    q = torch.clamp(torch.round(xb * idv[..., None]), -127, 127).to(torch.int8)
    s = torch.zeros_like(amax)
    for i in range(32):
        s = s + xb[..., i]
    hd = d.half().view(torch.int16)
    hs = (d * s).half().view(torch.int16)
    out = torch.zeros((N, K // 128, Q81), dtype=torch.uint8, device=x.device)
    out[..., :16] = torch.stack([hd, hs], dim=-1).reshape(N, K // 128, 8).contiguous().view(torch.uint8)
    out[..., 16:] = q.reshape(N, K // 128, 128).view(torch.uint8)
    return out


def moe_prefill(table: torch.Tensor, stride: int, g_off: int, u_off: int, d_off: int, down_type: int,
                x: torch.Tensor, idx, w, H: int, EFF: int, quantize=quantize_q8_1) -> torch.Tensor:
    """The reference's token-sequential MoE prefill (src/forward.c:1783-1830, per expert
    src/forward.c:876-893) in the GEMM semantics: per token and selected expert
    g, u = W_g x, W_u x (fp64, stored as fp32), act = silu(g) * u in fp32,
    out += w * (W_d Q8_1(act)).  Pairs are batched per expert only; every output row depends
    on its own token alone.  Returns the fp64 delta (T, H).  `quantize` maps fp32 rows to
    Q8_1 bytes (the caller passes the HIP quantizer, which is bit-exact against the oracle)."""
    import numpy as np
    T = x.shape[0]
    xq = quantize(x.float().contiguous()).reshape(T, -1)
    out = torch.zeros((T, H), dtype=torch.float64, device=x.device)
    for e in np.unique(idx):
        if e < 0 or (e + 1) * stride > table.numel():
            continue
        tok, slot = np.nonzero(idx == e)
        tt = torch.from_numpy(tok).to(x.device)
        base = int(e) * stride
        a = xq[tt]
        g = gemm(12, table[base + g_off: base + u_off], a, EFF, H, tok.size).float()
        u = gemm(12, table[base + u_off: base + d_off], a, EFF, H, tok.size).float()
        act = (g / (1.0 + torch.exp(-g)) * u).contiguous()
        d = gemm(down_type, table[base + d_off: base + stride], quantize(act), H, EFF, tok.size)
        out.index_add_(0, tt, d * torch.from_numpy(w[tok, slot]).to(x.device).double()[:, None])
    return out
