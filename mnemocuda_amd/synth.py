"""Seeded synthetic GGUF weights and activations with the value distributions of the
benchmark configurations (there are no checkpoints offline).

Q4_K super-block (144 B): d, dmin = f16(|N(0,1)| * 0.01); the 12 scale bytes uniform,
which is exactly (sc, m) ~ U{0..63}^8 each because the 6-bit packing is a bijection of
96 bits; 128 uniform nibble bytes.
Q6_K super-block (210 B): ql, qh uniform bytes; scales int8 = clip(round(N(0,32)), -128,
127); d = f16(|N(0,1)| * 0.01).

numpy generators serve the CPU oracle and parity tests; the torch generators build the
multi-GB benchmark tensors directly in HBM.
"""
from __future__ import annotations

import numpy as np

Q4K_BYTES, Q6K_BYTES = 144, 210


def q4k_blocks(rng: np.random.Generator, nblocks: int) -> np.ndarray:
    b = rng.integers(0, 256, size=(nblocks, Q4K_BYTES), dtype=np.uint8)
    dd = (np.abs(rng.standard_normal((nblocks, 2))) * 0.01).astype(np.float16)
    b[:, 0:4] = dd.view(np.uint8).reshape(nblocks, 4)
    return b


def q6k_blocks(rng: np.random.Generator, nblocks: int) -> np.ndarray:
    b = rng.integers(0, 256, size=(nblocks, Q6K_BYTES), dtype=np.uint8)
    sc = np.clip(np.rint(rng.standard_normal((nblocks, 16)) * 32.0), -128, 127).astype(np.int8)
    b[:, 192:208] = sc.view(np.uint8)
    d = (np.abs(rng.standard_normal(nblocks)) * 0.01).astype(np.float16)
    b[:, 208:210] = d.view(np.uint8).reshape(nblocks, 2)
    return b


def weights(rng: np.random.Generator, type_id: int, rows: int, cols: int) -> np.ndarray:
    """Row-major GGUF matrix [rows][cols] as a flat uint8 array."""
    bpr = (cols + 255) // 256
    if type_id == 12:
        return q4k_blocks(rng, rows * bpr).reshape(-1)
    if type_id == 14:
        return q6k_blocks(rng, rows * bpr).reshape(-1)
    if type_id == 0:
        return rng.standard_normal((rows, cols)).astype(np.float32).view(np.uint8).reshape(-1)
    raise ValueError(type_id)


# ------------------------------------------------------------------ torch (on device)
def q4k_blocks_torch(gen, nblocks: int, device):
    import torch
    b = torch.randint(0, 256, (nblocks, Q4K_BYTES), dtype=torch.uint8, device=device, generator=gen)
    dd = (torch.randn((nblocks, 2), device=device, generator=gen).abs() * 0.01).to(torch.float16)
    b[:, 0:4] = dd.view(torch.uint8).reshape(nblocks, 4)
    return b


def q6k_blocks_torch(gen, nblocks: int, device):
    import torch
    b = torch.randint(0, 256, (nblocks, Q6K_BYTES), dtype=torch.uint8, device=device, generator=gen)
    sc = torch.clamp(torch.round(torch.randn((nblocks, 16), device=device, generator=gen) * 32.0), -128, 127)
    b[:, 192:208] = sc.to(torch.int8).view(torch.uint8)
    d = (torch.randn(nblocks, device=device, generator=gen).abs() * 0.01).to(torch.float16)
    b[:, 208:210] = d.view(torch.uint8).reshape(nblocks, 2)
    return b


def weights_torch(gen, type_id: int, rows: int, cols: int, device):
    bpr = (cols + 255) // 256
    if type_id == 12:
        return q4k_blocks_torch(gen, rows * bpr, device).reshape(-1)
    if type_id == 14:
        return q6k_blocks_torch(gen, rows * bpr, device).reshape(-1)
    raise ValueError(type_id)


# ------------------------------------------------------------------ MoE routing / expert tables
def expert_layout(hidden: int, eff: int, down_type: int) -> tuple[int, int, int, int]:
    """(stride, gate_off, up_off, down_off) of one expert's [gate | up | down] record, the
    order of the reference's per-expert files (gate Q4_K, up Q4_K, down Q4_K or Q6_K)."""
    g = eff * ((hidden + 255) // 256) * Q4K_BYTES
    d = hidden * ((eff + 255) // 256) * (Q6K_BYTES if down_type == 14 else Q4K_BYTES)
    stride = (2 * g + d + 255) // 256 * 256
    return stride, 0, g, 2 * g


def expert_table(rng: np.random.Generator, n_experts: int, hidden: int, eff: int, down_type: int) -> np.ndarray:
    stride, _, up_off, down_off = expert_layout(hidden, eff, down_type)
    t = np.zeros((n_experts, stride), dtype=np.uint8)
    for e in range(n_experts):
        t[e, :up_off] = weights(rng, 12, eff, hidden)
        t[e, up_off:down_off] = weights(rng, 12, eff, hidden)
        dw = weights(rng, down_type, hidden, eff)
        t[e, down_off:down_off + dw.size] = dw
    return t.reshape(-1)


def expert_table_torch(gen, n_experts: int, hidden: int, eff: int, down_type: int, device):
    import torch
    stride, _, up_off, down_off = expert_layout(hidden, eff, down_type)
    t = torch.zeros((n_experts, stride), dtype=torch.uint8, device=device)
    g = up_off
    t[:, :up_off] = weights_torch(gen, 12, n_experts * eff, hidden, device).view(n_experts, g)
    t[:, up_off:down_off] = weights_torch(gen, 12, n_experts * eff, hidden, device).view(n_experts, g)
    dw = weights_torch(gen, down_type, n_experts * hidden, eff, device)
    t[:, down_off:down_off + dw.numel() // n_experts] = dw.view(n_experts, -1)
    return t.reshape(-1)


def zipf_routing(rng: np.random.Generator, n_tokens: int, n_experts: int, k: int, s: float = 1.1):
    """Top-k routing per token: k distinct experts drawn without replacement with
    P(expert of popularity rank r) ~ r^-s (rank order itself a random permutation), router
    weights = softmax over the k selected logits (normalised top-k).  Returns int32
    [n_tokens][k] ids and fp32 [n_tokens][k] weights."""
    p = 1.0 / np.arange(1, n_experts + 1) ** s
    p /= p.sum()
    order = rng.permutation(n_experts)
    idx = np.empty((n_tokens, k), dtype=np.int32)
    for t in range(n_tokens):
        idx[t] = order[rng.choice(n_experts, size=k, replace=False, p=p)]
    logits = np.sort(rng.standard_normal((n_tokens, k)), axis=1)[:, ::-1]
    w = np.exp(logits - logits[:, :1])
    w /= w.sum(axis=1, keepdims=True)
    return idx, w.astype(np.float32)
