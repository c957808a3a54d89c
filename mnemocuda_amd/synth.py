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
