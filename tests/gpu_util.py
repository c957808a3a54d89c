"""Helpers for the GPU parity tests (uploading oracle inputs, naming the case)."""
import sys

import numpy as np
import torch


def dev(a: np.ndarray) -> torch.Tensor:
    return torch.from_numpy(np.ascontiguousarray(a)).cuda()


def host(t: torch.Tensor) -> np.ndarray:
    torch.cuda.synchronize()
    return t.cpu().numpy()


def case(msg: str) -> None:
    """Name the case before a GPU step so that a crash log says what ran."""
    print(f"[gpu-case] {msg}", file=sys.stderr, flush=True)
