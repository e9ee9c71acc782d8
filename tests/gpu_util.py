"""Device-memory helpers for the GPU tests (torch is plumbing only)."""
from __future__ import annotations

import sys

import numpy as np

_VIEW = {np.uint16: np.int16, np.uint8: np.int8}


def announce(name: str) -> None:
    print(f"[gpu case] {name}", flush=True)
    sys.stdout.flush()


def to_dev(a: np.ndarray):
    import torch

    a = np.ascontiguousarray(a)
    v = a.view(_VIEW.get(a.dtype.type, a.dtype.type))
    return torch.from_numpy(v.copy()).to("cuda")


def from_dev(t, dtype) -> np.ndarray:
    import torch

    torch.cuda.synchronize()
    return t.cpu().numpy().view(dtype).copy()


def empty_dev(n: int, dtype):
    import torch

    tmap = {np.uint16: torch.int16, np.int8: torch.int8, np.float32: torch.float32,
            np.int32: torch.int32, np.uint8: torch.uint8}
    return torch.zeros(n, dtype=tmap[np.dtype(dtype).type], device="cuda")
