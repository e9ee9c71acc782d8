"""Host-side run tables and plans for the paged-KV path.

KVRunTable mirrors the reference's run table (kernels/attention_ops.mojo:54-89)
and AttentionPlan wraps ifr_plan_attention: the host half of the reference's
dispatcher (routing + plan_run_splits) producing the plan image the kernels
read.  Device memory comes from torch; torch is plumbing here, the compute is
in libinferno_hip.so.
"""
from __future__ import annotations

import ctypes as C
from dataclasses import dataclass

import numpy as np

from ._lib import INFO_LEN, P_I32, P_I64, check, lib

SLIDING, FULL = 0, 1


class KVRunTable:
    """KVRunTable (kernels/attention_ops.mojo:62-89): runs of
    {buf_start, base_pos, rows_off, page_count} and their page base rows."""

    def __init__(self) -> None:
        self.runs: list[list[int]] = []
        self.base_rows: list[int] = []

    def clear(self) -> None:
        self.runs.clear()
        self.base_rows.clear()

    def begin_run(self, buf_start: int, base_pos: int) -> None:
        self.runs.append([int(buf_start), int(base_pos), len(self.base_rows), 0])

    def add_base_row(self, row: int) -> None:
        self.base_rows.append(int(row))
        self.runs[-1][3] += 1

    def arrays(self) -> tuple[np.ndarray, np.ndarray]:
        runs = np.asarray(self.runs, dtype=np.int32).reshape(-1, 4)
        rows = np.asarray(self.base_rows if self.base_rows else [0], dtype=np.int32)
        return np.ascontiguousarray(runs), np.ascontiguousarray(rows)

    @property
    def num_runs(self) -> int:
        return len(self.runs)


def flash_partial_stride(num_q: int, head_dim: int) -> int:
    """flash_partial_stride (kernels/attention_ops.mojo:140-142)."""
    return int(lib().ifr_flash_partial_stride(num_q, head_dim))


def pow2_shift(value: int) -> int:
    """pow2_shift (kernels/attention_ops.mojo:32-37)."""
    s = 0
    while (1 << s) < value:
        s += 1
    return s


@dataclass
class PlanInfo:
    num_items: int
    num_units: int
    mode: int
    num_stripes: int
    image_bytes: int


class AttentionPlan:
    """A planned run table uploaded to the device.

    kind: SLIDING (window ring of cache_size positions) or FULL.
    cap: the reference's worker capacity; it fixes the split plan.
    """

    def __init__(self, table: KVRunTable, seq_len: int, *, kind: int, window: int,
                 cache_size: int, page_len: int, cache_rows: int, cap: int,
                 kv_row_bytes: int, device=None) -> None:
        import torch

        runs, rows = table.arrays()
        nbytes = int(lib().ifr_plan_bytes(runs.shape[0], rows.shape[0], seq_len, cap))
        self.host = np.zeros(max(nbytes // 4, 16), dtype=np.int32)
        self.info = (C.c_int64 * INFO_LEN)()
        check(lib().ifr_plan_attention(
            self.host.ctypes.data, self.host.nbytes,
            runs.ctypes.data_as(P_I32), runs.shape[0],
            rows.ctypes.data_as(P_I32), rows.shape[0],
            seq_len, kind, window, cache_size, page_len, cache_rows, cap,
            kv_row_bytes, self.info))
        used = int(self.info[4]) // 4
        dev = device if device is not None else torch.device("cuda")
        self.image = torch.from_numpy(self.host[:used].copy()).to(dev)
        self.kind = kind
        self.seq_len = seq_len
        self.page_len = page_len
        self.page_mask = cache_size // page_len - 1 if kind == SLIDING else -1
        self.page_shift = pow2_shift(page_len)

    @property
    def info_ptr(self):
        return C.cast(self.info, P_I64)

    @property
    def summary(self) -> PlanInfo:
        i = self.info
        return PlanInfo(int(i[0]), int(i[1]), int(i[2]), int(i[3]), int(i[4]))

    def items(self) -> np.ndarray:
        """Work items {q_row, run, start_pos, start, end, stripe} (host copy)."""
        off = int(self.host[11])
        n = int(self.info[0])
        return self.host[off:off + 8 * n].reshape(n, 8)[:, :6].copy()

    def units(self) -> np.ndarray:
        off = int(self.host[12])
        n = int(self.info[1])
        return self.host[off:off + 4 * n].reshape(n, 4)[:, :3].copy()
