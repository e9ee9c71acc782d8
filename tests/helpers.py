"""Scenario builders and comparisons shared by the tests (host side only)."""
from __future__ import annotations

from dataclasses import dataclass, field

import numpy as np

NUM_Q, NUM_KV, HEAD_DIM, PAGE_LEN = 16, 8, 256, 64
KV_STRIDE = NUM_KV * HEAD_DIM


def bf16_to_f32(b) -> np.ndarray:
    return (np.asarray(b, dtype=np.uint16).astype(np.uint32) << 16).view(np.float32)


def bf16_ulp(x: np.ndarray) -> np.ndarray:
    """Spacing of bf16 values at |x| (8 significant bits)."""
    ax = np.abs(x.astype(np.float64))
    e = np.floor(np.log2(np.maximum(ax, 2.0 ** -126)))
    return 2.0 ** (e - 7)


def compare_bf16(got_bits, ref_bits, tol: float = 1e-2) -> dict:
    """Max-abs comparison of bf16 outputs.  The bar is `tol` absolute; where
    the reference value's bf16 spacing exceeds tol (|x| >= 2), one spacing is
    allowed so that two f32 results a hair apart may round to neighbouring
    bf16 values."""
    a = bf16_to_f32(got_bits).astype(np.float64)
    b = bf16_to_f32(ref_bits).astype(np.float64)
    d = np.abs(a - b)
    allowed = np.maximum(tol, bf16_ulp(b))
    return {
        "max_abs": float(d.max()) if d.size else 0.0,
        "n_over_tol": int((d > tol).sum()),
        "n_fail": int((d > allowed).sum()),
        "n_nan": int(np.isnan(a).sum()),
        "n": int(d.size),
    }


# How many outputs may sit beyond 1e-2 (each within one bf16 spacing, so only
# where |x| >= 2).  A kernel whose f32 result is not the reference's bit for
# bit (MFMA sums in the matrix core's order, P in bf16 parts, the fused-FMA
# exp) lands on the neighbouring bf16 value when the two f32 results straddle
# a rounding boundary; the MFMA prefill tests measured up to about 1e-5 of
# their outputs doing so.  The cap is twice that plus a fixed margin of 8 for
# the small cases, so a change that moves many outputs by one spacing fails.
OVER_TOL_FIXED = 8
OVER_TOL_FRAC = 2e-5


def over_tol_cap(n: int) -> int:
    return OVER_TOL_FIXED + int(OVER_TOL_FRAC * n)


# Every assert_bar call of the session, printed as a table at its end (the
# test run's log then shows each comparison's count beyond 1e-2 and its cap).
BAR_LOG: list = []


def assert_bar(r: dict, label: str = "", strict: bool = False) -> dict:
    """Print the comparison and hold it to the bar: no NaN, every output within
    1e-2 or one bf16 spacing, and at most over_tol_cap(n) outputs beyond 1e-2
    (none when strict)."""
    import os

    cap = 0 if strict else over_tol_cap(r["n"])
    test = os.environ.get("PYTEST_CURRENT_TEST", "").split(" ")[0]
    BAR_LOG.append((test, label, r["n_over_tol"], cap, r["n"], r["max_abs"], r["n_fail"]))
    print(f"  {label}: n_over_tol={r['n_over_tol']} (cap {cap}) of {r['n']}, "
          f"max_abs={r['max_abs']:.6g}, n_fail={r['n_fail']}", flush=True)
    assert r["n_nan"] == 0 and r["n_fail"] == 0, (label, r)
    assert r["n_over_tol"] <= cap, (label, r, cap)
    return r


@dataclass
class PagedCase:
    """A paged KV cache with per-sequence page lists and one query token per
    sequence at position ctx[i] (the appended token)."""
    ctx: np.ndarray                 # cached tokens before the append, per seq
    pages: list                     # page ids per seq
    pool_pages: int
    page_len: int = PAGE_LEN
    runs: np.ndarray = field(default=None)
    base_rows: np.ndarray = field(default=None)

    @property
    def cache_rows(self) -> int:
        return self.pool_pages * self.page_len

    @property
    def seq_len(self) -> int:
        return int(self.runs.shape[0])


def make_decode_case(seed: int, ctx_list, page_len: int = PAGE_LEN,
                     extra_pages: int = 0) -> PagedCase:
    """Decode batch: sequence i holds ctx_list[i] tokens and appends one at
    position ctx_list[i]; its pages come from a seeded permutation of a shared
    pool (Fisher-Yates via numpy's PCG64)."""
    rng = np.random.default_rng(seed)
    ctx = np.asarray(ctx_list, dtype=np.int64)
    need = [(int(c) + 1 + page_len - 1) // page_len for c in ctx]
    pool = int(sum(need)) + extra_pages
    perm = rng.permutation(pool)
    pages, off = [], 0
    for n in need:
        pages.append([int(p) for p in perm[off:off + n]])
        off += n
    runs, rows = [], []
    for i, c in enumerate(ctx):
        runs.append([i, int(c), len(rows), len(pages[i])])
        rows.extend(p * page_len for p in pages[i])
    case = PagedCase(ctx=ctx, pages=pages, pool_pages=pool, page_len=page_len)
    case.runs = np.asarray(runs, dtype=np.int32)
    case.base_rows = np.asarray(rows, dtype=np.int32)
    return case


def make_prefill_case(seed: int, prefix_list, new_list, page_len: int = PAGE_LEN,
                      fixed_pages: int | None = None) -> PagedCase:
    """Prefill chunk: sequence i has prefix_list[i] cached tokens and appends
    new_list[i] tokens; runs are laid out back to back in the token buffer."""
    rng = np.random.default_rng(seed)
    pre = np.asarray(prefix_list, dtype=np.int64)
    new = np.asarray(new_list, dtype=np.int64)
    if fixed_pages is None:
        need = [(int(p + n) + page_len - 1) // page_len for p, n in zip(pre, new)]
    else:
        need = [fixed_pages] * len(pre)
    pool = int(sum(need))
    perm = rng.permutation(pool)
    pages, off = [], 0
    for n in need:
        pages.append([int(p) for p in perm[off:off + n]])
        off += n
    runs, rows, buf = [], [], 0
    for i in range(len(pre)):
        runs.append([buf, int(pre[i]), len(rows), len(pages[i])])
        rows.extend(p * page_len for p in pages[i])
        buf += int(new[i])
    case = PagedCase(ctx=pre, pages=pages, pool_pages=pool, page_len=page_len)
    case.runs = np.asarray(runs, dtype=np.int32)
    case.base_rows = np.asarray(rows, dtype=np.int32)
    return case


def seeded_bf16(n: int, seed: int) -> np.ndarray:
    """N(0,1) as bf16 bits from numpy (test inputs; not the device generator)."""
    rng = np.random.default_rng(seed)
    f = rng.standard_normal(n).astype(np.float32)
    u = f.view(np.uint32).astype(np.uint64)
    return ((u + ((u >> 16) & 1) + 0x7FFF) >> 16).astype(np.uint16)
