"""GPU parity of the bf16 decode and token-partitioned prefill routes for the
other head shapes the kernels are built for: head_dim 256 and 512, GQA 1 and
2, and head_dim 512 with GQA 8 (attention_shape_supported).  Both merge
kernels are reached: a unit of 32 or more splits takes merge_staged_kernel
(more than 128 splits: several staging rounds), fewer take merge_kernel.  Outputs
are within 1e-2 max-abs of the oracle (one bf16 spacing where |x| >= 2)."""
import numpy as np
import pytest

import oracle
from inferno_amd import attention as A
from inferno_amd.kv import FULL, SLIDING, AttentionPlan, KVRunTable
from tests.gpu_util import announce, empty_dev, from_dev, to_dev
from tests.helpers import (PAGE_LEN, assert_bar, compare_bf16, make_decode_case,
                           make_prefill_case, seeded_bf16)

pytestmark = pytest.mark.gpu

SHAPES = [(16, 8, 512), (8, 8, 256), (8, 8, 512), (4, 4, 256), (16, 2, 512)]


def _table(runs, rows) -> KVRunTable:
    t = KVRunTable()
    for r in runs:
        t.begin_run(int(r[0]), int(r[1]))
        for j in range(int(r[3])):
            t.add_base_row(int(rows[int(r[2]) + j]))
    return t


def _check(kind, runs, rows, cache_rows, seq_len, shape, cap, seed, window=0,
           cache_size=PAGE_LEN):
    nq, nkv, d = shape
    kvs = nkv * d
    q = seeded_bf16(seq_len * nq * d, seed)
    k = seeded_bf16(cache_rows * kvs, seed + 1)
    v = seeded_bf16(cache_rows * kvs, seed + 2)
    plan = AttentionPlan(_table(runs, rows), seq_len, kind=kind, window=window,
                         cache_size=cache_size, page_len=PAGE_LEN, cache_rows=cache_rows,
                         cap=cap, kv_row_bytes=kvs * 2)
    out = empty_dev(seq_len * nq * d, np.uint16)
    partials, ps = A.partials_buffer(plan, nq, d)
    A.attention_bf16(plan, to_dev(q), to_dev(k), to_dev(v), out, partials, ps, num_q=nq,
                     num_kv=nkv, head_dim=d, kv_stride=kvs)
    got = from_dev(out, np.uint16)
    ref = oracle.attention(kind, runs, rows, q, k, v, num_q=nq, num_kv=nkv, head_dim=d,
                           kv_stride=kvs, window=window, cache_size=cache_size,
                           page_len=PAGE_LEN, seq_len=seq_len, cap=cap, threads=8)
    assert_bar(compare_bf16(got, ref),
               f"mode={plan.summary.mode} stripes={plan.summary.num_stripes}")


@pytest.mark.parametrize("shape", SHAPES)
@pytest.mark.parametrize("cap", [16, 256, 1024, 4096])
def test_batched_decode_shapes(shape, cap):
    """cap is the worker count of the split plan: 16 workers over 5
    sequences give 1-5 splits a unit (merge_kernel), 256 about 50 and 1024
    about 115 (merge_staged_kernel, one staging round), 4096 up to one
    split per 16-position tile (several rounds)."""
    announce(f"decode shape={shape} cap={cap}")
    rng = np.random.default_rng(sum(shape) + cap)
    ctx = [int(x) for x in rng.integers(700, 3000, 5)]
    case = make_decode_case(31 + cap, ctx)
    _check(FULL, case.runs, case.base_rows, case.cache_rows, len(ctx), shape, cap,
           seed=40 + cap)


@pytest.mark.parametrize("shape", SHAPES)
def test_sliding_decode_shapes(shape):
    """Window 300 over 8-page rings: positions wrap onto the run's pages."""
    announce(f"sliding shape={shape}")
    rng = np.random.default_rng(5)
    B, ring = 4, 8
    pos = [int(x) for x in rng.integers(0, 2000, B)]
    perm = rng.permutation(B * ring)
    runs, rows = [], []
    for i in range(B):
        runs.append([i, pos[i], len(rows), ring])
        rows.extend(int(p) * PAGE_LEN for p in perm[i * ring:(i + 1) * ring])
    _check(SLIDING, np.asarray(runs, dtype=np.int32), np.asarray(rows, dtype=np.int32),
           B * ring * PAGE_LEN, B, shape, cap=3, seed=60, window=300,
           cache_size=ring * PAGE_LEN)


@pytest.mark.parametrize("shape", SHAPES)
def test_token_prefill_shapes(shape):
    """A prefill chunk of these shapes takes the token-partitioned route
    (the MFMA kernel covers head_dim 256 with GQA 2)."""
    announce(f"token prefill shape={shape}")
    case = make_prefill_case(9, [0, 300], [20, 45])
    n = 65
    _check(FULL, case.runs, case.base_rows, case.cache_rows, n, shape, cap=16, seed=80)
