"""GPU parity of the butterquant MFMA prefill -- sliding windows at head_dim
256 / GQA 2 (BqFlashPrefillSlidingKernel, butterquant_kernels/attention.mojo:
170-264) and full attention (BqFlashPrefillFullKernel, :267-351) at head_dim
256 / GQA 2 and at Gemma-4's full-layer shape, head_dim 512 / GQA 8 --
against the oracle's bq token
route: int8 K/V codes with f32 scales per row
and kv head, int8 queries with their bias (128 * sum q) and f_q.  The scores
come from an int8 MFMA and are formed in the reference's order, so they
equal the oracle's; the outputs are held to 1e-2 (one bf16 spacing where
|x| >= 2), the bar of the bf16 MFMA prefill.  The o_proj block quant of the
output (its own pass on this route) is bit-exact against the oracle's
quant of the GPU output."""
import numpy as np
import pytest

import oracle
from inferno_amd import attention as A
from inferno_amd.kv import FULL, SLIDING, AttentionPlan, KVRunTable
from tests.gpu_util import announce, empty_dev, from_dev, to_dev
from tests.helpers import assert_bar, compare_bf16, make_prefill_case

pytestmark = pytest.mark.gpu

NQ, NKV, D = 16, 8, 256
KVS = NKV * D
WNQ, WNKV, WD = 16, 2, 512


def _table(runs, rows) -> KVRunTable:
    t = KVRunTable()
    for r in runs:
        t.begin_run(int(r[0]), int(r[1]))
        for j in range(int(r[3])):
            t.add_base_row(int(rows[int(r[2]) + j]))
    return t


def _ring_case(seed, prefix, new, ring_pages, page_len):
    rng = np.random.default_rng(seed)
    perm = rng.permutation(len(prefix) * ring_pages)
    runs, rows, buf = [], [], 0
    for i in range(len(prefix)):
        runs.append([buf, prefix[i], len(rows), ring_pages])
        rows.extend(int(x) * page_len for x in perm[i * ring_pages:(i + 1) * ring_pages])
        buf += new[i]
    return np.asarray(runs, np.int32), np.asarray(rows, np.int32), len(prefix) * ring_pages * page_len


def _codes(n, seed, outliers=False):
    """Uniform int8 codes in [-127, 127]; with outliers, 1 % of them at
    +-127 in runs of one row."""
    rng = np.random.default_rng(seed)
    c = rng.integers(-127, 128, n).astype(np.int8)
    if outliers:
        idx = rng.random(n) < 0.01
        c[idx] = np.where(rng.random(int(idx.sum())) < 0.5, -127, 127).astype(np.int8)
    return c


def _run(window, prefix, new, ring, page_len, seed, q_scale=1.0, quant=False):
    runs, rows, cache_rows = _ring_case(seed, prefix, new, ring, page_len)
    n = sum(new)
    rng = np.random.default_rng(seed + 1)
    q = _codes(n * NQ * D, seed + 2)
    qb = (128.0 * q.reshape(n * NQ, D).astype(np.int64).sum(axis=1)).astype(np.float32)
    # Scores (raw - qb) * fq * ks / 127^2 with a spread of a few units.
    fq = (rng.uniform(0.5, 1.5, n * NQ) * q_scale).astype(np.float32)
    k = _codes(cache_rows * KVS, seed + 3, outliers=True)
    v = _codes(cache_rows * KVS, seed + 4)
    ks = rng.uniform(0.5, 1.5, cache_rows * NKV).astype(np.float32)
    vs = rng.uniform(0.5, 2.0, cache_rows * NKV).astype(np.float32)
    plan = AttentionPlan(_table(runs, rows), n, kind=SLIDING, window=window,
                         cache_size=ring * page_len, page_len=page_len, cache_rows=cache_rows,
                         cap=16, kv_row_bytes=KVS)
    assert plan.summary.mode == 1 and int(plan.info[14]) > 0, "not on the MFMA route"
    out = empty_dev(n * NQ * D, np.uint16)
    partials, ps = A.partials_buffer(plan, NQ, D)
    args = (plan, to_dev(q), to_dev(qb), to_dev(fq), to_dev(k), to_dev(ks), to_dev(v),
            to_dev(vs))
    kw = dict(num_q=NQ, num_kv=NKV, head_dim=D, kv_stride=KVS)
    A.bq_attention(*args, out, partials, ps, **kw)
    got = from_dev(out, np.uint16)
    if quant:
        out2 = empty_dev(n * NQ * D, np.uint16)
        o_i8 = empty_dev(n * NQ * D, np.int8)
        o_sa = empty_dev(n * NQ, np.float32)
        A.bq_attention(*args, out2, partials, ps, **kw, o_i8=o_i8, o_sa=o_sa)
        assert np.array_equal(from_dev(out2, np.uint16), got), "quant changed the output"
        want_i8, want_sa = oracle.bq_block_quant(got, cols=NQ * D, block=D)
        assert np.array_equal(from_dev(o_i8, np.int8).reshape(n, NQ * D), want_i8)
        assert np.array_equal(from_dev(o_sa, np.float32).view(np.uint32),
                              want_sa.reshape(-1).view(np.uint32))
    ref = oracle.bq_attention(SLIDING, runs, rows, q, qb, fq, k, ks, v, vs, num_q=NQ,
                              num_kv=NKV, head_dim=D, kv_stride=KVS, window=window,
                              cache_size=ring * page_len, page_len=page_len, seq_len=n,
                              cap=16, threads=16)
    return compare_bf16(got, ref)


@pytest.mark.parametrize("window", [16, 48, 64, 1024, 1, 17, 100, 1023])
def test_bq_sliding_prefill_windows(window):
    """Chunks from position 0, inside the first window and far past it; full
    and partial query blocks."""
    announce(f"bq mfma sliding prefill window={window}")
    prefix, new = [0, 5, max(0, window - 3), 700, 3000], [100, 64, 129, 77, 200]
    ring = 1 << int(np.ceil(np.log2((window + max(new) + 128) / 64)))
    r = _run(window, prefix, new, ring, 64, window, quant=window == 1024)
    assert_bar(r, f"window {window}")


def test_bq_sliding_prefill_diffuse():
    """f_q scaled by 1/16: attention spreads over the window."""
    announce("bq mfma sliding prefill diffuse")
    r = _run(1024, [0, 1500, 4000], [130, 64, 190], 32, 64, 7, q_scale=1.0 / 16)
    assert_bar(r, "diffuse")


@pytest.mark.parametrize("page_len,ring", [(8, 512), (1024, 2)])
def test_bq_sliding_prefill_page_sizes(page_len, ring):
    """8-row pages and Gemma-4's 1024-token pages on 2-page rings."""
    announce(f"bq mfma sliding prefill page_len={page_len}")
    r = _run(1024, [0, 900, 2500], [96, 129, 64], ring, page_len, 11)
    assert_bar(r, f"page_len {page_len}")


def _run_full(prefix, new, page_len, seed, quant=False, shape=(WNQ, WNKV, WD)):
    """Full attention over page lists (no ring): by default at head_dim 512 /
    GQA 8, or at the shape given (head_dim 256 / GQA 2)."""
    WNQ, WNKV, WD = shape
    case = make_prefill_case(seed, prefix, new, page_len=page_len)
    runs, rows, cache_rows = case.runs, case.base_rows, case.cache_rows
    kvs = WNKV * WD
    n = sum(new)
    rng = np.random.default_rng(seed + 1)
    q = _codes(n * WNQ * WD, seed + 2)
    qb = (128.0 * q.reshape(n * WNQ, WD).astype(np.int64).sum(axis=1)).astype(np.float32)
    # A 512-dim dot has sqrt(2) times the spread of a 256-dim one.
    fq = (rng.uniform(0.35, 1.05, n * WNQ) * np.sqrt(512 / WD)).astype(np.float32)
    k = _codes(cache_rows * kvs, seed + 3, outliers=True)
    v = _codes(cache_rows * kvs, seed + 4)
    ks = rng.uniform(0.5, 1.5, cache_rows * WNKV).astype(np.float32)
    vs = rng.uniform(0.5, 2.0, cache_rows * WNKV).astype(np.float32)
    plan = AttentionPlan(_table(runs, rows), n, kind=FULL, window=0, cache_size=page_len,
                         page_len=page_len, cache_rows=cache_rows, cap=16, kv_row_bytes=kvs)
    assert plan.summary.mode == 2 and int(plan.info[14]) > 0, "no query blocks"
    out = empty_dev(n * WNQ * WD, np.uint16)
    partials, ps = A.partials_buffer(plan, WNQ, WD)
    args = (plan, to_dev(q), to_dev(qb), to_dev(fq), to_dev(k), to_dev(ks), to_dev(v),
            to_dev(vs))
    kw = dict(num_q=WNQ, num_kv=WNKV, head_dim=WD, kv_stride=kvs)
    A.bq_attention(*args, out, partials, ps, **kw)
    got = from_dev(out, np.uint16)
    if quant:
        out2 = empty_dev(n * WNQ * WD, np.uint16)
        o_i8 = empty_dev(n * WNQ * WD, np.int8)
        o_sa = empty_dev(n * WNQ, np.float32)
        A.bq_attention(*args, out2, partials, ps, **kw, o_i8=o_i8, o_sa=o_sa)
        assert np.array_equal(from_dev(out2, np.uint16), got), "quant changed the output"
        want_i8, want_sa = oracle.bq_block_quant(got, cols=WNQ * WD, block=WD)
        assert np.array_equal(from_dev(o_i8, np.int8).reshape(n, WNQ * WD), want_i8)
        assert np.array_equal(from_dev(o_sa, np.float32).view(np.uint32),
                              want_sa.reshape(-1).view(np.uint32))
    ref = oracle.bq_attention(FULL, runs, rows, q, qb, fq, k, ks, v, vs, num_q=WNQ,
                              num_kv=WNKV, head_dim=WD, kv_stride=kvs, window=0,
                              cache_size=page_len, page_len=page_len, seq_len=n, cap=16,
                              threads=16)
    return compare_bf16(got, ref)


def test_bq_full_layer_prefill():
    """Chunks from position 0, short and long prefixes, blocks of 1-8 live
    tokens (pairs without live rows), a one-token chunk; the o_proj block
    quant on top."""
    announce("bq mfma full-layer prefill")
    r = _run_full([0, 100, 1000, 3000, 63, 5], [40, 33, 100, 64, 1, 7], 64, 21, quant=True)
    assert_bar(r, "full layer")


@pytest.mark.parametrize("page_len", [8, 1024])
def test_bq_full_layer_prefill_page_sizes(page_len):
    announce(f"bq mfma full-layer prefill page_len={page_len}")
    r = _run_full([0, 900, 2500], [96, 129, 64], page_len, 23)
    assert_bar(r, f"full layer page_len {page_len}")


@pytest.mark.parametrize("nkv", [1, 3])
def test_bq_full_layer_prefill_kv_head_counts(nkv):
    """8 and 24 q heads at head_dim 512 / GQA 8: both of the kernel's block
    placements over the XCDs (the kv head count divides 8, or not)."""
    announce(f"bq mfma full-layer prefill num_kv={nkv}")
    r = _run_full([0, 300, 1500, 70], [70, 129, 64, 9], 64, 41 + nkv, shape=(8 * nkv, nkv, WD))
    assert_bar(r, f"full layer num_kv {nkv}")


def test_bq_full_attention_prefill_hd256():
    """Full attention at 16 q / 8 kv x 256 on the int8 MFMA route: chunks from
    position 0, short and long prefixes, partial query blocks, a one-token
    chunk; the o_proj block quant on top."""
    announce("bq mfma full-attention prefill hd256")
    r = _run_full([0, 100, 1000, 3000, 63, 5], [40, 33, 100, 64, 1, 7], 64, 31, quant=True,
                  shape=(NQ, NKV, D))
    assert_bar(r, "full attention hd256")


@pytest.mark.parametrize("page_len", [8, 1024])
def test_bq_full_attention_prefill_hd256_page_sizes(page_len):
    """Pages of 8 rows (the per-row staging) and of 1,024."""
    announce(f"bq mfma full-attention prefill hd256 page_len={page_len}")
    r = _run_full([0, 900, 2500], [96, 129, 64], page_len, 33, shape=(NQ, NKV, D))
    assert_bar(r, f"full attention hd256 page_len {page_len}")


def test_bq_full_attention_prefill_hd256_long_run():
    """A run of 40,000 cached positions in pages of 8 rows (5,000 pages) moves
    the kernel's 4,096-entry page-table window once."""
    announce("bq mfma full-attention prefill hd256 long run")
    r = _run_full([40000, 50], [70, 30], 8, 35, shape=(NQ, NKV, D))
    assert_bar(r, "full attention hd256 long run")
