"""GPU parity at Gemma-4's production page geometry: 1024-token pages
(PAGE_LEN = SLIDING_WINDOW, modeling/gemma4_topology.mojo:36) with 2-page
sliding rings (SLIDING_RING_PAGES, :40), for both layer shapes.

- append bit-exact (positions cross page boundaries and ring wraps);
- bf16 decode (batched, full attention; sliding window 1024 on 2-page rings),
  the token-partitioned prefill (sliding) and the MFMA prefill (full, head_dim
  256): within 1e-2 of the oracle (one bf16 spacing where |x| >= 2);
- bq prep and decode bit-exact."""
import numpy as np
import pytest

import oracle
from inferno_amd import attention as A
from inferno_amd.kv import FULL, SLIDING, AttentionPlan, KVRunTable
from tests.gpu_util import announce, empty_dev, from_dev, to_dev
from tests.helpers import assert_bar, compare_bf16, make_decode_case, make_prefill_case, seeded_bf16

pytestmark = pytest.mark.gpu

PAGE = 1024
RING = 2
WINDOW = 1024
SHAPES = {"sliding": (16, 8, 256, 128, 128), "full": (16, 2, 512, 64, 256)}


def _table(runs, rows) -> KVRunTable:
    t = KVRunTable()
    for r in runs:
        t.begin_run(int(r[0]), int(r[1]))
        for j in range(int(r[3])):
            t.add_base_row(int(rows[int(r[2]) + j]))
    return t


def _ring_case(seed, pos_list, new=1):
    """Sequences on 2-page rings of a shared pool; sequence i attends at
    positions pos_i .. pos_i + new - 1 (tokens laid out back to back)."""
    rng = np.random.default_rng(seed)
    B = len(pos_list)
    perm = rng.permutation(B * RING)
    runs, rows = [], []
    for i, p in enumerate(pos_list):
        runs.append([i * new, p, len(rows), RING])
        rows.extend(int(x) * PAGE for x in perm[i * RING:(i + 1) * RING])
    return np.asarray(runs, np.int32), np.asarray(rows, np.int32), B * RING * PAGE


def _attend(kind, runs, rows, cache_rows, seq_len, shape, cap, seed):
    nq, nkv, d, half, pair = shape
    kvs = nkv * d
    q = seeded_bf16(seq_len * nq * d, seed)
    k = seeded_bf16(cache_rows * kvs, seed + 1)
    v = seeded_bf16(cache_rows * kvs, seed + 2)
    cache_size = RING * PAGE if kind == SLIDING else PAGE
    plan = AttentionPlan(_table(runs, rows), seq_len, kind=kind, window=WINDOW,
                         cache_size=cache_size, page_len=PAGE, cache_rows=cache_rows, cap=cap,
                         kv_row_bytes=kvs * 2)
    out = empty_dev(seq_len * nq * d, np.uint16)
    partials, ps = A.partials_buffer(plan, nq, d)
    A.attention_bf16(plan, to_dev(q), to_dev(k), to_dev(v), out, partials, ps, num_q=nq,
                     num_kv=nkv, head_dim=d, kv_stride=kvs)
    got = from_dev(out, np.uint16)
    ref = oracle.attention(kind, runs, rows, q, k, v, num_q=nq, num_kv=nkv, head_dim=d,
                           kv_stride=kvs, window=WINDOW, cache_size=cache_size, page_len=PAGE,
                           seq_len=seq_len, cap=cap, threads=16)
    assert_bar(compare_bf16(got, ref), f"mode={plan.summary.mode} "
               f"items={plan.summary.num_items} qblocks={int(plan.info[14])}")


@pytest.mark.parametrize("layer", ["sliding", "full"])
@pytest.mark.parametrize("cap", [16, 512])
def test_page1024_full_decode(layer, cap):
    announce(f"page 1024 full decode {layer} cap={cap}")
    rng = np.random.default_rng(cap)
    ctx = [int(x) for x in rng.integers(1, 9000, 7)] + [1023, 1024]
    case = make_decode_case(5 + cap, ctx, page_len=PAGE)
    _attend(FULL, case.runs, case.base_rows, case.cache_rows, len(ctx), SHAPES[layer], cap,
            60 + cap)


@pytest.mark.parametrize("layer", ["sliding", "full"])
def test_page1024_sliding_ring_decode(layer):
    """Window 1024 over 2-page rings: positions far past the ring wrap, and
    the window straddles the two pages."""
    announce(f"page 1024 sliding ring decode {layer}")
    pos = [0, 700, 1023, 1024, 2047, 2048, 5000, 31999]
    runs, rows, cache_rows = _ring_case(3, pos)
    _attend(SLIDING, runs, rows, cache_rows, len(pos), SHAPES[layer], 64, 70)


def test_page1024_sliding_prefill():
    """A sliding prefill chunk over 2-page rings (the MFMA sliding prefill)."""
    announce("page 1024 sliding prefill")
    runs, rows, cache_rows = _ring_case(4, [0, 1500, 6000], new=40)
    _attend(SLIDING, runs, rows, cache_rows, 120, SHAPES["sliding"], 16, 80)


def test_page1024_mfma_prefill():
    """A full-attention prefill chunk at head_dim 256 / GQA 2 on 1024-token
    pages: the MFMA prefill kernel."""
    announce("page 1024 mfma prefill")
    case = make_prefill_case(6, [0, 1100, 3000], [96, 64, 130], page_len=PAGE)
    _attend(FULL, case.runs, case.base_rows, case.cache_rows, 290, SHAPES["sliding"], 16, 90)


@pytest.mark.parametrize("layer", ["sliding", "full"])
def test_page1024_append(layer):
    """rope_cache_write bit-exact on 2-page rings, around page and ring
    boundaries."""
    announce(f"page 1024 append {layer}")
    nq, nkv, d, half, pair = SHAPES[layer]
    kvs = nkv * d
    pos = [0, 1023, 1024, 2047, 2048, 3071, 9000]
    runs, rows, cache_rows = _ring_case(8, pos)
    n = len(pos)
    rng = np.random.default_rng(9)
    ang = rng.uniform(-3, 3, (max(pos) + 2) * half)
    cos, sin = np.cos(ang).astype(np.float32), np.sin(ang).astype(np.float32)
    q = seeded_bf16(n * nq * d, 10)
    ks, vs = seeded_bf16(n * kvs, 11), seeded_bf16(n * kvs, 12)
    kc, vc = seeded_bf16(cache_rows * kvs, 13), seeded_bf16(cache_rows * kvs, 14)
    plan = AttentionPlan(_table(runs, rows), n, kind=SLIDING, window=WINDOW,
                         cache_size=RING * PAGE, page_len=PAGE, cache_rows=cache_rows, cap=16,
                         kv_row_bytes=kvs * 2)
    dq, dk, dv = to_dev(q), to_dev(kc), to_dev(vc)
    A.dispatch_rope_cache_write(plan, dq, to_dev(ks), to_dev(vs), dk, dv, to_dev(cos),
                                to_dev(sin), num_q=nq, num_kv=nkv, half=half, pair_stride=pair,
                                head_dim=d)
    oracle.rope_cache_write(runs, rows, q, ks, vs, kc, vc, cos, sin, num_q=nq, num_kv=nkv,
                            page_shift=10, row_mask=PAGE - 1, page_mask=RING - 1, seq_len=n,
                            half=half, pair_stride=pair, head_dim=d)
    assert np.array_equal(from_dev(dq, np.uint16), q)
    assert np.array_equal(from_dev(dk, np.uint16), kc)
    assert np.array_equal(from_dev(dv, np.uint16), vc)


@pytest.mark.parametrize("layer", ["sliding", "full"])
def test_page1024_bq_prefill_then_decode(layer):
    """bq on 1024-token pages: a prefill chunk quantises every position of
    each sequence's pages (codes bit-exact), then a decode step attends
    (outputs bit-exact); full attention over growing page lists."""
    announce(f"page 1024 bq {layer}")
    nq, nkv, d, half, pair = SHAPES[layer]
    kvs = nkv * d
    rng = np.random.default_rng(21)
    ctx = [int(x) for x in rng.integers(900, 3500, 4)]
    case = make_decode_case(22, ctx, page_len=PAGE)
    cos = np.cos(rng.uniform(-3, 3, (max(ctx) + 2) * half)).astype(np.float32)
    sin = np.sin(rng.uniform(-3, 3, (max(ctx) + 2) * half)).astype(np.float32)
    g = oracle.f32_to_bf16(rng.uniform(0.5, 1.5, d).astype(np.float32))
    rows_n = case.cache_rows
    k = np.zeros(rows_n * kvs, np.int8)
    v = np.zeros_like(k)
    ksc = np.zeros(rows_n * nkv, np.float32)
    vsc = np.zeros_like(ksc)
    dk, dv, dks, dvs = to_dev(k), to_dev(v), to_dev(ksc), to_dev(vsc)
    sqrt_n = float(np.sqrt(np.float32(d)))
    n_eps = float(np.float32(d) * np.float32(1e-6))

    def prep(runs, rows, n, seed):
        q = seeded_bf16(n * nq * d, seed)
        ks, vs = seeded_bf16(n * kvs, seed + 1), seeded_bf16(n * kvs, seed + 2)
        plan = AttentionPlan(_table(runs, rows), n, kind=FULL, window=0, cache_size=PAGE,
                             page_len=PAGE, cache_rows=rows_n, cap=32, kv_row_bytes=kvs)
        dq_i8 = empty_dev(n * nq * d, np.int8)
        dqb, dfq = empty_dev(n * nq, np.float32), empty_dev(n * nq, np.float32)
        A.dispatch_bq_attn_prep(plan, to_dev(q), to_dev(ks), to_dev(vs), to_dev(g), to_dev(g),
                                dq_i8, dqb, dfq, dk, dks, dv, dvs, to_dev(cos), to_dev(sin),
                                num_q=nq, num_kv=nkv, head_dim=d, rope_half=half,
                                pair_stride=pair, sqrt_n=sqrt_n, n_eps=n_eps)
        q_i8 = np.zeros(n * nq * d, np.int8)
        qb, fq = np.zeros(n * nq, np.float32), np.zeros(n * nq, np.float32)
        oracle.bq_attn_prep(runs, rows, q, ks, vs, g, g, q_i8, qb, fq, k, ksc, v, vsc, cos, sin,
                            num_q=nq, num_kv=nkv, page_shift=10, row_mask=PAGE - 1,
                            page_mask=-1, seq_len=n, head_dim=d, rope_half=half,
                            pair_stride=pair, sqrt_n=sqrt_n, n_eps=n_eps)
        assert np.array_equal(from_dev(dq_i8, np.int8), q_i8)
        for dev, host in ((dk, k), (dv, v)):
            assert np.array_equal(from_dev(dev, np.int8), host)
        for dev, host in ((dks, ksc), (dvs, vsc)):
            assert np.array_equal(from_dev(dev, np.float32).view(np.uint32), host.view(np.uint32))
        return plan, dq_i8, dqb, dfq, q_i8, qb, fq

    fill_runs, buf = [], 0
    for i, c in enumerate(ctx):
        fill_runs.append([buf, 0, int(case.runs[i][2]), int(case.runs[i][3])])
        buf += c
    prep(np.asarray(fill_runs, np.int32), case.base_rows, buf, 30)
    plan, dq_i8, dqb, dfq, q_i8, qb, fq = prep(case.runs, case.base_rows, len(ctx), 40)
    out = empty_dev(len(ctx) * nq * d, np.uint16)
    partials, ps = A.partials_buffer(plan, nq, d)
    A.bq_attention(plan, dq_i8, dqb, dfq, dk, dks, dv, dvs, out, partials, ps, num_q=nq,
                   num_kv=nkv, head_dim=d, kv_stride=kvs)
    ref = oracle.bq_attention(FULL, case.runs, case.base_rows, q_i8, qb, fq, k, ksc, v, vsc,
                              num_q=nq, num_kv=nkv, head_dim=d, kv_stride=kvs, window=0,
                              cache_size=PAGE, page_len=PAGE, seq_len=len(ctx), cap=32,
                              threads=16)
    got = from_dev(out, np.uint16)
    assert np.array_equal(got, ref), compare_bf16(got, ref)
