"""GPU parity of the bf16 paged-KV path against the CPU oracle: KV append
(bit-exact), split-KV decode + merge on every dispatch route, sliding rings,
token-partitioned prefill, and edge cases.  Attention outputs must be within
1e-2 max-abs of the oracle (one bf16 spacing allowed where |x| >= 2, see
tests/helpers.compare_bf16)."""
import numpy as np
import pytest

import oracle
from inferno_amd import attention as A
from inferno_amd.kv import FULL, SLIDING, AttentionPlan, KVRunTable
from tests.gpu_util import announce, empty_dev, from_dev, to_dev
from tests.helpers import (HEAD_DIM, KV_STRIDE, NUM_KV, NUM_Q, PAGE_LEN, assert_bar, compare_bf16,
                           make_decode_case, make_prefill_case, seeded_bf16)

pytestmark = pytest.mark.gpu


def _table(runs, rows) -> KVRunTable:
    t = KVRunTable()
    for r in runs:
        t.begin_run(int(r[0]), int(r[1]))
        for j in range(int(r[3])):
            t.add_base_row(int(rows[int(r[2]) + j]))
    return t


def _run_attention(kind, runs, rows, q, k, v, *, seq_len, cap, window=0, cache_size=PAGE_LEN,
                   cache_rows):
    table = _table(runs, rows)
    plan = AttentionPlan(table, seq_len, kind=kind, window=window, cache_size=cache_size,
                         page_len=PAGE_LEN, cache_rows=cache_rows, cap=cap,
                         kv_row_bytes=KV_STRIDE * 2)
    qd, kd, vd = to_dev(q), to_dev(k), to_dev(v)
    out = empty_dev(seq_len * NUM_Q * HEAD_DIM, np.uint16)
    partials, ps = A.partials_buffer(plan, NUM_Q, HEAD_DIM)
    A.attention_bf16(plan, qd, kd, vd, out, partials, ps, num_q=NUM_Q, num_kv=NUM_KV,
                     head_dim=HEAD_DIM, kv_stride=KV_STRIDE)
    got = from_dev(out, np.uint16)
    ref = oracle.attention(kind, runs, rows, q, k, v, num_q=NUM_Q, num_kv=NUM_KV,
                           head_dim=HEAD_DIM, kv_stride=KV_STRIDE, window=window,
                           cache_size=cache_size, page_len=PAGE_LEN, seq_len=seq_len,
                           cap=cap, threads=8)
    return got, ref, plan


def _assert_close(got, ref, what):
    assert_bar(compare_bf16(got, ref), what)


@pytest.mark.parametrize("cap", [1, 3, 64, 96, 128, 512])
def test_config1_append_then_decode(cap):
    """Config 1: B=1, ctx 4096 in 64-token pages drawn from a seeded permutation
    of a 128-page pool; append one token (RoPE + cache write), then decode."""
    announce(f"config1 cap={cap}")
    case = make_decode_case(2024, [4096], extra_pages=128 - 65)
    rows_cache = case.cache_rows
    k = seeded_bf16(rows_cache * KV_STRIDE, 1)
    v = seeded_bf16(rows_cache * KV_STRIDE, 2)
    q_src = seeded_bf16(NUM_Q * HEAD_DIM, 3)
    k_new = seeded_bf16(KV_STRIDE, 4)
    v_new = seeded_bf16(KV_STRIDE, 5)
    rng = np.random.default_rng(6)
    ang = rng.uniform(-np.pi, np.pi, (4097 + 8) * 128)
    cos = np.cos(ang).astype(np.float32)
    sin = np.sin(ang).astype(np.float32)

    table = _table(case.runs, case.base_rows)
    plan = AttentionPlan(table, 1, kind=FULL, window=0, cache_size=PAGE_LEN,
                         page_len=PAGE_LEN, cache_rows=rows_cache, cap=cap,
                         kv_row_bytes=KV_STRIDE * 2)
    qd, kd, vd = to_dev(q_src), to_dev(k), to_dev(v)
    A.dispatch_rope_cache_write(plan, qd, to_dev(k_new), to_dev(v_new), kd, vd, to_dev(cos),
                                to_dev(sin), num_q=NUM_Q, num_kv=NUM_KV, half=128,
                                pair_stride=128, head_dim=HEAD_DIM)
    out = empty_dev(NUM_Q * HEAD_DIM, np.uint16)
    partials, ps = A.partials_buffer(plan, NUM_Q, HEAD_DIM)
    A.attention_bf16(plan, qd, kd, vd, out, partials, ps, num_q=NUM_Q, num_kv=NUM_KV,
                     head_dim=HEAD_DIM, kv_stride=KV_STRIDE)

    q_ref, k_ref, v_ref = q_src.copy(), k.copy(), v.copy()
    oracle.rope_cache_write(case.runs, case.base_rows, q_ref, k_new, v_new, k_ref, v_ref,
                            cos, sin, num_q=NUM_Q, num_kv=NUM_KV, page_shift=6, row_mask=63,
                            page_mask=-1, seq_len=1, half=128, pair_stride=128,
                            head_dim=HEAD_DIM)
    assert np.array_equal(from_dev(qd, np.uint16), q_ref), "rotated q differs"
    assert np.array_equal(from_dev(kd, np.uint16), k_ref), "k cache differs"
    assert np.array_equal(from_dev(vd, np.uint16), v_ref), "v cache differs"
    ref = oracle.attention(FULL, case.runs, case.base_rows, q_ref, k_ref, v_ref,
                           num_q=NUM_Q, num_kv=NUM_KV, head_dim=HEAD_DIM,
                           kv_stride=KV_STRIDE, window=0, cache_size=PAGE_LEN,
                           page_len=PAGE_LEN, seq_len=1, cap=cap, threads=8)
    _assert_close(from_dev(out, np.uint16), ref, f"config1 cap={cap}")


@pytest.mark.parametrize("half,pair,d,q_off", [(128, 128, 256, 0), (64, 256, 512, 0),
                                               (40, 100, 256, 0), (128, 128, 256, 1)])
def test_append_vector_and_element_paths(half, pair, d, q_off):
    """The append's 16-byte path (rope half, pair stride and head_dim
    multiples of 8 and aligned bases: both Gemma-4 layer geometries, the
    second with unrotated chunks between and after the pairs) and its element
    path (a rope half of 40 with pair stride 100; a q base 2 bytes off
    16-byte alignment), bit-exact against the oracle over 5 runs of 1-40 new
    tokens whose positions cross page boundaries."""
    import torch

    announce(f"append paths half={half} pair={pair} d={d} q_off={q_off}")
    nq, nkv = 4, 2
    kvs = nkv * d
    prefix, new = [0, 63, 100, 1000, 5], [40, 2, 29, 1, 17]
    rng = np.random.default_rng(d + half + q_off)
    n_pages = [(p + m + PAGE_LEN - 1) // PAGE_LEN for p, m in zip(prefix, new)]
    perm = rng.permutation(sum(n_pages) + 3)
    runs, rows, buf, off = [], [], 0, 0
    for p, m, np_ in zip(prefix, new, n_pages):
        runs.append([buf, p, len(rows), np_])
        rows.extend(int(x) * PAGE_LEN for x in perm[off:off + np_])
        buf, off = buf + m, off + np_
    runs, rows = np.asarray(runs, np.int32), np.asarray(rows, np.int32)
    n, cache_rows = buf, (len(perm)) * PAGE_LEN
    ang = rng.uniform(-3, 3, (max(p + m for p, m in zip(prefix, new)) + 1) * half)
    cos, sin = np.cos(ang).astype(np.float32), np.sin(ang).astype(np.float32)
    q = seeded_bf16(n * nq * d, 31)
    ks, vs = seeded_bf16(n * kvs, 32), seeded_bf16(n * kvs, 33)
    kc, vc = seeded_bf16(cache_rows * kvs, 34), seeded_bf16(cache_rows * kvs, 35)
    plan = AttentionPlan(_table(runs, rows), n, kind=FULL, window=0, cache_size=PAGE_LEN,
                         page_len=PAGE_LEN, cache_rows=cache_rows, cap=16, kv_row_bytes=kvs * 2)
    q_store = to_dev(np.concatenate([np.zeros(q_off, np.uint16), q]))
    qd = q_store[q_off:]
    kd, vd = to_dev(kc), to_dev(vc)
    A.dispatch_rope_cache_write(plan, qd, to_dev(ks), to_dev(vs), kd, vd, to_dev(cos),
                                to_dev(sin), num_q=nq, num_kv=nkv, half=half, pair_stride=pair,
                                head_dim=d)
    torch.cuda.synchronize()
    oracle.rope_cache_write(runs, rows, q, ks, vs, kc, vc, cos, sin, num_q=nq, num_kv=nkv,
                            page_shift=6, row_mask=PAGE_LEN - 1, page_mask=-1, seq_len=n,
                            half=half, pair_stride=pair, head_dim=d)
    assert np.array_equal(from_dev(qd, np.uint16), q), "rotated q"
    assert np.array_equal(from_dev(kd, np.uint16), kc), "k cache"
    assert np.array_equal(from_dev(vd, np.uint16), vc), "v cache"


@pytest.mark.parametrize("cap,ctx_seed", [(64, 0), (1024, 1), (8, 2), (4096, 3)])
def test_batched_full_decode(cap, ctx_seed):
    """Config 2 shape at reduced batch: ctx ~ U[512, 8192], shared shuffled pool."""
    announce(f"batched full cap={cap}")
    rng = np.random.default_rng(ctx_seed)
    B = 12
    ctx = [int(x) for x in rng.integers(512, 8193, B)]
    case = make_decode_case(100 + ctx_seed, ctx)
    q = seeded_bf16(B * NUM_Q * HEAD_DIM, 11 + ctx_seed)
    k = seeded_bf16(case.cache_rows * KV_STRIDE, 12 + ctx_seed)
    v = seeded_bf16(case.cache_rows * KV_STRIDE, 13 + ctx_seed)
    got, ref, plan = _run_attention(FULL, case.runs, case.base_rows, q, k, v, seq_len=B,
                                    cap=cap, cache_rows=case.cache_rows)
    _assert_close(got, ref, f"batched cap={cap} mode={plan.summary.mode}")


@pytest.mark.parametrize("cap", [2, 256])
def test_sliding_ring_decode(cap):
    """Sliding window 256 over rings of 8 pages (cache_size 512 positions):
    positions beyond the ring wrap onto the run's fixed pages."""
    announce(f"sliding ring cap={cap}")
    rng = np.random.default_rng(7)
    B, ring, window = 6, 8, 256
    pos = [int(x) for x in rng.integers(0, 3000, B)]
    pos[0] = 10
    pool = B * ring
    perm = rng.permutation(pool)
    runs, rows = [], []
    for i in range(B):
        runs.append([i, pos[i], len(rows), ring])
        rows.extend(int(p) * PAGE_LEN for p in perm[i * ring:(i + 1) * ring])
    runs = np.asarray(runs, dtype=np.int32)
    rows = np.asarray(rows, dtype=np.int32)
    q = seeded_bf16(B * NUM_Q * HEAD_DIM, 21)
    k = seeded_bf16(pool * PAGE_LEN * KV_STRIDE, 22)
    v = seeded_bf16(pool * PAGE_LEN * KV_STRIDE, 23)
    got, ref, _ = _run_attention(SLIDING, runs, rows, q, k, v, seq_len=B, cap=cap,
                                 window=window, cache_size=ring * PAGE_LEN,
                                 cache_rows=pool * PAGE_LEN)
    _assert_close(got, ref, f"sliding cap={cap}")


@pytest.mark.parametrize("kind", [FULL, SLIDING])
def test_token_partitioned_prefill(kind):
    """Multi-token runs take the token-partitioned prefill route (one item per
    query token, causal range, direct or one-segment finalisation)."""
    announce(f"prefill kind={kind}")
    if kind == FULL:
        case = make_prefill_case(9, [0, 300, 77], [40, 25, 70])
        cache_size, window = PAGE_LEN, 0
        runs, rows = case.runs, case.base_rows
        cache_rows = case.cache_rows
    else:
        case = make_prefill_case(9, [0, 300, 77], [40, 25, 70], fixed_pages=4)
        cache_size, window = 4 * PAGE_LEN, 100
        runs, rows = case.runs, case.base_rows
        cache_rows = case.cache_rows
    n = 40 + 25 + 70
    q = seeded_bf16(n * NUM_Q * HEAD_DIM, 31)
    k = seeded_bf16(cache_rows * KV_STRIDE, 32)
    v = seeded_bf16(cache_rows * KV_STRIDE, 33)
    got, ref, plan = _run_attention(kind, runs, rows, q, k, v, seq_len=n, cap=16,
                                    window=window, cache_size=cache_size,
                                    cache_rows=cache_rows)
    assert plan.summary.mode in (1, 2)
    _assert_close(got, ref, f"prefill kind={kind}")


def test_edge_cases_single_position_and_tile_boundaries():
    """ctx 0 (one position), lengths at tile and page boundaries."""
    announce("edge cases")
    ctx = [0, 15, 16, 63, 64, 127, 1023]
    case = make_decode_case(55, ctx)
    B = len(ctx)
    q = seeded_bf16(B * NUM_Q * HEAD_DIM, 41)
    k = seeded_bf16(case.cache_rows * KV_STRIDE, 42)
    v = seeded_bf16(case.cache_rows * KV_STRIDE, 43)
    for cap in (8, 9, 100):
        got, ref, _ = _run_attention(FULL, case.runs, case.base_rows, q, k, v, seq_len=B,
                                     cap=cap, cache_rows=case.cache_rows)
        _assert_close(got, ref, f"edges cap={cap}")


def test_one_call_dispatch_wrappers_match_plan_path():
    """ifr_dispatch_full_attention / ifr_dispatch_sliding_attention (plan,
    upload and launch in one call) give the plan path's bits."""
    announce("one-call wrappers")
    ctx = [700, 2000, 65]
    case = make_decode_case(77, ctx)
    B = 3
    q = seeded_bf16(B * NUM_Q * HEAD_DIM, 51)
    k = seeded_bf16(case.cache_rows * KV_STRIDE, 52)
    v = seeded_bf16(case.cache_rows * KV_STRIDE, 53)
    got, _, _ = _run_attention(FULL, case.runs, case.base_rows, q, k, v, seq_len=B, cap=32,
                               cache_rows=case.cache_rows)
    out = empty_dev(B * NUM_Q * HEAD_DIM, np.uint16)
    A.dispatch_full_attention(to_dev(q), to_dev(k), to_dev(v), out,
                              _table(case.runs, case.base_rows), num_q=NUM_Q,
                              kv_stride=KV_STRIDE, seq_len=B, head_dim=HEAD_DIM,
                              gqa_ratio=2, page_len=PAGE_LEN, cache_rows=case.cache_rows,
                              cap=32)
    assert np.array_equal(from_dev(out, np.uint16), got)


def test_page_copy_and_gather_bit_exact():
    """Copy-on-write jobs (page_copy.mojo) and row gather (gather.mojo)."""
    announce("page copy + gather")
    rng = np.random.default_rng(8)
    arena = rng.integers(0, 256, 4 << 20, dtype=np.uint8)
    row_bytes = KV_STRIDE * 2
    jobs = np.array([
        [0 * row_bytes, 100 * row_bytes, 64 * row_bytes],    # whole page
        [200 * row_bytes, 300 * row_bytes, 5 * row_bytes],   # partial page
        [7, 1 << 21, 1000],                                  # unaligned bytes
    ], dtype=np.int64)
    dev = to_dev(arena)
    A.dispatch_copy_jobs(dev, jobs)
    ref = arena.copy()
    oracle.copy_jobs(ref, jobs)
    assert np.array_equal(from_dev(dev, np.uint8), ref)
    src = seeded_bf16(300 * 4096, 9)
    rows = rng.integers(0, 300, 77).astype(np.int32)
    dst = empty_dev(77 * 4096, np.uint16)
    A.dispatch_gather_rows(to_dev(src), dst, to_dev(rows), 77, 4096)
    assert np.array_equal(from_dev(dst, np.uint16), oracle.gather_rows(src, rows, 4096))


@pytest.mark.parametrize("base_off", [0, 3])
def test_page_copy_alignment_cases(base_off):
    """Each chunk picks its own path: co-aligned source and destination take
    the byte head / 16-byte body / byte tail path, others byte copies, in
    one call; the arena base itself may be unaligned (base_off 3)."""
    announce(f"page copy alignment base_off={base_off}")
    rng = np.random.default_rng(80 + base_off)
    n = 3 << 20
    arena = rng.integers(0, 256, n, dtype=np.uint8)
    # Sources below 1.5 MB, destinations above: no job reads another's output.
    jobs = np.array([
        [16, 1_500_000, 200_000],           # aligned, several 64 KiB chunks
        [200_021, 1_700_005, 70_001],       # co-aligned (offset 5): head/body/tail
        [300_009, 1_800_004, 131_077],      # offsets 9 and 4: bytes only
        [450_000, 1_950_003, 7],            # shorter than one vector
        [460_001, 1_960_001, 15],           # co-aligned, the head covers it all
        [470_000, 1_970_000, 0],            # empty job
        [500_000, 2_000_000, 4096 * 64],    # a whole bf16 page of rows
    ], dtype=np.int64)
    dev = to_dev(arena)
    A.dispatch_copy_jobs(dev[base_off:], jobs)
    ref = arena.copy()
    oracle.copy_jobs(ref[base_off:], jobs)
    got = from_dev(dev, np.uint8)
    assert np.array_equal(got, ref), int((got != ref).sum())
