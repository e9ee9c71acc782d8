"""GPU parity of chunked prefill over the paged cache (full attention):
append of the chunk (RoPE + cache write, bit-exact), then the MFMA prefill
kernel against the oracle's token-partitioned route
(FlashPrefillFullKernel + PrefillMergeKernel) within 1e-2 / one bf16 spacing."""
import numpy as np
import pytest

import oracle
from inferno_amd import attention as A
from inferno_amd.kv import FULL, AttentionPlan, KVRunTable
from tests.gpu_util import announce, empty_dev, from_dev, to_dev
from tests.helpers import (HEAD_DIM, KV_STRIDE, NUM_KV, NUM_Q, PAGE_LEN, assert_bar,
                           compare_bf16, make_prefill_case, seeded_bf16)

pytestmark = pytest.mark.gpu


def _table(runs, rows) -> KVRunTable:
    t = KVRunTable()
    for r in runs:
        t.begin_run(int(r[0]), int(r[1]))
        for j in range(int(r[3])):
            t.add_base_row(int(rows[int(r[2]) + j]))
    return t


def _prefill(case, n, q, k, v, cap=16, page_len=PAGE_LEN):
    plan = AttentionPlan(_table(case.runs, case.base_rows), n, kind=FULL, window=0,
                         cache_size=page_len, page_len=page_len, cache_rows=case.cache_rows,
                         cap=cap, kv_row_bytes=KV_STRIDE * 2)
    assert plan.summary.mode == 2 and int(plan.info[14]) > 0
    out = empty_dev(n * NUM_Q * HEAD_DIM, np.uint16)
    partials, ps = A.partials_buffer(plan, NUM_Q, HEAD_DIM)
    A.attention_bf16(plan, q, k, v, out, partials, ps, num_q=NUM_Q, num_kv=NUM_KV,
                     head_dim=HEAD_DIM, kv_stride=KV_STRIDE)
    return from_dev(out, np.uint16)


def test_prefill_small_all_tokens():
    announce("prefill small")
    prefix, new = [0, 100, 1000, 3000, 63], [40, 33, 100, 64, 1]
    case = make_prefill_case(3, prefix, new)
    n = sum(new)
    q = seeded_bf16(n * NUM_Q * HEAD_DIM, 1)
    k = seeded_bf16(case.cache_rows * KV_STRIDE, 2)
    v = seeded_bf16(case.cache_rows * KV_STRIDE, 3)
    got = _prefill(case, n, to_dev(q), to_dev(k), to_dev(v))
    ref = oracle.attention(FULL, case.runs, case.base_rows, q, k, v, num_q=NUM_Q,
                           num_kv=NUM_KV, head_dim=HEAD_DIM, kv_stride=KV_STRIDE, window=0,
                           cache_size=PAGE_LEN, page_len=PAGE_LEN, seq_len=n, cap=16,
                           threads=8)
    r = compare_bf16(got, ref)
    assert_bar(r, "prefill small")


def test_prefill_diffuse_scores():
    """Queries scaled by 1/16 (scores ~ N(0,1) instead of N(0,256)): attention
    spreads over many keys, so most tiles stay under the lo-part share and
    take only the bf16 hi parts of P."""
    announce("prefill diffuse")
    prefix, new = [0, 700, 3000, 4095], [64, 130, 200, 1]
    case = make_prefill_case(5, prefix, new)
    n = sum(new)
    rng = np.random.default_rng(11)
    qf = (rng.standard_normal(n * NUM_Q * HEAD_DIM) / 16.0).astype(np.float32)
    u = qf.view(np.uint32).astype(np.uint64)
    q = ((u + ((u >> 16) & 1) + 0x7FFF) >> 16).astype(np.uint16)
    k = seeded_bf16(case.cache_rows * KV_STRIDE, 12)
    v = seeded_bf16(case.cache_rows * KV_STRIDE, 13)
    got = _prefill(case, n, to_dev(q), to_dev(k), to_dev(v))
    ref = oracle.attention(FULL, case.runs, case.base_rows, q, k, v, num_q=NUM_Q,
                           num_kv=NUM_KV, head_dim=HEAD_DIM, kv_stride=KV_STRIDE, window=0,
                           cache_size=PAGE_LEN, page_len=PAGE_LEN, seq_len=n, cap=16,
                           threads=8)
    r = compare_bf16(got, ref)
    assert_bar(r, "prefill diffuse")


@pytest.mark.parametrize("page_len", [8, 128])
def test_prefill_page_sizes(page_len):
    """Pages of 8 rows (the kernel's per-row staging path) and of 128 rows
    (a staged iteration inside one page), with full and partial query blocks
    and prefixes that are not page multiples."""
    announce(f"prefill page_len={page_len}")
    prefix, new = [0, 70, 1500, 333], [64, 200, 129, 7]
    case = make_prefill_case(11 + page_len, prefix, new, page_len=page_len)
    n = sum(new)
    q = seeded_bf16(n * NUM_Q * HEAD_DIM, 21)
    k = seeded_bf16(case.cache_rows * KV_STRIDE, 22)
    v = seeded_bf16(case.cache_rows * KV_STRIDE, 23)
    got = _prefill(case, n, to_dev(q), to_dev(k), to_dev(v), page_len=page_len)
    ref = oracle.attention(FULL, case.runs, case.base_rows, q, k, v, num_q=NUM_Q,
                           num_kv=NUM_KV, head_dim=HEAD_DIM, kv_stride=KV_STRIDE, window=0,
                           cache_size=page_len, page_len=page_len, seq_len=n, cap=16,
                           threads=8)
    r = compare_bf16(got, ref)
    assert_bar(r, f"prefill page_len={page_len}")


@pytest.mark.parametrize("page_len", [4, 8])
def test_prefill_long_run_moves_the_page_window(page_len):
    """Runs whose page table outgrows the kernel's LDS window of 4,096
    entries (40,000 cached positions: 5,000 pages of 8 rows, 10,000 of 4)
    stay on the MFMA route; the window moves along the run once or twice."""
    announce(f"prefill beyond the LDS page window, page_len={page_len}")
    prefix, new = [40000, 100], [70, 64]
    case = make_prefill_case(31 + page_len, prefix, new, page_len=page_len)
    n = sum(new)
    q = seeded_bf16(n * NUM_Q * HEAD_DIM, 41)
    k = seeded_bf16(case.cache_rows * KV_STRIDE, 42)
    v = seeded_bf16(case.cache_rows * KV_STRIDE, 43)
    got = _prefill(case, n, to_dev(q), to_dev(k), to_dev(v), page_len=page_len)
    ref = oracle.attention(FULL, case.runs, case.base_rows, q, k, v, num_q=NUM_Q,
                           num_kv=NUM_KV, head_dim=HEAD_DIM, kv_stride=KV_STRIDE, window=0,
                           cache_size=page_len, page_len=page_len, seq_len=n, cap=16,
                           threads=16)
    assert_bar(compare_bf16(got, ref), f"prefill long run page_len={page_len}")


def test_prefill_config4_shape_append_then_attend():
    """Config 4: 8 sequences append 2048 tokens each onto prefixes ~ U[0,16384]
    (RoPE + cache write for the whole chunk, then causal prefill).  The cache
    writes are compared whole (bit-exact); attention outputs are checked for
    sampled query tokens against the oracle's token route."""
    announce("prefill config4 shape")
    rng = np.random.default_rng(44)
    prefix = [int(x) for x in rng.integers(0, 16385, 8)]
    new = [2048] * 8
    case = make_prefill_case(45, prefix, new)
    n = sum(new)
    k = seeded_bf16(case.cache_rows * KV_STRIDE, 4)
    v = seeded_bf16(case.cache_rows * KV_STRIDE, 5)
    q = seeded_bf16(n * NUM_Q * HEAD_DIM, 6)
    ks, vs = seeded_bf16(n * KV_STRIDE, 7), seeded_bf16(n * KV_STRIDE, 8)
    maxpos = max(p + m for p, m in zip(prefix, new)) + 1
    ang = rng.uniform(-3, 3, maxpos * 128)
    cos, sin = np.cos(ang).astype(np.float32), np.sin(ang).astype(np.float32)
    plan = AttentionPlan(_table(case.runs, case.base_rows), n, kind=FULL, window=0,
                         cache_size=PAGE_LEN, page_len=PAGE_LEN, cache_rows=case.cache_rows,
                         cap=16, kv_row_bytes=KV_STRIDE * 2)
    qd, kd, vd = to_dev(q), to_dev(k), to_dev(v)
    A.dispatch_rope_cache_write(plan, qd, to_dev(ks), to_dev(vs), kd, vd, to_dev(cos),
                                to_dev(sin), num_q=NUM_Q, num_kv=NUM_KV, half=128,
                                pair_stride=128, head_dim=HEAD_DIM)
    out = empty_dev(n * NUM_Q * HEAD_DIM, np.uint16)
    partials, ps = A.partials_buffer(plan, NUM_Q, HEAD_DIM)
    A.attention_bf16(plan, qd, kd, vd, out, partials, ps, num_q=NUM_Q, num_kv=NUM_KV,
                     head_dim=HEAD_DIM, kv_stride=KV_STRIDE)
    got = from_dev(out, np.uint16).reshape(n, NUM_Q * HEAD_DIM)
    q_ref, k_ref, v_ref = q.copy(), k.copy(), v.copy()
    oracle.rope_cache_write(case.runs, case.base_rows, q_ref, ks, vs, k_ref, v_ref, cos, sin,
                            num_q=NUM_Q, num_kv=NUM_KV, page_shift=6, row_mask=63,
                            page_mask=-1, seq_len=n, half=128, pair_stride=128,
                            head_dim=HEAD_DIM)
    assert np.array_equal(from_dev(kd, np.uint16), k_ref), "k cache after append"
    assert np.array_equal(from_dev(vd, np.uint16), v_ref), "v cache after append"
    assert np.array_equal(from_dev(qd, np.uint16), q_ref), "rotated q"
    # Sampled tokens, each as its own one-token run of a token plan (cap below
    # the run count): the same tiles-from-0 walk and one-segment merge.
    picks = []
    for r in range(8):
        for t in (0, 1, 15, 16, 777, 2046, 2047):
            picks.append((r, t))
    runs, q_s = [], []
    for i, (r, t) in enumerate(picks):
        runs.append([i, prefix[r] + t, case.runs[r, 2], case.runs[r, 3]])
        tok = r * 2048 + t
        q_s.append(q_ref[tok * NUM_Q * HEAD_DIM:(tok + 1) * NUM_Q * HEAD_DIM])
    runs = np.asarray(runs, dtype=np.int32)
    ref = oracle.attention(FULL, runs, case.base_rows, np.concatenate(q_s), k_ref, v_ref,
                           num_q=NUM_Q, num_kv=NUM_KV, head_dim=HEAD_DIM, kv_stride=KV_STRIDE,
                           window=0, cache_size=PAGE_LEN, page_len=PAGE_LEN,
                           seq_len=len(picks), cap=2, threads=16)
    sel = np.concatenate([got[r * 2048 + t] for r, t in picks])
    res = compare_bf16(sel, ref)
    assert_bar(res, "config4 sampled tokens")
