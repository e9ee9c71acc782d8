"""GPU parity of the MFMA chunked prefill at Gemma-4's full-attention shape
(head_dim 512, 16 q / 2 kv heads, modeling/gemma4_common.mojo:14-20;
FlashPrefillFullKernel + PrefillMergeKernel, kernels/
flash_attention_prefill.mojo:117-248): the chunk's tokens against the
oracle's token-partitioned route, within 1e-2 (one bf16 spacing where
|x| >= 2).  A wave owns 4 tokens x 8 q heads over all 512 dims and a block
16 tokens, so the cases cover partial blocks, waves without live rows, the
causal diagonal, page-table windows that move, and both of the kernel's
block placements (kv head counts that divide the 8 XCDs and one that does
not)."""
import numpy as np
import pytest

import oracle
from inferno_amd import attention as A
from inferno_amd.kv import FULL, AttentionPlan, KVRunTable
from tests.gpu_util import announce, empty_dev, from_dev, to_dev
from tests.helpers import assert_bar, compare_bf16, make_prefill_case, seeded_bf16

pytestmark = pytest.mark.gpu

NQ, NKV, D = 16, 2, 512
KVS = NKV * D
HALF, PAIR = 64, 256


def _table(runs, rows) -> KVRunTable:
    t = KVRunTable()
    for r in runs:
        t.begin_run(int(r[0]), int(r[1]))
        for j in range(int(r[3])):
            t.add_base_row(int(rows[int(r[2]) + j]))
    return t


def _plan(case, n, page_len, kvs=KVS):
    return AttentionPlan(_table(case.runs, case.base_rows), n, kind=FULL, window=0,
                         cache_size=page_len, page_len=page_len, cache_rows=case.cache_rows,
                         cap=16, kv_row_bytes=kvs * 2)


def _prefill(case, n, q, k, v, page_len=64, nq=NQ, nkv=NKV):
    kvs = nkv * D
    plan = _plan(case, n, page_len, kvs)
    assert plan.summary.mode == 2 and int(plan.info[14]) > 0, "no query blocks"
    out = empty_dev(n * nq * D, np.uint16)
    partials, ps = A.partials_buffer(plan, nq, D)
    A.attention_bf16(plan, to_dev(q), to_dev(k), to_dev(v), out, partials, ps, num_q=nq,
                     num_kv=nkv, head_dim=D, kv_stride=kvs)
    got = from_dev(out, np.uint16)
    ref = oracle.attention(FULL, case.runs, case.base_rows, q, k, v, num_q=nq, num_kv=nkv,
                           head_dim=D, kv_stride=kvs, window=0, cache_size=page_len,
                           page_len=page_len, seq_len=n, cap=16, threads=16)
    return compare_bf16(got, ref)


def test_wide_prefill_small_all_tokens():
    """Chunks from position 0, short and long prefixes, blocks of 1-8 live
    tokens (pairs without live rows), a chunk of one token."""
    announce("wide mfma prefill small")
    prefix, new = [0, 100, 1000, 3000, 63, 5], [40, 33, 100, 64, 1, 7]
    case = make_prefill_case(3, prefix, new)
    n = sum(new)
    r = _prefill(case, n, seeded_bf16(n * NQ * D, 1), seeded_bf16(case.cache_rows * KVS, 2),
                 seeded_bf16(case.cache_rows * KVS, 3))
    assert_bar(r, "wide prefill small")


def test_wide_prefill_diffuse_scores():
    """Queries scaled by 1/16: attention spreads over many keys (most tiles
    without lo parts)."""
    announce("wide mfma prefill diffuse")
    prefix, new = [0, 700, 2000], [130, 64, 90]
    case = make_prefill_case(7, prefix, new)
    n = sum(new)
    rng = np.random.default_rng(8)
    qf = (rng.standard_normal(n * NQ * D) / 16.0).astype(np.float32)
    u = qf.view(np.uint32).astype(np.uint64)
    q = ((u + ((u >> 16) & 1) + 0x7FFF) >> 16).astype(np.uint16)
    r = _prefill(case, n, q, seeded_bf16(case.cache_rows * KVS, 9),
                 seeded_bf16(case.cache_rows * KVS, 10))
    assert_bar(r, "wide prefill diffuse")


@pytest.mark.parametrize("nkv", [1, 3])
def test_wide_prefill_kv_head_counts(nkv):
    """8 and 24 q heads (1 and 3 kv heads at GQA 8): one kv head for every
    XCD, and a count that does not divide the 8 XCDs (the kernel then
    spreads each query block's kv heads over one XCD)."""
    announce(f"wide mfma prefill num_kv={nkv}")
    nq = 8 * nkv
    prefix, new = [0, 300, 1500, 70], [70, 129, 64, 9]
    case = make_prefill_case(21 + nkv, prefix, new)
    n = sum(new)
    r = _prefill(case, n, seeded_bf16(n * nq * D, 22), seeded_bf16(case.cache_rows * nkv * D, 23),
                 seeded_bf16(case.cache_rows * nkv * D, 24), nq=nq, nkv=nkv)
    assert_bar(r, f"wide prefill num_kv {nkv}")


@pytest.mark.parametrize("page_len", [8, 1024])
def test_wide_prefill_page_sizes(page_len):
    """Pages of 8 rows (each staged key row group spans pages) and Gemma-4's
    1024-token pages."""
    announce(f"wide mfma prefill page_len={page_len}")
    prefix, new = [0, 900, 2500], [96, 129, 64]
    case = make_prefill_case(11, prefix, new, page_len=page_len)
    n = sum(new)
    r = _prefill(case, n, seeded_bf16(n * NQ * D, 12), seeded_bf16(case.cache_rows * KVS, 13),
                 seeded_bf16(case.cache_rows * KVS, 14), page_len=page_len)
    assert_bar(r, f"wide prefill page_len {page_len}")


@pytest.mark.parametrize("page_len", [4, 8])
def test_wide_prefill_long_run_moves_the_page_window(page_len):
    """Runs whose page table outgrows the kernel's LDS window of 2,048
    entries (40,000 cached positions: 5,000 pages of 8 rows, 10,000 of 4)
    stay on the MFMA route; the window moves along the run two to four
    times."""
    announce(f"wide prefill beyond the LDS page window, page_len={page_len}")
    prefix, new = [40000, 40], [20, 30]
    case = make_prefill_case(15 + page_len, prefix, new, page_len=page_len)
    n = sum(new)
    r = _prefill(case, n, seeded_bf16(n * NQ * D, 16), seeded_bf16(case.cache_rows * KVS, 17),
                 seeded_bf16(case.cache_rows * KVS, 18), page_len=page_len)
    assert_bar(r, f"wide prefill long run page_len={page_len}")


def test_wide_prefill_8x2048_append_then_attend():
    """8 sequences in pairs sharing a prefix length append 2048 tokens each
    onto prefixes ~ U[0, 16384] (partial RoPE, half 64 / pair_stride 256),
    then the MFMA prefill; the cache writes bit-exact, sampled query tokens
    of every sequence against the oracle (each as a one-token run)."""
    announce("wide mfma prefill 8 x 2048")
    rng = np.random.default_rng(44)
    prefix = [int(x) for x in rng.integers(0, 16385, 4) for _ in range(2)]
    new = [2048] * 8
    case = make_prefill_case(45, prefix, new)
    n = sum(new)
    k = seeded_bf16(case.cache_rows * KVS, 4)
    v = seeded_bf16(case.cache_rows * KVS, 5)
    q = seeded_bf16(n * NQ * D, 6)
    ks, vs = seeded_bf16(n * KVS, 7), seeded_bf16(n * KVS, 8)
    maxpos = max(p + m for p, m in zip(prefix, new)) + 1
    ang = rng.uniform(-3, 3, maxpos * HALF)
    cos, sin = np.cos(ang).astype(np.float32), np.sin(ang).astype(np.float32)
    plan = _plan(case, n, 64)
    assert int(plan.info[14]) > 0
    qd, kd, vd = to_dev(q), to_dev(k), to_dev(v)
    A.dispatch_rope_cache_write(plan, qd, to_dev(ks), to_dev(vs), kd, vd, to_dev(cos),
                                to_dev(sin), num_q=NQ, num_kv=NKV, half=HALF, pair_stride=PAIR,
                                head_dim=D)
    out = empty_dev(n * NQ * D, np.uint16)
    partials, ps = A.partials_buffer(plan, NQ, D)
    A.attention_bf16(plan, qd, kd, vd, out, partials, ps, num_q=NQ, num_kv=NKV, head_dim=D,
                     kv_stride=KVS)
    got = from_dev(out, np.uint16).reshape(n, NQ * D)
    q_ref, k_ref, v_ref = q.copy(), k.copy(), v.copy()
    oracle.rope_cache_write(case.runs, case.base_rows, q_ref, ks, vs, k_ref, v_ref, cos, sin,
                            num_q=NQ, num_kv=NKV, page_shift=6, row_mask=63, page_mask=-1,
                            seq_len=n, half=HALF, pair_stride=PAIR, head_dim=D)
    assert np.array_equal(from_dev(kd, np.uint16), k_ref), "k cache after append"
    assert np.array_equal(from_dev(vd, np.uint16), v_ref), "v cache after append"
    assert np.array_equal(from_dev(qd, np.uint16), q_ref), "rotated q"
    picks = [(r, t) for r in range(8) for t in (0, 1, 7, 8, 15, 16, 31, 32, 63, 64, 1000,
                                                2046, 2047)]
    sruns, q_s = [], []
    for i, (r, t) in enumerate(picks):
        sruns.append([i, prefix[r] + t, case.runs[r, 2], case.runs[r, 3]])
        tok = r * 2048 + t
        q_s.append(q_ref[tok * NQ * D:(tok + 1) * NQ * D])
    sruns = np.asarray(sruns, dtype=np.int32)
    ref = oracle.attention(FULL, sruns, case.base_rows, np.concatenate(q_s), k_ref, v_ref,
                           num_q=NQ, num_kv=NKV, head_dim=D, kv_stride=KVS, window=0,
                           cache_size=64, page_len=64, seq_len=len(picks), cap=1, threads=16)
    sel = np.concatenate([got[r * 2048 + t] for r, t in picks])
    res = compare_bf16(sel, ref)
    assert_bar(res, "wide prefill 8 x 2048 sampled tokens")
