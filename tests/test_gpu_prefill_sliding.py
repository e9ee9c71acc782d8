"""GPU parity of the MFMA sliding-window prefill (FlashPrefillSlidingKernel,
kernels/flash_attention_prefill.mojo:18-114): every query token's tiles start
at its own window start lo = max(0, p - window + 1), which the kernel follows
through aligned 16-key tiles split at lo % 16.  Outputs within 1e-2 of the
oracle's token route (one bf16 spacing where |x| >= 2); the plan must take
the MFMA route (query blocks in info[14])."""
import numpy as np
import pytest

import oracle
from inferno_amd import attention as A
from inferno_amd.kv import SLIDING, AttentionPlan, KVRunTable
from tests.gpu_util import announce, empty_dev, from_dev, to_dev
from tests.helpers import (HEAD_DIM, KV_STRIDE, NUM_KV, NUM_Q, PAGE_LEN, assert_bar,
                           compare_bf16, seeded_bf16)

pytestmark = pytest.mark.gpu


def _table(runs, rows) -> KVRunTable:
    t = KVRunTable()
    for r in runs:
        t.begin_run(int(r[0]), int(r[1]))
        for j in range(int(r[3])):
            t.add_base_row(int(rows[int(r[2]) + j]))
    return t


def _ring_case(seed, prefix, new, ring_pages, page_len=PAGE_LEN):
    """Runs back to back in the token buffer, each on its own ring of
    ring_pages pages of a shuffled shared pool."""
    rng = np.random.default_rng(seed)
    B = len(prefix)
    perm = rng.permutation(B * ring_pages)
    runs, rows, buf = [], [], 0
    for i in range(B):
        runs.append([buf, prefix[i], len(rows), ring_pages])
        rows.extend(int(x) * page_len for x in perm[i * ring_pages:(i + 1) * ring_pages])
        buf += new[i]
    return np.asarray(runs, np.int32), np.asarray(rows, np.int32), B * ring_pages * page_len


def _run(runs, rows, cache_rows, n, window, ring_pages, q, k, v, page_len=PAGE_LEN):
    plan = AttentionPlan(_table(runs, rows), n, kind=SLIDING, window=window,
                         cache_size=ring_pages * page_len, page_len=page_len,
                         cache_rows=cache_rows, cap=16, kv_row_bytes=KV_STRIDE * 2)
    assert plan.summary.mode == 1 and int(plan.info[14]) > 0, "not on the MFMA route"
    out = empty_dev(n * NUM_Q * HEAD_DIM, np.uint16)
    partials, ps = A.partials_buffer(plan, NUM_Q, HEAD_DIM)
    A.attention_bf16(plan, to_dev(q), to_dev(k), to_dev(v), out, partials, ps, num_q=NUM_Q,
                     num_kv=NUM_KV, head_dim=HEAD_DIM, kv_stride=KV_STRIDE)
    return from_dev(out, np.uint16)


def _ref(runs, rows, n, window, ring_pages, q, k, v, page_len=PAGE_LEN):
    return oracle.attention(SLIDING, runs, rows, q, k, v, num_q=NUM_Q, num_kv=NUM_KV,
                            head_dim=HEAD_DIM, kv_stride=KV_STRIDE, window=window,
                            cache_size=ring_pages * page_len, page_len=page_len, seq_len=n,
                            cap=16, threads=16)


@pytest.mark.parametrize("window", [16, 48, 64, 304, 1024, 1, 5, 17, 100, 1000, 1023])
def test_sliding_prefill_windows(window):
    """Chunks that start at position 0, inside the first window, and far past
    it (the window start moves with every token), full and partial query
    blocks, windows of one tile, of three, not a power of two, and windows
    that are not a multiple of 16 (a row's last tile then ends past its
    position, with pads in the low or the high part of an aligned tile)."""
    announce(f"sliding mfma prefill window={window}")
    prefix = [0, 5, max(0, window - 3), 700, 3000]
    new = [100, 64, 129, 77, 200]
    ring = 1 << int(np.ceil(np.log2((window + max(new) + 2 * PAGE_LEN) / PAGE_LEN)))
    runs, rows, cache_rows = _ring_case(window, prefix, new, ring)
    n = sum(new)
    q = seeded_bf16(n * NUM_Q * HEAD_DIM, 1)
    k = seeded_bf16(cache_rows * KV_STRIDE, 2)
    v = seeded_bf16(cache_rows * KV_STRIDE, 3)
    got = _run(runs, rows, cache_rows, n, window, ring, q, k, v)
    r = compare_bf16(got, _ref(runs, rows, n, window, ring, q, k, v))
    assert_bar(r, f"window {window} ring {ring}")


def test_sliding_prefill_diffuse_scores():
    """Queries scaled by 1/16: attention spread over the whole window."""
    announce("sliding mfma prefill diffuse")
    prefix, new = [0, 1500, 4000], [130, 64, 190]
    runs, rows, cache_rows = _ring_case(7, prefix, new, 32)
    n = sum(new)
    rng = np.random.default_rng(8)
    qf = (rng.standard_normal(n * NUM_Q * HEAD_DIM) / 16.0).astype(np.float32)
    u = qf.view(np.uint32).astype(np.uint64)
    q = ((u + ((u >> 16) & 1) + 0x7FFF) >> 16).astype(np.uint16)
    k = seeded_bf16(cache_rows * KV_STRIDE, 9)
    v = seeded_bf16(cache_rows * KV_STRIDE, 10)
    got = _run(runs, rows, cache_rows, n, 1024, 32, q, k, v)
    r = compare_bf16(got, _ref(runs, rows, n, 1024, 32, q, k, v))
    assert_bar(r, "diffuse")


@pytest.mark.parametrize("page_len,ring_pages", [(8, 512), (1024, 4)])
def test_sliding_prefill_page_sizes(page_len, ring_pages):
    """Pages of 8 rows (several pages per staged row group) and Gemma-4's
    1024-token pages."""
    announce(f"sliding mfma prefill page_len={page_len}")
    prefix, new = [0, 900, 2500], [96, 129, 64]
    runs, rows, cache_rows = _ring_case(11, prefix, new, ring_pages, page_len)
    n = sum(new)
    q = seeded_bf16(n * NUM_Q * HEAD_DIM, 12)
    k = seeded_bf16(cache_rows * KV_STRIDE, 13)
    v = seeded_bf16(cache_rows * KV_STRIDE, 14)
    got = _run(runs, rows, cache_rows, n, 1024, ring_pages, q, k, v, page_len)
    r = compare_bf16(got, _ref(runs, rows, n, 1024, ring_pages, q, k, v, page_len))
    assert_bar(r, f"page_len {page_len}")


def test_sliding_prefill_chunk_8x2048_append_then_attend():
    """8 sequences append 2048 tokens each onto prefixes ~ U[0, 16384] on
    64-page rings (window 1024), then the MFMA sliding prefill; the cache
    writes bit-exact, sampled query tokens of every sequence against the
    oracle (each as a one-token run of a token plan)."""
    announce("sliding mfma prefill 8 x 2048")
    rng = np.random.default_rng(44)
    prefix = [int(x) for x in rng.integers(0, 16385, 8)]
    new = [2048] * 8
    ring = 64
    runs, rows, cache_rows = _ring_case(45, prefix, new, ring)
    n = sum(new)
    k = seeded_bf16(cache_rows * KV_STRIDE, 4)
    v = seeded_bf16(cache_rows * KV_STRIDE, 5)
    q = seeded_bf16(n * NUM_Q * HEAD_DIM, 6)
    ks, vs = seeded_bf16(n * KV_STRIDE, 7), seeded_bf16(n * KV_STRIDE, 8)
    maxpos = max(p + m for p, m in zip(prefix, new)) + 1
    ang = rng.uniform(-3, 3, maxpos * 128)
    cos, sin = np.cos(ang).astype(np.float32), np.sin(ang).astype(np.float32)
    plan = AttentionPlan(_table(runs, rows), n, kind=SLIDING, window=1024,
                         cache_size=ring * PAGE_LEN, page_len=PAGE_LEN, cache_rows=cache_rows,
                         cap=16, kv_row_bytes=KV_STRIDE * 2)
    assert int(plan.info[14]) > 0
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
    oracle.rope_cache_write(runs, rows, q_ref, ks, vs, k_ref, v_ref, cos, sin, num_q=NUM_Q,
                            num_kv=NUM_KV, page_shift=6, row_mask=63, page_mask=ring - 1,
                            seq_len=n, half=128, pair_stride=128, head_dim=HEAD_DIM)
    assert np.array_equal(from_dev(kd, np.uint16), k_ref), "k cache after append"
    assert np.array_equal(from_dev(vd, np.uint16), v_ref), "v cache after append"
    assert np.array_equal(from_dev(qd, np.uint16), q_ref), "rotated q"
    picks = [(r, t) for r in range(8) for t in (0, 1, 15, 16, 17, 63, 64, 1022, 1023, 1024,
                                                1025, 1500, 2046, 2047)]
    sruns, q_s = [], []
    for i, (r, t) in enumerate(picks):
        sruns.append([i, prefix[r] + t, runs[r, 2], runs[r, 3]])
        tok = r * 2048 + t
        q_s.append(q_ref[tok * NUM_Q * HEAD_DIM:(tok + 1) * NUM_Q * HEAD_DIM])
    sruns = np.asarray(sruns, dtype=np.int32)
    ref = oracle.attention(SLIDING, sruns, rows, np.concatenate(q_s), k_ref, v_ref,
                           num_q=NUM_Q, num_kv=NUM_KV, head_dim=HEAD_DIM, kv_stride=KV_STRIDE,
                           window=1024, cache_size=ring * PAGE_LEN, page_len=PAGE_LEN,
                           seq_len=len(picks), cap=2, threads=16)
    sel = np.concatenate([got[r * 2048 + t] for r, t in picks])
    res = compare_bf16(sel, ref)
    assert_bar(res, "8 x 2048 sampled tokens")
