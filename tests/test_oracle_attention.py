"""CPU tests pinning the oracle's attention, append, copy, gather and
butterquant paths against closed forms, textbook softmax and the reference's
own scalar parity harness."""
import numpy as np
import pytest

import oracle
from tests import bq_schedule as bq
from tests.helpers import (HEAD_DIM, KV_STRIDE, NUM_KV, NUM_Q, PAGE_LEN, bf16_to_f32,
                           make_decode_case, make_prefill_case, seeded_bf16)


def _tile_weights(kv_len, splits):
    """Per-position weight of the q = 0 closed form.  All scores are 0, so the
    running max is 0 from the first tile on, every later tile multiplies the
    state by c0 = fexp(0), and every split is merged with the same factor.
    Position t of split s, tile j gets c0^(T_s - 1 - j)."""
    c0 = float(oracle.fexp(np.float32(0.0))[()])
    w = np.zeros(kv_len)
    for a, b in splits:
        n_tiles = (b - a + 15) // 16
        for t in range(a, b):
            j = (t - a) // 16
            w[t] = c0 ** (n_tiles - 1 - j)
    return w


def _closed_form_out(v_rows, w):
    acc = (w[:, None] * v_rows.astype(np.float64)).sum(0)
    return acc / w.sum()


@pytest.mark.parametrize("route", ["single", "batched", "token_full", "token_sliding"])
def test_attention_q_zero_closed_form(route):
    ctx = {"single": [700], "batched": [1000, 37, 300], "token_full": [200, 90],
           "token_sliding": [300, 41]}[route]
    case = make_decode_case(11, ctx)
    cap = {"single": 5, "batched": 9, "token_full": 2, "token_sliding": 2}[route]
    kind = 0 if route == "token_sliding" else 1
    window = 128
    if route == "token_sliding":
        kind = 0
    B = len(ctx)
    q = np.zeros(B * NUM_Q * HEAD_DIM, dtype=np.uint16)
    k = seeded_bf16(case.cache_rows * KV_STRIDE, 1)
    v = seeded_bf16(case.cache_rows * KV_STRIDE, 2)
    cache_size = case.pool_pages * PAGE_LEN  # ring never wraps here
    pages_pow2 = 1 << (max(len(p) for p in case.pages) - 1).bit_length()
    if kind == 0:
        cache_size = pages_pow2 * PAGE_LEN
        runs = case.runs.copy()
        runs[:, 3] = pages_pow2
        rows = []
        for i, p in enumerate(case.pages):
            runs[i, 2] = len(rows)
            rows.extend([x * PAGE_LEN for x in p] + [0] * (pages_pow2 - len(p)))
        base_rows = np.asarray(rows, dtype=np.int32)
    else:
        runs, base_rows = case.runs, case.base_rows
    out = oracle.attention(kind, runs, base_rows, q, k, v, num_q=NUM_Q, num_kv=NUM_KV,
                           head_dim=HEAD_DIM, kv_stride=KV_STRIDE, window=window,
                           cache_size=cache_size, page_len=PAGE_LEN, seq_len=B, cap=cap)
    out = bf16_to_f32(out).reshape(B, NUM_Q, HEAD_DIM)
    for i in range(B):
        pos = int(case.ctx[i])
        if kind == 0:
            kv_len = min(pos + 1, window)
            first = pos - kv_len + 1
        else:
            kv_len, first = pos + 1, 0
        if route == "single":
            nw = min(oracle.recommended_workers(kv_len * KV_STRIDE * 2, cap), cap, kv_len)
            splits = [oracle.worker_range(kv_len, nw, w) for w in range(nw)]
        elif route == "batched":
            kvs = [int(c) + 1 for c in case.ctx]
            bands = oracle.plan_run_splits(kvs, list(range(B)), cap, 16)
            n = int(bands[i, 2])
            splits = [oracle.worker_range(kv_len, n, s) for s in range(n)]
        else:
            splits = [(0, kv_len)]
        w = _tile_weights(kv_len, splits)
        positions = np.arange(first, first + kv_len)
        slots = [oracle.paged_slot(base_rows[runs[i, 2]:], 6, 63,
                                   (cache_size // PAGE_LEN - 1) if kind == 0 else -1, 0, p)
                 for p in positions]
        vf = bf16_to_f32(v).reshape(-1, NUM_KV, HEAD_DIM)
        for h in range(NUM_Q):
            want = _closed_form_out(vf[slots, h // 2], w)
            got = out[i, h]
            err = np.abs(got - want)
            assert np.all(err <= 2.0 ** -8 * np.abs(want) + 1e-6), (route, i, h, err.max())


def test_attention_single_tile_matches_textbook_softmax():
    # One tile, one split: softmax with the biased exp differs from the
    # textbook one only through the per-weight relative error in [-6.9e-3, 0].
    ctx = [9, 15, 3]
    case = make_decode_case(5, ctx)
    B = len(ctx)
    q = seeded_bf16(B * NUM_Q * HEAD_DIM, 7)
    qf = bf16_to_f32(q).reshape(B, NUM_Q, HEAD_DIM).astype(np.float64) / 8.0
    q = ((qf.astype(np.float32).view(np.uint32) >> 16).astype(np.uint16)).reshape(-1)
    k = seeded_bf16(case.cache_rows * KV_STRIDE, 8)
    v = seeded_bf16(case.cache_rows * KV_STRIDE, 9)
    out = oracle.attention(1, case.runs, case.base_rows, q, k, v, num_q=NUM_Q,
                           num_kv=NUM_KV, head_dim=HEAD_DIM, kv_stride=KV_STRIDE,
                           window=0, cache_size=PAGE_LEN, page_len=PAGE_LEN, seq_len=B,
                           cap=1)
    out = bf16_to_f32(out).reshape(B, NUM_Q, HEAD_DIM).astype(np.float64)
    qf = bf16_to_f32(q).reshape(B, NUM_Q, HEAD_DIM).astype(np.float64)
    kf = bf16_to_f32(k).reshape(-1, NUM_KV, HEAD_DIM).astype(np.float64)
    vf = bf16_to_f32(v).reshape(-1, NUM_KV, HEAD_DIM).astype(np.float64)
    for i in range(B):
        slots = [int(case.base_rows[case.runs[i, 2] + p // 64]) + p % 64
                 for p in range(ctx[i] + 1)]
        for h in range(NUM_Q):
            s = kf[slots, h // 2] @ qf[i, h]          # no 1/sqrt(d): Gemma4 scale 1
            w = np.exp(s - s.max())
            vv = vf[slots, h // 2]
            want = (w[:, None] * vv).sum(0) / w.sum()
            bound = 7e-3 * (vv.max(0) - vv.min(0)) + 2.0 ** -8 * np.abs(want) + 1e-4
            assert np.all(np.abs(out[i, h] - want) <= bound), (i, h)


def test_rope_cache_write_identity_and_quarter_turn():
    case = make_decode_case(3, [70, 5])
    B = 2
    q0 = seeded_bf16(B * NUM_Q * HEAD_DIM, 1)
    ks = seeded_bf16(B * KV_STRIDE, 2)
    vs = seeded_bf16(B * KV_STRIDE, 3)
    half = 128
    for mode in ("identity", "quarter"):
        cos = np.full(1024 * half, 1.0 if mode == "identity" else 0.0, dtype=np.float32)
        sin = np.full(1024 * half, 0.0 if mode == "identity" else 1.0, dtype=np.float32)
        q = q0.copy()
        kc = np.zeros(case.cache_rows * KV_STRIDE, dtype=np.uint16)
        vc = np.zeros_like(kc)
        oracle.rope_cache_write(case.runs, case.base_rows, q, ks, vs, kc, vc, cos, sin,
                                num_q=NUM_Q, num_kv=NUM_KV, page_shift=6, row_mask=63,
                                page_mask=-1, seq_len=B, half=half, pair_stride=128,
                                head_dim=HEAD_DIM)
        for i in range(B):
            pos = int(case.ctx[i])
            slot = int(case.base_rows[case.runs[i, 2] + pos // 64]) + pos % 64
            kd = kc[slot * KV_STRIDE:(slot + 1) * KV_STRIDE].reshape(NUM_KV, HEAD_DIM)
            kin = ks[i * KV_STRIDE:(i + 1) * KV_STRIDE].reshape(NUM_KV, HEAD_DIM)
            assert np.array_equal(vc[slot * KV_STRIDE:(slot + 1) * KV_STRIDE],
                                  vs[i * KV_STRIDE:(i + 1) * KV_STRIDE])
            qo = q[i * NUM_Q * HEAD_DIM:(i + 1) * NUM_Q * HEAD_DIM].reshape(NUM_Q, HEAD_DIM)
            qi = q0[i * NUM_Q * HEAD_DIM:(i + 1) * NUM_Q * HEAD_DIM].reshape(NUM_Q, HEAD_DIM)
            if mode == "identity":
                assert np.array_equal(kd, kin) and np.array_equal(qo, qi)
            else:  # (lo, hi) -> (-hi, lo)
                assert np.array_equal(kd[:, :128], kin[:, 128:] ^ 0x8000)
                assert np.array_equal(kd[:, 128:], kin[:, :128])
                assert np.array_equal(qo[:, :128], qi[:, 128:] ^ 0x8000)


def test_copy_jobs_and_gather_closed_form():
    rng = np.random.default_rng(4)
    arena = rng.integers(0, 255, 1 << 16, dtype=np.uint8)
    ref = arena.copy()
    jobs = np.array([[0, 40000, 4096], [8192, 20000, 100], [30000, 50000, 7]])
    oracle.copy_jobs(arena, jobs)
    for s, d, n in jobs:
        ref[d:d + n] = ref[s:s + n]
    assert np.array_equal(arena, ref)
    src = seeded_bf16(50 * 64, 5)
    rows = np.array([3, 3, 49, 0, 17], dtype=np.int32)
    got = oracle.gather_rows(src, rows, 64).reshape(5, 64)
    assert np.array_equal(got, src.reshape(50, 64)[rows])


@pytest.mark.parametrize("workers,threads", [(1, 1), (3, 2), (16, 8), (200, 8)])
def test_fanned_out_copy_and_gather_closed_form(workers, threads):
    """dispatch_copy_jobs' 64-byte aligned worker shares (page_copy.mojo:18-60)
    and dispatch_gather_rows' row shares write what the jobs and rows say,
    whatever the worker count: shares that end mid-job, jobs shorter than 64
    bytes, an empty job and more workers than aligned shares."""
    rng = np.random.default_rng(40 + workers)
    arena = rng.integers(0, 255, 1 << 18, dtype=np.uint8)
    ref = arena.copy()
    jobs = np.array([[0, 140000, 65536], [70000, 210000, 333], [80001, 220001, 7],
                     [90000, 230000, 0], [100003, 240007, 5000]])
    oracle.copy_jobs_workers(arena, jobs, workers, threads)
    for s, d, n in jobs:
        ref[d:d + n] = ref[s:s + n]
    assert np.array_equal(arena, ref)
    src = seeded_bf16(300 * 96, 6)
    rows = rng.integers(0, 300, 257).astype(np.int32)
    got = oracle.gather_rows_workers(src, rows, 96, workers, threads).reshape(-1, 96)
    assert np.array_equal(got, src.reshape(300, 96)[rows])


def test_bq_oracle_against_reference_head_schedule():
    """tests/test_sliding_attention_degree_parity.mojo at degree 1: the oracle's
    prep + bq sliding attention over the reference's 10-step schedule must stay
    within the reference's 0.05 of its exact-exp scalar reference_head."""
    cos, sin, norm = bq.constant_tables()
    k_cache = np.zeros(bq.CACHE_ROWS * bq.KV_STRIDE, dtype=np.int8)
    v_cache = np.zeros_like(k_cache)
    k_scale = np.zeros(bq.CACHE_ROWS * bq.NUM_KV, dtype=np.float32)
    v_scale = np.zeros_like(k_scale)
    worst_all = 0.0
    for spec in bq.schedule():
        tok_seq, tok_pos, runs, rows, q, k, v, n = bq.step_inputs(spec)
        q_i8 = np.zeros(n * bq.Q_STRIDE, dtype=np.int8)
        qi_bias = np.zeros(n * bq.NUM_Q, dtype=np.float32)
        f_q = np.zeros_like(qi_bias)
        oracle.bq_attn_prep(runs, rows, q, k, v, norm, norm, q_i8, qi_bias, f_q, k_cache,
                            k_scale, v_cache, v_scale, cos, sin, num_q=bq.NUM_Q,
                            num_kv=bq.NUM_KV, page_shift=6, row_mask=63,
                            page_mask=bq.RING_PAGES - 1, seq_len=n, head_dim=bq.HEAD_DIM,
                            rope_half=bq.ROPE_HALF, pair_stride=bq.PAIR_STRIDE,
                            sqrt_n=bq.SQRT_HD, n_eps=bq.HD_EPS)
        out = oracle.bq_attention(0, runs, rows, q_i8, qi_bias, f_q, k_cache, k_scale,
                                  v_cache, v_scale, num_q=bq.NUM_Q, num_kv=bq.NUM_KV,
                                  head_dim=bq.HEAD_DIM, kv_stride=bq.KV_STRIDE,
                                  window=bq.WINDOW, cache_size=bq.CACHE_SIZE,
                                  page_len=bq.PAGE_LEN, seq_len=n, cap=bq.POOL_WORKERS)
        worst = bq.check_step(tok_seq, tok_pos, spec, q_i8, f_q, k_cache, k_scale, v_cache,
                              v_scale, out)
        worst_all = max(worst_all, worst)
    assert worst_all <= bq.TOL, worst_all
