"""GPU parity of the MiniMax-M3 block-sparse path through the C ABI:

- lightning indexer: selected blocks bit-exact with the oracle (and the
  reference smoke test's expectation), block scores equal as values, on
  random paged decode batches, a one-run prefill and an all-ties case that
  exercises the bank's tie order;
- block-sparse attention: within the bar (1e-2, one bf16 spacing where
  |x| >= 2) of the oracle, on the indexer's own selections and on
  hand-picked block lists with clipped last blocks."""
import numpy as np
import pytest

import oracle
from inferno_amd import attention as A
from inferno_amd.kv import FULL, AttentionPlan, KVRunTable
from tests.gpu_util import announce, empty_dev, from_dev, to_dev
from tests.helpers import assert_bar, compare_bf16, make_decode_case

pytestmark = pytest.mark.gpu

BLOCK, TOPK, IH, HD = 128, 16, 4, 128
NUM_Q, NUM_KV = 64, 4
KV_STRIDE = NUM_KV * HD
SCALE = np.float32(1.0) / np.sqrt(np.float32(HD))


def _bf(x) -> np.ndarray:
    return oracle.f32_to_bf16(np.asarray(x, dtype=np.float32).ravel())


def _plan(runs, rows, seq_len, cache_rows, page_len):
    t = KVRunTable()
    for r in runs:
        t.begin_run(int(r[0]), int(r[1]))
        for j in range(int(r[3])):
            t.add_base_row(int(rows[int(r[2]) + j]))
    return AttentionPlan(t, seq_len, kind=FULL, window=0, cache_size=page_len,
                         page_len=page_len, cache_rows=cache_rows, cap=16,
                         kv_row_bytes=KV_STRIDE * 2)


def _run_indexer(plan, index_q, index_k):
    seq = plan.seq_len
    scores = A.index_scores_buffer(plan, IH, BLOCK)
    bi = empty_dev(seq * IH * TOPK, np.int32)
    A.dispatch_lightning_indexer(plan, to_dev(index_q), to_dev(index_k), bi, scores)
    stride = scores.numel() // (seq * IH)
    return (from_dev(bi, np.int32).reshape(seq, IH, TOPK),
            from_dev(scores, np.float32).reshape(seq, IH, stride))


def _check_indexer(runs, rows, index_q, index_k, cache_rows, page_len):
    """Decode runs (one token each): GPU block ids == oracle block ids."""
    plan = _plan(runs, rows, len(runs), cache_rows, page_len)
    got, got_sc = _run_indexer(plan, index_q, index_k)
    want, want_sc = oracle.lightning_indexer(runs, rows, index_q, index_k, num_heads=IH,
                                             head_dim=HD, block_size=BLOCK, topk=TOPK,
                                             local_blocks=1, init_blocks=0, scale=SCALE,
                                             page_len=page_len, seq_len=plan.seq_len)
    assert np.array_equal(got, want), np.argwhere(got != want)[:5]
    return got, got_sc, want_sc


@pytest.mark.parametrize("page_len", [16, 64, 128])
def test_indexer_random_decode_bit_exact(page_len):
    """Pages of 16 rows take the per-lane page-table reads; pages of >= 64
    rows the scalar page-row reads (a 64-position round spans <= 2 pages)."""
    announce(f"indexer random decode page_len={page_len}")
    rng = np.random.default_rng(page_len)
    ctx = [0, 5, 127, 128, 2047, 2048, 5000, 9999]
    case = make_decode_case(17, ctx, page_len=page_len)
    index_q = _bf(rng.standard_normal(len(ctx) * IH * HD))
    index_k = _bf(rng.standard_normal(case.cache_rows * HD))
    got, got_sc, want_sc = _check_indexer(case.runs, case.base_rows, index_q, index_k,
                                          case.cache_rows, page_len)
    for i, c in enumerate(ctx):
        nb = c // BLOCK + 1
        assert np.array_equal(got_sc[i, :, :nb], want_sc[i, :, :nb]), i


def test_indexer_long_row_takes_the_bank():
    """A context past 2048 blocks (270,000 positions) skips the radix-select
    shortcut and runs the streaming bank on random scores."""
    announce("indexer long row (bank path)")
    rng = np.random.default_rng(5)
    page_len = 128
    case = make_decode_case(19, [270_000, 5], page_len=page_len)
    index_q = _bf(rng.standard_normal(2 * IH * HD))
    index_k = _bf(rng.standard_normal(case.cache_rows * HD))
    got, _, _ = _check_indexer(case.runs, case.base_rows, index_q, index_k, case.cache_rows,
                               page_len)
    assert got[0, 0, -1] == 270_000 // BLOCK


def test_indexer_reference_smoke_prefill():
    """prototypes/smoke_lightning_indexer.mojo: one run of 5000 tokens from
    position 0, identity 128-row pages, index_q = 0.01, index_k[g] = (5120 - g)
    * 0.001; probes 0, 1, 299, 2560, 4999 select blocks 0..14 and the local
    block.  A sample of tokens is also checked against the oracle."""
    announce("indexer reference smoke (5000-token prefill)")
    seq_len, page_len = 5000, BLOCK
    rows_n = (seq_len + page_len - 1) // page_len * page_len
    g = np.arange(rows_n)
    index_k = np.repeat(_bf((rows_n - g).astype(np.float32) * np.float32(0.001)), HD)
    index_q = np.full(seq_len * IH * HD, _bf([0.01])[0], dtype=np.uint16)
    rows = np.arange(rows_n // page_len, dtype=np.int32) * page_len
    runs = np.asarray([[0, 0, 0, len(rows)]], dtype=np.int32)
    plan = _plan(runs, rows, seq_len, rows_n, page_len)
    got, _ = _run_indexer(plan, index_q, index_k)
    for tok in [0, 1, 299, 2560, 4999]:
        nb = tok // BLOCK + 1
        want = (list(range(nb)) + [-1] * (TOPK - nb) if nb <= TOPK
                else list(range(TOPK - 1)) + [nb - 1])
        for h in range(IH):
            assert got[tok, h].tolist() == want, (tok, h)
    sample = [0, 1, 127, 128, 1000, 2047, 2048, 3333, 4095, 4999]
    druns = np.asarray([[i, t, 0, len(rows)] for i, t in enumerate(sample)], dtype=np.int32)
    want, _ = oracle.lightning_indexer(druns, rows, index_q[:len(sample) * IH * HD], index_k,
                                       num_heads=IH, head_dim=HD, block_size=BLOCK, topk=TOPK,
                                       local_blocks=1, init_blocks=0, scale=SCALE,
                                       page_len=page_len, seq_len=len(sample))
    assert np.array_equal(got[sample], want)


def test_indexer_all_ties_follow_the_bank_order():
    """Equal keys make every block score equal: the selection is decided by
    the bank's tie order alone (hand-derived answers for 20 and 40 blocks)."""
    announce("indexer all ties")
    page_len = 128
    ctx = [20 * BLOCK - 1, 40 * BLOCK - 1, 3 * BLOCK + 5]
    case = make_decode_case(3, ctx, page_len=page_len)
    index_k = np.full(case.cache_rows * HD, _bf([0.25])[0], dtype=np.uint16)
    index_q = np.full(len(ctx) * IH * HD, _bf([0.5])[0], dtype=np.uint16)
    got, _, _ = _check_indexer(case.runs, case.base_rows, index_q, index_k, case.cache_rows,
                               page_len)
    assert got[0, 0].tolist() == list(range(12)) + [16, 17, 18, 19]
    assert got[1, 0].tolist() == [0, 1, 2, 3, 16, 17, 18, 19, 32, 33, 34, 35, 36, 37, 38, 39]
    assert got[2, 0].tolist() == [0, 1, 2, 3] + [-1] * 12


def _sparse_inputs(rng, n_tok, cache_rows):
    q = _bf(rng.standard_normal(n_tok * NUM_Q * HD) * float(SCALE))
    k = _bf(rng.standard_normal(cache_rows * KV_STRIDE))
    v = _bf(rng.standard_normal(cache_rows * KV_STRIDE))
    return q, k, v


def _check_sparse(plan, runs, rows, q, k, v, bi, page_len):
    seq = plan.seq_len
    out = empty_dev(seq * NUM_Q * HD, np.uint16)
    A.dispatch_block_sparse_attention(plan, to_dev(q), to_dev(k), to_dev(v), to_dev(bi), out)
    got = from_dev(out, np.uint16)
    want = oracle.block_sparse_attention(runs, rows, q, k, v, bi, num_q=NUM_Q, num_kv=NUM_KV,
                                         head_dim=HD, kv_stride=KV_STRIDE, block_size=BLOCK,
                                         topk=TOPK, page_len=page_len, seq_len=seq)
    return assert_bar(compare_bf16(got, want), f"sparse seq={seq} page_len={page_len}")


@pytest.mark.parametrize("page_len", [64, 128])
def test_sparse_attention_on_indexer_selection(page_len):
    announce(f"sparse attention on indexer selection page_len={page_len}")
    rng = np.random.default_rng(100 + page_len)
    ctx = [0, 77, 300, 2048, 4100, 7000]
    case = make_decode_case(23, ctx, page_len=page_len)
    index_q = _bf(rng.standard_normal(len(ctx) * IH * HD))
    index_k = _bf(rng.standard_normal(case.cache_rows * HD))
    plan = _plan(case.runs, case.base_rows, len(ctx), case.cache_rows, page_len)
    bi, _ = _run_indexer(plan, index_q, index_k)
    q, k, v = _sparse_inputs(rng, len(ctx), case.cache_rows)
    r = _check_sparse(plan, case.runs, case.base_rows, q, k, v, bi, page_len)
    print(f"  sparse attention vs oracle: {r}", flush=True)


def test_sparse_attention_hand_picked_blocks_and_prefill_chunk():
    """A prefill chunk of 24 tokens at positions 1000..1023 (one run), each kv
    head with its own list: unsorted, early -1, a block past the causal end
    (clipped to nothing) and the partial last block."""
    announce("sparse attention hand-picked blocks, prefill chunk")
    rng = np.random.default_rng(7)
    page_len = 64
    n_tok, base = 24, 1000
    need = (base + n_tok + page_len - 1) // page_len
    rows = rng.permutation(need + 3).astype(np.int32)[:need] * page_len
    cache_rows = (need + 3) * page_len
    runs = np.asarray([[0, base, 0, need]], dtype=np.int32)
    plan = _plan(runs, rows, n_tok, cache_rows, page_len)
    bi = np.full((n_tok, NUM_KV, TOPK), -1, np.int32)
    for t in range(n_tok):
        bi[t, 0, :3] = [7, 0, 3]
        bi[t, 1, :2] = [7, 7]
        bi[t, 2, :4] = [1, 2, -1, 5]
        bi[t, 3, :3] = [9, 6, 7]
    q, k, v = _sparse_inputs(rng, n_tok, cache_rows)
    _check_sparse(plan, runs, rows, q, k, v, bi, page_len)


def test_sparse_rejects_unsupported_shapes():
    from inferno_amd._lib import InfernoHipError

    case = make_decode_case(1, [100], page_len=64)
    plan = _plan(case.runs, case.base_rows, 1, case.cache_rows, 64)
    q = empty_dev(NUM_Q * HD, np.uint16)
    kv = empty_dev(case.cache_rows * KV_STRIDE, np.uint16)
    bi = empty_dev(NUM_KV * TOPK, np.int32)
    out = empty_dev(NUM_Q * HD, np.uint16)
    with pytest.raises(InfernoHipError):
        A.dispatch_block_sparse_attention(plan, q, kv, kv, bi, out, num_q=32)   # gqa 8
    with pytest.raises(InfernoHipError):
        A.dispatch_block_sparse_attention(plan, q, kv, kv, bi, out, head_dim=256)
    scores = A.index_scores_buffer(plan, IH, BLOCK)
    with pytest.raises(InfernoHipError):
        A.dispatch_lightning_indexer(plan, q, kv, bi, scores, topk_blocks=33)


def _bq_inputs(rng, n_tok, cache_rows):
    q = rng.integers(-127, 128, n_tok * NUM_Q * HD).astype(np.int8)
    qb = (q.reshape(-1, HD).astype(np.int64).sum(axis=1) * 128).astype(np.float32)
    fq = rng.uniform(0.002, 0.02, n_tok * NUM_Q).astype(np.float32)
    k = rng.integers(-127, 128, cache_rows * KV_STRIDE).astype(np.int8)
    v = rng.integers(-127, 128, cache_rows * KV_STRIDE).astype(np.int8)
    ks = rng.uniform(0.5, 4.0, cache_rows * NUM_KV).astype(np.float32)
    vs = rng.uniform(0.5, 4.0, cache_rows * NUM_KV).astype(np.float32)
    return q, qb, fq, k, ks, v, vs


def _check_bq_sparse(plan, runs, rows, inputs, bi, page_len, cap):
    q, qb, fq, k, ks, v, vs = inputs
    seq = plan.seq_len
    out = empty_dev(seq * NUM_Q * HD, np.uint16)
    A.dispatch_bq_block_sparse_attention(plan, to_dev(q), to_dev(qb), to_dev(fq), to_dev(k),
                                         to_dev(ks), to_dev(v), to_dev(vs), to_dev(bi), out,
                                         cap=cap)
    got = from_dev(out, np.uint16)
    want = oracle.bq_block_sparse_attention(runs, rows, q, qb, fq, k, ks, v, vs, bi,
                                            num_q=NUM_Q, num_kv=NUM_KV, head_dim=HD,
                                            kv_stride=KV_STRIDE, block_size=BLOCK, topk=TOPK,
                                            page_len=page_len, seq_len=seq, cap=cap)
    return assert_bar(compare_bf16(got, want), f"sparse seq={seq} page_len={page_len}")


@pytest.mark.parametrize("cap", [1, 7, 64])
def test_bq_sparse_decode_worker_bands(cap):
    """seq_len 1: the (kv head, slot) units banded over min(cap, units)
    workers, selections from the GPU indexer plus a list with -1 holes."""
    announce(f"bq sparse decode cap={cap}")
    rng = np.random.default_rng(300 + cap)
    page_len = 128
    case = make_decode_case(31, [7000], page_len=page_len)
    plan = _plan(case.runs, case.base_rows, 1, case.cache_rows, page_len)
    index_q = _bf(rng.standard_normal(IH * HD))
    index_k = _bf(rng.standard_normal(case.cache_rows * HD))
    bi, _ = _run_indexer(plan, index_q, index_k)
    bi[0, 2, 3] = -1
    bi[0, 2, 9] = -1
    inputs = _bq_inputs(rng, 1, case.cache_rows)
    r = _check_bq_sparse(plan, case.runs, case.base_rows, inputs, bi, page_len, cap)
    print(f"  bq sparse decode cap={cap}: {r}", flush=True)


def test_bq_sparse_prefill_chunk():
    """seq_len > 1: a 20-token chunk at positions 1000..1019, per-head lists
    with an early -1, a repeated block and a block past the causal end."""
    announce("bq sparse prefill chunk")
    rng = np.random.default_rng(41)
    page_len = 64
    n_tok, base = 20, 1000
    need = (base + n_tok + page_len - 1) // page_len
    rows = rng.permutation(need + 2).astype(np.int32)[:need] * page_len
    cache_rows = (need + 2) * page_len
    runs = np.asarray([[0, base, 0, need]], dtype=np.int32)
    plan = _plan(runs, rows, n_tok, cache_rows, page_len)
    bi = np.full((n_tok, NUM_KV, TOPK), -1, np.int32)
    for t in range(n_tok):
        bi[t, 0, :3] = [7, 0, 3]
        bi[t, 1, :2] = [7, 7]
        bi[t, 2, :4] = [1, 2, -1, 5]
        bi[t, 3, :3] = [9, 6, 7]
    _check_bq_sparse(plan, runs, rows, _bq_inputs(rng, n_tok, cache_rows), bi, page_len, cap=8)


@pytest.mark.parametrize("page_len", [64, 128])
def test_bq_sparse_batched_decode_on_indexer_selection(page_len):
    """seq_len > 1 with one token per sequence (config 6's batched decode):
    the four-waves-per-(token, kv head) int8 kernel with its rotating tile
    registers, over the GPU indexer's selections, including a sequence of
    position 0 and a long one that fills all 16 slots."""
    announce(f"bq sparse batched decode page_len={page_len}")
    rng = np.random.default_rng(500 + page_len)
    ctx = [0, 77, 300, 2048, 4100, 7000, 20000]
    case = make_decode_case(29, ctx, page_len=page_len)
    index_q = _bf(rng.standard_normal(len(ctx) * IH * HD))
    index_k = _bf(rng.standard_normal(case.cache_rows * HD))
    plan = _plan(case.runs, case.base_rows, len(ctx), case.cache_rows, page_len)
    bi, _ = _run_indexer(plan, index_q, index_k)
    inputs = _bq_inputs(rng, len(ctx), case.cache_rows)
    r = _check_bq_sparse(plan, case.runs, case.base_rows, inputs, bi, page_len, cap=8)
    print(f"  bq sparse batched decode vs oracle: {r}", flush=True)
