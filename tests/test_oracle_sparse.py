"""CPU pins of the oracle's MiniMax-M3 block-sparse path (prototypes/, degree 1):

- the reference's own lightning-indexer smoke test
  (prototypes/smoke_lightning_indexer.mojo:73-150: monotone keys select
  blocks 0..14 plus the local block) at its probe tokens;
- hand-derived known answers for the top-k bank's tie order (reduce_argmax
  prefers the smaller lane, then register), with and without a bank refill;
- invariants of the selection on random scores (sorted, local block kept,
  the rest the largest scores);
- block scores against a float64 max over each block's causal positions;
- sparse attention: the q = 0 closed form over the selected blocks' tiles,
  and bit-equality with the dense oracle when every block is selected."""
import numpy as np
import pytest

import oracle

BLOCK, TOPK, HEADS, HD = 128, 16, 4, 128
SCALE = np.float32(1.0) / np.sqrt(np.float32(HD))


def _bf(x) -> np.ndarray:
    return oracle.f32_to_bf16(np.asarray(x, dtype=np.float32).ravel())


def _identity_pages(num_rows: int, page_len: int) -> np.ndarray:
    return np.arange((num_rows + page_len - 1) // page_len, dtype=np.int32) * page_len


def _decode_runs(positions, pages_per_run: int) -> np.ndarray:
    """One single-token run per position, all over the same identity page table."""
    return np.asarray([[i, p, 0, pages_per_run] for i, p in enumerate(positions)],
                      dtype=np.int32)


def test_reference_smoke_monotone_keys():
    seq_len, page_len = 5000, BLOCK
    num_key_rows = (seq_len + page_len - 1) // page_len * page_len
    g = np.arange(num_key_rows)
    kval = (num_key_rows - g).astype(np.float32) * np.float32(0.001)
    index_k = np.repeat(_bf(kval), HD)
    probes = [0, 1, 299, 2560, 4999]
    index_q = np.full(len(probes) * HEADS * HD, _bf([0.01])[0], dtype=np.uint16)
    rows = _identity_pages(num_key_rows, page_len)
    runs = _decode_runs(probes, len(rows))
    idx, _ = oracle.lightning_indexer(runs, rows, index_q, index_k, num_heads=HEADS,
                                      head_dim=HD, block_size=BLOCK, topk=TOPK,
                                      local_blocks=1, init_blocks=0, scale=SCALE,
                                      page_len=page_len, seq_len=len(probes))
    for i, tok in enumerate(probes):
        nb = tok // BLOCK + 1
        if nb <= TOPK:
            want = list(range(nb)) + [-1] * (TOPK - nb)
        else:
            want = list(range(TOPK - 1)) + [nb - 1]
        for h in range(HEADS):
            assert idx[i, h].tolist() == want, (tok, h)


def test_bank_tie_order_without_refill():
    # 20 equal scores, block 19 forced: after it the ties go by lane, then
    # register: slots 0, 16, 1, 17, 2, 18, 3, 4, ..., 11.
    got = oracle.select_blocks(np.full(20, 0.5, np.float32), 20, topk=TOPK, local_blocks=1,
                               init_blocks=0)
    assert got.tolist() == list(range(12)) + [16, 17, 18, 19]


def test_bank_tie_order_with_refill():
    # 40 equal scores: the first full bank (blocks 0..31) keeps slots 0,16,1,17,
    # ..,7,23 = blocks 0..7 and 16..23 in that order; blocks 32..39 refill slots
    # 16..23 (39 forced); the final pass then takes 39 and
    # 0,32,16,33,1,34,17,35,2,36,18,37,3,38,19.
    got = oracle.select_blocks(np.full(40, 0.5, np.float32), 40, topk=TOPK, local_blocks=1,
                               init_blocks=0)
    assert got.tolist() == [0, 1, 2, 3, 16, 17, 18, 19, 32, 33, 34, 35, 36, 37, 38, 39]


@pytest.mark.parametrize("nb,local,init", [(1, 1, 0), (7, 1, 0), (16, 1, 0), (17, 1, 0),
                                           (100, 1, 0), (333, 2, 1), (1000, 1, 3)])
def test_selection_invariants_on_random_scores(nb, local, init):
    rng = np.random.default_rng(nb)
    scores = rng.standard_normal(nb).astype(np.float32)
    got = oracle.select_blocks(scores, nb, topk=TOPK, local_blocks=local, init_blocks=init)
    sel = [int(b) for b in got if b >= 0]
    assert all(b == -1 for b in got[len(sel):])
    assert sel == sorted(set(sel)) and len(sel) == min(TOPK, nb)
    forced = {b for b in range(nb) if b >= nb - local or b < init}
    assert forced <= set(sel)
    free = [b for b in range(nb) if b not in forced]
    want_free = sorted(free, key=lambda b: -scores[b])[:min(TOPK, nb) - len(forced)]
    assert set(sel) - forced == set(want_free)


def test_block_scores_match_float64_block_max():
    rng = np.random.default_rng(3)
    page_len = 64
    positions = [0, 130, 700, 1023]
    num_rows = 1024 + page_len
    rows = rng.permutation(num_rows // page_len).astype(np.int32) * page_len
    runs = _decode_runs(positions, len(rows))
    index_q = _bf(rng.standard_normal(len(positions) * HEADS * HD))
    index_k = _bf(rng.standard_normal(num_rows * HD))
    sc = oracle.index_block_scores(runs, rows, index_q, index_k, num_heads=HEADS, head_dim=HD,
                                   block_size=BLOCK, scale=SCALE, page_len=page_len,
                                   seq_len=len(positions))
    qf = oracle.bf16_to_f32(index_q).astype(np.float64).reshape(len(positions), HEADS, HD)
    kf = oracle.bf16_to_f32(index_k).astype(np.float64).reshape(num_rows, HD)
    for i, p in enumerate(positions):
        slots = np.array([rows[x // page_len] + x % page_len for x in range(p + 1)])
        d = (kf[slots] @ qf[i].T) * float(SCALE)          # [pos][head]
        nb = p // BLOCK + 1
        for b in range(nb):
            want = d[b * BLOCK:min((b + 1) * BLOCK, p + 1)].max(axis=0)
            assert np.allclose(sc[i, :, b], want, rtol=0, atol=2e-5 * np.abs(d).max()), (i, b)


def _sparse_case(rng, positions, num_q, num_kv, page_len=64):
    D = HD
    kv_stride = num_kv * D
    num_rows = (max(positions) // page_len + 2) * page_len
    rows = rng.permutation(num_rows // page_len).astype(np.int32) * page_len
    runs = _decode_runs(positions, len(rows))
    k = _bf(rng.standard_normal(num_rows * kv_stride))
    v = _bf(rng.standard_normal(num_rows * kv_stride))
    return runs, rows, k, v, kv_stride


def test_sparse_attention_q0_closed_form():
    rng = np.random.default_rng(4)
    positions = [1000, 77]
    num_q, num_kv = 64, 4
    gqa = num_q // num_kv
    runs, rows, k, v, kv_stride = _sparse_case(rng, positions, num_q, num_kv)
    # Token 0 (position 1000, 8 blocks, the last one clipped to 105
    # positions): different block lists per kv head; token 1: block 0 only.
    bi = np.full((len(positions), num_kv, TOPK), -1, np.int32)
    bi[0, 0, :3] = [0, 3, 7]
    bi[0, 1, :3] = [1, 2, 7]
    bi[0, 2, :1] = [7]
    bi[0, 3, :3] = [0, 5, 6]
    bi[1, :, 0] = 0
    q = np.zeros(len(positions) * num_q * HD, np.uint16)
    out = oracle.block_sparse_attention(runs, rows, q, k, v, bi, num_q=num_q, num_kv=num_kv,
                                        head_dim=HD, kv_stride=kv_stride, block_size=BLOCK,
                                        topk=TOPK, page_len=64, seq_len=len(positions))
    got = oracle.bf16_to_f32(out).astype(np.float64).reshape(len(positions), num_q, HD)
    c = float(oracle.fexp(np.zeros(1, np.float32))[0])
    vf = oracle.bf16_to_f32(v).astype(np.float64).reshape(-1, num_kv, HD)
    for i, p in enumerate(positions):
        for h in range(num_kv):
            tiles = []
            for b in bi[i, h]:
                if b < 0:
                    break
                lo, hi = b * BLOCK, min((b + 1) * BLOCK, p + 1)
                tiles += [list(range(s, min(s + 16, hi))) for s in range(lo, hi, 16)]
            n = len(tiles)
            num = np.zeros(HD)
            den = 0.0
            for j, tile in enumerate(tiles):
                wgt = c ** (n - j)
                slots = [rows[x // 64] + x % 64 for x in tile]
                num += wgt * vf[slots, h].sum(axis=0)
                den += wgt * len(tile)
            want = num / den
            for r in range(gqa):
                assert np.allclose(got[i, h * gqa + r], want, atol=1e-2, rtol=0), (i, h, r)


def test_sparse_equals_dense_when_every_block_is_selected():
    rng = np.random.default_rng(5)
    num_q, num_kv = 16, 2
    for p in [5, 200, 1500]:
        runs, rows, k, v, kv_stride = _sparse_case(rng, [p], num_q, num_kv)
        q = _bf(rng.standard_normal(num_q * HD))
        nb = p // BLOCK + 1
        bi = np.full((1, num_kv, TOPK), -1, np.int32)
        bi[0, :, :nb] = np.arange(nb)
        sparse = oracle.block_sparse_attention(runs, rows, q, k, v, bi, num_q=num_q,
                                               num_kv=num_kv, head_dim=HD, kv_stride=kv_stride,
                                               block_size=BLOCK, topk=TOPK, page_len=64,
                                               seq_len=1)
        dense = oracle.attention(1, runs, rows, q, k, v, num_q=num_q, num_kv=num_kv,
                                 head_dim=HD, kv_stride=kv_stride, window=0, cache_size=64,
                                 page_len=64, seq_len=1, cap=1)
        assert np.array_equal(sparse, dense), p


def _bq_case(rng, positions, num_q, num_kv, kv_stride, page_len=64):
    D = HD
    num_rows = (max(positions) // page_len + 2) * page_len
    rows = rng.permutation(num_rows // page_len).astype(np.int32) * page_len
    runs = _decode_runs(positions, len(rows))
    q = rng.integers(-127, 128, len(positions) * num_q * D).astype(np.int8)
    qb = (q.reshape(-1, D).astype(np.int64).sum(axis=1) * 128).astype(np.float32)
    fq = rng.uniform(0.5, 2.0, len(positions) * num_q).astype(np.float32)
    k = rng.integers(-127, 128, num_rows * kv_stride).astype(np.int8)
    v = rng.integers(-127, 128, num_rows * kv_stride).astype(np.int8)
    ks = rng.uniform(0.5, 4.0, num_rows * num_kv).astype(np.float32)
    vs = rng.uniform(0.5, 4.0, num_rows * num_kv).astype(np.float32)
    return runs, rows, q, qb, fq, k, ks, v, vs


@pytest.mark.parametrize("cap,nb", [(1, 5), (32, 16)])
def test_bq_sparse_decode_equals_dense_decode(cap, nb):
    """Every block selected: with one worker (cap 1) the decode route is the
    dense decode's single split; with 16 blocks and one (head, block) unit per
    worker, each head's stripes are exactly the dense decode's 16 block-aligned
    splits (16 = one merge batch), so the outputs are bit-equal."""
    rng = np.random.default_rng(cap + nb)
    num_q, num_kv, kv_stride = 16, 2, 1024
    p = nb * BLOCK - 1
    runs, rows, q, qb, fq, k, ks, v, vs = _bq_case(rng, [p], num_q, num_kv, kv_stride)
    bi = np.full((1, num_kv, TOPK), -1, np.int32)
    bi[0, :, :nb] = np.arange(nb)
    sparse = oracle.bq_block_sparse_attention(runs, rows, q, qb, fq, k, ks, v, vs, bi,
                                              num_q=num_q, num_kv=num_kv, head_dim=HD,
                                              kv_stride=kv_stride, block_size=BLOCK, topk=TOPK,
                                              page_len=64, seq_len=1, cap=cap)
    dense_cap = 1 if cap == 1 else nb
    assert oracle.recommended_workers((p + 1) * kv_stride, dense_cap) == dense_cap
    dense = oracle.bq_attention(1, runs, rows, q, qb, fq, k, ks, v, vs, num_q=num_q,
                                num_kv=num_kv, head_dim=HD, kv_stride=kv_stride, window=0,
                                cache_size=64, page_len=64, seq_len=1, cap=dense_cap)
    assert np.array_equal(sparse, dense)


def test_bq_sparse_routes_q0_closed_form():
    """q = 0 makes every score 0: each stripe weights its tiles by powers of
    fexp(0) in walk order, so the output pins the decode route's worker bands
    (cap 3 over 4 kv heads x 5 slots, -1 slots skipped) and the prefill route's
    stop at -1."""
    rng = np.random.default_rng(9)
    num_q, num_kv = 64, 4
    gqa, kv_stride = num_q // num_kv, num_kv * HD
    c = float(oracle.fexp(np.zeros(1, np.float32))[0])
    for positions in ([1000], [1000, 300]):
        runs, rows, q, qb, fq, k, ks, v, vs = _bq_case(rng, positions, num_q, num_kv,
                                                       kv_stride)
        q[:] = 0
        qb[:] = 0
        bi = np.full((len(positions), num_kv, TOPK), -1, np.int32)
        lists = [[7, 0, 3, -1, 5], [1, -1, 2, 2, 6], [7, 6, 5, 4, 3], [-1, -1, 0, 1, 2]]
        for i in range(len(positions)):
            for h in range(num_kv):
                bi[i, h, :5] = lists[h]
        seq = len(positions)
        out = oracle.bq_block_sparse_attention(runs, rows, q, qb, fq, k, ks, v, vs, bi,
                                               num_q=num_q, num_kv=num_kv, head_dim=HD,
                                               kv_stride=kv_stride, block_size=BLOCK,
                                               topk=TOPK, page_len=64, seq_len=seq, cap=3)
        got = oracle.bf16_to_f32(out).astype(np.float64).reshape(seq, num_q, HD)
        vf = v.astype(np.float64).reshape(-1, num_kv, HD)
        vsf = vs.astype(np.float64).reshape(-1, num_kv)

        def walk(tok, h, slots, stop):
            tiles = []
            for sidx in slots:
                b = int(bi[tok, h, sidx])
                if b < 0:
                    if stop:
                        break
                    continue
                lo, hi = b * BLOCK, min((b + 1) * BLOCK, positions[tok] + 1)
                tiles += [list(range(s0, min(s0 + 16, hi))) for s0 in range(lo, hi, 16)]
            n = len(tiles)
            num, den = np.zeros(HD), 0.0
            for j, tile in enumerate(tiles):
                wgt = c ** (n - j)
                sl = [rows[x // 64] + x % 64 for x in tile]
                num += wgt * (vf[sl, h] * vsf[sl, h][:, None] / 127.0).sum(axis=0)
                den += wgt * len(tile)
            return num, den

        for i, p in enumerate(positions):
            for h in range(num_kv):
                if seq == 1:
                    slots_n = min(TOPK, p // BLOCK + 1)
                    total, workers = num_kv * slots_n, min(3, num_kv * slots_n)
                    per = -(-total // workers)
                    num, den = np.zeros(HD), 0.0
                    for w in range(workers):
                        lo, hi = min(w * per, total), min(w * per + per, total)
                        s_lo = max(lo, h * slots_n) - h * slots_n
                        s_hi = min(hi, (h + 1) * slots_n) - h * slots_n
                        if s_lo >= s_hi:
                            continue
                        a, d = walk(i, h, range(s_lo, s_hi), stop=False)
                        num, den = num + c * a, den + c * d
                else:
                    num, den = walk(i, h, range(TOPK), stop=True)
                want = num / den if den > 0 else np.zeros(HD)  # no tiles: zeros
                for r in range(gqa):
                    assert np.allclose(got[i, h * gqa + r], want, atol=1e-2, rtol=0), (seq, i, h)
