"""GPU parity at Gemma-4's full-attention layer shape: head_dim 512, 16 q / 2 kv
heads (GQA 8), partial RoPE over 64 pairs at pair_stride 256
(modeling/gemma4_common.mojo:14-20), as dispatch_full_attention_qkv and
dispatch_bq_full_attention_qkv call the path (modeling/gemma_4_moe.mojo:
395-490, modeling/gemma_4_moe_bq.mojo:527-620).

- append (rope_cache_write) bit-exact, and the fused head norm + append with
  V taken from the raw K projection (the full layer's V, gemma_4_moe.mojo:
  441-448), bit-exact;
- bf16 decode (batched, all merge routes) and a prefill chunk within 1e-2
  of the oracle (one bf16 spacing where |x| >= 2);
- bq prep (codes, scales, q bias and f_q) bit-exact with partial RoPE and
  gains, and bq decode outputs bit-exact (integer MFMA scores, the
  reference's softmax and per-element P.V order), with the o_proj block
  quant fused into the merge at block 512; a bq prefill chunk (MFMA route)
  within 1e-2."""
import numpy as np
import pytest

import oracle
from inferno_amd import attention as A
from inferno_amd.kv import FULL, AttentionPlan, KVRunTable
from tests.gpu_util import announce, empty_dev, from_dev, to_dev
from tests.helpers import assert_bar, compare_bf16, make_decode_case, make_prefill_case, seeded_bf16

pytestmark = pytest.mark.gpu

NQ, NKV, D = 16, 2, 512
KVS = NKV * D
HALF, PAIR = 64, 256
SQRT_HD = float(np.sqrt(np.float32(D)))
HD_EPS = float(np.float32(D) * np.float32(1e-6))
PAGE = 64


def _table(runs, rows) -> KVRunTable:
    t = KVRunTable()
    for r in runs:
        t.begin_run(int(r[0]), int(r[1]))
        for j in range(int(r[3])):
            t.add_base_row(int(rows[int(r[2]) + j]))
    return t


def _bf16(x: np.ndarray) -> np.ndarray:
    u = np.ascontiguousarray(x, dtype=np.float32).view(np.uint32).astype(np.uint64)
    return ((u + ((u >> 16) & 1) + 0x7FFF) >> 16).astype(np.uint16)


def _tables(max_pos: int, seed: int):
    ang = np.random.default_rng(seed).uniform(-3, 3, (max_pos + 2) * HALF)
    return np.cos(ang).astype(np.float32), np.sin(ang).astype(np.float32)


def _plan(case, seq_len, cap, kv_row_bytes):
    return AttentionPlan(_table(case.runs, case.base_rows), seq_len, kind=FULL, window=0,
                         cache_size=PAGE, page_len=PAGE, cache_rows=case.cache_rows, cap=cap,
                         kv_row_bytes=kv_row_bytes)


def test_full_layer_append_partial_rope():
    """rope_cache_write at half 64 / pair_stride 256, then the fused norm +
    append with v_src = k_src: q, k and v cache rows bit-exact."""
    announce("full layer append")
    case = make_decode_case(3, [100, 1300, 7, 640])
    n = len(case.ctx)
    cos, sin = _tables(int(case.ctx.max()) + 1, 4)
    rng = np.random.default_rng(5)
    gq = _bf16(rng.uniform(0.5, 1.5, D))
    gk = _bf16(rng.uniform(0.5, 1.5, D))
    q = seeded_bf16(n * NQ * D, 6)
    kn = seeded_bf16(n * KVS, 7)
    vn = seeded_bf16(n * KVS, 8)
    rows = case.cache_rows
    kc = seeded_bf16(rows * KVS, 9)
    vc = seeded_bf16(rows * KVS, 10)
    plan = _plan(case, n, 16, KVS * 2)

    dq, dk, dv = to_dev(q), to_dev(kc), to_dev(vc)
    A.dispatch_rope_cache_write(plan, dq, to_dev(kn), to_dev(vn), dk, dv, to_dev(cos),
                                to_dev(sin), num_q=NQ, num_kv=NKV, half=HALF,
                                pair_stride=PAIR, head_dim=D)
    q_ref, k_ref, v_ref = q.copy(), kc.copy(), vc.copy()
    oracle.rope_cache_write(case.runs, case.base_rows, q_ref, kn, vn, k_ref, v_ref, cos, sin,
                            num_q=NQ, num_kv=NKV, page_shift=6, row_mask=63, page_mask=-1,
                            seq_len=n, half=HALF, pair_stride=PAIR, head_dim=D)
    assert np.array_equal(from_dev(dq, np.uint16), q_ref), "q differs"
    assert np.array_equal(from_dev(dk, np.uint16), k_ref), "k cache differs"
    assert np.array_equal(from_dev(dv, np.uint16), v_ref), "v cache differs"

    # The full layer's V is the raw K projection normalised without a gain.
    dq2, dk2, dv2 = to_dev(q), to_dev(kc), to_dev(vc)
    dkn = to_dev(kn)
    A.dispatch_rms_norm_rope_cache_write(plan, dq2, dkn, dkn, dk2, dv2, to_dev(gq), to_dev(gk),
                                         to_dev(cos), to_dev(sin), num_q=NQ, num_kv=NKV,
                                         half=HALF, pair_stride=PAIR, head_dim=D,
                                         sqrt_n=SQRT_HD, n_eps=HD_EPS)
    q_ref, k_ref, v_ref = q.copy(), kc.copy(), vc.copy()
    kk, vv = kn.copy(), kn.copy()
    oracle.rms_norm_qkv_heads(q_ref, kk, vv, gq, gk, num_q=NQ, num_kv=NKV, seq_len=n,
                              head_dim=D, sqrt_n=SQRT_HD, n_eps=HD_EPS)
    oracle.rope_cache_write(case.runs, case.base_rows, q_ref, kk, vv, k_ref, v_ref, cos, sin,
                            num_q=NQ, num_kv=NKV, page_shift=6, row_mask=63, page_mask=-1,
                            seq_len=n, half=HALF, pair_stride=PAIR, head_dim=D)
    assert np.array_equal(from_dev(dq2, np.uint16), q_ref), "normed q differs"
    assert np.array_equal(from_dev(dk2, np.uint16), k_ref), "normed k cache differs"
    assert np.array_equal(from_dev(dv2, np.uint16), v_ref), "normed v cache differs"
    assert np.array_equal(from_dev(dkn, np.uint16), kn), "k_src was modified"


def _bf16_attention(case, seq_len, cap, seed):
    q = seeded_bf16(seq_len * NQ * D, seed)
    k = seeded_bf16(case.cache_rows * KVS, seed + 1)
    v = seeded_bf16(case.cache_rows * KVS, seed + 2)
    plan = _plan(case, seq_len, cap, KVS * 2)
    out = empty_dev(seq_len * NQ * D, np.uint16)
    partials, ps = A.partials_buffer(plan, NQ, D)
    A.attention_bf16(plan, to_dev(q), to_dev(k), to_dev(v), out, partials, ps, num_q=NQ,
                     num_kv=NKV, head_dim=D, kv_stride=KVS)
    got = from_dev(out, np.uint16)
    ref = oracle.attention(FULL, case.runs, case.base_rows, q, k, v, num_q=NQ, num_kv=NKV,
                           head_dim=D, kv_stride=KVS, window=0, cache_size=PAGE,
                           page_len=PAGE, seq_len=seq_len, cap=cap, threads=8)
    return assert_bar(compare_bf16(got, ref), f"mode={plan.summary.mode} "
                      f"items={plan.summary.num_items} stripes={plan.summary.num_stripes}")


@pytest.mark.parametrize("cap", [1, 16, 256, 1024, 4096])
def test_full_layer_decode(cap):
    """Batched decode over ragged contexts: cap 1 gives one split per
    sequence seeded then capped, 16 a few splits per unit (merge_kernel), 256
    and 1024 tens to a hundred (merge_staged_kernel), 4096 a split per tile."""
    announce(f"full layer decode cap={cap}")
    rng = np.random.default_rng(100 + cap)
    ctx = [int(x) for x in rng.integers(1, 3000, 6)] + [0, 15, 16, 17]
    case = make_decode_case(200 + cap, ctx)
    _bf16_attention(case, len(ctx), cap, 300 + cap)


def test_full_layer_single_sequence():
    """seq_len 1 routes through recommended_workers (config-1-like)."""
    announce("full layer single sequence")
    case = make_decode_case(41, [4095])
    _bf16_attention(case, 1, 128, 42)


def test_full_layer_token_prefill():
    """A short prefill chunk at this shape (the MFMA prefill route;
    test_gpu_prefill_wide.py covers it in depth)."""
    announce("full layer token prefill")
    case = make_prefill_case(9, [0, 300, 77], [20, 45, 33])
    _bf16_attention(case, 98, 16, 80)


class _BqCache:
    def __init__(self, rows):
        self.k = np.zeros(rows * KVS, dtype=np.int8)
        self.v = np.zeros(rows * KVS, dtype=np.int8)
        self.ks = np.zeros(rows * NKV, dtype=np.float32)
        self.vs = np.zeros(rows * NKV, dtype=np.float32)
        self.dk, self.dv = to_dev(self.k), to_dev(self.v)
        self.dks, self.dvs = to_dev(self.ks), to_dev(self.vs)

    def assert_equal(self):
        for dev, host, dt, name in ((self.dk, self.k, np.int8, "k codes"),
                                    (self.dv, self.v, np.int8, "v codes"),
                                    (self.dks, self.ks, np.float32, "k scales"),
                                    (self.dvs, self.vs, np.float32, "v scales")):
            got = from_dev(dev, dt)
            if dt == np.float32:
                got, host = got.view(np.uint32), host.view(np.uint32)
            assert np.array_equal(got, host), (name, int((got != host).sum()))


def _outliers(x, seed):
    f = (x.astype(np.uint32) << 16).view(np.float32).copy()
    f[np.random.default_rng(seed).random(f.size) < 0.01] *= 20
    return _bf16(f)


def _bq_step(cache, runs, rows, cache_rows, seq_len, cap, q, kraw, gq, gk, cos, sin,
             attend=True):
    """bq prep with v_src = k_src (the full layer's raw K projection), then
    (attend) bq attention with and without the o_proj block quant; prep,
    decode and the quant against the oracle bit for bit, a prefill chunk on
    the MFMA route within 1e-2 (one bf16 spacing where |x| >= 2)."""
    table = _table(runs, rows)
    plan = AttentionPlan(table, seq_len, kind=FULL, window=0, cache_size=PAGE, page_len=PAGE,
                         cache_rows=cache_rows, cap=cap, kv_row_bytes=KVS)
    dq_i8 = empty_dev(seq_len * NQ * D, np.int8)
    dqb = empty_dev(seq_len * NQ, np.float32)
    dfq = empty_dev(seq_len * NQ, np.float32)
    dkraw = to_dev(kraw)
    A.dispatch_bq_attn_prep(plan, to_dev(q), dkraw, dkraw, to_dev(gq), to_dev(gk), dq_i8, dqb,
                            dfq, cache.dk, cache.dks, cache.dv, cache.dvs, to_dev(cos),
                            to_dev(sin), num_q=NQ, num_kv=NKV, head_dim=D, rope_half=HALF,
                            pair_stride=PAIR, sqrt_n=SQRT_HD, n_eps=HD_EPS)
    q_i8 = np.zeros(seq_len * NQ * D, dtype=np.int8)
    qb = np.zeros(seq_len * NQ, dtype=np.float32)
    fq = np.zeros_like(qb)
    oracle.bq_attn_prep(runs, rows, q, kraw, kraw, gq, gk, q_i8, qb, fq, cache.k, cache.ks,
                        cache.v, cache.vs, cos, sin, num_q=NQ, num_kv=NKV, page_shift=6,
                        row_mask=63, page_mask=-1, seq_len=seq_len, head_dim=D,
                        rope_half=HALF, pair_stride=PAIR, sqrt_n=SQRT_HD, n_eps=HD_EPS)
    assert np.array_equal(from_dev(dq_i8, np.int8), q_i8), "q codes differ"
    assert np.array_equal(from_dev(dqb, np.float32).view(np.uint32), qb.view(np.uint32))
    assert np.array_equal(from_dev(dfq, np.float32).view(np.uint32), fq.view(np.uint32))
    cache.assert_equal()
    if not attend:
        return

    out = empty_dev(seq_len * NQ * D, np.uint16)
    partials, ps = A.partials_buffer(plan, NQ, D)
    A.bq_attention(plan, dq_i8, dqb, dfq, cache.dk, cache.dks, cache.dv, cache.dvs, out,
                   partials, ps, num_q=NQ, num_kv=NKV, head_dim=D, kv_stride=KVS)
    out2 = empty_dev(seq_len * NQ * D, np.uint16)
    o_i8 = empty_dev(seq_len * NQ * D, np.int8)
    o_sa = empty_dev(seq_len * NQ, np.float32)
    A.bq_attention(plan, dq_i8, dqb, dfq, cache.dk, cache.dks, cache.dv, cache.dvs, out2,
                   partials, ps, num_q=NQ, num_kv=NKV, head_dim=D, kv_stride=KVS, o_i8=o_i8,
                   o_sa=o_sa)
    got = from_dev(out, np.uint16)
    ref = oracle.bq_attention(FULL, runs, rows, q_i8, qb, fq, cache.k, cache.ks, cache.v,
                              cache.vs, num_q=NQ, num_kv=NKV, head_dim=D, kv_stride=KVS,
                              window=0, cache_size=PAGE, page_len=PAGE, seq_len=seq_len,
                              cap=cap, threads=8)
    r = compare_bf16(got, ref)
    mfma = plan.summary.mode == 2 and int(plan.info[14]) > 0
    label = f"bq mode={plan.summary.mode} stripes={plan.summary.num_stripes} mfma={mfma}"
    if mfma:  # the MFMA prefill: the bf16 prefill's bar
        assert_bar(r, label)
    else:
        print(f"  {label}: {r}", flush=True)
        assert np.array_equal(got, ref), r
    assert np.array_equal(from_dev(out2, np.uint16), got), "fused quant changed the output"
    want_i8, want_sa = oracle.bq_block_quant(got, cols=NQ * D, block=D)
    assert np.array_equal(from_dev(o_i8, np.int8).reshape(seq_len, NQ * D), want_i8)
    assert np.array_equal(from_dev(o_sa, np.float32).view(np.uint32),
                          want_sa.reshape(-1).view(np.uint32))


@pytest.mark.parametrize("cap", [16, 512])
def test_full_layer_bq_prefill_then_decode(cap):
    """bq full layer: a prefill chunk quantises every position (codes
    checked), then a decode step appends one token per sequence and attends
    (batched split route); K/V ~ N(0,1) with 1 % outliers x20, RoPE over 64
    pairs, non-unit gains."""
    announce(f"full layer bq cap={cap}")
    rng = np.random.default_rng(7 + cap)
    B = 5
    ctx = [int(x) for x in rng.integers(200, 2500, B)]
    case = make_decode_case(8 + cap, ctx)
    cos, sin = _tables(max(ctx) + 1, 9)
    gq = _bf16(rng.uniform(0.5, 1.5, D))
    gk = _bf16(rng.uniform(0.5, 1.5, D))
    cache = _BqCache(case.cache_rows)
    runs, rows, buf = [], [], 0
    for i, c in enumerate(ctx):
        runs.append([buf, 0, len(rows), len(case.pages[i])])
        rows.extend(p * PAGE for p in case.pages[i])
        buf += c
    runs = np.asarray(runs, dtype=np.int32)
    rows = np.asarray(rows, dtype=np.int32)
    n = buf
    q = seeded_bf16(n * NQ * D, 21)
    kraw = _outliers(seeded_bf16(n * KVS, 22), 23)
    _bq_step(cache, runs, rows, case.cache_rows, n, cap, q, kraw, gq, gk, cos, sin,
             attend=False)
    qd = seeded_bf16(B * NQ * D, 31)
    kd = _outliers(seeded_bf16(B * KVS, 32), 33)
    _bq_step(cache, case.runs, case.base_rows, case.cache_rows, B, cap, qd, kd, gq, gk, cos,
             sin)


def test_full_layer_bq_token_prefill():
    """A short bq prefill chunk over cached prefixes (the MFMA prefill route
    at this shape; test_gpu_bq_prefill.py covers it in depth)."""
    announce("full layer bq token prefill")
    case = make_prefill_case(11, [0, 90, 300], [40, 25, 17])
    n = 82
    rng = np.random.default_rng(12)
    cos, sin = _tables(400, 13)
    gq = _bf16(rng.uniform(0.5, 1.5, D))
    gk = _bf16(rng.uniform(0.5, 1.5, D))
    cache = _BqCache(case.cache_rows)
    # Fill the prefixes first (codes only), then the chunk attends over them.
    runs, rows, buf = [], [], 0
    for i, p in enumerate(case.ctx):
        if p == 0:
            continue
        runs.append([buf, 0, int(case.runs[i][2]), int(case.runs[i][3])])
        buf += int(p)
    runs = np.asarray(runs, dtype=np.int32)
    _bq_step(cache, runs, case.base_rows, case.cache_rows, buf, 16,
             seeded_bf16(buf * NQ * D, 14), _outliers(seeded_bf16(buf * KVS, 15), 16),
             gq, gk, cos, sin, attend=False)
    _bq_step(cache, case.runs, case.base_rows, case.cache_rows, n, 16,
             seeded_bf16(n * NQ * D, 17), _outliers(seeded_bf16(n * KVS, 18), 19),
             gq, gk, cos, sin)
