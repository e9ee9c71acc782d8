"""Randomized GPU parity sweep over the attention routes: seeded cases
drawing the layer shape (16q/8kv x 256 or 16q/2kv x 512), full attention or
sliding windows (multiples of 16 and not, so both prefill kernels and the
token route run), page sizes 8-1024, rings that wrap, batches of 1-12 runs,
contexts including 0, 15/16/17 and page edges, decode steps or prefill
chunks, and worker caps 1-512.  Every output element against the oracle,
within 1e-2 (one bf16 spacing where |x| >= 2); each case prints its draw.
The butterquant routes run on the same draws (at the bq layer shapes), bit-
exact off the MFMA prefill."""
import numpy as np
import pytest

import oracle
from inferno_amd import attention as A
from inferno_amd.kv import FULL, SLIDING, AttentionPlan, KVRunTable
from tests.gpu_util import announce, empty_dev, from_dev, to_dev
from tests.helpers import assert_bar, compare_bf16, seeded_bf16

pytestmark = pytest.mark.gpu

SHAPES = [(16, 8, 256), (16, 2, 512)]
SPECIAL = [0, 1, 15, 16, 17, 63, 64, 65, 1023, 1024]


def _table(runs, rows) -> KVRunTable:
    t = KVRunTable()
    for r in runs:
        t.begin_run(int(r[0]), int(r[1]))
        for j in range(int(r[3])):
            t.add_base_row(int(rows[int(r[2]) + j]))
    return t


def _draw(seed):
    rng = np.random.default_rng(1000 + seed)
    nq, nkv, d = SHAPES[int(rng.integers(0, 2))]
    kind = SLIDING if rng.random() < 0.5 else FULL
    page_len = int(rng.choice([8, 16, 64, 1024]))
    window = int(rng.choice([16, 48, 100, 1024])) if kind == SLIDING else 0
    decode = rng.random() < 0.5
    B = int(rng.integers(1, 13))
    prefix = [int(rng.choice(SPECIAL)) if rng.random() < 0.3 else int(rng.integers(0, 3000))
              for _ in range(B)]
    new = [1] * B if decode else [int(rng.integers(1, 150)) for _ in range(B)]
    cap = int(rng.choice([1, 3, 16, 64, 512]))
    return dict(nq=nq, nkv=nkv, d=d, kind=kind, page_len=page_len, window=window,
                decode=decode, prefix=prefix, new=new, cap=cap, seed=seed)


def _layout(c, rng):
    """Runs back to back in the token buffer; full attention: each run's pages
    cover its positions; sliding: a power-of-two ring holding the window and
    the chunk."""
    pl = c["page_len"]
    if c["kind"] == SLIDING:
        need = (c["window"] + max(c["new"]) + 2 * pl + pl - 1) // pl
        ring = 1 << int(np.ceil(np.log2(max(need, 2))))
        counts = [ring] * len(c["prefix"])
    else:
        ring = 0
        counts = [max(1, (p + n + pl - 1) // pl) for p, n in zip(c["prefix"], c["new"])]
    perm = rng.permutation(sum(counts))
    runs, rows, buf, off = [], [], 0, 0
    for p, n, k in zip(c["prefix"], c["new"], counts):
        runs.append([buf, p, len(rows), k])
        rows.extend(int(x) * pl for x in perm[off:off + k])
        buf, off = buf + n, off + k
    return (np.asarray(runs, np.int32), np.asarray(rows, np.int32), sum(counts) * pl, ring,
            buf)


@pytest.mark.parametrize("seed", range(32))
def test_random_plan(seed):
    c = _draw(seed)
    rng = np.random.default_rng(2000 + seed)
    runs, rows, cache_rows, ring, n = _layout(c, rng)
    nq, nkv, d, pl = c["nq"], c["nkv"], c["d"], c["page_len"]
    kvs = nkv * d
    cache_size = ring * pl if c["kind"] == SLIDING else pl
    announce(f"random plan {seed}: {'sliding' if c['kind'] == SLIDING else 'full'} "
             f"{nq}q/{nkv}kv x {d} page {pl} window {c['window']} "
             f"{'decode' if c['decode'] else 'prefill'} B={len(c['prefix'])} cap={c['cap']} "
             f"prefix={c['prefix']} new={c['new']}")
    q = seeded_bf16(n * nq * d, 3 * seed + 1)
    k = seeded_bf16(cache_rows * kvs, 3 * seed + 2)
    v = seeded_bf16(cache_rows * kvs, 3 * seed + 3)
    plan = AttentionPlan(_table(runs, rows), n, kind=c["kind"], window=c["window"],
                         cache_size=cache_size, page_len=pl, cache_rows=cache_rows,
                         cap=c["cap"], kv_row_bytes=kvs * 2)
    out = empty_dev(n * nq * d, np.uint16)
    partials, ps = A.partials_buffer(plan, nq, d)
    A.attention_bf16(plan, to_dev(q), to_dev(k), to_dev(v), out, partials, ps, num_q=nq,
                     num_kv=nkv, head_dim=d, kv_stride=kvs)
    got = from_dev(out, np.uint16)
    ref = oracle.attention(c["kind"], runs, rows, q, k, v, num_q=nq, num_kv=nkv, head_dim=d,
                           kv_stride=kvs, window=c["window"], cache_size=cache_size,
                           page_len=pl, seq_len=n, cap=c["cap"], threads=16)
    assert_bar(compare_bf16(got, ref), f"{c} mode={plan.summary.mode} "
               f"items={plan.summary.num_items} qblocks={int(plan.info[14])}")


def _codes(n, rng):
    return rng.integers(-127, 128, n).astype(np.int8)


@pytest.mark.parametrize("seed", range(16))
def test_random_bq_plan(seed):
    """The butterquant routes on the same draws (synthetic codes, scales with
    O(1) outputs): bit-exact off the MFMA prefill, within the bar on it."""
    c = _draw(100 + seed)
    if c["kind"] == SLIDING and (c["nq"], c["d"]) == (16, 512):
        c["kind"], c["window"] = FULL, 0  # bq sliding layers are 16q/8kv x 256
    if c["kind"] == FULL and c["d"] == 256:
        c["nq"], c["nkv"], c["d"] = 16, 2, 512  # bq full layers are 16q/2kv x 512
    rng = np.random.default_rng(3000 + seed)
    runs, rows, cache_rows, ring, n = _layout(c, rng)
    nq, nkv, d, pl = c["nq"], c["nkv"], c["d"], c["page_len"]
    kvs = nkv * d
    cache_size = ring * pl if c["kind"] == SLIDING else pl
    announce(f"random bq plan {seed}: {'sliding' if c['kind'] == SLIDING else 'full'} "
             f"{nq}q/{nkv}kv x {d} page {pl} window {c['window']} "
             f"{'decode' if c['decode'] else 'prefill'} B={len(c['prefix'])} cap={c['cap']} "
             f"prefix={c['prefix']} new={c['new']}")
    q = _codes(n * nq * d, rng)
    qb = (128.0 * q.reshape(n * nq, d).astype(np.int64).sum(axis=1)).astype(np.float32)
    fq = (rng.uniform(0.5, 1.5, n * nq) / np.sqrt(d / 256)).astype(np.float32)
    k, v = _codes(cache_rows * kvs, rng), _codes(cache_rows * kvs, rng)
    ks = rng.uniform(0.5, 1.5, cache_rows * nkv).astype(np.float32)
    vs = rng.uniform(0.5, 2.0, cache_rows * nkv).astype(np.float32)
    plan = AttentionPlan(_table(runs, rows), n, kind=c["kind"], window=c["window"],
                         cache_size=cache_size, page_len=pl, cache_rows=cache_rows,
                         cap=c["cap"], kv_row_bytes=kvs)
    out = empty_dev(n * nq * d, np.uint16)
    partials, ps = A.partials_buffer(plan, nq, d)
    A.bq_attention(plan, to_dev(q), to_dev(qb), to_dev(fq), to_dev(k), to_dev(ks), to_dev(v),
                   to_dev(vs), out, partials, ps, num_q=nq, num_kv=nkv, head_dim=d,
                   kv_stride=kvs)
    got = from_dev(out, np.uint16)
    ref = oracle.bq_attention(c["kind"], runs, rows, q, qb, fq, k, ks, v, vs, num_q=nq,
                              num_kv=nkv, head_dim=d, kv_stride=kvs, window=c["window"],
                              cache_size=cache_size, page_len=pl, seq_len=n, cap=c["cap"],
                              threads=16)
    r = compare_bf16(got, ref)
    mfma = int(plan.info[14]) > 0 and plan.summary.mode in (1, 2)
    assert_bar(r, f"{c} mode={plan.summary.mode} items={plan.summary.num_items} mfma={mfma}")
    if not mfma:
        assert np.array_equal(got, ref), (c, r)
