"""Parity at the benchmark's own sizes: bench.py builds each timed workload
(seed 20241, its batch, its cap and its page tables, K/V generated on the
device), one step runs (append, then attention), and every output element is
compared with the oracle run on host copies of the same caches.

- configs 2 and 3 (bf16): every output within 1e-2 of the oracle, with no
  widening (n_over_tol == 0); config 3 reads the ring pages of the rotated
  layer cache the step used;
- config 7 (bf16, head_dim 512 with 8 q heads per kv head): its scores are
  MFMA sums, exact products added in the matrix core's order rather than the
  reference's VDPBF16PS chain, so a near-tie of two scores can move an output
  across a bf16 rounding boundary: every output within one bf16 spacing where
  |x| >= 2 and 1e-2 elsewhere, and at most 1e-5 of the outputs beyond 1e-2;
- configs 5 and 8 (bq): outputs bit-exact;
- config 6 (MiniMax-M3 sparse decode, bf16 and int8 KV): the indexer's
  selected blocks bit-exact over every cached position of the 64 sequences,
  the sparse attention on them within 1e-2 (one bf16 spacing where |x| >=
  2);
- the append of every config: the appended K/V rows and the rotated q
  bit-exact against the oracle's rope_cache_write / bq prep, computed on a
  compact copy of the appended pages.

The oracle runs on 16 threads (the box's CPU share); each test takes seconds
of GPU time and up to about a minute of host time."""
import argparse
import time

import numpy as np
import pytest

import bench
import oracle
from tests.gpu_util import announce
from tests.helpers import compare_bf16

pytestmark = pytest.mark.gpu

SEED = 20241
THREADS = 16


def _args(cap):
    return argparse.Namespace(cap=cap, norm="none", oproj=False, oquant="none", kv="bf16")


def _host(t, dtype):
    import torch

    torch.cuda.synchronize()
    return np.ascontiguousarray(t.cpu().numpy().view(dtype))


def _compact_append_case(w):
    """A run table whose appended position of sequence i lands on compact page
    i (every other ordinal maps to page B, never written), so the oracle's
    append can run on B + 1 pages."""
    B = len(w.pos)
    runs, rows = [], []
    for i, p in enumerate(w.pos):
        npg = w.ring if w.ring else p // bench.PAGE_LEN + 1
        target = (p // bench.PAGE_LEN) & (npg - 1) if w.ring else p // bench.PAGE_LEN
        runs.append([i, p, len(rows), npg])
        rows.extend((i if o == target else B) * bench.PAGE_LEN for o in range(npg))
    return np.asarray(runs, np.int32), np.asarray(rows, np.int32), (B + 1) * bench.PAGE_LEN


def _slots(w):
    """Cache row of each sequence's appended position in the real tables."""
    out = []
    for i, p in enumerate(w.pos):
        pages = w.pages[i]
        o = (p // bench.PAGE_LEN) & (len(pages) - 1) if w.ring else p // bench.PAGE_LEN
        out.append(int(pages[o]) * bench.PAGE_LEN + p % bench.PAGE_LEN)
    return np.asarray(out)


def _run_bf16(config, cap, strict=True):
    import torch

    announce(f"fullsize config {config} cap {cap}: setup")
    t0 = time.time()
    w = bench.DecodeBf16(config, SEED)
    dev = torch.device("cuda:0")
    w.setup(dev, _args(cap))
    q_pre = _host(w.q, np.uint16)
    ks, vs = _host(w.ks, np.uint16), _host(w.vs, np.uint16)
    for ph in w.phases:
        w.launch(ph)
    kc, vc = w.kl[w.layer]
    got = _host(w.out, np.uint16)
    q_post = _host(w.q, np.uint16)
    k_host, v_host = _host(kc, np.uint16), _host(vc, np.uint16)
    announce(f"  step done, caches on host ({(k_host.nbytes + v_host.nbytes) / 1e9:.1f} GB, "
             f"{time.time() - t0:.1f} s)")

    # The append: q rotated in place and the appended rows, against the oracle.
    runs_c, rows_c, crow = _compact_append_case(w)
    kcomp = np.zeros(crow * w.kvs, np.uint16)
    vcomp = np.zeros_like(kcomp)
    q_ref = q_pre.copy()
    cos, sin = (x.cpu().numpy() for x in (w.cos, w.sin))
    oracle.rope_cache_write(runs_c, rows_c, q_ref, ks, vs, kcomp, vcomp, cos, sin,
                            num_q=w.nq, num_kv=w.nkv, page_shift=6, row_mask=63,
                            page_mask=w.plan.page_mask, seq_len=len(w.pos), half=w.half,
                            pair_stride=w.pair, head_dim=w.hd)
    assert np.array_equal(q_post, q_ref), "rotated q differs"
    sl = _slots(w)
    B = len(w.pos)
    crows = np.arange(B) * bench.PAGE_LEN + np.asarray(w.pos) % bench.PAGE_LEN
    kv = w.kvs
    for name, host, comp in (("k", k_host, kcomp), ("v", v_host, vcomp)):
        g = host.reshape(-1, kv)[sl]
        r = comp.reshape(-1, kv)[crows]
        assert np.array_equal(g, r), f"appended {name} rows differ"

    t1 = time.time()
    runs, rows = w.table.arrays()
    ref = oracle.attention(w.kind, runs, rows, q_post, k_host, v_host, num_q=w.nq,
                           num_kv=w.nkv, head_dim=w.hd, kv_stride=w.kvs, window=w.window,
                           cache_size=w.cache_size, page_len=bench.PAGE_LEN, seq_len=B,
                           cap=cap, threads=THREADS)
    r = compare_bf16(got, ref)
    announce(f"  oracle {time.time() - t1:.1f} s, items {w.plan.summary.num_items}, "
             f"stripes {w.plan.summary.num_stripes}: {r}")
    assert r["n_nan"] == 0 and r["n_fail"] == 0, r
    if strict:
        assert r["n_over_tol"] == 0, r
    else:
        assert r["n_over_tol"] <= got.size * 1e-5, r


def test_fullsize_config2_headline():
    """The headline plan: B=64, ctx ~ U[512, 32768], cap 512."""
    _run_bf16(2, bench.DEFAULT_CAP[2])


def test_fullsize_config3_sliding_rings():
    """B=64 sliding window 1024 over 32-page rings, cap 256."""
    _run_bf16(3, bench.DEFAULT_CAP[3])


def test_fullsize_config7_full_layer():
    """Gemma-4's full-attention layer (16q/2kv hd512), B=64, cap 512."""
    _run_bf16(7, bench.DEFAULT_CAP[7], strict=False)


def _run_bq(config, cap):
    import torch

    announce(f"fullsize bq config {config} cap {cap}: setup")
    t0 = time.time()
    w = bench.DecodeBq(config, SEED)
    dev = torch.device("cuda:0")
    w.setup(dev, _args(cap))
    qs, kss, vss = (_host(t, np.uint16) for t in (w.qs, w.kss, w.vss))
    for ph in w.phases:
        w.launch(ph)
    got = _host(w.out, np.uint16)
    q_i8, qb, fq = _host(w.q_i8, np.int8), _host(w.qb, np.float32), _host(w.fq, np.float32)
    kc, vc = _host(w.kc, np.int8), _host(w.vc, np.int8)
    ksc, vsc = _host(w.ksc, np.float32), _host(w.vsc, np.float32)
    announce(f"  step done, caches on host ({(kc.nbytes + vc.nbytes) / 1e9:.1f} GB, "
             f"{time.time() - t0:.1f} s)")

    # The quantizing append against the oracle's prep on compact pages.
    B = len(w.pos)
    runs_c, rows_c = [], []
    for i, p in enumerate(w.pos):
        npg = p // bench.PAGE_LEN + 1
        runs_c.append([i, p, len(rows_c), npg])
        rows_c.extend((i if o == npg - 1 else B) * bench.PAGE_LEN for o in range(npg))
    runs_c, rows_c = np.asarray(runs_c, np.int32), np.asarray(rows_c, np.int32)
    crow = (B + 1) * bench.PAGE_LEN
    kcomp = np.zeros(crow * w.kvs, np.int8)
    vcomp = np.zeros_like(kcomp)
    kscomp = np.zeros(crow * w.nkv, np.float32)
    vscomp = np.zeros_like(kscomp)
    q_ref = np.zeros_like(q_i8)
    qb_ref, fq_ref = np.zeros_like(qb), np.zeros_like(fq)
    cos, sin = (x.cpu().numpy() for x in (w.cos, w.sin))
    qn = _host(w.qn, np.uint16)
    vsrc = kss if config == 8 else vss
    oracle.bq_attn_prep(runs_c, rows_c, qs, kss, vsrc, qn, qn, q_ref, qb_ref, fq_ref, kcomp,
                        kscomp, vcomp, vscomp, cos, sin, num_q=w.nq, num_kv=w.nkv,
                        page_shift=6, row_mask=63, page_mask=-1, seq_len=B, head_dim=w.hd,
                        rope_half=w.half, pair_stride=w.pair,
                        sqrt_n=float(np.sqrt(np.float32(w.hd))),
                        n_eps=float(np.float32(w.hd) * np.float32(1e-6)))
    assert np.array_equal(q_i8, q_ref), "q codes differ"
    assert np.array_equal(qb.view(np.uint32), qb_ref.view(np.uint32)), "q bias differs"
    assert np.array_equal(fq.view(np.uint32), fq_ref.view(np.uint32)), "f_q differs"
    runs, rows = w.table.arrays()
    sl = np.asarray([int(rows[runs[i][2] + p // bench.PAGE_LEN]) + p % bench.PAGE_LEN
                     for i, p in enumerate(w.pos)])
    crows = np.arange(B) * bench.PAGE_LEN + np.asarray(w.pos) % bench.PAGE_LEN
    for name, host, comp, width in (("k", kc, kcomp, w.kvs), ("v", vc, vcomp, w.kvs),
                                    ("k scale", ksc, kscomp, w.nkv),
                                    ("v scale", vsc, vscomp, w.nkv)):
        g = host.reshape(-1, width)[sl]
        r = comp.reshape(-1, width)[crows]
        if g.dtype == np.float32:
            g, r = g.view(np.uint32), r.view(np.uint32)
        assert np.array_equal(g, r), f"appended {name} differ"

    t1 = time.time()
    ref = oracle.bq_attention(1, runs, rows, q_i8, qb, fq, kc, ksc, vc, vsc, num_q=w.nq,
                              num_kv=w.nkv, head_dim=w.hd, kv_stride=w.kvs, window=0,
                              cache_size=bench.PAGE_LEN, page_len=bench.PAGE_LEN, seq_len=B,
                              cap=cap, threads=THREADS)
    r = compare_bf16(got, ref)
    announce(f"  oracle {time.time() - t1:.1f} s, items {w.plan.summary.num_items}: {r}")
    assert np.array_equal(got, ref), r


def test_fullsize_config5_bq():
    """B=128, ctx ~ U[1024, 65536], cap 2048: outputs bit-exact."""
    _run_bq(5, bench.DEFAULT_CAP[5])


def test_fullsize_config8_bq_full_layer():
    """The bq full-attention layer (16q/2kv hd512), B=128, cap 2048."""
    _run_bq(8, bench.DEFAULT_CAP[8])


def _run_sparse(kv):
    import torch

    announce(f"fullsize config 6 kv {kv}: setup")
    t0 = time.time()
    w = bench.SparseM3(SEED)
    dev = torch.device("cuda:0")
    w.setup(dev, _args(0) if kv == "bf16" else argparse.Namespace(cap=0, kv=kv))
    for ph in w.phases:
        w.launch(ph)
    ik, kc, vc, ks, vs = w.kl[w.layer]
    B, IH, TOPK = len(w.pos), w.IH, w.TOPK
    got_bi = _host(w.block_idx, np.int32).reshape(B, IH, TOPK)
    got = _host(w.out, np.uint16)
    iq, ikh = _host(w.index_q, np.uint16), _host(ik, np.uint16)
    announce(f"  step done, index keys on host ({ikh.nbytes / 1e9:.1f} GB, "
             f"{time.time() - t0:.1f} s)")

    t1 = time.time()
    runs, rows = w.table.arrays()
    scale = float(np.float32(1.0) / np.sqrt(np.float32(w.HD)))
    want_bi, _ = oracle.lightning_indexer(runs, rows, iq, ikh, num_heads=IH, head_dim=w.HD,
                                          block_size=w.BLOCK, topk=TOPK, local_blocks=1,
                                          init_blocks=0, scale=scale, page_len=w.PLEN,
                                          seq_len=B)
    assert np.array_equal(got_bi, want_bi), np.argwhere(got_bi != want_bi)[:5]
    announce(f"  indexer oracle {time.time() - t1:.1f} s: block ids bit-exact")
    del ikh

    t2 = time.time()
    common = dict(num_q=w.NQ, num_kv=w.NKV, head_dim=w.HD, kv_stride=w.NKV * w.HD,
                  block_size=w.BLOCK, topk=TOPK, page_len=w.PLEN, seq_len=B)
    if kv == "bf16":
        q, kh, vh = _host(w.q, np.uint16), _host(kc, np.uint16), _host(vc, np.uint16)
        ref = oracle.block_sparse_attention(runs, rows, q, kh, vh, want_bi, **common)
    else:
        q, kh, vh = _host(w.q, np.int8), _host(kc, np.int8), _host(vc, np.int8)
        qb, fq = _host(w.qb, np.float32), _host(w.fq, np.float32)
        ksh, vsh = _host(ks, np.float32), _host(vs, np.float32)
        ref = oracle.bq_block_sparse_attention(runs, rows, q, qb, fq, kh, ksh, vh, vsh,
                                               want_bi, cap=128, **common)
    r = compare_bf16(got, ref)
    announce(f"  attention oracle {time.time() - t2:.1f} s, "
             f"bit-exact {bool(np.array_equal(got, ref))}: {r}")
    assert r["n_nan"] == 0 and r["n_fail"] == 0, r


def test_fullsize_config6_sparse():
    """MiniMax-M3 sparse decode, B=64, ctx ~ U[1024, 131072]: the indexer's
    block ids bit-exact over every cached position, the sparse attention
    within the bar on them."""
    _run_sparse("bf16")


def test_fullsize_config6_bq_sparse():
    """The same over int8 KV (bench.py's random codes and scales, cap 128)."""
    _run_sparse("bq")
