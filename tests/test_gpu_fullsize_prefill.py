"""Parity of the chunked-prefill workloads exactly as bench.py times them
(seed 20241, the default cap, the plan bench.py builds): one step runs on the
GPU and every output of every query token is compared with the oracle.

- config 4 (bf16, 16q/8kv hd256) and config 12 (Gemma-4's full layer, 16q/2kv
  hd512): 8 sequences x 2048 new tokens on prefixes shared by sequence pairs.
  The step is the copy-on-write of each pair's partial prefix page
  (ContinuousBatchScheduler.fork_prefix, continuous_batching/scheduler.mojo:
  427-436; dispatch_copy_jobs, kernels/page_copy.mojo:63-94), the append
  (RoPE + cache write of the whole chunk, kernels/rope.mojo:53-171) and the
  causal MFMA prefill (FlashPrefillFullKernel + PrefillMergeKernel,
  kernels/flash_attention_prefill.mojo:117-248).  The whole K/V arena after
  the step must equal the oracle's copy jobs and rope_cache_write applied to
  a host copy of the arena taken before it, bit for bit, and the rotated q
  likewise; the outputs of all 16,384 query tokens are held to the bf16
  bar (1e-2, one spacing where |x| >= 2) with a bounded count beyond 1e-2.
- config 11 (sliding window 1024 on 64-page rings): append + sliding MFMA
  prefill (FlashPrefillSlidingKernel, kernels/flash_attention_prefill.mojo:
  18-114), checked the same way.
- --kv bq forms of configs 4, 11 and 12: the append is bq prep
  (butterquant_kernels/attention.mojo:494-632), whose codes, scales, q codes,
  q biases and f_q are compared whole and bit for bit; the attention
  (BqFlashPrefill{Sliding,Full}Kernel, :170-351) is held to the same bar.

The oracle runs on 16 threads (the box's CPU share), on the token route
(every query token walks its keys from its first tile), as the reference's
prefill kernels do."""
import argparse
import time

import numpy as np
import pytest

import bench
import oracle
from tests.gpu_util import announce
from tests.helpers import assert_bar, compare_bf16

pytestmark = pytest.mark.gpu

SEED = 20241
THREADS = 16


def _host(t, dtype):
    import torch

    torch.cuda.synchronize()
    return np.ascontiguousarray(t.cpu().numpy().view(dtype))


def _args(config):
    return argparse.Namespace(cap=bench.DEFAULT_CAP[config], norm="none", oproj=False,
                              oquant="none")


def _geom(w):
    """Page geometry of the workload's plan: shift, row mask, page mask."""
    return 6, 63, int(w.plan.page_mask)


def _check_bf16(w, kind, window, cache_size, label):
    import torch

    arena_pre = _host(w.arena if hasattr(w, "arena") else torch.cat([w.k, w.v]), np.uint16)
    q_pre, ks, vs = _host(w.q, np.uint16), _host(w.ks, np.uint16), _host(w.vs, np.uint16)
    t0 = time.time()
    for ph in w.phases:
        w.launch(ph)
    got = _host(w.out, np.uint16)
    q_post = _host(w.q, np.uint16)
    arena_post = _host(w.arena if hasattr(w, "arena") else torch.cat([w.k, w.v]), np.uint16)
    announce(f"  {label}: step done ({time.time() - t0:.1f} s)")

    # Copy-on-write, then the append, on the host copy.
    arena_ref = arena_pre.copy()
    jobs = getattr(w, "jobs", np.zeros((0, 3), np.int64))
    if jobs.size:
        oracle.copy_jobs(arena_ref.view(np.uint8), jobs)
    half_n = arena_ref.size // 2
    k_ref, v_ref = arena_ref[:half_n], arena_ref[half_n:]
    q_ref = q_pre.copy()
    cos, sin = (x.cpu().numpy() for x in (w.cos, w.sin))
    shift, row_mask, page_mask = _geom(w)
    runs, rows = w.table.arrays()
    oracle.rope_cache_write(runs, rows, q_ref, ks, vs, k_ref, v_ref, cos, sin, num_q=w.nq,
                            num_kv=w.nkv, page_shift=shift, row_mask=row_mask,
                            page_mask=page_mask, seq_len=w.n, half=w.half,
                            pair_stride=w.pair, head_dim=w.hd)
    assert np.array_equal(q_post, q_ref), "rotated q differs"
    bad = np.flatnonzero(arena_post != arena_ref)
    assert bad.size == 0, f"K/V arena differs at {bad.size} elements, first {bad[:4]}"
    announce(f"  {label}: copy-on-write ({jobs.shape[0]} jobs) and append bit-exact over the "
             f"whole arena ({arena_ref.nbytes / 1e6:.0f} MB)")

    t1 = time.time()
    ref = oracle.attention(kind, runs, rows, q_ref, k_ref, v_ref, num_q=w.nq, num_kv=w.nkv,
                           head_dim=w.hd, kv_stride=w.kvs, window=window,
                           cache_size=cache_size, page_len=bench.PAGE_LEN, seq_len=w.n,
                           cap=w.cap, threads=THREADS)
    announce(f"  {label}: oracle {time.time() - t1:.1f} s over {w.n} query tokens, "
             f"{int(w.plan.info[14])} query blocks")
    assert_bar(compare_bf16(got, ref), f"{label} all tokens")


def test_fullsize_config4_prefill():
    """bench --config 4: COW + append + causal MFMA prefill, as timed."""
    import torch

    announce("fullsize prefill config 4: setup")
    w = bench.PrefillBf16(SEED, 4)
    w.setup(torch.device("cuda:0"), _args(4))
    assert int(w.plan.info[14]) > 0, "config 4 must take the MFMA prefill route"
    _check_bf16(w, 1, 0, bench.PAGE_LEN, "config 4")


def test_fullsize_config12_prefill():
    """bench --config 12: the same at Gemma-4's full-attention layer shape."""
    import torch

    announce("fullsize prefill config 12: setup")
    w = bench.PrefillBf16(SEED, 12)
    w.setup(torch.device("cuda:0"), _args(12))
    assert int(w.plan.info[14]) > 0, "config 12 must take the MFMA prefill route"
    _check_bf16(w, 1, 0, bench.PAGE_LEN, "config 12")


def test_fullsize_config11_sliding_prefill():
    """bench --config 11: append + sliding-window (1024) MFMA prefill."""
    import torch

    announce("fullsize prefill config 11: setup")
    w = bench.PrefillSliding(SEED, 1024)
    w.setup(torch.device("cuda:0"), _args(11))
    assert int(w.plan.info[14]) > 0, "config 11 must take the MFMA prefill route"
    _check_bf16(w, 0, w.window, w.RING * bench.PAGE_LEN, "config 11")


def _check_bq(w, kind, window, cache_size, vsrc_is_k, label):
    k_pre, v_pre = _host(w.k, np.int8), _host(w.v, np.int8)
    ksc_pre, vsc_pre = _host(w.ksc, np.float32), _host(w.vsc, np.float32)
    qs, ks, vs = _host(w.q, np.uint16), _host(w.ks, np.uint16), _host(w.vs, np.uint16)
    gain = _host(w.gain, np.uint16)
    t0 = time.time()
    for ph in w.phases:
        w.launch(ph)
    got = _host(w.out, np.uint16)
    q_i8, qb, fq = _host(w.q_i8, np.int8), _host(w.qb, np.float32), _host(w.fq, np.float32)
    kc, vc = _host(w.k, np.int8), _host(w.v, np.int8)
    ksc, vsc = _host(w.ksc, np.float32), _host(w.vsc, np.float32)
    announce(f"  {label}: step done ({time.time() - t0:.1f} s)")

    jobs = getattr(w, "jobs", np.zeros((0, 3), np.int64))
    if jobs.size:
        # K/V code jobs address the code arena, scale jobs the scale arena.
        n_code = w.cow.jobs.shape[0] if w.cow is not None else 0
        codes = np.concatenate([k_pre, v_pre])
        oracle.copy_jobs(codes.view(np.uint8), jobs[:n_code])
        k_pre, v_pre = codes[:k_pre.size].copy(), codes[k_pre.size:].copy()
        scales = np.concatenate([ksc_pre, vsc_pre])
        oracle.copy_jobs(scales.view(np.uint8), jobs[n_code:])
        ksc_pre, vsc_pre = scales[:ksc_pre.size].copy(), scales[ksc_pre.size:].copy()
    q_ref = np.zeros_like(q_i8)
    qb_ref, fq_ref = np.zeros_like(qb), np.zeros_like(fq)
    cos, sin = (x.cpu().numpy() for x in (w.cos, w.sin))
    shift, row_mask, page_mask = _geom(w)
    runs, rows = w.table.arrays()
    oracle.bq_attn_prep(runs, rows, qs, ks, ks if vsrc_is_k else vs, gain, gain, q_ref,
                        qb_ref, fq_ref, k_pre, ksc_pre, v_pre, vsc_pre, cos, sin,
                        num_q=w.nq, num_kv=w.nkv, page_shift=shift, row_mask=row_mask,
                        page_mask=page_mask, seq_len=w.n, head_dim=w.hd, rope_half=w.half,
                        pair_stride=w.pair, sqrt_n=float(np.sqrt(np.float32(w.hd))),
                        n_eps=float(np.float32(w.hd) * np.float32(1e-6)))
    assert np.array_equal(q_i8, q_ref), "q codes differ"
    assert np.array_equal(qb.view(np.uint32), qb_ref.view(np.uint32)), "q bias differs"
    assert np.array_equal(fq.view(np.uint32), fq_ref.view(np.uint32)), "f_q differs"
    for name, g, r in (("k codes", kc, k_pre), ("v codes", vc, v_pre),
                       ("k scales", ksc.view(np.uint32), ksc_pre.view(np.uint32)),
                       ("v scales", vsc.view(np.uint32), vsc_pre.view(np.uint32))):
        bad = np.flatnonzero(g != r)
        assert bad.size == 0, f"{name} differ at {bad.size} elements, first {bad[:4]}"
    announce(f"  {label}: copy-on-write ({jobs.shape[0]} jobs) and bq prep bit-exact over "
             "the whole cache")

    t1 = time.time()
    ref = oracle.bq_attention(kind, runs, rows, q_i8, qb, fq, kc, ksc, vc, vsc, num_q=w.nq,
                              num_kv=w.nkv, head_dim=w.hd, kv_stride=w.kvs, window=window,
                              cache_size=cache_size, page_len=bench.PAGE_LEN, seq_len=w.n,
                              cap=w.cap, threads=THREADS)
    announce(f"  {label}: oracle {time.time() - t1:.1f} s over {w.n} query tokens, "
             f"{int(w.plan.info[14])} query blocks")
    assert_bar(compare_bf16(got, ref), f"{label} all tokens")


def test_fullsize_config12_bq_prefill():
    """bench --config 12 --kv bq: COW of codes and scales, bq prep, bq MFMA
    prefill at the full-attention layer shape (V is the raw K projection,
    modeling/gemma_4_moe_bq.mojo:566-573)."""
    import torch

    announce("fullsize prefill config 12 bq: setup")
    w = bench.PrefillBf16(SEED, 12, kv="bq")
    w.setup(torch.device("cuda:0"), _args(12))
    assert int(w.plan.info[14]) > 0, "config 12 bq must take the MFMA prefill route"
    _check_bq(w, 1, 0, bench.PAGE_LEN, True, "config 12 bq")


def test_fullsize_config11_bq_sliding_prefill():
    """bench --config 11 --kv bq: bq prep into the rings + sliding bq prefill."""
    import torch

    announce("fullsize prefill config 11 bq: setup")
    w = bench.PrefillSliding(SEED, 1024, kv="bq")
    w.setup(torch.device("cuda:0"), _args(11))
    assert int(w.plan.info[14]) > 0, "config 11 bq must take the MFMA prefill route"
    _check_bq(w, 0, w.window, w.RING * bench.PAGE_LEN, False, "config 11 bq")


def test_fullsize_config4_bq_prefill():
    """bench --config 4 --kv bq: COW of codes and scales, bq prep, and the
    int8 MFMA prefill at 16 q / 8 kv x 256."""
    import torch

    announce("fullsize prefill config 4 bq: setup")
    w = bench.PrefillBf16(SEED, 4, kv="bq")
    w.setup(torch.device("cuda:0"), _args(4))
    assert int(w.plan.info[14]) > 0, "config 4 bq must take the MFMA prefill route"
    _check_bq(w, 1, 0, bench.PAGE_LEN, False, "config 4 bq")
