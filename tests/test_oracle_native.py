"""The -march=native build of the oracle (the timed CPU baseline: AVX-512,
with VDPBF16PS and VPDPBUSD dots where the host has AVX-512 BF16 / VNNI)
returns the portable x86-64-v3 build's outputs bit for bit on every attention
route: decode splits and merges, the sliding and full token routes of
prefill, head_dim 512 with GQA 8, and the int8 (bq) forms."""
import numpy as np
import pytest

import oracle
from tests.helpers import (HEAD_DIM, KV_STRIDE, NUM_KV, NUM_Q, PAGE_LEN, make_decode_case,
                           make_prefill_case, seeded_bf16)


@pytest.fixture(scope="module")
def native():
    try:
        return oracle.native_lib()
    except Exception as e:  # no compiler for this host
        pytest.skip(f"native oracle build unavailable: {e}")


def _both(native, fn):
    a = fn()
    with oracle.using(native):
        b = fn()
    return a, b


@pytest.mark.parametrize("kind,window,cache", [(1, 0, PAGE_LEN), (0, 100, PAGE_LEN * 128)])
def test_native_matches_portable_bf16_prefill(native, kind, window, cache):
    case = make_prefill_case(3, [4000, 100, 0], [64, 70, 33])
    n = 167
    q = seeded_bf16(n * NUM_Q * HEAD_DIM, 1)
    k = seeded_bf16(case.cache_rows * KV_STRIDE, 2)
    v = seeded_bf16(case.cache_rows * KV_STRIDE, 3)
    a, b = _both(native, lambda: oracle.attention(
        kind, case.runs, case.base_rows, q, k, v, num_q=NUM_Q, num_kv=NUM_KV,
        head_dim=HEAD_DIM, kv_stride=KV_STRIDE, window=window, cache_size=cache,
        page_len=PAGE_LEN, seq_len=n, cap=8, threads=8))
    assert np.array_equal(a, b)


@pytest.mark.parametrize("nq,nkv,hd", [(16, 8, 256), (16, 2, 512)])
def test_native_matches_portable_bf16_decode(native, nq, nkv, hd):
    dc = make_decode_case(5, [3000, 500, 7000, 16, 1])
    kvs = nkv * hd
    q = seeded_bf16(5 * nq * hd, 4)
    k = seeded_bf16(dc.cache_rows * kvs, 5)
    v = seeded_bf16(dc.cache_rows * kvs, 6)
    for cap in (4, 64):
        a, b = _both(native, lambda: oracle.attention(
            1, dc.runs, dc.base_rows, q, k, v, num_q=nq, num_kv=nkv, head_dim=hd,
            kv_stride=kvs, window=0, cache_size=PAGE_LEN, page_len=PAGE_LEN, seq_len=5,
            cap=cap, threads=8))
        assert np.array_equal(a, b), cap


@pytest.mark.parametrize("kind,cache", [(1, PAGE_LEN), (0, PAGE_LEN * 128)])
def test_native_matches_portable_bq(native, kind, cache):
    case = make_prefill_case(3, [4000, 100, 0], [64, 70, 33])
    n = 167
    rng = np.random.default_rng(9)
    qi = rng.integers(-128, 128, n * NUM_Q * HEAD_DIM, dtype=np.int8)
    qb = (128 * qi.reshape(-1, HEAD_DIM).astype(np.int64).sum(1)).astype(np.float32)
    fq = rng.uniform(0.01, 0.1, n * NUM_Q).astype(np.float32)
    ki = rng.integers(-128, 128, case.cache_rows * KV_STRIDE, dtype=np.int8)
    vi = rng.integers(-128, 128, case.cache_rows * KV_STRIDE, dtype=np.int8)
    ks = rng.uniform(0.5, 4, case.cache_rows * NUM_KV).astype(np.float32)
    vs = rng.uniform(0.5, 4, case.cache_rows * NUM_KV).astype(np.float32)
    a, b = _both(native, lambda: oracle.bq_attention(
        kind, case.runs, case.base_rows, qi, qb, fq, ki, ks, vi, vs, num_q=NUM_Q,
        num_kv=NUM_KV, head_dim=HEAD_DIM, kv_stride=KV_STRIDE, window=100, cache_size=cache,
        page_len=PAGE_LEN, seq_len=n, cap=8, threads=8))
    assert np.array_equal(a, b)
