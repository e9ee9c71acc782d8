"""CPU tests pinning the oracle's numeric primitives and planning helpers
against closed forms, published vectors and brute force."""
import math

import numpy as np
import pytest

import oracle


def test_fexp_error_envelope_matches_reference_comment():
    # simd_math/exponential.mojo:167-171: max rel. error ~ -6.88e-3, the fit
    # never overshoots exp on [-30, 0].
    x = np.linspace(-30, 0, 300001).astype(np.float32)
    rel = oracle.fexp(x).astype(np.float64) / np.exp(x.astype(np.float64)) - 1
    assert -6.9e-3 < rel.min() < -6.8e-3
    assert rel.max() <= 0.0


def test_fexp_closed_form_bit_path():
    # Float64 evaluation of the same integer bit path; only the final float
    # roundings may differ, so agreement within 2 f32 ulp pins the constants,
    # the truncating int conversion and the mantissa-fraction polynomial.
    def ref(x):
        a = np.float32(12102203.16156148)
        b = np.float32(1059208216.0)
        t = np.float32(np.float32(a * np.float32(x)) + b)
        i = int(t)  # truncation toward zero
        u = i & 0xFFFFFFFF
        k = np.array([u], dtype=np.uint32).view(np.float32)[0]
        f = (u & 0x7FFFFF) / 2.0 ** 23
        p = 1.6501418352127075 + f * (-0.37554836273193359 + f * 0.38696467876434326)
        return float(k) * p

    for x in [0.0, -0.5, -1.0, -3.25, -10.0, -40.0, -86.9, -87.0]:
        got = float(oracle.fexp(np.float32(x)))
        want = ref(x)
        assert abs(got - want) <= 2 * np.spacing(np.float32(abs(want))), (x, got, want)
    # fexp(0) < 1: every online-softmax tile rescales earlier tiles.
    assert float(oracle.fexp(np.float32(0.0))) == pytest.approx(0.99963, abs=1e-5)


def test_splitmix64_published_vectors():
    # SplitMix64 with state starting at 0 (Vigna's reference): the first
    # outputs are splitmix64(k * golden) in this counter formulation.
    golden = 0x9E3779B97F4A7C15
    expected = [0xE220A8397B1DCDAF, 0x6E789E6AA1B965F4, 0x06C45D188009454F]
    for k, e in enumerate(expected):
        assert oracle.splitmix64((k * golden) & (2**64 - 1)) == e


def test_bf16_round_to_nearest_even():
    f = np.array([1.0, 1.00390625, 1.01171875, 1.0078125, -2.5, 0.0, -0.0,
                  3.0e38, 1e-40], dtype=np.float32)
    b = oracle.f32_to_bf16(f)
    back = oracle.bf16_to_f32(b)
    # 1 + 2^-8 is a tie between 1 and 1 + 2^-7: even mantissa (1.0) wins.
    assert back[1] == 1.0
    # 1 + 3*2^-8 is a tie between 1+2^-7 and 1+2^-6: even is 1 + 2^-6.
    assert back[2] == np.float32(1.015625)
    assert back[3] == np.float32(1.0078125)
    assert back[4] == -2.5 and back[0] == 1.0
    assert b[5] == 0 and b[6] == 0x8000
    for i in range(len(f)):
        assert oracle.lib().ifo_f32_to_bf16(float(f[i])) == b[i]


def test_tree_sum16_is_halving_tree():
    v = np.array([1e8, 1, -1e8, 1, 3, 5, 7, 9, 2, 4, 6, 8, 10, 12, 14, 16],
                 dtype=np.float32)
    a = v.copy()
    w = 8
    while w >= 1:
        a[:w] = a[:w] + a[w:2 * w]
        w //= 2
    got = oracle.lib().ifo_tree_sum16(v.ctypes.data)
    assert np.float32(got) == a[0]


def _brute_plan(kv, cap, min_split):
    n = [0] * len(kv)
    ceil = [(k + min_split - 1) // min_split if k > 0 else 0 for k in kv]
    rem = cap
    for i in range(len(kv)):
        if ceil[i] > 0 and rem > 0:
            n[i] = 1
            rem -= 1
    while rem > 0:
        cands = [i for i in range(len(kv)) if 0 < n[i] < ceil[i]]
        if not cands:
            break
        # largest kv per split; exact rational comparison, first index on ties
        best = max(cands, key=lambda i: (kv[i] / n[i], -i))
        ties = [i for i in cands if kv[i] * n[best] == kv[best] * n[i]]
        best = min(ties)
        n[best] += 1
        rem -= 1
    return n


@pytest.mark.parametrize("seed", range(6))
def test_plan_run_splits_against_brute_force(seed):
    rng = np.random.default_rng(seed)
    R = int(rng.integers(1, 40))
    kv = [int(x) for x in rng.integers(0, 3000, R)]
    if seed == 0:
        kv = [16, 16, 16, 32]  # ties
    cap = int(rng.integers(1, 300))
    got = oracle.plan_run_splits(kv, list(range(R)), cap, 16)
    want = _brute_plan(kv, cap, 16)
    assert list(got[:, 2]) == want
    assert list(got[:, 1]) == list(np.concatenate([[0], np.cumsum(want)[:-1]]))
    assert got[:, 2].sum() <= cap
    total_ceil = sum((k + 15) // 16 for k in kv if k > 0)
    assert got[:, 2].sum() == min(cap, total_ceil) or got[:, 2].sum() == cap


@pytest.mark.parametrize("total,nw", [(10, 4), (9, 4), (4097, 128), (1, 1), (33, 3), (0, 2)])
def test_worker_range_partitions(total, nw):
    spans = [oracle.worker_range(total, nw, w) for w in range(nw)]
    covered = []
    for s, e in spans:
        assert 0 <= s <= e <= total
        covered.extend(range(s, e))
    assert covered == list(range(total))


def test_recommended_workers_heuristic():
    # helpers.mojo:206-219: capacity when >= 1 MiB, else isqrt(bytes/2280).
    assert oracle.recommended_workers(2 << 20, 96) == 96
    assert oracle.recommended_workers(100 * 2280, 96) == 10
    assert oracle.recommended_workers(0, 96) == 1
    assert oracle.recommended_workers(123, 1) == 1


def test_paged_slot_matches_reference_ring_slot():
    # tests/test_sliding_attention_degree_parity.mojo:83-86 ring_slot with the
    # test's 2-page rings of 64-token pages.
    def ring_slot(pos, pages):
        return pages[(pos // 64) % 2] * 64 + pos % 64

    pages = [3, 1]
    rows = np.array([p * 64 for p in pages], dtype=np.int32)
    for pos in [0, 5, 63, 64, 100, 127, 128, 200, 1000]:
        assert oracle.paged_slot(rows, 6, 63, 1, 0, pos) == ring_slot(pos, pages)
    # full cache: page_mask -1
    rows = np.array([7, 2, 9], dtype=np.int32) * 64
    assert oracle.paged_slot(rows, 6, 63, -1, 0, 130) == 9 * 64 + 2
    assert oracle.paged_slot(rows, 6, 63, -1, 100, 30) == 9 * 64 + 2


def test_flash_partial_stride():
    # attention_ops.mojo:140-142 at the config shapes: 4128 floats.
    assert oracle.flash_partial_stride(16, 256) == 4128
    assert oracle.flash_partial_stride(16, 512) == ((16 * 512 + 32) * 4 + 63) // 64 * 16


def test_fwht_matches_sylvester_hadamard():
    from scipy.linalg import hadamard

    rng = np.random.default_rng(1)
    for n in (16, 256):
        H = hadamard(n).astype(np.float64) / math.sqrt(n)
        x = rng.standard_normal(n).astype(np.float32)
        got = oracle.fwht(x)
        want = H @ x.astype(np.float64)
        assert np.max(np.abs(got - want)) < 1e-5 * np.sqrt(n)
    imp = np.zeros(256, dtype=np.float32)
    imp[0] = 1.0
    assert np.all(oracle.fwht(imp) == np.float32(1 / 16))
    const = np.ones(256, dtype=np.float32)
    out = oracle.fwht(const)
    assert out[0] == 16.0 and np.all(out[1:] == 0.0)


def test_absmax_quantize_definition():
    rng = np.random.default_rng(2)
    x = (rng.standard_normal(256) * 3).astype(np.float32)
    q, amax, qsum = oracle.absmax_quantize(x)
    assert amax == np.max(np.abs(x))
    assert np.max(np.abs(q.astype(int))) == 127
    assert qsum == int(q.astype(np.int64).sum())
    deq = q.astype(np.float64) * amax / 127
    assert np.max(np.abs(deq - x)) <= amax / 254 * (1 + 1e-6)
    # half-way values round to even
    y = np.array([127.0, 0.5, 1.5, 2.5, -0.5, -1.5], dtype=np.float32)
    q, amax, _ = oracle.absmax_quantize(y)
    assert list(q) == [127, 0, 2, 2, 0, -2]
    z = np.zeros(8, dtype=np.float32)
    q, amax, _ = oracle.absmax_quantize(z)
    assert amax == np.float32(1e-10) and not q.any()


def _bf16(vals) -> np.ndarray:
    return oracle.f32_to_bf16(np.asarray(vals, dtype=np.float32))


def test_bq_block_quant_known_answers():
    # amax 127 gives inv exactly 1 and amax 254 gives 0.5, so the codes are
    # the values themselves (halved); ties at .5 go to even, not away from 0.
    block = 16
    row0 = [127.0, 0.5, 1.5, 2.5, 3.5, -0.5, -1.5, -2.5, -3.5, 4.0, -127.0, 0, 0, 0, 0, 0]
    row1 = [254.0, 5.0, 7.0, -5.0, -7.0, 1.0, 3.0, 0, 0, 0, 0, 0, 0, 0, 0, -254.0]
    zero = [0.0] * block
    src = _bf16(row0 + row1 + zero + row1)
    codes, scales = oracle.bq_block_quant(src, cols=2 * block, block=block)
    assert codes.shape == (2, 32) and scales.shape == (2, 2)
    assert list(codes[0, :16]) == [127, 0, 2, 2, 4, 0, -2, -2, -4, 4, -127, 0, 0, 0, 0, 0]
    assert list(codes[0, 16:]) == [127, 2, 4, -2, -4, 0, 2, 0, 0, 0, 0, 0, 0, 0, 0, -127]
    assert not codes[1, :16].any()
    assert list(codes[1, 16:]) == list(codes[0, 16:])
    assert scales.tolist() == [[127.0, 254.0], [0.0, 254.0]]


def test_bq_block_quant_bounds_and_block_independence():
    rng = np.random.default_rng(5)
    cols, block = 512, 256
    x = (rng.standard_normal((7, cols)) * rng.uniform(0.01, 50, (7, 1))).astype(np.float32)
    x[3, :block] *= 1e4  # a loud block must not change its neighbour's codes
    src = _bf16(x)
    xf = oracle.bf16_to_f32(src).astype(np.float64).reshape(7, cols)
    codes, scales = oracle.bq_block_quant(src, cols=cols, block=block)
    for t in range(7):
        for b in range(2):
            blk = xf[t, b * block:(b + 1) * block]
            amax = np.max(np.abs(blk))
            assert scales[t, b] == np.float32(amax)
            c = codes[t, b * block:(b + 1) * block].astype(np.int64)
            i = int(np.argmax(np.abs(blk)))
            assert c[i] == (127 if blk[i] > 0 else -127)
            assert np.all(np.abs(c) <= 127)
            assert np.max(np.abs(c * amax / 127 - blk)) <= amax / 254 * (1 + 1e-5)
    alone, alone_sa = oracle.bq_block_quant(src.reshape(7, cols)[3, block:], cols=block,
                                            block=block)
    assert np.array_equal(alone[0], codes[3, block:]) and alone_sa[0, 0] == scales[3, 1]


def test_head_inv_rms_chain():
    rng = np.random.default_rng(3)
    x = rng.standard_normal(256).astype(np.float32)
    got = oracle.head_inv_rms(x, 16.0, np.float32(256) * np.float32(1e-6))
    want = 16.0 / math.sqrt(float(np.sum(x.astype(np.float64) ** 2)) + 256e-6)
    assert got == pytest.approx(want, rel=2e-6)
