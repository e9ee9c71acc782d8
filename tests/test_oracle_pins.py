"""CPU pins of the oracle's tile-wise online softmax and log-sum-exp merge
against an independent float64 model of the same algorithm.

The model follows the reference's steps -- 16-position tiles from each
split's first position (FlashAttentionKernel, kernels/flash_attention.mojo:
44-54), per tile m_new = max(tile max, m), corr = fexp(max(-87, m - m_new)),
w = fexp(max(-87, s - m_new)) with pads at -1e30, acc = acc * corr + sum w v,
l = l * corr + sum w (online_softmax_tile / process_kv_tile,
kernels/attention_ops.mojo:165-253), and merge_segments (kernels/
logsum_merge.mojo:28-92): M = max m_s, c_s = fexp(max(-87, m_s - M)) (0 when
l_s = 0), out = sum c_s acc_s / sum c_s l_s -- in float64, with exact bf16
dot products.  Only fexp itself is shared with the oracle (pinned on its own
in test_oracle_numerics.py).

The score profiles make the tile structure matter: one position in an early
tile dominates every later score, and a later tile raises the maximum again,
so a missing carry of m across tiles, a rescale of the tile's own weights by
corr, or l updated without corr each moves the partials by far more than the
tolerance (the fexp(0) = 0.99963 bias alone is 3.7e-4 per misplaced tile)."""
import ctypes as C

import numpy as np
import pytest

import oracle
from tests.helpers import bf16_to_f32

W = 16


def _bf16(x):
    u = np.ascontiguousarray(x, dtype=np.float32).view(np.uint32).astype(np.uint64)
    return ((u + ((u >> 16) & 1) + 0x7FFF) >> 16).astype(np.uint16)


def _fexp(x):
    """The reference's biased exp on float32(x) (the oracle's, pinned
    separately), returned as float64."""
    return np.asarray(oracle.fexp(np.asarray(x, dtype=np.float32)), dtype=np.float64)


def model_partial(scores, v, start, end):
    """float64 online softmax over [start, end) in 16-position tiles."""
    m, l = -1e30, 0.0
    acc = np.zeros(v.shape[1])
    for t0 in range(start, end, W):
        n = min(W, end - t0)
        s = np.full(W, -1e30)
        s[:n] = scores[t0:t0 + n]
        m_new = max(s.max(), m)
        corr = float(_fexp(max(-87.0, m - m_new)))
        w = _fexp(np.maximum(-87.0, s - m_new))
        acc = acc * corr + w[:n] @ v[t0:t0 + n]
        l = l * corr + w.sum()
        m = m_new
    return m, l, acc


def model_merge(parts):
    M = max(p[0] for p in parts)
    num, den = 0.0, 0.0
    for m, l, acc in parts:
        c = float(_fexp(max(-87.0, m - M))) if l > 0 else 0.0
        num = num + c * acc
        den = den + c * l
    return num / den


def _profile(n, D, seed, dominant_at, later_max_at):
    """q and k (bf16) with dot products ~ N(0, 4) plus a dominant score at one
    position and a higher one later; v ~ N(0, 1)."""
    rng = np.random.default_rng(seed)
    q = rng.standard_normal(D).astype(np.float32)
    q /= np.linalg.norm(q)
    k = rng.standard_normal((n, D)).astype(np.float32) * 2.0 / np.sqrt(D) * np.sqrt(D)
    k = k - np.outer(k @ q, q) + np.outer(rng.standard_normal(n) * 2.0, q)
    k[dominant_at] += 14.0 * q
    if later_max_at is not None:
        k[later_max_at] += 17.0 * q
    v = rng.standard_normal((n, D)).astype(np.float32)
    qb, kb, vb = _bf16(q * 2.0), _bf16(k), _bf16(v)
    scores = bf16_to_f32(kb).astype(np.float64).reshape(n, D) @ bf16_to_f32(qb).astype(np.float64)
    return qb, kb, vb, scores


def _oracle_partial(qb, kb, vb, D, n, start, end):
    """ifo_flash_partial over [start, end) of one sequence laid out in one page
    (one q head, one kv head)."""
    ps = oracle.flash_partial_stride(1, D)
    part = np.zeros(ps, dtype=np.float32)
    page = 1 << int(np.ceil(np.log2(max(n, 2))))
    rows = np.zeros(1, dtype=np.int32)
    kpad = np.zeros(page * D, np.uint16)
    vpad = np.zeros(page * D, np.uint16)
    kpad[:n * D] = kb.reshape(-1)
    vpad[:n * D] = vb.reshape(-1)
    shift = int(np.log2(page))
    oracle.lib().ifo_flash_partial(rows.ctypes.data, shift, page - 1, -1, qb.ctypes.data,
                                   kpad.ctypes.data, vpad.ctypes.data, part.ctypes.data, 1, D,
                                   1, D, 0, start, end)
    return float(part[D]), float(part[D + 1]), part[:D].astype(np.float64)


@pytest.mark.parametrize("dominant_at,later_max_at", [(5, None), (5, 150), (40, 190)])
def test_partial_matches_float64_tile_model(dominant_at, later_max_at):
    n, D = 200, 32  # 13 tiles, the last partial
    qb, kb, vb, scores = _profile(n, D, 3 + dominant_at, dominant_at, later_max_at)
    v64 = bf16_to_f32(vb).astype(np.float64).reshape(n, D)
    for start, end in [(0, n), (16, n), (48, 177)]:
        m_o, l_o, acc_o = _oracle_partial(qb, kb, vb, D, n, start, end)
        m_m, l_m, acc_m = model_partial(scores, v64, start, end)
        assert abs(m_o - m_m) <= 1e-5 * abs(m_m), (start, end, m_o, m_m)
        assert abs(l_o - l_m) <= 2e-5 * abs(l_m), (start, end, l_o, l_m)
        assert np.allclose(acc_o, acc_m, rtol=2e-5, atol=2e-5 * np.abs(acc_m).max())


def test_model_separates_the_plausible_mistakes():
    """The model's own sensitivity: each mistake moves l or acc by far more
    than the 2e-5 tolerance on this profile."""
    n, D = 200, 32
    qb, kb, vb, scores = _profile(n, D, 8, 5, 150)
    v64 = bf16_to_f32(vb).astype(np.float64).reshape(n, D)
    m, l, acc = model_partial(scores, v64, 0, n)

    def variant(kind):
        mm, ll, aa = -1e30, 0.0, np.zeros(D)
        for t0 in range(0, n, W):
            k = min(W, n - t0)
            s = np.full(W, -1e30)
            s[:k] = scores[t0:t0 + k]
            m_new = s.max() if kind == "no_carry" else max(s.max(), mm)
            corr = float(_fexp(max(-87.0, mm - m_new)))
            w = _fexp(np.maximum(-87.0, s - m_new))
            if kind == "rescale_after_add":
                aa = (aa + w[:k] @ v64[t0:t0 + k]) * corr
                ll = (ll + w.sum()) * corr
            elif kind == "l_without_corr":
                aa = aa * corr + w[:k] @ v64[t0:t0 + k]
                ll = ll + w.sum()
            else:
                aa = aa * corr + w[:k] @ v64[t0:t0 + k]
                ll = ll * corr + w.sum()
            mm = m_new
        return ll, aa

    for kind in ("no_carry", "rescale_after_add", "l_without_corr"):
        ll, aa = variant(kind)
        dev = max(abs(ll - l) / l, np.abs(aa / ll - acc / l).max() / np.abs(acc / l).max())
        assert dev > 1e-3, (kind, dev)


def _finalize(parts32, D):
    """ifo_finalize_head over stripes of one q head; returns the bf16 row."""
    ps = oracle.flash_partial_stride(1, D)
    segs = np.zeros((len(parts32), ps), dtype=np.float32)
    for i, (m, l, acc) in enumerate(parts32):
        segs[i, :D] = acc
        segs[i, D] = m
        segs[i, D + 1] = l
    out = np.zeros(D, dtype=np.uint16)
    oracle.lib().ifo_finalize_head(out.ctypes.data, segs.ctypes.data, ps, len(parts32), 1, D, 0)
    return bf16_to_f32(out).astype(np.float64)


@pytest.mark.parametrize("n_splits", [2, 5, 17, 40])
def test_merge_matches_float64_model(n_splits):
    """Merging the oracle's own f32 partials: the model's merge of the same
    partials rounds to the same bf16 outputs (at most 1 % one spacing apart,
    from f32 vs f64 sums), with maxima spread over 12 units so that the
    corrections, the 16-split batches of L and the empty stripes (l = 0,
    c = 0) all matter."""
    rng = np.random.default_rng(n_splits)
    D = 256
    rows_same = 0
    total = 0
    for trial in range(16):
        parts = []
        for s in range(n_splits):
            if s % 7 == 6:
                parts.append((-1e30, 0.0, np.zeros(D, np.float32)))  # an empty split
                continue
            m = float(np.float32(rng.uniform(-6, 6)))
            l = float(np.float32(rng.uniform(0.5, 40)))
            acc = (rng.standard_normal(D) * l).astype(np.float32)
            parts.append((m, l, acc))
        got = _finalize(parts, D)
        want = model_merge([(m, float(l), acc.astype(np.float64)) for m, l, acc in parts])
        want_bf16 = bf16_to_f32(_bf16(want.astype(np.float32))).astype(np.float64)
        diff = np.abs(got - want_bf16)
        spacing = 2.0 ** (np.floor(np.log2(np.maximum(np.abs(want), 2.0 ** -126))) - 7)
        assert (diff <= spacing * 1.0001).all(), (trial, diff.max())
        rows_same += int((diff == 0).sum())
        total += D
    assert rows_same >= 0.99 * total, (rows_same, total)


def test_merge_model_separates_exp_from_fexp():
    """With true exp in place of the biased exp, the merged outputs of the
    same partials move by more than a bf16 spacing in many elements: the
    merge test above would fail such a mistake."""
    rng = np.random.default_rng(7)
    D = 256
    parts = [(float(rng.uniform(-6, 6)), float(rng.uniform(0.5, 40)),
              rng.standard_normal(D) * 10) for _ in range(8)]
    a = model_merge(parts)
    M = max(p[0] for p in parts)
    num = sum(np.exp(m - M) * acc for m, _, acc in parts)
    den = sum(np.exp(m - M) * l for m, l, _ in parts)
    b = num / den
    spacing = 2.0 ** (np.floor(np.log2(np.abs(a))) - 7)
    assert (np.abs(a - b) > spacing).mean() > 0.1
