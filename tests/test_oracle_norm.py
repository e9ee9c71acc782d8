"""CPU pins of the oracle's head RMS norm (dispatch_rms_norm_qkv_heads,
kernels/rmsnorm.mojo:168-215): closed forms, exact power-of-two scale
invariance, unit RMS of the output, gains on q and k only, and agreement
with a float64 RMS norm to one bf16 rounding."""
import numpy as np
import pytest

import oracle
from tests.helpers import bf16_to_f32, bf16_ulp

D = 256


def _norm(q, k, v, qw, kw, num_q, num_kv, seq_len, sqrt_n=16.0, n_eps=D * 1e-6, head_dim=D):
    q, k, v = q.copy(), k.copy(), v.copy()
    oracle.rms_norm_qkv_heads(q, k, v, qw, kw, num_q=num_q, num_kv=num_kv, seq_len=seq_len,
                              head_dim=head_dim, sqrt_n=sqrt_n, n_eps=n_eps)
    return q, k, v


def _bf(x):
    return oracle.f32_to_bf16(np.asarray(x, dtype=np.float32).ravel())


def test_constant_row_closed_form():
    # x = 1.5 everywhere: ssq = 256 * 2.25 = 576 exactly, inv = 16/24 = 2/3,
    # y = bf16(1.5 * f32(2/3)) = 1.0 (w = 1); with w = 2 (exact), 2.0.
    x = _bf(np.full(D, 1.5))
    one, two = _bf(np.ones(D)), _bf(np.full(D, 2.0))
    q, k, v = _norm(x, x, x, one, two, 1, 1, 1, n_eps=0.0)
    assert np.all(bf16_to_f32(q) == 1.0)
    assert np.all(bf16_to_f32(k) == 2.0)
    assert np.all(bf16_to_f32(v) == 1.0), "v heads take no gain"


def test_power_of_two_scaling_is_exact():
    rng = np.random.default_rng(3)
    x = _bf(rng.normal(0, 1, 4 * D))
    w = _bf(rng.uniform(0.5, 1.5, D))
    base = _norm(x, x[:2 * D], x[2 * D:], w, w, 4, 2, 1, n_eps=0.0)
    for s in (2.0, 0.125, 1024.0):
        xs = _bf(bf16_to_f32(x) * s)
        got = _norm(xs, xs[:2 * D], xs[2 * D:], w, w, 4, 2, 1, n_eps=0.0)
        for a, b in zip(base, got):
            assert np.array_equal(a, b)


def test_unit_rms_and_float64_agreement():
    rng = np.random.default_rng(4)
    T, NQ, NKV = 3, 16, 8
    q = _bf(rng.normal(0, 3, T * NQ * D))
    k = _bf(rng.normal(0, 0.2, T * NKV * D))
    v = _bf(rng.normal(5, 1, T * NKV * D))
    qw = _bf(rng.uniform(0.5, 1.5, D))
    kw = _bf(rng.uniform(0.5, 1.5, D))
    eps = 1e-6
    qn, kn, vn = _norm(q, k, v, qw, kw, NQ, NKV, T, n_eps=D * eps)
    for src, out, w in ((q, qn, qw), (k, kn, kw), (v, vn, None)):
        x = bf16_to_f32(src).astype(np.float64).reshape(-1, D)
        ref = x / np.sqrt((x * x).mean(1, keepdims=True) + eps)
        if w is not None:
            ref = ref * bf16_to_f32(w).astype(np.float64)
        got = bf16_to_f32(out).astype(np.float64).reshape(-1, D)
        assert np.all(np.abs(got - ref) <= 1.01 * bf16_ulp(ref)), "within one bf16 rounding"
        if w is None:
            rms = np.sqrt((got ** 2).mean(1))
            assert np.all(np.abs(rms - 1.0) < 2 ** -7)


@pytest.mark.parametrize("head_dim", [128, 512])
def test_other_head_dims(head_dim):
    rng = np.random.default_rng(head_dim)
    x = _bf(rng.normal(0, 1, 2 * head_dim))
    w = _bf(np.ones(head_dim))
    q, _, _ = _norm(x, x[:head_dim], x[head_dim:], w, w, 2, 1, 1, sqrt_n=float(np.sqrt(head_dim)),
                    n_eps=0.0, head_dim=head_dim)
    y = bf16_to_f32(q).astype(np.float64).reshape(2, head_dim)
    assert np.all(np.abs(np.sqrt((y ** 2).mean(1)) - 1) < 2 ** -7)
