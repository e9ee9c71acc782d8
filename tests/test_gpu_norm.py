"""GPU parity of the head RMS norm (dispatch_rms_norm_qkv_heads,
kernels/rmsnorm.mojo:168-215), alone and fused ahead of the append
(dispatch_rope_cache_write, kernels/rope.mojo:128-171): bit-exact against
the oracle's norm followed by the oracle's append."""
import numpy as np
import pytest

import oracle
from inferno_amd import attention as A
from inferno_amd.kv import FULL, SLIDING, AttentionPlan, KVRunTable
from tests.gpu_util import announce, from_dev, to_dev
from tests.helpers import make_prefill_case, seeded_bf16

pytestmark = pytest.mark.gpu

NUM_Q, NUM_KV = 16, 8


def _table(runs, rows) -> KVRunTable:
    t = KVRunTable()
    for r in runs:
        t.begin_run(int(r[0]), int(r[1]))
        for j in range(int(r[3])):
            t.add_base_row(int(rows[int(r[2]) + j]))
    return t


def _gains(d, seed):
    rng = np.random.default_rng(seed)
    return oracle.f32_to_bf16(rng.uniform(0.25, 2.0, d).astype(np.float32))


@pytest.mark.parametrize("head_dim", [256, 512])
def test_norm_alone_bit_exact(head_dim):
    announce(f"rms norm alone D={head_dim}")
    T = 37
    q = seeded_bf16(T * NUM_Q * head_dim, 1)
    k = seeded_bf16(T * NUM_KV * head_dim, 2)
    v = seeded_bf16(T * NUM_KV * head_dim, 3)
    v[: head_dim] = 0  # an all-zero head: inv = sqrt_n / sqrt(n_eps)
    qw, kw = _gains(head_dim, 4), _gains(head_dim, 5)
    sqrt_n, n_eps = float(np.sqrt(head_dim)), head_dim * 1e-6
    qd, kd, vd = to_dev(q), to_dev(k), to_dev(v)
    A.dispatch_rms_norm_qkv_heads(qd, kd, vd, to_dev(qw), to_dev(kw), num_q=NUM_Q,
                                  num_kv=NUM_KV, seq_len=T, head_dim=head_dim, sqrt_n=sqrt_n,
                                  n_eps=n_eps)
    oracle.rms_norm_qkv_heads(q, k, v, qw, kw, num_q=NUM_Q, num_kv=NUM_KV, seq_len=T,
                              head_dim=head_dim, sqrt_n=sqrt_n, n_eps=n_eps)
    assert np.array_equal(from_dev(qd, np.uint16), q)
    assert np.array_equal(from_dev(kd, np.uint16), k)
    assert np.array_equal(from_dev(vd, np.uint16), v)


@pytest.mark.parametrize("kind,half,pair_stride", [(FULL, 128, 128), (SLIDING, 64, 128)])
def test_norm_fused_into_append_bit_exact(kind, half, pair_stride):
    """A prefill chunk over three sequences (ring pages for the sliding
    case); partial rotary (half 64 of pair stride 128) leaves elements that
    are normalised but not rotated."""
    announce(f"rms norm + append kind={kind} half={half}")
    D = 256
    kv_stride = NUM_KV * D
    prefix, new = [0, 70, 1500], [5, 64, 33]
    if kind == SLIDING:
        case = make_prefill_case(8, prefix, new, fixed_pages=32)
        cache_size, window = 32 * 64, 1024
    else:
        case = make_prefill_case(8, prefix, new)
        cache_size, window = 64, 0
    n = sum(new)
    q = seeded_bf16(n * NUM_Q * D, 11)
    ks, vs = seeded_bf16(n * kv_stride, 12), seeded_bf16(n * kv_stride, 13)
    kc, vc = seeded_bf16(case.cache_rows * kv_stride, 14), seeded_bf16(case.cache_rows * kv_stride, 15)
    qw, kw = _gains(D, 16), _gains(D, 17)
    rng = np.random.default_rng(18)
    maxpos = max(p + m for p, m in zip(prefix, new)) + 1
    ang = rng.uniform(-3, 3, maxpos * half)
    cos, sin = np.cos(ang).astype(np.float32), np.sin(ang).astype(np.float32)
    plan = AttentionPlan(_table(case.runs, case.base_rows), n, kind=kind, window=window,
                         cache_size=cache_size, page_len=64, cache_rows=case.cache_rows, cap=16,
                         kv_row_bytes=kv_stride * 2)
    qd, ksd, vsd, kcd, vcd = to_dev(q), to_dev(ks), to_dev(vs), to_dev(kc), to_dev(vc)
    A.dispatch_rms_norm_rope_cache_write(plan, qd, ksd, vsd, kcd, vcd, to_dev(qw), to_dev(kw),
                                         to_dev(cos), to_dev(sin), num_q=NUM_Q, num_kv=NUM_KV,
                                         half=half, pair_stride=pair_stride, head_dim=D,
                                         sqrt_n=16.0, n_eps=D * 1e-6)
    # Reference: the norm in place, then the append.
    q_r, k_r, v_r = q.copy(), ks.copy(), vs.copy()
    oracle.rms_norm_qkv_heads(q_r, k_r, v_r, qw, kw, num_q=NUM_Q, num_kv=NUM_KV, seq_len=n,
                              head_dim=D, sqrt_n=16.0, n_eps=D * 1e-6)
    kc_r, vc_r = kc.copy(), vc.copy()
    oracle.rope_cache_write(case.runs, case.base_rows, q_r, k_r, v_r, kc_r, vc_r, cos, sin,
                            num_q=NUM_Q, num_kv=NUM_KV, page_shift=6, row_mask=63,
                            page_mask=plan.page_mask, seq_len=n, half=half,
                            pair_stride=pair_stride, head_dim=D)
    assert np.array_equal(from_dev(qd, np.uint16), q_r), "normalised, rotated q"
    assert np.array_equal(from_dev(kcd, np.uint16), kc_r), "k cache"
    assert np.array_equal(from_dev(vcd, np.uint16), vc_r), "v cache"
    assert np.array_equal(from_dev(ksd, np.uint16), ks), "k_src is only read"
