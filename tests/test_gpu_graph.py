"""HIP graph capture of a decode step.  The plan-based entry points
(ifr_rope_cache_write, ifr_attention_bf16, ifr_bq_attention) launch kernels
only -- no allocation, memset or copy -- so a host can capture a layer's
append + attention once and replay it.  Each test replays its graph several
times, with eager launches and synchronisations between the replays, and
checks every replay against the eager outputs bit for bit (the attention
outputs, the rotated queries and the appended cache rows)."""
import numpy as np
import pytest

from inferno_amd import attention as A
from inferno_amd.kv import FULL, SLIDING, AttentionPlan, KVRunTable
from tests.gpu_util import announce, empty_dev, from_dev, to_dev
from tests.helpers import make_decode_case, seeded_bf16

pytestmark = pytest.mark.gpu

NQ, NKV, D = 16, 8, 256
KVS = NKV * D
HALF = PAIR = 128
REPLAYS = 4


def _table(runs, rows) -> KVRunTable:
    t = KVRunTable()
    for r in runs:
        t.begin_run(int(r[0]), int(r[1]))
        for j in range(int(r[3])):
            t.add_base_row(int(rows[int(r[2]) + j]))
    return t


def _rope(maxpos, seed):
    rng = np.random.default_rng(seed)
    ang = rng.uniform(-3, 3, maxpos * HALF)
    return to_dev(np.cos(ang).astype(np.float32)), to_dev(np.sin(ang).astype(np.float32))


@pytest.mark.parametrize("ctx,cap,kind", [
    ([4096], 128, FULL),                       # one sequence: the LDS-staged merge
    ([300, 5000, 1200, 64, 9000, 17, 2048, 700], 64, FULL),   # batched: merge_kernel
    ([1500, 3000, 1023, 4000], 96, SLIDING),   # sliding rings
])
def test_graph_replays_decode_step_bf16(ctx, cap, kind):
    import torch

    announce(f"graph decode bf16 kind={kind} B={len(ctx)} cap={cap}")
    B = len(ctx)
    if kind == SLIDING:
        ring = 32
        runs = np.asarray([[i, c, ring * i, ring] for i, c in enumerate(ctx)], np.int32)
        rows = np.asarray([p * 64 for p in range(ring * B)], np.int32)
        cache_rows, cache_size, window = ring * B * 64, ring * 64, 1024
    else:
        case = make_decode_case(31 + B, ctx)
        runs, rows = case.runs, case.base_rows
        cache_rows, cache_size, window = case.pool_pages * 64, 64, 0
    plan = AttentionPlan(_table(runs, rows), B, kind=kind, window=window,
                         cache_size=cache_size, page_len=64, cache_rows=cache_rows, cap=cap,
                         kv_row_bytes=KVS * 2, device=torch.device("cuda"))
    q0 = to_dev(seeded_bf16(B * NQ * D, 1))
    k0 = to_dev(seeded_bf16(cache_rows * KVS, 2))
    v0 = to_dev(seeded_bf16(cache_rows * KVS, 3))
    ks, vs = to_dev(seeded_bf16(B * KVS, 4)), to_dev(seeded_bf16(B * KVS, 5))
    cos, sin = _rope(max(ctx) + 2, 6)
    q, k, v = q0.clone(), k0.clone(), v0.clone()
    out = empty_dev(B * NQ * D, np.uint16)
    partials, ps = A.partials_buffer(plan, NQ, D)

    def step():
        A.dispatch_rope_cache_write(plan, q, ks, vs, k, v, cos, sin, num_q=NQ, num_kv=NKV,
                                    half=HALF, pair_stride=PAIR, head_dim=D)
        A.attention_bf16(plan, q, k, v, out, partials, ps, num_q=NQ, num_kv=NKV, head_dim=D,
                         kv_stride=KVS)

    def reset():
        q.copy_(q0)
        k.copy_(k0)
        v.copy_(v0)
        out.zero_()

    step()
    torch.cuda.synchronize()
    want = [from_dev(t, np.uint16) for t in (out, q, k, v)]
    reset()
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        step()
    other = empty_dev(B * NQ * D, np.uint16)
    for r in range(REPLAYS):
        reset()
        # Eager work of the program between replays: the attention into
        # another buffer on the unrotated queries.
        A.attention_bf16(plan, q0, k0, v0, other, partials, ps, num_q=NQ, num_kv=NKV,
                         head_dim=D, kv_stride=KVS)
        torch.cuda.synchronize()
        g.replay()
        torch.cuda.synchronize()
        got = [from_dev(t, np.uint16) for t in (out, q, k, v)]
        for name, a, b in zip(("output", "rotated q", "k cache", "v cache"), got, want):
            assert np.array_equal(a, b), f"replay {r}: {name} differs from the eager step"
        print(f"  replay {r}: outputs, rotated q and caches bit-exact", flush=True)
    del g


def test_graph_replays_bq_attention():
    """The int8 (butterquant) attention at Gemma-4's full-layer shape (head_dim
    512, 16q/2kv): one sequence and a batch, each captured and replayed."""
    import torch

    nq, nkv, d = 16, 2, 512
    kvs = nkv * d
    for ctx, cap in (([6000], 256), ([700, 3000, 64, 9000], 32)):
        announce(f"graph bq attention B={len(ctx)} cap={cap}")
        B = len(ctx)
        case = make_decode_case(50 + B, ctx)
        rows_n = case.pool_pages * 64
        rng = np.random.default_rng(7 + B)
        plan = AttentionPlan(_table(case.runs, case.base_rows), B, kind=FULL, window=0,
                             cache_size=64, page_len=64, cache_rows=rows_n, cap=cap,
                             kv_row_bytes=kvs, device=torch.device("cuda"))
        q = rng.integers(-127, 128, B * nq * d).astype(np.int8)
        qb = (128.0 * q.reshape(B * nq, d).astype(np.int64).sum(axis=1)).astype(np.float32)
        fq = rng.uniform(0.02, 0.06, B * nq).astype(np.float32)
        kc = rng.integers(-127, 128, rows_n * kvs).astype(np.int8)
        vc = rng.integers(-127, 128, rows_n * kvs).astype(np.int8)
        ksc = rng.uniform(0.5, 1.5, rows_n * nkv).astype(np.float32)
        vsc = rng.uniform(0.5, 2.0, rows_n * nkv).astype(np.float32)
        dev = [to_dev(x) for x in (q, qb, fq, kc, ksc, vc, vsc)]
        out = empty_dev(B * nq * d, np.uint16)
        partials, ps = A.partials_buffer(plan, nq, d)

        def attend(o):
            A.bq_attention(plan, *dev, o, partials, ps, num_q=nq, num_kv=nkv, head_dim=d,
                           kv_stride=kvs)

        attend(out)
        want = from_dev(out, np.uint16)
        out.zero_()
        torch.cuda.synchronize()
        g = torch.cuda.CUDAGraph()
        with torch.cuda.graph(g):
            attend(out)
        other = empty_dev(B * nq * d, np.uint16)
        for r in range(REPLAYS):
            out.zero_()
            attend(other)
            torch.cuda.synchronize()
            g.replay()
            torch.cuda.synchronize()
            assert np.array_equal(from_dev(out, np.uint16), want), f"replay {r} differs"
            print(f"  replay {r}: bit-exact", flush=True)
        del g


@pytest.mark.parametrize("nq,nkv,d,half,pair", [(16, 8, 256, 128, 128), (16, 2, 512, 64, 256)])
def test_graph_replays_bq_prep_and_attention(nq, nkv, d, half, pair):
    """The butterquant decode step as bench.py captures it for its int8 decode
    workloads (16q/8kv x 256 and 16q/2kv x 512): the quantising append (ifr_bq_attn_prep: RMS norm, RoPE, FWHT, int8 codes of
    q, k, v) and the int8 attention, at both layer shapes.  Every replay's
    outputs, query codes and cache codes/scales equal the eager step's."""
    import torch

    announce(f"graph bq prep + attention {nq}q/{nkv}kv x {d}")
    ctx = [3000, 700, 12000, 64]
    B = len(ctx)
    case = make_decode_case(61 + d, ctx)
    rows_n = case.pool_pages * 64
    kvs = nkv * d
    plan = AttentionPlan(_table(case.runs, case.base_rows), B, kind=FULL, window=0,
                         cache_size=64, page_len=64, cache_rows=rows_n, cap=64,
                         kv_row_bytes=kvs, device=torch.device("cuda"))
    q_src = to_dev(seeded_bf16(B * nq * d, 11))
    k_src = to_dev(seeded_bf16(B * kvs, 12))
    v_src = to_dev(seeded_bf16(B * kvs, 13))
    norm_q, norm_k = to_dev(seeded_bf16(d, 14)), to_dev(seeded_bf16(d, 15))
    cos, sin = _rope(max(ctx) + 2, 16)
    rng = np.random.default_rng(17)
    kc0 = to_dev(rng.integers(-127, 128, rows_n * kvs).astype(np.int8))
    vc0 = to_dev(rng.integers(-127, 128, rows_n * kvs).astype(np.int8))
    ks0 = to_dev(rng.uniform(0.5, 1.5, rows_n * nkv).astype(np.float32))
    vs0 = to_dev(rng.uniform(0.5, 2.0, rows_n * nkv).astype(np.float32))
    kc, vc, ks, vs = kc0.clone(), vc0.clone(), ks0.clone(), vs0.clone()
    q_i8 = empty_dev(B * nq * d, np.int8)
    qb, fq = empty_dev(B * nq, np.float32), empty_dev(B * nq, np.float32)
    out = empty_dev(B * nq * d, np.uint16)
    partials, ps = A.partials_buffer(plan, nq, d)

    def step():
        A.dispatch_bq_attn_prep(plan, q_src, k_src, v_src, norm_q, norm_k, q_i8, qb, fq, kc, ks,
                                vc, vs, cos, sin, num_q=nq, num_kv=nkv, head_dim=d,
                                rope_half=half, pair_stride=pair,
                                sqrt_n=float(np.sqrt(np.float32(d))),
                                n_eps=float(np.float32(d) * np.float32(1e-6)))
        A.bq_attention(plan, q_i8, qb, fq, kc, ks, vc, vs, out, partials, ps, num_q=nq,
                       num_kv=nkv, head_dim=d, kv_stride=kvs)

    def reset():
        for t, t0 in ((kc, kc0), (vc, vc0), (ks, ks0), (vs, vs0)):
            t.copy_(t0)
        for t in (q_i8, qb, fq, out):
            t.zero_()

    def state():
        return [from_dev(out, np.uint16), from_dev(q_i8, np.int8), from_dev(kc, np.int8),
                from_dev(vc, np.int8), from_dev(ks, np.float32).view(np.uint32),
                from_dev(vs, np.float32).view(np.uint32)]

    step()
    torch.cuda.synchronize()
    want = state()
    reset()
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        step()
    for r in range(REPLAYS):
        reset()
        A.bq_attention(plan, q_i8, qb, fq, kc0, ks0, vc0, vs0, empty_dev(B * nq * d, np.uint16),
                       partials, ps, num_q=nq, num_kv=nkv, head_dim=d, kv_stride=kvs)
        torch.cuda.synchronize()
        g.replay()
        torch.cuda.synchronize()
        for name, a, b in zip(("output", "q codes", "k codes", "v codes", "k scales",
                               "v scales"), state(), want):
            assert np.array_equal(a, b), f"replay {r}: {name} differs from the eager step"
        print(f"  replay {r}: bit-exact", flush=True)
    del g


def test_graph_replays_full_layer_decode_bf16():
    """The bf16 decode step at Gemma-4's full-attention shape (16q/2kv x 512,
    partial RoPE): the append and the wide-kernel attention, replayed."""
    import torch

    nq, nkv, d, half, pair = 16, 2, 512, 64, 256
    kvs = nkv * d
    announce("graph full-layer decode bf16")
    ctx = [5000, 300, 16000, 2048, 77]
    B = len(ctx)
    case = make_decode_case(71, ctx)
    rows_n = case.pool_pages * 64
    plan = AttentionPlan(_table(case.runs, case.base_rows), B, kind=FULL, window=0,
                         cache_size=64, page_len=64, cache_rows=rows_n, cap=128,
                         kv_row_bytes=kvs * 2, device=torch.device("cuda"))
    q0 = to_dev(seeded_bf16(B * nq * d, 21))
    k0 = to_dev(seeded_bf16(rows_n * kvs, 22))
    v0 = to_dev(seeded_bf16(rows_n * kvs, 23))
    ks, vs = to_dev(seeded_bf16(B * kvs, 24)), to_dev(seeded_bf16(B * kvs, 25))
    cos, sin = _rope(max(ctx) + 2, 26)
    q, k, v = q0.clone(), k0.clone(), v0.clone()
    out = empty_dev(B * nq * d, np.uint16)
    partials, ps = A.partials_buffer(plan, nq, d)

    def step():
        A.dispatch_rope_cache_write(plan, q, ks, vs, k, v, cos, sin, num_q=nq, num_kv=nkv,
                                    half=half, pair_stride=pair, head_dim=d)
        A.attention_bf16(plan, q, k, v, out, partials, ps, num_q=nq, num_kv=nkv, head_dim=d,
                         kv_stride=kvs)

    def reset():
        q.copy_(q0)
        k.copy_(k0)
        v.copy_(v0)
        out.zero_()

    step()
    torch.cuda.synchronize()
    want = [from_dev(t, np.uint16) for t in (out, q, k, v)]
    reset()
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        step()
    for r in range(REPLAYS):
        reset()
        torch.cuda.synchronize()
        g.replay()
        torch.cuda.synchronize()
        for name, a, b in zip(("output", "rotated q", "k cache", "v cache"),
                              [from_dev(t, np.uint16) for t in (out, q, k, v)], want):
            assert np.array_equal(a, b), f"replay {r}: {name} differs from the eager step"
        print(f"  replay {r}: bit-exact", flush=True)
    del g
