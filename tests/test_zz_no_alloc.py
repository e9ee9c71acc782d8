"""ifr_attention_bf16_noalloc (partials in the library's static device array)
against ifr_attention_bf16 (caller partials): both run the same kernels, so
the outputs are bit-identical.  Two calls in a row, the second with a smaller
plan, so the second reuses the array the first left behind; a plan whose
partials exceed IFR_STATIC_SCRATCH_BYTES is refused on the host; prefill
chunks on the MFMA routes (no partials) run whatever their stripe count; a
decode step through the entry point is captured in a HIP graph and replayed."""
import ctypes as C

import numpy as np
import pytest

from inferno_amd import attention as A
from inferno_amd._lib import lib
from inferno_amd.kv import FULL, AttentionPlan, KVRunTable, flash_partial_stride
from tests.gpu_util import announce, empty_dev, from_dev, to_dev
from tests.helpers import make_decode_case, make_prefill_case, seeded_bf16

pytestmark = pytest.mark.gpu

STATIC_BYTES = 32 << 20
IFR_ESPACE = -4


def _table(case) -> KVRunTable:
    t = KVRunTable()
    for r in case.runs:
        t.begin_run(int(r[0]), int(r[1]))
        for j in range(int(r[3])):
            t.add_base_row(int(case.base_rows[int(r[2]) + j]))
    return t


def _noalloc(plan, q, k, v, out, nq, nkv, d):
    import torch

    return lib().ifr_attention_bf16_noalloc(
        int(plan.image.data_ptr()), plan.info_ptr, int(q.data_ptr()), int(k.data_ptr()),
        int(v.data_ptr()), int(out.data_ptr()), nq, nkv, d, nkv * d, plan.page_len,
        plan.page_mask, int(torch.cuda.current_stream().cuda_stream))


@pytest.mark.parametrize("shape", [(16, 8, 256), (16, 2, 512)])
def test_noalloc_matches_caller_partials(shape):
    nq, nkv, d = shape
    kvs = nkv * d
    for call, (B, cap, seed) in enumerate([(12, 512, 1), (3, 64, 2)]):
        announce(f"noalloc shape={shape} call={call} B={B} cap={cap}")
        rng = np.random.default_rng(seed)
        ctx = [int(x) for x in rng.integers(500, 6000, B)]
        case = make_decode_case(seed + 10, ctx)
        plan = AttentionPlan(_table(case), B, kind=FULL, window=0, cache_size=64, page_len=64,
                             cache_rows=case.cache_rows, cap=cap, kv_row_bytes=kvs * 2)
        assert plan.summary.num_stripes * flash_partial_stride(nq, d) * 4 <= STATIC_BYTES
        q = to_dev(seeded_bf16(B * nq * d, seed + 20))
        k = to_dev(seeded_bf16(case.cache_rows * kvs, seed + 21))
        v = to_dev(seeded_bf16(case.cache_rows * kvs, seed + 22))
        want = empty_dev(B * nq * d, np.uint16)
        partials, ps = A.partials_buffer(plan, nq, d)
        A.attention_bf16(plan, q, k, v, want, partials, ps, num_q=nq, num_kv=nkv, head_dim=d,
                         kv_stride=kvs)
        got = empty_dev(B * nq * d, np.uint16)
        assert _noalloc(plan, q, k, v, got, nq, nkv, d) == 0
        w, g = from_dev(want, np.uint16), from_dev(got, np.uint16)
        print(f"  stripes={plan.summary.num_stripes} differing={int((w != g).sum())}",
              flush=True)
        assert np.array_equal(w, g)


def test_noalloc_refuses_oversized_plan():
    """4096 stripes of 16 x 512 partials (134 MB) exceed the array: IFR_ESPACE
    before any launch.  The K and V bases are null, which the host's own
    argument checks reject too, so a call that got past the size check would
    return an error rather than launch on buffers the plan does not fit."""
    import torch

    announce("noalloc oversized plan")
    case = make_decode_case(5, [60000, 60000])
    plan = AttentionPlan(_table(case), 2, kind=FULL, window=0, cache_size=64, page_len=64,
                         cache_rows=case.cache_rows, cap=4096, kv_row_bytes=2 * 1024)
    assert plan.summary.num_stripes * flash_partial_stride(16, 512) * 4 > STATIC_BYTES
    q = empty_dev(2 * 16 * 512, np.uint16)
    out = empty_dev(2 * 16 * 512, np.uint16)
    st = lib().ifr_attention_bf16_noalloc(
        int(plan.image.data_ptr()), plan.info_ptr, int(q.data_ptr()), 0, 0,
        int(out.data_ptr()), 16, 2, 512, 2 * 512, plan.page_len, plan.page_mask,
        int(torch.cuda.current_stream().cuda_stream))
    assert st == IFR_ESPACE
    buf = C.create_string_buffer(512)
    lib().ifr_last_error(buf, 512)
    assert b"static scratch" in buf.value


@pytest.mark.parametrize("shape", [(16, 8, 256), (16, 2, 512)])
def test_noalloc_runs_long_prefill_chunks(shape):
    """A prefill chunk of 3,000 tokens: its token plan has one stripe per token
    (3,000 x 16.5 KB or 33 KB of partials, beyond the static array), but the
    MFMA prefill route writes no partials, so the entry point runs it, bit for
    bit as ifr_attention_bf16 does."""
    nq, nkv, d = shape
    kvs = nkv * d
    announce(f"noalloc long prefill chunk shape={shape}")
    prefix, new = [5000, 0], [1800, 1200]
    case = make_prefill_case(71, prefix, new)
    n = sum(new)
    plan = AttentionPlan(_table(case), n, kind=FULL, window=0, cache_size=64, page_len=64,
                         cache_rows=case.cache_rows, cap=16, kv_row_bytes=kvs * 2)
    assert int(plan.info[14]) > 0
    assert plan.summary.num_stripes * flash_partial_stride(nq, d) * 4 > STATIC_BYTES
    q = to_dev(seeded_bf16(n * nq * d, 72))
    k = to_dev(seeded_bf16(case.cache_rows * kvs, 73))
    v = to_dev(seeded_bf16(case.cache_rows * kvs, 74))
    want = empty_dev(n * nq * d, np.uint16)
    partials, ps = A.partials_buffer(plan, nq, d)
    A.attention_bf16(plan, q, k, v, want, partials, ps, num_q=nq, num_kv=nkv, head_dim=d,
                     kv_stride=kvs)
    got = empty_dev(n * nq * d, np.uint16)
    assert _noalloc(plan, q, k, v, got, nq, nkv, d) == 0
    assert np.array_equal(from_dev(want, np.uint16), from_dev(got, np.uint16))


@pytest.mark.parametrize("shape", [(16, 8, 256), (16, 2, 512)])
def test_noalloc_graph_replays_decode_step(shape):
    """A decode step through the entry point captured in a HIP graph: each
    replay (with eager calls of the entry point on another plan, which reuse
    the static array, and synchronisations in between) gives the eager
    step's outputs bit for bit."""
    import torch

    nq, nkv, d = shape
    kvs = nkv * d
    announce(f"noalloc graph decode shape={shape}")
    ctx = [300, 5000, 1200, 64, 9000, 17, 2048, 700]
    B = len(ctx)
    case = make_decode_case(81, ctx)
    plan = AttentionPlan(_table(case), B, kind=FULL, window=0, cache_size=64, page_len=64,
                         cache_rows=case.cache_rows, cap=256, kv_row_bytes=kvs * 2,
                         device=torch.device("cuda"))
    assert plan.summary.num_stripes * flash_partial_stride(nq, d) * 4 <= STATIC_BYTES
    q = to_dev(seeded_bf16(B * nq * d, 82))
    k = to_dev(seeded_bf16(case.cache_rows * kvs, 83))
    v = to_dev(seeded_bf16(case.cache_rows * kvs, 84))
    out = empty_dev(B * nq * d, np.uint16)
    assert _noalloc(plan, q, k, v, out, nq, nkv, d) == 0
    want = from_dev(out, np.uint16)
    other_case = make_decode_case(85, [4000, 100])
    other_plan = AttentionPlan(_table(other_case), 2, kind=FULL, window=0, cache_size=64,
                               page_len=64, cache_rows=other_case.cache_rows, cap=64,
                               kv_row_bytes=kvs * 2, device=torch.device("cuda"))
    oq = to_dev(seeded_bf16(2 * nq * d, 86))
    ok_ = to_dev(seeded_bf16(other_case.cache_rows * kvs, 87))
    ov = to_dev(seeded_bf16(other_case.cache_rows * kvs, 88))
    other = empty_dev(2 * nq * d, np.uint16)
    out.zero_()
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        assert _noalloc(plan, q, k, v, out, nq, nkv, d) == 0
    for r in range(4):
        out.zero_()
        assert _noalloc(other_plan, oq, ok_, ov, other, nq, nkv, d) == 0
        torch.cuda.synchronize()
        g.replay()
        torch.cuda.synchronize()
        assert np.array_equal(from_dev(out, np.uint16), want), f"replay {r} differs"
        print(f"  replay {r}: bit-exact", flush=True)
    del g
