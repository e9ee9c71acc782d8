"""GPU parity of the whole step path as a serving loop drives it: the C++
scheduler's run tables and copy-on-write page copies feed the append and
attention kernels (ring pool -> sliding layer, growing pool -> full layer),
checked step by step against the oracle scheduler and a CPU mirror of the
KV arena (see tests/serving_harness.py)."""
import numpy as np
import pytest

from inferno_amd.kv import FULL, SLIDING
from tests.gpu_util import announce
from tests.serving_harness import PoolLayer, ServingHarness

pytestmark = pytest.mark.gpu


def test_config3_ring_serving_loop():
    """Config 3 at one GPU's share: 16 sequences on 32-page rings (window
    1024) plus a growing pool for the full layer, prompts of 1100-2600
    tokens (most rings wrap), chunked prefill, then 256 decode steps."""
    announce("serving loop config3 ring")
    rng = np.random.default_rng(7)
    B, ring = 16, 32
    ctx = [int(x) for x in rng.integers(1100, 2601, B)]
    new_tokens = 300
    grow_pages = sum((c + new_tokens) // 64 + 1 for c in ctx) + 8
    h = ServingHarness(max_seqs=B, max_slots=B, max_step_tokens=1024, step_budget=1024,
                       pools=[PoolLayer(B * ring, ring, ring, SLIDING, window=1024),
                              PoolLayer(grow_pages, 0, 64, FULL)],
                       cap=128, max_pos=4096, seed=8)
    for i in range(B):
        toks = [int(x) for x in rng.integers(0, 30000, ctx[i])]
        toks[0] = 40000 + i
        h.submit(toks, new_tokens)
    decode_steps = steps = 0
    while decode_steps < 256:
        check = steps < 3 or steps % 32 == 0
        rep = h.step(check_attention=check, rng=rng)
        assert rep is not None
        if rep["tokens"] == rep["slots"] == B:
            decode_steps += 1
        if steps % 64 == 0:
            h.compare_arena()
        if check:
            print(f"  step {steps}: {rep['tokens']} tokens {rep['slots']} slots "
                  f"{rep['checks']}", flush=True)
        steps += 1
    h.compare_arena()
    wrapped = sum(h.ps.registry.length(s) > ring * 64 for s in range(B))
    print(f"  {steps} steps, {len(h.checked)} attention checks, {wrapped} rings wrapped",
          flush=True)
    assert wrapped >= B // 2
    assert h.ps.invariant_failures == (0, 0)


def test_config4_prefix_sharing_copy_on_write():
    """Config 4's sharing pattern at reduced length: four donors prefill
    prompts of P_k + 256 tokens (P_k ~ U[64, 2000]); while they decode, four
    requests sharing their first P_k tokens fork: sealed pages are shared,
    the divergent partial page and the ring's live window are copied on the
    GPU, and the forks prefill their own 512 tokens over the shared pages."""
    announce("serving loop config4 prefix sharing")
    rng = np.random.default_rng(9)
    pairs = 4
    prefix = [int(x) for x in rng.integers(64, 2001, pairs)]
    prefix[0] = 1280  # one page-aligned prefix: sealed pages only
    grow_pages = sum((p + 1024) // 64 + 2 for p in prefix) * 2
    h = ServingHarness(max_seqs=2 * pairs, max_slots=2 * pairs, max_step_tokens=2048,
                       step_budget=2048,
                       pools=[PoolLayer(2 * pairs * 32, 32, 32, SLIDING, window=1024),
                              PoolLayer(grow_pages, 0, 64, FULL)],
                       cap=16, max_pos=4096, seed=10)
    base = [[int(x) for x in rng.integers(0, 30000, p)] for p in prefix]
    for k in range(pairs):
        base[k][0] = 41000 + k
        h.submit(base[k] + [int(x) for x in rng.integers(0, 30000, 256)], 64)
    steps = 0
    while True:  # donors prefill and start decoding
        rep = h.step(check_attention=steps % 2 == 0, rng=rng)
        steps += 1
        if all(h.ps.request(k).generated for k in range(pairs)):
            break
        assert steps < 100
    forks = [h.submit(base[k] + [int(x) for x in rng.integers(30000, 31000, 512)], 2)
             for k in range(pairs)]
    copies = 0
    while any(not h.ps.request(r).done for r in forks):
        rep = h.step(check_attention=True, rng=rng)
        copies += rep["copies"]
        print(f"  step {steps}: {rep['tokens']} tokens, {rep['copies']} copy jobs "
              f"{rep['checks']}", flush=True)
        steps += 1
        assert steps < 200
    h.compare_arena()
    for k, r in enumerate(forks):
        sid, donor = h.ps.request(r).seq_id, h.ps.request(k).seq_id
        sealed = prefix[k] // 64
        for o in range(sealed):
            assert (h.ps.pages.page_index(1, sid, o) == h.ps.pages.page_index(1, donor, o)), \
                f"fork {k} ordinal {o} shares the donor's page"
    assert copies > 0 and h.copies_done > 0
    assert h.ps.invariant_failures == (0, 0)


def test_config3_ring_serving_loop_page1024():
    """The same loop at Gemma-4's production geometry: 1024-token pages, the
    sliding pool on 2-page rings (modeling/gemma4_topology.mojo:36,40), the
    full layer's pool growing in 1024-token pages; prompts of 1100-2600
    tokens wrap most rings, then 256 decode steps."""
    announce("serving loop config3 ring, 1024-token pages")
    rng = np.random.default_rng(17)
    B, ring, page = 8, 2, 1024
    ctx = [int(x) for x in rng.integers(1100, 2601, B)]
    new_tokens = 300
    grow_pages = sum((c + new_tokens) // page + 1 for c in ctx) + 2
    h = ServingHarness(max_seqs=B, max_slots=B, max_step_tokens=1024, step_budget=1024,
                       pools=[PoolLayer(B * ring, ring, ring, SLIDING, window=1024,
                                        page_len=page),
                              PoolLayer(grow_pages, 0, 4, FULL, page_len=page)],
                       cap=128, max_pos=4096, seed=18, page_len=page)
    for i in range(B):
        toks = [int(x) for x in rng.integers(0, 30000, ctx[i])]
        toks[0] = 42000 + i
        h.submit(toks, new_tokens)
    decode_steps = steps = 0
    while decode_steps < 256:
        check = steps < 3 or steps % 32 == 0
        rep = h.step(check_attention=check, rng=rng)
        assert rep is not None
        if rep["tokens"] == rep["slots"] == B:
            decode_steps += 1
        if steps % 64 == 0:
            h.compare_arena()
        if check:
            print(f"  step {steps}: {rep['tokens']} tokens {rep['slots']} slots "
                  f"{rep['checks']}", flush=True)
        steps += 1
    h.compare_arena()
    wrapped = sum(h.ps.registry.length(s) > ring * page for s in range(B))
    print(f"  {steps} steps, {len(h.checked)} attention checks, {wrapped} rings wrapped",
          flush=True)
    assert wrapped >= B // 2
    assert h.ps.invariant_failures == (0, 0)
