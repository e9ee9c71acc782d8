"""Host-side page state: the C++ library (inferno_amd.host) against the
oracle restatement (oracle/host.py) in lockstep on randomized workloads,
conservation invariants after every action, textbook pins for the prefix
hash, and closed-form run tables / copy jobs for kv_policy.  CPU only."""
import numpy as np
import pytest

import oracle.host as O
from inferno_amd import host as P
from inferno_amd.host import HostStateError
from inferno_amd._lib import InfernoHipError

PPP = 4


# ---------------------------------------------------------------------------
# prefix hash
# ---------------------------------------------------------------------------
def test_splitmix64_published_vectors():
    # SplitMix64 from seed 0: its outputs are splitmix64(k * golden) for
    # k = 0, 1, 2 in this stateless form (Steele, Lea, Flood 2014).
    golden = 0x9E3779B97F4A7C15
    want = [0xE220A8397B1DCDAF, 0x6E789E6AA1B965F4, 0x06C45D188009454F]
    for k, w in enumerate(want):
        x = (k * golden) & O.M64
        assert O.splitmix64(x) == w
        assert P.splitmix64(x) == w


def _fmix32(h):
    h ^= h >> 16
    h = (h * 0x85EBCA6B) & O.M32
    h ^= h >> 13
    h = (h * 0xC2B2AE35) & O.M32
    return h ^ (h >> 16)


def _oracle_lane_step(lane, token):
    """One lane of the oracle's block loop, isolated by hashing a 16-token
    block whose other lanes are fixed: lane j's update is the MurmurHash3
    x86_32 body step with the lane value as running state."""
    m = ((token & O.M32) * O.BLOCK_C1) & O.M32
    m = (O._rotl32(m, 15) * O.BLOCK_C2) & O.M32
    x = lane ^ m
    return ((O._rotl32(x, 13) * 5) + O.BLOCK_C3) & O.M32


@pytest.mark.parametrize("key,seed,want", [
    (0x00000000, 0x00000000, 0x2362F9DE),
    (0xFFFFFFFF, 0x00000000, 0x76293B50),
    (0x87654321, 0x00000000, 0xF55B516B),
    (0x87654321, 0x5082EDEE, 0x2362F9DE),
])
def test_block_step_is_murmur3_body(key, seed, want):
    """murmur3_x86_32(4-byte key, seed) = fmix32(body(seed, key) ^ 4): the
    published test vectors pin the oracle's per-lane mixing constants and
    rotations."""
    assert _fmix32(_oracle_lane_step(seed, key) ^ 4) == want


def test_hash_block_product_matches_oracle():
    rng = np.random.default_rng(5)
    for count in list(range(0, 40)) + [63, 64, 65, 1024]:
        toks = [int(x) for x in rng.integers(-2**31, 2**31, count + 3)]
        start = int(rng.integers(0, 3))
        assert P.hash_token_block(toks, start, count) == O.hash_token_block(toks, start, count)
    # A 16-token block that differs in one position in each lane changes.
    base = list(range(16))
    h0 = P.hash_token_block(base, 0, 16)
    for j in range(16):
        t = list(base)
        t[j] += 1
        assert P.hash_token_block(t, 0, 16) != h0


def test_chain_and_hashed_prefix_product_matches_oracle():
    rng = np.random.default_rng(6)
    for _ in range(200):
        n = int(rng.integers(0, 60))
        a = [int(x) for x in rng.integers(0, 5, n)]
        b = list(a)
        if n and rng.random() < 0.8:
            k = int(rng.integers(0, n))
            b[k] += 1
        b += [int(x) for x in rng.integers(0, 5, int(rng.integers(0, 9)))]
        ppp = int(rng.choice([1, 2, 4, 16]))
        ca, cb, oa, ob = [], [], [], []
        P.refresh_chain(ppp, ca, a)
        P.refresh_chain(ppp, cb, b)
        O.refresh_chain(ppp, oa, a)
        O.refresh_chain(ppp, ob, b)
        assert ca == oa and cb == ob
        got = P.hashed_prefix_len(ppp, a, ca, b, cb)
        assert got == O.hashed_prefix_len(ppp, a, oa, b, ob)
        assert got == O.token_prefix_len(a, b), "hashed prefix equals exact prefix"
    # Trimming: a shorter token list pops links.
    c = []
    P.refresh_chain(4, c, list(range(20)))
    assert len(c) == 5
    P.refresh_chain(4, c, list(range(9)))
    assert len(c) == 2


# ---------------------------------------------------------------------------
# page accountant: random operations, product vs oracle, invariants
# ---------------------------------------------------------------------------
def _state(acc, pools):
    return [tuple(np.asarray(x).tolist() for x in acc.export(p)) for p in range(pools)]


def _check_conservation(acc, n_pools, max_seqs, pins=()):
    for p in range(n_pools):
        table, holds, free = (np.asarray(x) for x in acc.export(p))
        refs = np.zeros_like(holds)
        for page in table.ravel():
            if page >= 0:
                refs[page] += 1
        for pp, page in pins:
            if pp == p:
                refs[page] += 1
        assert np.array_equal(refs, holds), "holds == table references + pins"
        assert sorted(free.tolist()) == sorted(np.nonzero(holds == 0)[0].tolist())
        assert len(set(free.tolist())) == len(free)


def test_accountant_random_ops_match_oracle():
    rng = np.random.default_rng(11)
    specs = [(10, 2, 2), (24, 0, 8)]
    max_seqs = 5
    pa = P.KVPageAccountant(max_seqs, [P.PagePoolSpec(*s) for s in specs])
    oa = O.KVPageAccountant(O.BatchGeometry(max_seqs, 4, 8, [O.PagePoolSpec(*s) for s in specs]))
    for it in range(3000):
        op = int(rng.integers(0, 7))
        seq = int(rng.integers(0, max_seqs))
        if op == 0:
            assert pa.admit() == oa.admit()
        elif op == 1:
            pa.release(seq)
            oa.release(seq)
        elif op == 2 and oa.active[seq]:
            last = int(rng.integers(0, 8))
            r1 = pa.reserve(seq, last)
            assert r1 == oa.reserve(seq, last)
        elif op == 3 and oa.active[seq]:
            keep = int(rng.integers(-1, 8))
            pa.truncate(seq, keep)
            oa.truncate(seq, keep)
        elif op == 4:
            dst = int(rng.integers(0, max_seqs))
            o = int(rng.integers(0, 8))
            if (oa.active[seq] and oa.active[dst] and seq != dst
                    and oa.page_index(1, seq, o) >= 0 and oa.page_index(1, dst, o) < 0):
                pa.share(1, seq, dst, o)
                oa.share(1, seq, dst, o)
        elif op == 5:
            o = int(rng.integers(0, 8))
            if oa.active[seq] and oa.page_index(1, seq, o) >= 0:
                assert pa.replace_with_private(1, seq, o) == oa.replace_with_private(1, seq, o)
        elif op == 6:
            last = int(rng.integers(0, 8))
            n1, n2 = [0, 0], [0, 0]
            pa.pages_needed(seq, last, n1)
            oa.pages_needed(seq, last, n2)
            assert n1 == n2 and pa.fits(n1) == oa.fits(n2)
        assert _state(pa, 2) == _state(oa, 2), f"diverged at op {it}"
        _check_conservation(pa, 2, max_seqs)


def test_accountant_contract_violations_are_errors():
    pa = P.KVPageAccountant(2, [P.PagePoolSpec(4, 0, 4)])
    s = pa.admit()
    with pytest.raises(InfernoHipError):
        pa.release_page(0, 3)  # unheld page
    with pytest.raises(InfernoHipError):
        pa.share(0, s, 1, 0)  # source unmapped
    assert pa.reserve(s, 1)
    with pytest.raises(InfernoHipError):
        pa.reserve(s, 4)  # ordinal beyond the per-sequence bound
    with pytest.raises(HostStateError):
        pa.page_index(0, 0, 9)


# ---------------------------------------------------------------------------
# scheduler: product vs oracle in lockstep on randomized serving workloads
# ---------------------------------------------------------------------------
class Clock:
    def __init__(self):
        self.t = 0

    def __call__(self):
        self.t += 1000
        return self.t


class EchoModel:
    """Samples token 7000 + (step * 7 + slot) % vocab for each emitting slot,
    so generated continuations repeat and create prefix matches."""

    def __init__(self, vocab):
        self.steps = 0
        self.vocab = vocab
        self.cancel_rid = None
        self.log = []

    def execute(self, sched, schedule, pages):
        self.steps += 1
        if self.cancel_rid is not None:
            sched.cancel(self.cancel_rid)
            self.cancel_rid = None
        self.log.append(([(s.seq_id, s.request_id, s.base_pos, s.n_tokens, s.prompt_len, s.emit)
                          for s in schedule.slots], list(schedule.tokens),
                         [(c.pool, c.src_page, c.dst_page, c.pos_start, c.pos_count)
                          for c in schedule.copies]))
        if sched.fully_cancelled():
            return []
        return [7000 + (self.steps * 7 + k) % self.vocab
                for k, s in enumerate(schedule.slots) if s.emit]


def _snapshot(sched, is_oracle, n_pools):
    reg = sched.registry
    pages = [tuple(np.asarray(x).tolist() for x in sched.pages.export(p)) for p in range(n_pools)]
    regs = []
    for sid in range(reg.max_seqs):
        toks = reg.tokens_of(sid) if is_oracle else reg.tokens(sid)
        chain = reg.chain_of(sid) if is_oracle else reg.chain(sid)
        regs.append((reg.is_resident(sid), reg.owner_of(sid), toks, chain, reg.last_used(sid),
                     sched.ring_floor(sid)))
    reqs = []
    for rid in range(sched.num_requests):
        r = sched.request(rid)
        reqs.append((r.seq_id, r.done, r.live, r.cancelled, list(r.tokens), list(r.generated)))
    return pages, regs, reqs, sched.pending()


def _family_prompt(rng, families):
    f = families[int(rng.integers(0, len(families)))]
    n = int(rng.integers(1, len(f) + 6))
    toks = list(f[:n])
    while len(toks) < n:
        toks.append(int(rng.integers(0, 50)))
    if rng.random() < 0.3 and toks:
        k = int(rng.integers(0, len(toks)))
        toks[k] = int(rng.integers(50, 60))
    return toks


@pytest.mark.parametrize("seed", range(6))
def test_scheduler_lockstep_random_workload(seed):
    rng = np.random.default_rng(100 + seed)
    max_seqs = int(rng.integers(3, 7))
    ring = (max_seqs * 2, 2, 2)
    grow_pages = int(rng.integers(8, 26))
    grow = (grow_pages, 0, int(rng.integers(6, 12)))
    max_slots = int(rng.integers(1, 5))
    max_step = int(rng.integers(4, 17))
    budget = int(rng.integers(4, 17))
    stops = [7003] if seed % 2 else [-1]
    pg = P.BatchGeometry(max_seqs, max_slots, max_step, [P.PagePoolSpec(*ring),
                                                         P.PagePoolSpec(*grow)])
    og = O.BatchGeometry(max_seqs, max_slots, max_step, [O.PagePoolSpec(*ring),
                                                         O.PagePoolSpec(*grow)])
    ps = P.ContinuousBatchScheduler(PPP, pg, budget, stops)
    os_ = O.ContinuousBatchScheduler(PPP, og, budget, stops)
    pclock, oclock = Clock(), Clock()
    pm, om = EchoModel(5), EchoModel(5)
    families = [[int(x) for x in rng.integers(0, 50, 24)] for _ in range(3)]
    actions = {"submit": 0, "step": 0, "cancel": 0, "retire": 0, "evict": 0}
    for it in range(400):
        r = rng.random()
        if r < 0.25:
            toks = _family_prompt(rng, families)
            mx = int(rng.integers(1, 6))
            ns = bool(rng.random() < 0.1)
            a, b = ps.submit(toks, mx, ns), os_.submit(toks, mx, ns)
            assert a == b
            actions["submit"] += 1
        elif r < 0.30 and os_.num_requests:
            rid = int(rng.integers(0, os_.num_requests))
            if os_.request(rid).live and not os_.request(rid).done:
                if rng.random() < 0.5:
                    ps.cancel(rid)
                    os_.cancel(rid)
                else:  # cancelled mid-step, from inside the model
                    pm.cancel_rid = om.cancel_rid = rid
                actions["cancel"] += 1
        elif r < 0.38 and os_.num_requests:
            rid = int(rng.integers(0, os_.num_requests))
            assert ps.retire(rid) == os_.retire(rid)
            actions["retire"] += 1
        elif r < 0.40:
            assert ps.evict_warm() == os_.evict_warm()
            actions["evict"] += 1
        else:
            assert ps.step(pm, pclock) == os_.step(om, oclock)
            actions["step"] += 1
            assert pm.log == om.log
        assert _snapshot(ps, False, 2) == _snapshot(os_, True, 2), f"diverged at action {it}"
        assert ps.invariant_failures == os_.invariant_failures
        _check_conservation(ps.pages, 2, max_seqs)
    assert actions["step"] > 100 and actions["submit"] > 50
    # The workload exercised sharing and copy-on-write.
    assert any(log[2] for log in om.log), "no prefix copy was scheduled"


# ---------------------------------------------------------------------------
# kv_policy
# ---------------------------------------------------------------------------
def test_prefix_copy_jobs_closed_form():
    ring = P.KVPoolMirror(64, 1, 1000, 10_000_000, 2, [(0, 4096), (5_000_000, 4096)],
                          P.PagePoolSpec(32, 2, 2))
    full = P.KVPoolMirror(64, 2, 50_000_000, 20_000_000, 1, [(0, 2048), (8_000_000, 2048)],
                          P.PagePoolSpec(100, 0, 50))
    copies = [P.PageCopy(0, 3, 7, 5, 10), P.PageCopy(1, 9, 4, 5, 10)]
    jobs = P.prefix_copy_jobs([ring, full], copies).tolist()
    # Ring pool: rows 5..14 of page 3 -> page 7, per layer (2) x component (2).
    want = []
    for l in range(2):
        for off in (0, 5_000_000):
            base = 1000 + l * 10_000_000 + off
            want.append([base + (3 * 64 + 5) * 4096, base + (7 * 64 + 5) * 4096, 10 * 4096])
    # Position-sharded pool (pos_shard 2, 32 rows per page): positions 5..14
    # are rows 2..7 (row_end = ceil(15 / 2) = 8).
    for off in (0, 8_000_000):
        base = 50_000_000 + off
        want.append([base + (9 * 32 + 2) * 2048, base + (4 * 32 + 2) * 2048, 6 * 2048])
    assert jobs == want
    # The oracle restatement agrees.
    ojobs = []
    for c, m in zip(copies, [ring, full]):
        om = O.KVPoolMirror(m.page_len, m.pos_shard, m.region_off, m.stride, m.layers,
                            m.components, O.PagePoolSpec(*m.spec.__dict__.values()))
        O.append_prefix_copy_jobs(om, O.PageCopy(c.pool, c.src_page, c.dst_page, c.pos_start,
                                                 c.pos_count), ojobs)
    assert [list(j) for j in ojobs] == want


def test_bind_pool_run_table_matches_pages_and_oracle():
    geom = P.BatchGeometry(4, 4, 64, [P.PagePoolSpec(8, 2, 2), P.PagePoolSpec(40, 0, 10)])
    ogeom = O.BatchGeometry(4, 4, 64, [O.PagePoolSpec(8, 2, 2), O.PagePoolSpec(40, 0, 10)])
    ps = P.ContinuousBatchScheduler(PPP, geom, 64, [-1])
    os_ = O.ContinuousBatchScheduler(PPP, ogeom, 64, [-1])
    for toks in ([1, 2, 3, 4, 5, 6, 7, 8, 9, 10], [1, 2, 3, 4, 5, 6, 7, 8, 11], [20, 21, 22]):
        ps.submit(toks, 3)
        os_.submit(toks, 3)
    pc, oc = Clock(), Clock()
    pm, om = EchoModel(9), EchoModel(9)
    mirrors = [P.KVPoolMirror(PPP, 1, 0, 0, 1, [(0, 16)], P.PagePoolSpec(8, 2, 2)),
               P.KVPoolMirror(PPP, 2, 0, 0, 1, [(0, 16)], P.PagePoolSpec(40, 0, 10))]
    for _ in range(6):
        assert ps.build_schedule(pc()) == os_.build_schedule(oc())
        sched = ps.schedule
        for pool, mirror in enumerate(mirrors):
            t = P.bind_pool_run_table(ps, pool, mirror)
            om_ = O.KVPoolMirror(mirror.page_len, mirror.pos_shard, 0, 0, 1, [(0, 16)],
                                 O.PagePoolSpec(*mirror.spec.__dict__.values()))
            oruns, orows = O.bind_pool_run_table(os_.schedule, os_.pages, pool, om_)
            assert t.runs == oruns and t.base_rows == orows
            buf = 0
            for s, run in zip(sched.slots, t.runs):
                assert run[0] == buf and run[1] == s.base_pos
                pages = [ps.pages.page_index(pool, s.seq_id, o) for o in range(run[3])]
                assert t.base_rows[run[2]:run[2] + run[3]] == [
                    pg * mirror.rows_per_page() for pg in pages]
                buf += s.n_tokens
        outs = pm.execute(ps, sched, ps.pages)
        ps.absorb(outs, pc())
        os_.absorb(om.execute(os_, os_.schedule, os_.pages), oc())


@pytest.mark.parametrize("ring_pages,ppp", [(32, 64), (2, 1024)])
def test_config3_ring_256_decode_steps_lockstep(ring_pages, ppp):
    """Config 3's page-state check: 64 sequences on rings of window 1024 x 2
    positions -- 32 pages of 64 tokens, or Gemma-4's production 2 pages of
    1024 (modeling/gemma4_topology.mojo:36,40) -- plus a growing pool,
    prefilled past the ring wrap, then 256 decode steps of the whole batch;
    page tables, holds, free stacks and ring floors of the C++ scheduler
    equal the oracle's after every step."""
    rng = np.random.default_rng(33)
    B = 64
    ctx = [int(x) for x in rng.integers(1023, 4096, B)]
    new_tokens = 700
    grow_pages = sum((c + new_tokens) // ppp + 1 for c in ctx)
    specs = [(B * ring_pages, ring_pages, ring_pages), (grow_pages, 0, 5120 // ppp)]
    pg = P.BatchGeometry(B, B, 1024, [P.PagePoolSpec(*s) for s in specs])
    og = O.BatchGeometry(B, B, 1024, [O.PagePoolSpec(*s) for s in specs])
    ps = P.ContinuousBatchScheduler(ppp, pg, 1024, [-1])
    os_ = O.ContinuousBatchScheduler(ppp, og, 1024, [-1])
    for i in range(B):
        toks = [int(x) for x in rng.integers(0, 30000, ctx[i])]
        toks[0] = 40000 + i  # no shared prefixes
        assert ps.submit(toks, new_tokens) == os_.submit(toks, new_tokens)
    pc, oc = Clock(), Clock()
    pm, om = EchoModel(997), EchoModel(997)
    decode_steps = steps = 0
    while decode_steps < 256:
        n = ps.step(pm, pc)
        assert n == os_.step(om, oc) and n > 0
        assert pm.log[-1] == om.log[-1]
        slots = pm.log[-1][0]
        if len(slots) == B and all(s[3] == 1 for s in slots):
            decode_steps += 1
        assert _snapshot(ps, False, 2) == _snapshot(os_, True, 2)
        _check_conservation(ps.pages, 2, B)
        steps += 1
        assert steps < 2000
    wrapped = sum(ps.registry.length(sid) > ring_pages * ppp for sid in range(B))
    assert wrapped > B // 2, "most rings wrapped"
    assert ps.invariant_failures == (0, 0)


def test_export_schedule_checks_every_capacity():
    """ifr_scheduler_export_schedule refuses a slots, tokens or copies
    capacity below the built schedule's count with IFR_ESPACE and writes
    nothing, like the other exports."""
    import ctypes as C

    from inferno_amd._lib import lib

    geo = P.BatchGeometry(4, 4, 64, [P.PagePoolSpec(8, 2, 2), P.PagePoolSpec(40, 0, 10)])
    s = P.ContinuousBatchScheduler(PPP, geo, 64, [-1])
    s.submit(list(range(10)), 3, False)
    s.submit(list(range(20, 27)), 3, False)
    assert s.build_schedule(1000)
    ns, nt = s._query("NUM_SLOTS"), s._query("NUM_TOKENS")
    assert ns == 2 and nt == 17
    slots = np.full((ns, 6), -7, dtype=np.int64)
    toks = np.full(nt, -7, dtype=np.int32)
    vp = lambda a: a.ctypes.data_as(C.c_void_p)
    f = lib().ifr_scheduler_export_schedule
    assert f(s._h, vp(slots), ns - 1, vp(toks), nt, None, 0) == -4
    assert f(s._h, vp(slots), ns, vp(toks), nt - 1, None, 0) == -4
    assert (slots == -7).all() and (toks == -7).all(), "a refused export wrote"
    assert f(s._h, vp(slots), ns, vp(toks), nt, None, 0) == 0
    assert list(slots[:, 3]) == [10, 7] and list(toks[:10]) == list(range(10))
    # With no copies in the schedule a zero copies capacity is enough.
    copies = np.full((1, 5), -7, dtype=np.int64)
    assert f(s._h, None, 0, None, 0, vp(copies), 0) == 0 and (copies == -7).all()
