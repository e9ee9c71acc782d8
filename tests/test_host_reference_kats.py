"""The reference's own known-answer tests for the host-side page state, run
against both the oracle restatement (oracle/host.py) and the product C++
library (inferno_amd.host over include/inferno_host.h).

Ported from tests/test_slot_registry.mojo:48-242 and
tests/test_scheduler_reuse.mojo:18-491 with the same inputs, the same
expected integers and the same StubModel.  CPU only."""
import types

import pytest

import oracle.host as O
from inferno_amd import host as P


def _impl(name):
    if name == "oracle":
        return types.SimpleNamespace(
            name=name, PagePoolSpec=O.PagePoolSpec, BatchGeometry=O.BatchGeometry,
            SlotRegistry=lambda ppp, n: O.SlotRegistry(ppp, n), refresh_chain=O.refresh_chain,
            Scheduler=O.ContinuousBatchScheduler)
    return types.SimpleNamespace(
        name=name, PagePoolSpec=P.PagePoolSpec, BatchGeometry=P.BatchGeometry,
        SlotRegistry=lambda ppp, n: P.SlotRegistry(ppp, n), refresh_chain=P.refresh_chain,
        Scheduler=P.ContinuousBatchScheduler)


@pytest.fixture(params=["oracle", "product"])
def impl(request):
    return _impl(request.param)


# ---------------------------------------------------------------------------
# tests/test_slot_registry.mojo
# ---------------------------------------------------------------------------
REG_PPP = 2


def plen(impl, reg, sid, q, ppp=REG_PPP):
    chain = []
    impl.refresh_chain(ppp, chain, q)
    return reg.prefix_len(sid, q, chain)


def best_prefix(impl, reg, incoming, want_owned, ppp=REG_PPP):
    chain = []
    impl.refresh_chain(ppp, chain, incoming)
    best, best_lcp = -1, 0
    for sid in range(reg.max_seqs):
        if not reg.is_resident(sid):
            continue
        if (reg.owner_of(sid) >= 0) != want_owned:
            continue
        lcp = reg.prefix_len(sid, incoming, chain)
        if lcp > best_lcp:
            best, best_lcp = sid, lcp
    return best, best_lcp


def test_registry_match_on_empty(impl):
    reg = impl.SlotRegistry(REG_PPP, 4)
    assert best_prefix(impl, reg, [1, 2, 3], False)[0] == -1
    assert best_prefix(impl, reg, [1, 2, 3], True)[0] == -1
    assert reg.lru_victim() == -1


def test_registry_prefix_len(impl):
    reg = impl.SlotRegistry(REG_PPP, 4)
    reg.open(0, 10, 100)
    reg.extend(0, [1, 2, 3], 0, 0, 3, 100)
    reg.set_warm(0)
    assert plen(impl, reg, 0, [1, 2, 3, 4, 5]) == 3, "continuation matches whole history"
    assert reg.length(0) == 3
    assert plen(impl, reg, 0, [9, 9, 9, 9]) == 0
    assert plen(impl, reg, 0, [1, 2, 9, 9]) == 2
    assert plen(impl, reg, 0, [1, 2, 3]) == 3
    assert plen(impl, reg, 0, [1, 2]) == 2


def test_registry_owner_partition(impl):
    reg = impl.SlotRegistry(REG_PPP, 4)
    reg.open(2, 5, 50)
    reg.extend(2, [7, 8], 0, 0, 2, 50)
    cont = [7, 8, 9]
    assert best_prefix(impl, reg, cont, False)[0] == -1
    assert best_prefix(impl, reg, cont, True) == (2, 2)
    assert reg.lru_victim() == -1
    reg.set_warm(2)
    assert best_prefix(impl, reg, cont, False)[0] == 2
    assert best_prefix(impl, reg, cont, True)[0] == -1
    assert reg.lru_victim() == 2


def test_registry_longest_prefix_wins(impl):
    reg = impl.SlotRegistry(REG_PPP, 4)
    reg.open(0, 1, 10)
    reg.extend(0, [1, 2], 0, 0, 2, 10)
    reg.set_warm(0)
    reg.open(1, 2, 20)
    reg.extend(1, [1, 2, 3, 4], 0, 0, 4, 20)
    reg.set_warm(1)
    assert best_prefix(impl, reg, [1, 2, 3, 4, 5, 6], False) == (1, 4)
    assert best_prefix(impl, reg, [1, 2, 9, 9], False)[1] == 2


def test_registry_lru_victim(impl):
    reg = impl.SlotRegistry(REG_PPP, 4)
    for sid, (tok, t) in enumerate([(1, 300), (2, 100), (3, 200)]):
        reg.open(sid, sid + 1, t)
        reg.extend(sid, [tok], 0, 0, 1, t)
        reg.set_warm(sid)
    assert reg.lru_victim() == 1
    reg.close(1)
    assert reg.lru_victim() == 2
    assert reg.length(1) == 0
    assert not reg.is_resident(1)
    assert best_prefix(impl, reg, [2, 2], False)[0] == -1


def test_registry_seed_and_truncate(impl):
    reg = impl.SlotRegistry(REG_PPP, 4)
    reg.open(0, 1, 100)
    reg.seed(0, [5, 6, 7, 8], 3, 100)
    assert reg.length(0) == 3
    cont = [5, 6, 7, 9, 9]
    reg.set_warm(0)
    assert best_prefix(impl, reg, cont, False) == (0, 3)
    reg.adopt(0, 7, 200)
    reg.seed(0, cont, 2, 200)
    assert reg.length(0) == 2
    assert reg.owner_of(0) == 7


def test_registry_divergent_reseed(impl):
    reg = impl.SlotRegistry(REG_PPP, 4)
    original = [1, 2, 3, 4]
    reg.open(0, 1, 10)
    reg.extend(0, original, 0, 0, 4, 10)
    reg.set_warm(0)
    assert plen(impl, reg, 0, original) == 4
    divergent = [1, 9, 3, 4]
    reg.adopt(0, 2, 20)
    reg.seed(0, divergent, 4, 20)
    assert plen(impl, reg, 0, divergent) == 4
    assert plen(impl, reg, 0, original) == 1, "stale chain entries must not survive"


def test_registry_hashed_matches_exact(impl):
    wide = 16
    reg = impl.SlotRegistry(wide, 2)
    history = [1000 + i * 7 for i in range(64)]
    reg.open(0, 1, 10)
    reg.extend(0, history, 0, 0, 64, 10)
    reg.set_warm(0)
    mismatched = 0
    for divergence in range(65):
        q = list(history)
        if divergence < 64:
            q[divergence] = -1
        hashed = plen(impl, reg, 0, q, wide)
        exact = reg.exact_prefix_len(0, q)
        if hashed != exact or exact != min(divergence, 64):
            mismatched += 1
    assert mismatched == 0
    longer = [1000 + i * 7 for i in range(80)]
    assert plen(impl, reg, 0, longer, wide) == 64


# ---------------------------------------------------------------------------
# tests/test_scheduler_reuse.mojo
# ---------------------------------------------------------------------------
PPP = 4
RING_POOL, GROW_POOL = 0, 1
RING_PAGES, GROW_PAGES = 8, 16


class Clock:
    """Strictly increasing stand-in for perf_counter_ns()."""

    def __init__(self):
        self.t = 0

    def __call__(self):
        self.t += 1000
        return self.t


class StubModel:
    """tests/test_scheduler_reuse.mojo:18-73."""

    def __init__(self):
        self.steps = 0
        self.fed_tokens = 0
        self.ring_copy_positions = 0
        self.grow_copy_positions = 0
        self.next_token = 9000
        self.cancel_at_step = -1
        self.victim = None
        self.aborted_steps = 0

    def execute(self, sched, schedule, pages):
        self.steps += 1
        if self.steps == self.cancel_at_step:
            sched.cancel(self.victim)
        if sched.fully_cancelled():
            self.aborted_steps += 1
            return []
        self.fed_tokens += len(schedule.tokens)
        for c in schedule.copies:
            if c.pool == RING_POOL:
                self.ring_copy_positions += c.pos_count
            else:
                self.grow_copy_positions += c.pos_count
        outs = []
        for s in schedule.slots:
            if s.emit:
                outs.append(self.next_token)
                self.next_token += 1
        return outs


def stub_geometry(impl):
    return impl.BatchGeometry(4, 4, 8, [impl.PagePoolSpec(RING_PAGES, 2, 2),
                                        impl.PagePoolSpec(GROW_PAGES, 0, GROW_PAGES)])


def run_until_idle(sched, model, clock):
    steps = 0
    while sched.pending_work():
        if sched.step(model, clock) == 0:
            break
        steps += 1
    return steps


def test_scheduler_reuse_main_sequence(impl):
    """test_scheduler_reuse.mojo:95-290: fresh prefill, adoption + fork,
    privatization, cancellation, retirement, mid-step abort, drain."""
    clock = Clock()
    model = StubModel()
    sched = impl.Scheduler(PPP, stub_geometry(impl), 8, [-1])
    pages, reg = sched.pages, sched.registry

    # fresh prefill
    rf = sched.submit([100 + t for t in range(9)], 1)
    assert run_until_idle(sched, model, clock) == 2, "9-token prompt prefills in two steps"
    assert model.fed_tokens == 9
    assert sched.request(rf).done
    sid_f = sched.request(rf).seq_id

    # adoption (take) and fork (point + copy)
    rk = sched.submit(list(sched.request(rf).tokens) + [111], 1)
    rl = sched.submit([100 + t for t in range(9)] + [222], 1)
    fed_before = model.fed_tokens
    assert run_until_idle(sched, model, clock) == 1, "adoption and fork settle in one step"
    assert model.fed_tokens - fed_before == 3, "21 requested tokens cost 3 fed tokens"
    assert sched.request(rk).seq_id == sid_f, "warm sequence is donated to the continuation"
    sid_l = sched.request(rl).seq_id
    assert sid_l != sid_f
    assert pages.page_index(GROW_POOL, sid_f, 0) == pages.page_index(GROW_POOL, sid_l, 0)
    assert pages.page_index(GROW_POOL, sid_f, 1) == pages.page_index(GROW_POOL, sid_l, 1)
    assert pages.page_holds(GROW_POOL, pages.page_index(GROW_POOL, sid_f, 0)) == 2
    assert pages.page_index(GROW_POOL, sid_f, 2) != pages.page_index(GROW_POOL, sid_l, 2)
    assert model.grow_copy_positions == 1, "divergence copy moves one position"
    assert model.ring_copy_positions == 4, "ring copy moves exactly the live window"

    # adoption with truncation privatizes a shared page
    rm = sched.submit([100 + t for t in range(7)] + [333], 1)
    fed_before = model.fed_tokens
    grow_before, ring_before = model.grow_copy_positions, model.ring_copy_positions
    assert run_until_idle(sched, model, clock) == 1
    assert sched.request(rm).seq_id == sid_f, "intact warm sequence wins over the stale fork"
    assert model.fed_tokens - fed_before == 1
    assert model.grow_copy_positions - grow_before == 3, "privatization copies the kept rows"
    assert model.ring_copy_positions == ring_before, "adoption never copies the ring"
    assert pages.page_index(GROW_POOL, sid_f, 1) != pages.page_index(GROW_POOL, sid_l, 1)
    assert pages.page_holds(GROW_POOL, pages.page_index(GROW_POOL, sid_f, 1)) == 1
    assert pages.page_holds(GROW_POOL, pages.page_index(GROW_POOL, sid_l, 1)) == 1

    # cancellation demotes the sequence to a warm prefix
    rx = sched.submit([600 + t for t in range(9)], 1)
    sched.step(model, clock)
    assert not sched.request(rx).done
    sid_x = sched.request(rx).seq_id
    sched.cancel(rx)
    run_until_idle(sched, model, clock)
    assert sched.request(rx).done
    assert reg.is_resident(sid_x) and reg.owner_of(sid_x) == -1
    assert reg.length(sid_x) == 8, "partial prefill survives cancellation"
    fed_before_retry = model.fed_tokens
    ry = sched.submit([600 + t for t in range(9)] + [777], 1)
    run_until_idle(sched, model, clock)
    assert sched.request(ry).seq_id == sid_x, "retry re-adopts the cancelled prefix"
    assert model.fed_tokens - fed_before_retry == 2, "retry pays only the unprefilled tail"

    # retirement recycles request slots
    table_len = sched.num_requests
    assert sched.retire(rx)
    assert sched.retire(ry)
    assert not sched.retire(rx), "double retirement is refused"
    rz = sched.submit([800 + t for t in range(4)], 1)
    assert rz < table_len, "new request reuses a retired slot"
    assert sched.num_requests == table_len
    run_until_idle(sched, model, clock)
    assert sched.request(rz).done

    # mid-step cancellation aborts and discards the step
    rw = sched.submit([900 + t for t in range(9)], 1)
    sched.step(model, clock)
    sid_w = sched.request(rw).seq_id
    assert reg.length(sid_w) == 8, "first step prefills the budget"
    model.victim = rw
    model.cancel_at_step = model.steps + 1
    fed_before_abort = model.fed_tokens
    assert sched.step(model, clock) == 1, "aborted step still reports its slot"
    assert model.aborted_steps == 1
    assert model.fed_tokens == fed_before_abort
    assert reg.length(sid_w) == 8, "discarded step leaves the history unextended"
    assert len(sched.request(rw).generated) == 0
    assert sched.ring_floor(sid_w) == 1, "discard raises the ring floor over the partial writes"
    run_until_idle(sched, model, clock)
    assert sched.request(rw).done
    assert reg.is_resident(sid_w) and reg.owner_of(sid_w) == -1

    assert sched.invariant_failures == (0, 0)

    # hold balance after eviction
    while sched.evict_warm():
        pass
    assert pages.pool_available(RING_POOL) == RING_PAGES
    assert pages.pool_available(GROW_POOL) == GROW_PAGES


def test_scheduler_pressure_rig(impl):
    """test_scheduler_reuse.mojo:292-398: decode-first scheduling, productive
    eviction, demote-on-preempt, chained warm survival, clean drain."""
    clock = Clock()
    m2 = StubModel()
    geom = impl.BatchGeometry(4, 2, 8, [impl.PagePoolSpec(8, 2, 2), impl.PagePoolSpec(6, 0, 8)])
    sched2 = impl.Scheduler(PPP, geom, 8, [-1])
    reg2, pages2 = sched2.registry, sched2.pages

    rpa = sched2.submit([100 + t for t in range(20)], 1)
    sched2.step(m2, clock)
    assert not sched2.request(rpa).done
    rpd = sched2.submit([200, 201], 2)
    sched2.step(m2, clock)
    assert len(sched2.request(rpd).generated) >= 1, "late short request emits"
    assert not sched2.request(rpa).done
    run_until_idle(sched2, m2, clock)
    assert sched2.request(rpa).done and sched2.request(rpd).done
    sid_pa = sched2.request(rpa).seq_id
    sid_pd = sched2.request(rpd).seq_id

    rad = sched2.submit([300 + t for t in range(12)], 5)
    sched2.step(m2, clock)
    sid_ad = sched2.request(rad).seq_id
    assert not reg2.is_resident(sid_pa), "eviction reclaims the oldest cache that frees pages"
    assert reg2.is_resident(sid_pd), "eviction stops once the shortage is covered"
    sched2.step(m2, clock)
    rfb = sched2.submit([300 + t for t in range(8)] + [400, 401], 1)
    sched2.step(m2, clock)
    sid_fb = sched2.request(rfb).seq_id
    assert sched2.request(rfb).done and sid_fb != sid_ad, "fork against the active donor"

    rdd = sched2.submit([500 + t for t in range(16)], 1)
    rcc = sched2.submit([300 + t for t in range(8)] + [600 + t for t in range(6)], 1)
    sched2.step(m2, clock)
    sid_dd = sched2.request(rdd).seq_id
    assert sched2.request(rcc).seq_id == sid_fb, "unslotted edit adopts the warm fork"
    assert pages2.page_index(GROW_POOL, sid_fb, 2) < 0, "truncation released the tail page"
    sched2.cancel(rcc)
    sched2.step(m2, clock)
    assert reg2.is_resident(sid_fb), "shared-only warm cache survives the page shortage"
    assert (sched2.request(rdd).seq_id == -1 and reg2.is_resident(sid_dd)
            and reg2.owner_of(sid_dd) == -1), "preempted prefill demotes to warm"
    assert reg2.length(sid_dd) == 7, "preempted prefill keeps its absorbed history"
    run_until_idle(sched2, m2, clock)
    assert sched2.request(rdd).done and sched2.request(rad).done
    assert sched2.request(rdd).seq_id == sid_dd, "re-attachment reuses the preserved sequence"
    while sched2.evict_warm():
        pass
    assert pages2.pool_available(RING_POOL) == 8 and pages2.pool_available(GROW_POOL) == 6


def test_scheduler_submit_validation_and_ceiling(impl):
    """test_scheduler_reuse.mojo:400-427."""
    clock = Clock()
    m3 = StubModel()
    sched3 = impl.Scheduler(PPP, stub_geometry(impl), 8, [-1])
    assert sched3.submit([], 1) is None
    assert sched3.submit(list(range(65)), 1) is None, "beyond the page ceiling"
    rcl = sched3.submit([1000 + t for t in range(64)], 8)
    assert rcl is not None
    run_until_idle(sched3, m3, clock)
    assert sched3.request(rcl).done
    assert len(sched3.request(rcl).generated) == 1, "generation stops at the ceiling"


def test_scheduler_stop_token_list(impl):
    """test_scheduler_reuse.mojo:429-444."""
    clock = Clock()
    m4 = StubModel()
    sched4 = impl.Scheduler(PPP, stub_geometry(impl), 8, [42, 9000])
    rs = sched4.submit([50 + t for t in range(4)], 5)
    run_until_idle(sched4, m4, clock)
    assert sched4.request(rs).done and len(sched4.request(rs).generated) == 1


def test_scheduler_same_step_chaining_defers(impl):
    """test_scheduler_reuse.mojo:446-485."""
    clock = Clock()
    m5 = StubModel()
    sched5 = impl.Scheduler(PPP, stub_geometry(impl), 8, [-1])
    rw0 = sched5.submit([700 + t for t in range(8)], 1)
    run_until_idle(sched5, m5, clock)
    sid_w0 = sched5.request(rw0).seq_id
    rca = sched5.submit([700 + t for t in range(8)], 3)
    rcb = sched5.submit([700 + t for t in range(8)] + [666, 667], 1)
    fed_chain = m5.fed_tokens
    sched5.step(m5, clock)
    assert sched5.request(rca).seq_id == sid_w0, "page-aligned replay adopts the warm donor"
    assert sched5.request(rcb).seq_id == -1, "chained match defers"
    run_until_idle(sched5, m5, clock)
    sid_cb = sched5.request(rcb).seq_id
    assert sched5.request(rcb).done and sid_cb != sid_w0
    pg = sched5.pages
    assert pg.page_index(GROW_POOL, sid_w0, 0) == pg.page_index(GROW_POOL, sid_cb, 0)
    assert m5.fed_tokens - fed_chain == 5, "deferral pays only the divergent tails"
