"""Pure-Python restatement of the reference's host-side page state: page
allocator, page table, multi-pool accountant, prefix hash, slot registry,
continuous-batching scheduler and the kv_policy run-table / copy-job helpers.

TEST INFRASTRUCTURE ONLY.  Imported by tests/ (as the checker the C++ host
library is compared against, step by step) and never by the product package.

Each class or function names the reference lines it follows.  Pins:
  * paging, registry, scheduler: the reference's own known-answer tests
    (tests/test_slot_registry.mojo:48-242, tests/test_scheduler_reuse.mojo:
    95-491) run against this restatement in tests/test_host_reference_kats.py,
    plus conservation invariants (holds == table references + pins, free
    stack == unheld pages) checked after every step of randomized workloads.
  * prefix hash: the SplitMix64 finalizer's published vectors, MurmurHash3's
    block constants, a closed-form recomputation of a 16-token block and the
    hashed == exact prefix invariant at every divergence point.
  * kv_policy: closed-form byte offsets on hand-made mirrors.
"""
from __future__ import annotations

from dataclasses import dataclass, field
from typing import List, Optional

M32 = 0xFFFFFFFF
M64 = 0xFFFFFFFFFFFFFFFF

# simd_width_of[DType.int32]() on the AVX-512 hosts the reference targets
# (continuous_batching/prefix_hash.mojo:6).
TOKEN_LANES = 16
BLOCK_C1 = 0xCC9E2D51
BLOCK_C2 = 0x1B873593
BLOCK_C3 = 0xE6546B64
CHAIN_SEED = 0x9AE16A3B2F90404F


# ---------------------------------------------------------------------------
# paging.mojo
# ---------------------------------------------------------------------------
@dataclass(frozen=True)
class PagePoolSpec:
    """continuous_batching/paging.mojo:1-5."""
    num_pages: int
    fixed_pages_per_seq: int
    max_pages_per_seq: int


@dataclass
class BatchGeometry:
    """continuous_batching/paging.mojo:8-13."""
    max_seqs: int
    max_slots: int
    max_step_tokens: int
    pools: List[PagePoolSpec]


class KVPageAllocator:
    """LIFO free stack + hold counts (paging.mojo:16-58).  The stack starts
    as [n-1, ..., 0], so acquire() hands out 0, 1, 2, ... first."""

    def __init__(self, num_pages: int):
        self.free_stack = [num_pages - 1 - i for i in range(num_pages)]
        self.holds = [0] * num_pages

    def acquire(self) -> int:
        if not self.free_stack:
            return -1
        page = self.free_stack.pop()
        self.holds[page] = 1
        return page

    def retain(self, page: int) -> None:
        assert self.holds[page] > 0, "page allocator: retain of an unheld page"
        self.holds[page] += 1

    def release(self, page: int) -> None:
        assert self.holds[page] > 0, "page allocator: release of an unheld page"
        self.holds[page] -= 1
        if self.holds[page] == 0:
            self.free_stack.append(page)

    def hold_count(self, page: int) -> int:
        return self.holds[page]

    def available(self) -> int:
        return len(self.free_stack)


class KVPageTable:
    """entries[seq * max_pages + ordinal] = page or -1 (paging.mojo:61-86)."""

    def __init__(self, max_seqs: int, max_pages_per_seq: int):
        self.max_seqs = max_seqs
        self.max_pages_per_seq = max_pages_per_seq
        self.entries = [-1] * (max_seqs * max_pages_per_seq)

    def entry_index(self, seq_id: int, ordinal: int) -> int:
        assert ordinal < self.max_pages_per_seq, "page table: ordinal beyond per-sequence bound"
        return seq_id * self.max_pages_per_seq + ordinal

    def map_page(self, seq_id: int, ordinal: int, page: int) -> None:
        self.entries[self.entry_index(seq_id, ordinal)] = page

    def page_index(self, seq_id: int, ordinal: int) -> int:
        return self.entries[self.entry_index(seq_id, ordinal)]


class PagePool:
    def __init__(self, spec: PagePoolSpec, max_seqs: int):
        self.spec = spec
        self.pages = KVPageAllocator(spec.num_pages)
        self.table = KVPageTable(max_seqs, spec.max_pages_per_seq)


class KVPageAccountant:
    """Multi-pool page accounting (paging.mojo:96-242)."""

    def __init__(self, geometry: BatchGeometry):
        self.max_seqs = geometry.max_seqs
        self.pools = [PagePool(s, geometry.max_seqs) for s in geometry.pools]
        self.active = [False] * geometry.max_seqs

    def pool_count(self) -> int:
        return len(self.pools)

    def pool_available(self, p: int) -> int:
        return self.pools[p].pages.available()

    def pool_fixed_pages(self, p: int) -> int:
        return self.pools[p].spec.fixed_pages_per_seq

    def page_index(self, p: int, seq_id: int, ordinal: int) -> int:
        return self.pools[p].table.page_index(seq_id, ordinal)

    def page_holds(self, p: int, page: int) -> int:
        return self.pools[p].pages.hold_count(page)

    def pool_pages(self, p: int) -> int:
        return self.pools[p].spec.num_pages

    def pool_seq_page_limit(self, p: int) -> int:
        return self.pools[p].spec.max_pages_per_seq

    def freeable_pages(self, p: int, seq_id: int) -> int:
        pool = self.pools[p]
        n = 0
        for o in range(pool.spec.max_pages_per_seq):
            page = pool.table.page_index(seq_id, o)
            if page >= 0 and pool.pages.hold_count(page) == 1:
                n += 1
        return n

    def export(self, p: int):
        """(table [max_seqs][max_pages_per_seq], holds, free stack bottom
        first), the layout the C++ library's export returns."""
        import numpy as np
        pool = self.pools[p]
        table = np.asarray(pool.table.entries, dtype=np.int32).reshape(
            self.max_seqs, pool.spec.max_pages_per_seq)
        return (table, np.asarray(pool.pages.holds, dtype=np.int32),
                np.asarray(pool.pages.free_stack, dtype=np.int32))

    def is_active(self, seq_id: int) -> bool:
        return self.active[seq_id]

    def retain_page(self, p: int, page: int) -> None:
        self.pools[p].pages.retain(page)

    def release_page(self, p: int, page: int) -> None:
        self.pools[p].pages.release(page)

    def admit(self) -> int:
        """paging.mojo:156-170: first inactive seq; fails (-1) as soon as a
        pool cannot cover its fixed ring pages."""
        for sid in range(self.max_seqs):
            if self.active[sid]:
                continue
            for pool in self.pools:
                if pool.spec.fixed_pages_per_seq > pool.pages.available():
                    return -1
            for pool in self.pools:
                for o in range(pool.spec.fixed_pages_per_seq):
                    pool.table.map_page(sid, o, pool.pages.acquire())
            self.active[sid] = True
            return sid
        return -1

    def release(self, seq_id: int) -> None:
        if not self.active[seq_id]:
            return
        for pool in self.pools:
            for o in range(pool.spec.max_pages_per_seq):
                page = pool.table.page_index(seq_id, o)
                if page >= 0:
                    pool.pages.release(page)
                    pool.table.map_page(seq_id, o, -1)
        self.active[seq_id] = False

    def share(self, p: int, src_seq: int, dst_seq: int, ordinal: int) -> None:
        pool = self.pools[p]
        page = pool.table.page_index(src_seq, ordinal)
        assert page >= 0, "share: source ordinal is unmapped"
        assert pool.table.page_index(dst_seq, ordinal) < 0, "share: destination ordinal already mapped"
        pool.pages.retain(page)
        pool.table.map_page(dst_seq, ordinal, page)

    def truncate(self, seq_id: int, last_keep: int) -> None:
        for pool in self.pools:
            if pool.spec.fixed_pages_per_seq > 0:
                continue
            for o in range(last_keep + 1, pool.spec.max_pages_per_seq):
                page = pool.table.page_index(seq_id, o)
                if page >= 0:
                    pool.pages.release(page)
                    pool.table.map_page(seq_id, o, -1)

    def replace_with_private(self, p: int, seq_id: int, ordinal: int) -> int:
        pool = self.pools[p]
        fresh = pool.pages.acquire()
        if fresh < 0:
            return -1
        old = pool.table.page_index(seq_id, ordinal)
        assert old >= 0, "replace_with_private: ordinal is unmapped"
        pool.pages.release(old)
        pool.table.map_page(seq_id, ordinal, fresh)
        return fresh

    def pages_needed(self, seq_id: int, last_ordinal: int, need: List[int]) -> None:
        for p, pool in enumerate(self.pools):
            if pool.spec.fixed_pages_per_seq > 0:
                continue
            for o in range(last_ordinal + 1):
                if pool.table.page_index(seq_id, o) < 0:
                    need[p] += 1

    def fits(self, need: List[int]) -> bool:
        return all(need[p] <= pool.pages.available() for p, pool in enumerate(self.pools))

    def reserve(self, seq_id: int, last_ordinal: int) -> bool:
        for pool in self.pools:
            if pool.spec.fixed_pages_per_seq > 0:
                continue
            for o in range(last_ordinal + 1):
                if pool.table.page_index(seq_id, o) >= 0:
                    continue
                page = pool.pages.acquire()
                if page < 0:
                    return False
                pool.table.map_page(seq_id, o, page)
        return True


# ---------------------------------------------------------------------------
# prefix_hash.mojo
# ---------------------------------------------------------------------------
def splitmix64(x: int) -> int:
    """SplitMix64 finalizer (simd_math/sampling_rng.mojo:11-19)."""
    z = (x + 0x9E3779B97F4A7C15) & M64
    z = ((z ^ (z >> 30)) * 0xBF58476D1CE4E5B9) & M64
    z = ((z ^ (z >> 27)) * 0x94D049BB133111EB) & M64
    return z ^ (z >> 31)


def _rotl32(x: int, b: int) -> int:
    return ((x << b) | (x >> (32 - b))) & M32


def hash_token_block(tokens, start: int, count: int) -> int:
    """prefix_hash.mojo:22-39: 16 uint32 lanes of MurmurHash3-style block
    mixing over whole 16-token groups, then a SplitMix64 fold of
    (count, each lane tagged with its index, each tail token)."""
    lanes = [0] * TOKEN_LANES
    i = 0
    while i + TOKEN_LANES <= count:
        for j in range(TOKEN_LANES):
            m = ((int(tokens[start + i + j]) & M32) * BLOCK_C1) & M32
            m = (_rotl32(m, 15) * BLOCK_C2) & M32
            x = lanes[j] ^ m
            lanes[j] = ((_rotl32(x, 13) * 5) + BLOCK_C3) & M32
        i += TOKEN_LANES
    acc = splitmix64(count & M64)
    for lane in range(TOKEN_LANES):
        acc = splitmix64(acc ^ ((lane << 32) | lanes[lane]))
    while i < count:
        acc = splitmix64(acc ^ (int(tokens[start + i]) & M32))
        i += 1
    return acc


def chain_link(prev: int, block_hash: int) -> int:
    """prefix_hash.mojo:42-44."""
    return splitmix64(prev ^ splitmix64(block_hash))


def refresh_chain(ppp: int, chain: List[int], tokens) -> None:
    """prefix_hash.mojo:47-57: one link per sealed page, extended or popped
    to len(tokens) // ppp."""
    sealed = len(tokens) // ppp
    while len(chain) > sealed:
        chain.pop()
    while len(chain) < sealed:
        o = len(chain)
        prev = chain[o - 1] if o > 0 else CHAIN_SEED
        chain.append(chain_link(prev, hash_token_block(tokens, o * ppp, ppp)))


def first_mismatch(a, b, start: int, limit: int) -> int:
    """prefix_hash.mojo:60-78 (the SIMD scan returns the first differing
    index, as this scalar loop does)."""
    i = start
    while i < limit:
        if a[i] != b[i]:
            return i
        i += 1
    return limit


def token_prefix_len(a, b) -> int:
    return first_mismatch(a, b, 0, min(len(a), len(b)))


def hashed_prefix_len(ppp: int, a_tokens, a_chain, b_tokens, b_chain) -> int:
    """prefix_hash.mojo:86-97: equal chain links, then an exact scan of at
    most one page after the last matching link."""
    pages = min(len(a_chain), len(b_chain))
    matched = 0
    while matched < pages and a_chain[matched] == b_chain[matched]:
        matched += 1
    n = min(len(a_tokens), len(b_tokens))
    base = matched * ppp
    return first_mismatch(a_tokens, b_tokens, base, min(n, base + ppp))


# ---------------------------------------------------------------------------
# slot_registry.mojo
# ---------------------------------------------------------------------------
class SlotRegistry:
    """continuous_batching/slot_registry.mojo:6-107."""

    def __init__(self, ppp: int, max_seqs: int):
        self.ppp = ppp
        self.max_seqs = max_seqs
        self.resident = [False] * max_seqs
        self.owner = [-1] * max_seqs
        self.last_used_at = [0] * max_seqs
        self.tokens: List[List[int]] = [[] for _ in range(max_seqs)]
        self.chains: List[List[int]] = [[] for _ in range(max_seqs)]

    def length(self, sid: int) -> int:
        return len(self.tokens[sid])

    def owner_of(self, sid: int) -> int:
        return self.owner[sid]

    def open(self, sid: int, owner_id: int, now: int) -> None:
        self.resident[sid] = True
        self.owner[sid] = owner_id
        self.last_used_at[sid] = now
        self.tokens[sid] = []
        self.chains[sid] = []

    def adopt(self, sid: int, owner_id: int, now: int) -> None:
        self.owner[sid] = owner_id
        self.last_used_at[sid] = now

    def extend(self, sid: int, source, start: int, base_pos: int, count: int, now: int) -> None:
        assert base_pos <= len(self.tokens[sid]), "slot registry: extend would leave a position gap"
        for t in range(count):
            if base_pos + t < len(self.tokens[sid]):
                continue
            self.tokens[sid].append(int(source[start + t]))
        refresh_chain(self.ppp, self.chains[sid], self.tokens[sid])
        self.last_used_at[sid] = now

    def seed(self, sid: int, source, count: int, now: int) -> None:
        same = token_prefix_len(self.tokens[sid], source)
        keep = min(same, count) // self.ppp
        del self.chains[sid][keep:]
        self.tokens[sid] = [int(source[i]) for i in range(count)]
        refresh_chain(self.ppp, self.chains[sid], self.tokens[sid])
        self.last_used_at[sid] = now

    def set_warm(self, sid: int) -> None:
        self.owner[sid] = -1

    def close(self, sid: int) -> None:
        self.resident[sid] = False
        self.owner[sid] = -1
        self.tokens[sid] = []
        self.chains[sid] = []

    def is_resident(self, sid: int) -> bool:
        return self.resident[sid]

    def prefix_len(self, sid: int, incoming, incoming_chain) -> int:
        return hashed_prefix_len(self.ppp, self.tokens[sid], self.chains[sid], incoming,
                                 incoming_chain)

    def exact_prefix_len(self, sid: int, incoming) -> int:
        return token_prefix_len(self.tokens[sid], incoming)

    def last_used(self, sid: int) -> int:
        return self.last_used_at[sid]

    def tokens_of(self, sid: int) -> List[int]:
        return list(self.tokens[sid])

    def chain_of(self, sid: int) -> List[int]:
        return list(self.chains[sid])

    def lru_victim(self) -> int:
        victim, oldest = -1, 0
        for sid in range(self.max_seqs):
            if not self.resident[sid] or self.owner[sid] >= 0:
                continue
            if victim < 0 or self.last_used_at[sid] < oldest:
                victim, oldest = sid, self.last_used_at[sid]
        return victim


# ---------------------------------------------------------------------------
# schedule.mojo / scheduler.mojo
# ---------------------------------------------------------------------------
@dataclass
class BatchSlot:
    """continuous_batching/schedule.mojo:29-51 (sampling parameters and the
    cancel token are looked up through request_id)."""
    seq_id: int
    request_id: int
    base_pos: int
    n_tokens: int
    prompt_len: int
    emit: bool

    def prefill_count(self) -> int:
        pre = self.prompt_len - self.base_pos
        if pre < 0:
            return 0
        return min(pre, self.n_tokens)

    def decode_count(self) -> int:
        return self.n_tokens - self.prefill_count()


@dataclass
class PageCopy:
    """schedule.mojo:54-60."""
    pool: int
    src_page: int
    dst_page: int
    pos_start: int
    pos_count: int


@dataclass
class Schedule:
    """schedule.mojo:63-90."""
    slots: List[BatchSlot] = field(default_factory=list)
    tokens: List[int] = field(default_factory=list)
    copies: List[PageCopy] = field(default_factory=list)
    prefill_tokens: int = 0
    decode_tokens: int = 0

    def clear(self) -> None:
        self.slots, self.tokens, self.copies = [], [], []
        self.prefill_tokens = self.decode_tokens = 0


@dataclass
class PrefixReuse:
    """scheduler.mojo:15-21."""
    seq_id: int
    adopted: bool
    trim_len: int
    copy_start: int
    copy_count: int


class Request:
    """scheduler.mojo:30-58 (the cancel token is a flag on the request)."""

    def __init__(self, tokens, max_new_tokens: int, no_share: bool = False):
        self.tokens = [int(t) for t in tokens]
        self.chain: List[int] = []
        self.generated: List[int] = []
        self.max_new_tokens = max_new_tokens
        self.seq_id = -1
        self.done = False
        self.live = True
        self.no_share = no_share
        self.cancelled = False

    def rehash(self, ppp: int) -> None:
        refresh_chain(ppp, self.chain, self.tokens)


BIG = 1 << 62


class ContinuousBatchScheduler:
    """continuous_batching/scheduler.mojo:61-780."""

    def __init__(self, ppp: int, geometry: BatchGeometry, step_budget: int, stop_tokens,
                 decode_band: int = 4):
        self.ppp = ppp
        self.pages = KVPageAccountant(geometry)
        self.registry = SlotRegistry(ppp, geometry.max_seqs)
        self.requests: List[Request] = []
        self.schedule = Schedule()
        self.need = [0] * len(geometry.pools)
        self.max_slots = geometry.max_slots
        self.step_budget = min(step_budget, geometry.max_step_tokens)
        self.decode_band = decode_band
        self.stop_tokens = [int(t) for t in (stop_tokens if hasattr(stop_tokens, "__len__")
                                              else [stop_tokens])]
        self.pending_ids: List[int] = []
        self.free_slots: List[int] = []
        ring_capacity, seq_ceiling = BIG, BIG
        for spec in geometry.pools:
            if spec.fixed_pages_per_seq > 0:
                ring_capacity = min(ring_capacity, spec.fixed_pages_per_seq * ppp)
            else:
                seq_ceiling = min(seq_ceiling,
                                  min(spec.max_pages_per_seq, spec.num_pages) * ppp)
        self.ring_capacity = ring_capacity
        self.seq_ceiling = seq_ceiling
        self.ring_floors = [0] * geometry.max_seqs
        self.reuse: List[PrefixReuse] = []
        self.reuse_copies: List[PageCopy] = []
        self.pins: List[tuple] = []
        self.reuse_dirty = [False] * geometry.max_seqs
        self.unsharable = [False] * geometry.max_seqs
        self.shared_writes = 0
        self.unsharable_shared = 0

    @property
    def invariant_failures(self) -> tuple:
        return self.shared_writes, self.unsharable_shared

    # -- views used by the tests (same names as the C++ library's mirror) -----
    def request(self, rid: int) -> Request:
        return self.requests[rid]

    def ring_floor(self, sid: int) -> int:
        return self.ring_floors[sid]

    def pending(self) -> List[int]:
        return list(self.pending_ids)

    @property
    def num_requests(self) -> int:
        return len(self.requests)

    # -- requests -----------------------------------------------------------
    def is_stop_token(self, token: int) -> bool:
        return token in self.stop_tokens

    def submit(self, tokens, max_new_tokens: int, no_share: bool = False) -> Optional[int]:
        """scheduler.mojo:137-154."""
        if len(tokens) == 0 or len(tokens) > self.seq_ceiling:
            return None
        req = Request(tokens, max_new_tokens, no_share)
        if self.free_slots:
            rid = self.free_slots.pop()
            self.requests[rid] = req
        else:
            rid = len(self.requests)
            self.requests.append(req)
        self.requests[rid].rehash(self.ppp)
        self.pending_ids.append(rid)
        return rid

    def cancel(self, rid: int) -> None:
        self.requests[rid].cancelled = True

    def retire(self, rid: int) -> bool:
        """scheduler.mojo:159-174."""
        r = self.requests[rid]
        if not r.live or not r.done:
            return False
        r.live = False
        r.tokens, r.chain, r.generated = [], [], []
        self.pending_ids = [k for k in self.pending_ids if k != rid]
        self.free_slots.append(rid)
        return True

    def pending_work(self) -> bool:
        return any(not self.requests[k].done for k in self.pending_ids)

    # -- eviction -----------------------------------------------------------
    def evict_warm(self) -> bool:
        """scheduler.mojo:182-189."""
        victim = self.registry.lru_victim()
        if victim < 0:
            return False
        self.pages.release(victim)
        self.registry.close(victim)
        self.unsharable[victim] = False
        return True

    def is_warm(self, sid: int) -> bool:
        return self.registry.is_resident(sid) and self.registry.owner_of(sid) < 0

    def evict_warm_for(self) -> bool:
        """scheduler.mojo:196-220: oldest warm sequence that frees a page of
        a short pool, else the oldest warm member of a warm-only share chain."""
        victim, oldest = -1, 0
        for sid in range(self.registry.max_seqs):
            if not self.is_warm(sid):
                continue
            frees = False
            for p in range(self.pages.pool_count()):
                if self.need[p] <= self.pages.pool_available(p):
                    continue
                if self.pages.freeable_pages(p, sid) > 0:
                    frees = True
            if not frees:
                continue
            if victim < 0 or self.registry.last_used_at[sid] < oldest:
                victim, oldest = sid, self.registry.last_used_at[sid]
        if victim < 0:
            victim = self.chained_warm_victim()
        if victim < 0:
            return False
        self.pages.release(victim)
        self.registry.close(victim)
        self.unsharable[victim] = False
        return True

    def chained_warm_victim(self) -> int:
        """scheduler.mojo:222-254."""
        victim, oldest = -1, 0
        for p in range(self.pages.pool_count()):
            if self.need[p] <= self.pages.pool_available(p):
                continue
            warm_holds = [0] * self.pages.pool_pages(p)
            for sid in range(self.registry.max_seqs):
                if not self.is_warm(sid):
                    continue
                for o in range(self.pages.pool_seq_page_limit(p)):
                    page = self.pages.page_index(p, sid, o)
                    if page >= 0:
                        warm_holds[page] += 1
            for sid in range(self.registry.max_seqs):
                if not self.is_warm(sid):
                    continue
                chained = False
                for o in range(self.pages.pool_seq_page_limit(p)):
                    page = self.pages.page_index(p, sid, o)
                    if page < 0:
                        continue
                    if (self.pages.page_holds(p, page) > 1
                            and warm_holds[page] == self.pages.page_holds(p, page)):
                        chained = True
                if not chained:
                    continue
                if victim < 0 or self.registry.last_used_at[sid] < oldest:
                    victim, oldest = sid, self.registry.last_used_at[sid]
        return victim

    # -- prefix reuse -------------------------------------------------------
    def window_intact(self, sid: int, lcp: int) -> bool:
        """scheduler.mojo:256-267."""
        seq_len = self.registry.length(sid)
        if lcp >= seq_len:
            return True
        live_start = max(lcp - self.ppp, 0)
        floor = max(self.ring_floors[sid], seq_len - self.ring_capacity)
        return live_start >= floor

    def release_copy_pins(self) -> None:
        for p, page in self.pins:
            self.pages.release_page(p, page)
        self.pins = []

    def best_reusable(self, rid: int, want_owned: bool):
        """scheduler.mojo:274-304."""
        req = self.requests[rid]
        best, best_lcp = -1, 0
        for sid in range(self.registry.max_seqs):
            if not self.registry.is_resident(sid) or self.unsharable[sid] or self.reuse_dirty[sid]:
                continue
            if (self.registry.owner_of(sid) >= 0) != want_owned:
                continue
            lcp = self.registry.prefix_len(sid, req.tokens, req.chain)
            if lcp <= best_lcp:
                continue
            if not self.window_intact(sid, lcp):
                continue
            best, best_lcp = sid, lcp
        if best >= 0:
            exact = self.registry.exact_prefix_len(best, req.tokens)
            if exact < best_lcp:
                best_lcp = exact
                if best_lcp == 0 or not self.window_intact(best, best_lcp):
                    return -1, 0
        return best, best_lcp

    def dirty_donor_exists(self, rid: int) -> bool:
        """scheduler.mojo:306-319."""
        req = self.requests[rid]
        for sid in range(self.registry.max_seqs):
            if not self.reuse_dirty[sid] or not self.registry.is_resident(sid):
                continue
            lcp = self.registry.prefix_len(sid, req.tokens, req.chain)
            if lcp < self.ppp:
                continue
            if self.window_intact(sid, lcp):
                return True
        return False

    def adopt_prefix(self, sid: int, rid: int, lcp: int, now: int) -> bool:
        """scheduler.mojo:321-393: hand a warm sequence to the request,
        truncating past the match and privatizing a shared partial page."""
        ppp = self.ppp
        req = self.requests[rid]
        req_len = len(req.tokens)
        seq_len = self.registry.length(sid)
        take = lcp
        resume = take - 1 if take == req_len else take
        keep_last = (take - 1) // ppp
        private_ordinal = resume // ppp
        do_private = False
        if private_ordinal <= keep_last:
            for p in range(self.pages.pool_count()):
                if self.pages.pool_fixed_pages(p) > 0:
                    continue
                page = self.pages.page_index(p, sid, private_ordinal)
                if self.pages.page_holds(p, page) > 1:
                    do_private = True
        if do_private:
            for p in range(len(self.need)):
                self.need[p] = 0
            for p in range(self.pages.pool_count()):
                if self.pages.pool_fixed_pages(p) > 0:
                    continue
                page = self.pages.page_index(p, sid, private_ordinal)
                if self.pages.page_holds(p, page) > 1:
                    self.need[p] += 1
            while not self.pages.fits(self.need):
                if self.evict_warm_for():
                    continue
                take = private_ordinal * ppp
                do_private = False
                break
            if not do_private:
                if take < 1:
                    return False
                keep_last = (take - 1) // ppp
        self.registry.adopt(sid, rid, now)
        copy_start = len(self.reuse_copies)
        trim = take
        if do_private:
            valid_rows = take - private_ordinal * ppp
            for p in range(self.pages.pool_count()):
                if self.pages.pool_fixed_pages(p) > 0:
                    continue
                old_page = self.pages.page_index(p, sid, private_ordinal)
                if self.pages.page_holds(p, old_page) <= 1:
                    continue
                fresh = self.pages.replace_with_private(p, sid, private_ordinal)
                assert fresh >= 0, "adopt: privatization page must fit"
                self.pages.retain_page(p, old_page)
                self.pins.append((p, old_page))
                self.reuse_copies.append(PageCopy(p, old_page, fresh, 0, valid_rows))
            trim = private_ordinal * ppp
        if take < seq_len:
            stale_floor = seq_len - self.ring_capacity
            if stale_floor > self.ring_floors[sid]:
                self.ring_floors[sid] = stale_floor
            self.pages.truncate(sid, keep_last)
            self.registry.seed(sid, req.tokens, take, now)
        self.reuse.append(PrefixReuse(sid, True, trim, copy_start,
                                       len(self.reuse_copies) - copy_start))
        if len(self.reuse_copies) > copy_start or (take == req_len and take % ppp == 0):
            self.reuse_dirty[sid] = True
        self.unsharable[sid] = req.no_share
        req.seq_id = sid
        return True

    def fork_prefix(self, donor: int, rid: int, lcp: int, now: int) -> bool:
        """scheduler.mojo:395-466: new sequence sharing the donor's sealed
        pages, with copies of the partial page and the live ring window."""
        ppp = self.ppp
        req = self.requests[rid]
        req_len = len(req.tokens)
        resume = lcp - 1 if lcp == req_len else lcp
        sid = self.pages.admit()
        if sid < 0:
            if not self.evict_warm():
                return False
            sid = self.pages.admit()
            if sid < 0:
                return False
        sealed = resume // ppp
        last_ordinal = (lcp - 1) // ppp
        for p in range(self.pages.pool_count()):
            if self.pages.pool_fixed_pages(p) > 0:
                continue
            for o in range(sealed):
                self.pages.share(p, donor, sid, o)
        while True:
            for p in range(len(self.need)):
                self.need[p] = 0
            self.pages.pages_needed(sid, last_ordinal, self.need)
            if self.pages.fits(self.need):
                break
            if not self.evict_warm_for():
                self.pages.release(sid)
                return False
        if not self.pages.reserve(sid, last_ordinal):
            self.pages.release(sid)
            return False
        copy_start = len(self.reuse_copies)
        partial_rows = lcp - sealed * ppp
        if partial_rows > 0:
            for p in range(self.pages.pool_count()):
                if self.pages.pool_fixed_pages(p) > 0:
                    continue
                self.reuse_copies.append(PageCopy(
                    p, self.pages.page_index(p, donor, sealed),
                    self.pages.page_index(p, sid, sealed), 0, partial_rows))
        live_start = max(lcp - ppp, 0)
        for p in range(self.pages.pool_count()):
            ring_pages = self.pages.pool_fixed_pages(p)
            if ring_pages == 0:
                continue
            a = live_start
            while a < lcp:
                page_end = (a // ppp + 1) * ppp
                seg_end = min(lcp, page_end)
                ring_slot = (a // ppp) % ring_pages
                self.reuse_copies.append(PageCopy(
                    p, self.pages.page_index(p, donor, ring_slot),
                    self.pages.page_index(p, sid, ring_slot), a % ppp, seg_end - a))
                a = seg_end
        self.registry.open(sid, rid, now)
        self.registry.seed(sid, req.tokens, lcp, now)
        self.ring_floors[sid] = live_start
        self.unsharable[sid] = req.no_share
        req.seq_id = sid
        self.reuse.append(PrefixReuse(sid, False, 0, copy_start,
                                       len(self.reuse_copies) - copy_start))
        self.reuse_dirty[sid] = True
        return True

    def request_common_prefix(self, a: int, b: int) -> int:
        ra, rb = self.requests[a], self.requests[b]
        return hashed_prefix_len(self.ppp, ra.tokens, ra.chain, rb.tokens, rb.chain)

    def slot_want(self, rid: int) -> int:
        req = self.requests[rid]
        base = min(self.registry.length(req.seq_id), len(req.tokens) - 1)
        return len(req.tokens) - base

    def admit_slot(self, rid: int, budget: int) -> int:
        """scheduler.mojo:481-511; returns the remaining budget."""
        ppp = self.ppp
        req = self.requests[rid]
        sid = req.seq_id
        base_pos = min(self.registry.length(sid), len(req.tokens) - 1)
        want = len(req.tokens) - base_pos
        feed = min(want, budget)
        for j in self.pending_ids:
            if j == rid or self.requests[j].seq_id >= 0:
                continue
            common = self.request_common_prefix(rid, j)
            if common < ppp:
                continue
            limit = common + ppp - base_pos
            if 1 <= limit < feed:
                feed = limit
        emit = base_pos + feed == len(req.tokens)
        self.schedule.tokens.extend(req.tokens[base_pos:base_pos + feed])
        prompt_len = len(req.tokens) - len(req.generated)
        slot = BatchSlot(sid, rid, base_pos, feed, prompt_len, emit)
        self.schedule.prefill_tokens += slot.prefill_count()
        self.schedule.decode_tokens += slot.decode_count()
        self.schedule.slots.append(slot)
        return budget - feed

    def preempt_last_slot(self, now: int) -> None:
        """scheduler.mojo:513-542."""
        dropped = self.schedule.slots.pop()
        if dropped.n_tokens:
            del self.schedule.tokens[-dropped.n_tokens:]
        self.schedule.prefill_tokens -= dropped.prefill_count()
        self.schedule.decode_tokens -= dropped.decode_count()
        sid = dropped.seq_id
        owner = self.registry.owner_of(sid)
        adopted_record, fork_record = -1, -1
        for k, r in enumerate(self.reuse):
            if r.seq_id != sid:
                continue
            if r.adopted:
                adopted_record = k
            else:
                fork_record = k
            r.seq_id = -1
        if adopted_record >= 0:
            self.registry.seed(sid, self.requests[owner].tokens,
                               self.reuse[adopted_record].trim_len, now)
            self.registry.set_warm(sid)
        elif fork_record >= 0:
            self.pages.release(sid)
            self.registry.close(sid)
            self.unsharable[sid] = False
        else:
            self.registry.set_warm(sid)
        self.requests[owner].seq_id = -1

    def unwind_prefix_reuse(self, now: int) -> None:
        """scheduler.mojo:544-565."""
        for r in self.reuse:
            sid = r.seq_id
            if sid < 0:
                continue
            owner = self.registry.owner_of(sid)
            if r.adopted:
                if owner >= 0:
                    self.requests[owner].seq_id = -1
                    self.registry.seed(sid, self.requests[owner].tokens, r.trim_len, now)
                self.registry.set_warm(sid)
            else:
                if owner >= 0:
                    self.requests[owner].seq_id = -1
                self.pages.release(sid)
                self.registry.close(sid)
                self.unsharable[sid] = False
        self.reuse = []
        self.reuse_copies = []
        self.release_copy_pins()

    def build_schedule(self, now: int) -> bool:
        """scheduler.mojo:567-729."""
        ppp = self.ppp
        kept = []
        for i in self.pending_ids:
            r = self.requests[i]
            if r.done:
                continue
            if r.cancelled:
                r.done = True
                if r.seq_id >= 0:
                    self.registry.set_warm(r.seq_id)
                    r.seq_id = -1
                continue
            kept.append(i)
        self.pending_ids = kept
        self.reuse = []
        self.reuse_copies = []
        self.reuse_dirty = [False] * len(self.reuse_dirty)

        for i in self.pending_ids:
            r = self.requests[i]
            if r.seq_id >= 0:
                continue
            if not r.no_share:
                warm_sid, warm_lcp = self.best_reusable(i, False)
                active_sid, active_lcp = self.best_reusable(i, True)
                can_adopt = warm_sid >= 0 and warm_lcp >= 1
                can_fork = active_sid >= 0 and active_lcp >= ppp
                matched = False
                if can_adopt and (not can_fork or warm_lcp + ppp > active_lcp):
                    matched = self.adopt_prefix(warm_sid, i, warm_lcp, now)
                    if not matched and can_fork:
                        matched = self.fork_prefix(active_sid, i, active_lcp, now)
                elif can_fork:
                    matched = self.fork_prefix(active_sid, i, active_lcp, now)
                    if not matched and can_adopt:
                        matched = self.adopt_prefix(warm_sid, i, warm_lcp, now)
                if matched:
                    continue
                if self.dirty_donor_exists(i):
                    continue
            sid = self.pages.admit()
            if sid < 0:
                if not self.evict_warm():
                    continue
                sid = self.pages.admit()
                if sid < 0:
                    continue
            self.registry.open(sid, i, now)
            self.unsharable[sid] = r.no_share
            self.ring_floors[sid] = 0
            r.seq_id = sid

        self.schedule.clear()
        budget = self.step_budget
        prefill_waiting = any(self.requests[i].seq_id >= 0 and self.slot_want(i) > self.decode_band
                              for i in self.pending_ids)
        decode_cap = self.max_slots - 1 if prefill_waiting else self.max_slots
        slotted = [False] * len(self.pending_ids)
        for k, i in enumerate(self.pending_ids):
            if self.requests[i].seq_id < 0:
                continue
            if len(self.schedule.slots) >= decode_cap or budget < 1:
                break
            if self.slot_want(i) > self.decode_band:
                continue
            budget = self.admit_slot(i, budget)
            slotted[k] = True
        for k, i in enumerate(self.pending_ids):
            if slotted[k] or self.requests[i].seq_id < 0:
                continue
            if len(self.schedule.slots) >= self.max_slots or budget < 1:
                break
            budget = self.admit_slot(i, budget)

        while self.schedule.slots:
            for p in range(len(self.need)):
                self.need[p] = 0
            for s in self.schedule.slots:
                self.pages.pages_needed(s.seq_id, (s.base_pos + s.n_tokens - 1) // ppp, self.need)
            if self.pages.fits(self.need):
                break
            if self.evict_warm_for():
                continue
            if len(self.schedule.slots) == 1:
                self.unwind_prefix_reuse(now)
                return False
            self.preempt_last_slot(now)

        if not self.schedule.slots:
            self.unwind_prefix_reuse(now)
            return False

        for s in self.schedule.slots:
            if not self.pages.reserve(s.seq_id, (s.base_pos + s.n_tokens - 1) // ppp):
                self.unwind_prefix_reuse(now)
                return False

        # scheduler.mojo:688-720 are debug_asserts; the reference's release
        # build runs on, so they are counted here rather than raised.
        for s in self.schedule.slots:
            first = s.base_pos // ppp
            last = (s.base_pos + s.n_tokens - 1) // ppp
            for p in range(self.pages.pool_count()):
                if self.pages.pool_fixed_pages(p) > 0:
                    continue
                for o in range(first, last + 1):
                    if self.pages.page_holds(p, self.pages.page_index(p, s.seq_id, o)) != 1:
                        self.shared_writes += 1
        for s in self.schedule.slots:
            if not self.unsharable[s.seq_id]:
                continue
            last = (s.base_pos + s.n_tokens - 1) // ppp
            for p in range(self.pages.pool_count()):
                if self.pages.pool_fixed_pages(p) > 0:
                    continue
                for o in range(last + 1):
                    if self.pages.page_holds(p, self.pages.page_index(p, s.seq_id, o)) != 1:
                        self.unsharable_shared += 1

        for r in self.reuse:
            if r.seq_id < 0:
                continue
            self.schedule.copies.extend(self.reuse_copies[r.copy_start:r.copy_start + r.copy_count])
        self.release_copy_pins()
        return True

    def absorb(self, emitted, now: int) -> None:
        """scheduler.mojo:731-759: extend histories with the fed tokens and
        append each emitting slot's sampled token."""
        buf_start, emit_idx = 0, 0
        for s in self.schedule.slots:
            rid = self.registry.owner_of(s.seq_id)
            self.registry.extend(s.seq_id, self.schedule.tokens, buf_start, s.base_pos,
                                 s.n_tokens, now)
            buf_start += s.n_tokens
            if s.emit:
                token = int(emitted[emit_idx])
                emit_idx += 1
                req = self.requests[rid]
                req.generated.append(token)
                req.tokens.append(token)
                req.rehash(self.ppp)
                if (self.is_stop_token(token) or len(req.generated) >= req.max_new_tokens
                        or len(req.tokens) > self.seq_ceiling):
                    req.done = True
                    self.registry.set_warm(s.seq_id)

    def discard_step(self) -> None:
        """scheduler.mojo:761-768."""
        for s in self.schedule.slots:
            floor = s.base_pos + s.n_tokens - self.ring_capacity
            if floor > self.ring_floors[s.seq_id]:
                self.ring_floors[s.seq_id] = floor

    def fully_cancelled(self) -> bool:
        """schedule.mojo:84-90."""
        if not self.schedule.slots:
            return False
        return all(self.requests[s.request_id].cancelled for s in self.schedule.slots)

    def step(self, model, clock) -> int:
        """scheduler.mojo:770-780; clock() stands for perf_counter_ns()."""
        if not self.build_schedule(clock()):
            return 0
        outs = model.execute(self, self.schedule, self.pages)
        if self.fully_cancelled():
            self.discard_step()
        else:
            self.absorb(outs, clock())
        return len(self.schedule.slots)


# ---------------------------------------------------------------------------
# modeling/kv_policy.mojo
# ---------------------------------------------------------------------------
@dataclass
class KVPoolMirror:
    """kv_policy.mojo:18-35: one pool's physical layout in the arena."""
    page_len: int
    pos_shard: int
    region_off: int
    stride: int
    layers: int
    components: List[tuple]  # (offset, row_bytes)
    spec: PagePoolSpec

    def rows_per_page(self) -> int:
        return self.page_len // self.pos_shard


def append_prefix_copy_jobs(mirror: KVPoolMirror, copy: PageCopy, jobs: list) -> None:
    """kv_policy.mojo:59-78: one byte job per layer x component."""
    rpp = mirror.rows_per_page()
    row_start = copy.pos_start // mirror.pos_shard
    row_end = (copy.pos_start + copy.pos_count + mirror.pos_shard - 1) // mirror.pos_shard
    rows = row_end - row_start
    for l in range(mirror.layers):
        base = mirror.region_off + l * mirror.stride
        for off, row_bytes in mirror.components:
            src = (copy.src_page * rpp + row_start) * row_bytes
            dst = (copy.dst_page * rpp + row_start) * row_bytes
            jobs.append((base + off + src, base + off + dst, rows * row_bytes))


def bind_pool_run_table(schedule: Schedule, pages: KVPageAccountant, pool_id: int,
                        mirror: KVPoolMirror):
    """kv_policy.mojo:99-123: runs [buf_start, base_pos, rows_off, page_count]
    and base rows (page * rows_per_page) per slot."""
    rpp = mirror.rows_per_page()
    runs, rows = [], []
    buf_start = 0
    for s in schedule.slots:
        if mirror.spec.fixed_pages_per_seq > 0:
            ordinals = mirror.spec.fixed_pages_per_seq
        else:
            ordinals = (s.base_pos + s.n_tokens - 1) // mirror.page_len + 1
        runs.append([buf_start, s.base_pos, len(rows), ordinals])
        for o in range(ordinals):
            page = pages.page_index(pool_id, s.seq_id, o)
            assert page >= 0, "run references unmapped page"
            rows.append(page * rpp)
        buf_start += s.n_tokens
    return runs, rows
