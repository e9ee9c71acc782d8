"""Python mirror of the reference's host-side page state, over the C ABI of
include/inferno_host.h (the state itself is C++ inside libinferno_hip.so).

Names and argument meanings follow the reference:
  KVPageAccountant        continuous_batching/paging.mojo:96-242
  SlotRegistry            continuous_batching/slot_registry.mojo:6-107
  ContinuousBatchScheduler continuous_batching/scheduler.mojo:61-780
  splitmix64 / hash_token_block / chain_link / refresh_chain /
  hashed_prefix_len       continuous_batching/prefix_hash.mojo:22-97
  KVPoolMirror / bind_pool_run_table / append_prefix_copy_jobs /
  dispatch_prefix_copies  modeling/kv_policy.mojo:18-123
Differences of form: clocks are explicit (`now`, default perf_counter_ns());
a request's CancelToken is `scheduler.cancel(request_id)`; a model's
`execute(scheduler, schedule, pages)` returns the sampled token ids of the
emitting slots in slot order.
"""
from __future__ import annotations

import ctypes as C
import time
from dataclasses import dataclass, field
from typing import List, Optional, Sequence

import numpy as np

from ._lib import P_I64, QUERY_ERROR, VP, check, last_error, lib
from .kv import KVRunTable

_PQ = dict(POOL_COUNT=0, MAX_SEQS=1, AVAILABLE=2, FIXED_PAGES=3, POOL_PAGES=4, SEQ_LIMIT=5,
           PAGE_INDEX=6, PAGE_HOLDS=7, FREEABLE=8, ACTIVE=9)
_RQ = dict(LENGTH=0, OWNER=1, RESIDENT=2, LAST_USED=3, CHAIN_LEN=4, MAX_SEQS=5, PPP=6)
_SQ = dict(PENDING_WORK=0, FULLY_CANCELLED=1, NUM_SLOTS=2, NUM_TOKENS=3, NUM_COPIES=4,
           PREFILL_TOKENS=5, DECODE_TOKENS=6, NUM_REQUESTS=7, NUM_PENDING=8,
           RING_CAPACITY=9, SEQ_CEILING=10, RING_FLOOR=11, REQ_SEQ_ID=12, REQ_DONE=13,
           REQ_LIVE=14, REQ_CANCELLED=15, REQ_NUM_TOKENS=16, REQ_NUM_GENERATED=17, PPP=18,
           SHARED_WRITES=19, UNSHARABLE_SHARED=20)


class HostStateError(RuntimeError):
    pass


def _q(value: int) -> int:
    if value == QUERY_ERROR:
        raise HostStateError(last_error())
    return int(value)


def _i32(xs: Sequence[int]) -> np.ndarray:
    return np.ascontiguousarray(np.asarray(xs, dtype=np.int64).astype(np.int32))


def _u64(xs: Sequence[int]) -> np.ndarray:
    return np.ascontiguousarray(np.asarray(list(xs), dtype=np.uint64))


def _vp(a: np.ndarray):
    return a.ctypes.data_as(VP) if a.size else None


def _now(now: Optional[int]) -> int:
    return time.perf_counter_ns() if now is None else int(now)


# ---------------------------------------------------------------------------
# prefix hash
# ---------------------------------------------------------------------------
def splitmix64(x: int) -> int:
    return int(lib().ifr_splitmix64(int(x) & 0xFFFFFFFFFFFFFFFF))


def hash_token_block(tokens: Sequence[int], start: int, count: int) -> int:
    t = _i32(tokens)
    if start < 0 or count < 0 or start + count > t.size:
        raise ValueError("hash_token_block: range outside tokens")
    return int(lib().ifr_hash_token_block(_vp(t), start, count))


def chain_link(prev: int, block_hash: int) -> int:
    return int(lib().ifr_chain_link(int(prev), int(block_hash)))


def refresh_chain(positions_per_page: int, chain: List[int], tokens: Sequence[int]) -> None:
    """Updates `chain` in place to one link per sealed page of `tokens`."""
    t = _i32(tokens)
    cap = max(len(chain), t.size // positions_per_page, 1)
    buf = np.zeros(cap, dtype=np.uint64)
    buf[:len(chain)] = np.asarray(chain, dtype=np.uint64)
    n = int(lib().ifr_refresh_chain(_vp(buf), len(chain), cap, _vp(t), t.size,
                                    positions_per_page))
    if n < 0:
        raise HostStateError(last_error())
    chain[:] = [int(x) for x in buf[:n]]


def hashed_prefix_len(positions_per_page: int, a_tokens, a_chain, b_tokens, b_chain) -> int:
    a, b = _i32(a_tokens), _i32(b_tokens)
    ac, bc = _u64(a_chain), _u64(b_chain)
    return _q(lib().ifr_hashed_prefix_len(positions_per_page, _vp(a), a.size, _vp(ac), ac.size,
                                          _vp(b), b.size, _vp(bc), bc.size))


# ---------------------------------------------------------------------------
# pages
# ---------------------------------------------------------------------------
@dataclass(frozen=True)
class PagePoolSpec:
    """paging.mojo:1-5."""
    num_pages: int
    fixed_pages_per_seq: int
    max_pages_per_seq: int


@dataclass
class BatchGeometry:
    """paging.mojo:8-13."""
    max_seqs: int
    max_slots: int
    max_step_tokens: int
    pools: List[PagePoolSpec]


def _specs(pools: Sequence[PagePoolSpec]) -> np.ndarray:
    return np.ascontiguousarray(np.asarray(
        [[p.num_pages, p.fixed_pages_per_seq, p.max_pages_per_seq] for p in pools],
        dtype=np.int64).reshape(-1, 3))


class KVPageAccountant:
    """Multi-pool page accounting (paging.mojo:96-242).  Built standalone
    from (max_seqs, pools), or lent out by a scheduler (`_borrow`)."""

    def __init__(self, max_seqs: int, pools: Sequence[PagePoolSpec]):
        h = VP()
        specs = _specs(pools)
        check(lib().ifr_pages_create(max_seqs, _vp(specs), len(pools), C.byref(h)))
        self._h, self._owner = h, None
        self._owned = True

    @classmethod
    def _borrow(cls, handle, owner) -> "KVPageAccountant":
        obj = cls.__new__(cls)
        obj._h, obj._owner, obj._owned = VP(handle), owner, False
        return obj

    def __del__(self):
        if getattr(self, "_owned", False) and self._h:
            lib().ifr_pages_destroy(self._h)
            self._h = VP()

    def _query(self, what: str, a: int = 0, b: int = 0, c: int = 0) -> int:
        return _q(lib().ifr_pages_query(self._h, _PQ[what], a, b, c))

    def pool_count(self) -> int:
        return self._query("POOL_COUNT")

    def pool_available(self, pool: int) -> int:
        return self._query("AVAILABLE", pool)

    def pool_fixed_pages(self, pool: int) -> int:
        return self._query("FIXED_PAGES", pool)

    def pool_pages(self, pool: int) -> int:
        return self._query("POOL_PAGES", pool)

    def pool_seq_page_limit(self, pool: int) -> int:
        return self._query("SEQ_LIMIT", pool)

    def page_index(self, pool: int, seq_id: int, ordinal: int) -> int:
        return self._query("PAGE_INDEX", pool, seq_id, ordinal)

    def page_holds(self, pool: int, page: int) -> int:
        return self._query("PAGE_HOLDS", pool, page)

    def freeable_pages(self, pool: int, seq_id: int) -> int:
        return self._query("FREEABLE", pool, seq_id)

    def is_active(self, seq_id: int) -> bool:
        return bool(self._query("ACTIVE", seq_id))

    def retain_page(self, pool: int, page: int) -> None:
        check(lib().ifr_pages_retain_page(self._h, pool, page))

    def release_page(self, pool: int, page: int) -> None:
        check(lib().ifr_pages_release_page(self._h, pool, page))

    def admit(self) -> int:
        out = C.c_int64()
        check(lib().ifr_pages_admit(self._h, C.byref(out)))
        return out.value

    def release(self, seq_id: int) -> None:
        check(lib().ifr_pages_release(self._h, seq_id))

    def share(self, pool: int, src_seq: int, dst_seq: int, ordinal: int) -> None:
        check(lib().ifr_pages_share(self._h, pool, src_seq, dst_seq, ordinal))

    def truncate(self, seq_id: int, last_keep_ordinal: int) -> None:
        check(lib().ifr_pages_truncate(self._h, seq_id, last_keep_ordinal))

    def replace_with_private(self, pool: int, seq_id: int, ordinal: int) -> int:
        out = C.c_int64()
        check(lib().ifr_pages_replace_with_private(self._h, pool, seq_id, ordinal,
                                                   C.byref(out)))
        return out.value

    def pages_needed(self, seq_id: int, last_ordinal: int, need: List[int]) -> None:
        arr = np.ascontiguousarray(np.asarray(need, dtype=np.int64))
        check(lib().ifr_pages_pages_needed(self._h, seq_id, last_ordinal, _vp(arr)))
        need[:] = [int(x) for x in arr]

    def fits(self, need: Sequence[int]) -> bool:
        arr = np.ascontiguousarray(np.asarray(need, dtype=np.int64))
        out = C.c_int64()
        check(lib().ifr_pages_fits(self._h, _vp(arr), C.byref(out)))
        return bool(out.value)

    def reserve(self, seq_id: int, last_ordinal: int) -> bool:
        out = C.c_int64()
        check(lib().ifr_pages_reserve(self._h, seq_id, last_ordinal, C.byref(out)))
        return bool(out.value)

    def export(self, pool: int):
        """(table [max_seqs][max_pages_per_seq], holds [num_pages],
        free_stack bottom first) as int32 arrays."""
        max_seqs = self._query("MAX_SEQS")
        limit, n = self.pool_seq_page_limit(pool), self.pool_pages(pool)
        table = np.empty((max_seqs, limit), dtype=np.int32)
        holds = np.empty(max(n, 1), dtype=np.int32)
        free = np.empty(max(n, 1), dtype=np.int32)
        fl = C.c_int64()
        check(lib().ifr_pages_export(self._h, pool, _vp(table), _vp(holds), _vp(free),
                                     C.byref(fl)))
        return table, holds[:n].copy(), free[:fl.value].copy()


# ---------------------------------------------------------------------------
# slot registry
# ---------------------------------------------------------------------------
class SlotRegistry:
    """slot_registry.mojo:6-107 (positions_per_page is a constructor
    argument instead of a compile-time parameter)."""

    def __init__(self, positions_per_page: int, max_seqs: int):
        h = VP()
        check(lib().ifr_registry_create(positions_per_page, max_seqs, C.byref(h)))
        self._h, self._owner, self._owned = h, None, True

    @classmethod
    def _borrow(cls, handle, owner) -> "SlotRegistry":
        obj = cls.__new__(cls)
        obj._h, obj._owner, obj._owned = VP(handle), owner, False
        return obj

    def __del__(self):
        if getattr(self, "_owned", False) and self._h:
            lib().ifr_registry_destroy(self._h)
            self._h = VP()

    def _query(self, what: str, sid: int = 0) -> int:
        return _q(lib().ifr_registry_query(self._h, _RQ[what], sid))

    @property
    def max_seqs(self) -> int:
        return self._query("MAX_SEQS")

    def length(self, sid: int) -> int:
        return self._query("LENGTH", sid)

    def owner_of(self, sid: int) -> int:
        return self._query("OWNER", sid)

    def is_resident(self, sid: int) -> bool:
        return bool(self._query("RESIDENT", sid))

    def last_used(self, sid: int) -> int:
        return self._query("LAST_USED", sid)

    def open(self, sid: int, owner_id: int, now: Optional[int] = None) -> None:
        check(lib().ifr_registry_open(self._h, sid, owner_id, _now(now)))

    def adopt(self, sid: int, owner_id: int, now: Optional[int] = None) -> None:
        check(lib().ifr_registry_adopt(self._h, sid, owner_id, _now(now)))

    def extend(self, sid: int, source: Sequence[int], start: int, base_pos: int, count: int,
               now: Optional[int] = None) -> None:
        s = _i32(source)
        check(lib().ifr_registry_extend(self._h, sid, _vp(s), s.size, start, base_pos, count,
                                        _now(now)))

    def seed(self, sid: int, source: Sequence[int], count: int,
             now: Optional[int] = None) -> None:
        s = _i32(source)
        check(lib().ifr_registry_seed(self._h, sid, _vp(s), s.size, count, _now(now)))

    def set_warm(self, sid: int) -> None:
        check(lib().ifr_registry_set_warm(self._h, sid))

    def close(self, sid: int) -> None:
        check(lib().ifr_registry_close(self._h, sid))

    def prefix_len(self, sid: int, incoming: Sequence[int], incoming_chain) -> int:
        t, c = _i32(incoming), _u64(incoming_chain)
        return _q(lib().ifr_registry_prefix_len(self._h, sid, _vp(t), t.size, _vp(c), c.size))

    def exact_prefix_len(self, sid: int, incoming: Sequence[int]) -> int:
        t = _i32(incoming)
        return _q(lib().ifr_registry_exact_prefix_len(self._h, sid, _vp(t), t.size))

    def lru_victim(self) -> int:
        return _q(lib().ifr_registry_lru_victim(self._h))

    def tokens(self, sid: int) -> List[int]:
        n = self.length(sid)
        buf = np.empty(max(n, 1), dtype=np.int32)
        check(lib().ifr_registry_export(self._h, sid, _vp(buf), n, None, 0))
        return [int(x) for x in buf[:n]]

    def chain(self, sid: int) -> List[int]:
        n = self._query("CHAIN_LEN", sid)
        buf = np.empty(max(n, 1), dtype=np.uint64)
        check(lib().ifr_registry_export(self._h, sid, None, 0, _vp(buf), n))
        return [int(x) for x in buf[:n]]


# ---------------------------------------------------------------------------
# scheduler
# ---------------------------------------------------------------------------
@dataclass
class BatchSlot:
    """schedule.mojo:29-51."""
    seq_id: int
    request_id: int
    base_pos: int
    n_tokens: int
    prompt_len: int
    emit: bool

    def prefill_count(self) -> int:
        pre = self.prompt_len - self.base_pos
        return 0 if pre < 0 else min(pre, self.n_tokens)

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
    """schedule.mojo:63-90 (a snapshot of the scheduler's current step)."""
    slots: List[BatchSlot] = field(default_factory=list)
    tokens: List[int] = field(default_factory=list)
    copies: List[PageCopy] = field(default_factory=list)
    prefill_tokens: int = 0
    decode_tokens: int = 0


@dataclass
class RequestView:
    seq_id: int
    done: bool
    live: bool
    cancelled: bool
    tokens: List[int]
    generated: List[int]


class ContinuousBatchScheduler:
    """scheduler.mojo:61-780."""

    def __init__(self, positions_per_page: int, geometry: BatchGeometry, step_budget: int,
                 stop_tokens, decode_band: int = 4):
        stops = [int(stop_tokens)] if np.isscalar(stop_tokens) else [int(t) for t in stop_tokens]
        st = _i32(stops)
        specs = _specs(geometry.pools)
        h = VP()
        check(lib().ifr_scheduler_create(
            positions_per_page, geometry.max_seqs, geometry.max_slots,
            geometry.max_step_tokens, _vp(specs), len(geometry.pools), step_budget,
            _vp(st), st.size, decode_band, C.byref(h)))
        self._h = h
        self.positions_per_page = positions_per_page
        self.pages = KVPageAccountant._borrow(lib().ifr_scheduler_pages(h), self)
        self.registry = SlotRegistry._borrow(lib().ifr_scheduler_registry(h), self)

    def __del__(self):
        if getattr(self, "_h", None):
            lib().ifr_scheduler_destroy(self._h)
            self._h = VP()

    def _query(self, what: str, arg: int = 0) -> int:
        return _q(lib().ifr_scheduler_query(self._h, _SQ[what], arg))

    # -- requests
    def submit(self, tokens: Sequence[int], max_new_tokens: int,
               no_share: bool = False) -> Optional[int]:
        t = _i32(tokens)
        out = C.c_int64()
        check(lib().ifr_scheduler_submit(self._h, _vp(t), t.size, max_new_tokens,
                                         1 if no_share else 0, C.byref(out)))
        return None if out.value < 0 else out.value

    def cancel(self, request_id: int) -> None:
        check(lib().ifr_scheduler_cancel(self._h, request_id))

    def retire(self, request_id: int) -> bool:
        out = C.c_int64()
        check(lib().ifr_scheduler_retire(self._h, request_id, C.byref(out)))
        return bool(out.value)

    def pending_work(self) -> bool:
        return bool(self._query("PENDING_WORK"))

    def evict_warm(self) -> bool:
        out = C.c_int64()
        check(lib().ifr_scheduler_evict_warm(self._h, C.byref(out)))
        return bool(out.value)

    def request(self, request_id: int) -> RequestView:
        nt = self._query("REQ_NUM_TOKENS", request_id)
        ng = self._query("REQ_NUM_GENERATED", request_id)
        tb = np.empty(max(nt, 1), dtype=np.int32)
        gb = np.empty(max(ng, 1), dtype=np.int32)
        check(lib().ifr_scheduler_export_request(self._h, request_id, _vp(tb), nt, _vp(gb), ng))
        return RequestView(self._query("REQ_SEQ_ID", request_id),
                           bool(self._query("REQ_DONE", request_id)),
                           bool(self._query("REQ_LIVE", request_id)),
                           bool(self._query("REQ_CANCELLED", request_id)),
                           [int(x) for x in tb[:nt]], [int(x) for x in gb[:ng]])

    @property
    def num_requests(self) -> int:
        return self._query("NUM_REQUESTS")

    def pending(self) -> List[int]:
        n = C.c_int64()
        check(lib().ifr_scheduler_export_pending(self._h, None, 0, C.byref(n)))
        buf = np.empty(max(n.value, 1), dtype=np.int64)
        check(lib().ifr_scheduler_export_pending(self._h, _vp(buf), n.value, C.byref(n)))
        return [int(x) for x in buf[:n.value]]

    def ring_floor(self, seq_id: int) -> int:
        return self._query("RING_FLOOR", seq_id)

    @property
    def invariant_failures(self) -> tuple:
        """(shared-page writes, unsharable-with-shared-page) counts of the
        reference's debug-build schedule checks (scheduler.mojo:688-720)."""
        return self._query("SHARED_WRITES"), self._query("UNSHARABLE_SHARED")

    @property
    def ring_capacity(self) -> int:
        return self._query("RING_CAPACITY")

    @property
    def seq_ceiling(self) -> int:
        return self._query("SEQ_CEILING")

    # -- steps
    def build_schedule(self, now: Optional[int] = None) -> bool:
        out = C.c_int64()
        check(lib().ifr_scheduler_build_schedule(self._h, _now(now), C.byref(out)))
        return bool(out.value)

    @property
    def schedule(self) -> Schedule:
        ns, nt, nc = (self._query("NUM_SLOTS"), self._query("NUM_TOKENS"),
                      self._query("NUM_COPIES"))
        slots = np.empty((max(ns, 1), 6), dtype=np.int64)
        toks = np.empty(max(nt, 1), dtype=np.int32)
        copies = np.empty((max(nc, 1), 5), dtype=np.int64)
        check(lib().ifr_scheduler_export_schedule(self._h, _vp(slots), slots.shape[0],
                                                  _vp(toks), toks.size, _vp(copies),
                                                  copies.shape[0]))
        return Schedule(
            [BatchSlot(int(r[0]), int(r[1]), int(r[2]), int(r[3]), int(r[4]), bool(r[5]))
             for r in slots[:ns]],
            [int(x) for x in toks[:nt]],
            [PageCopy(*(int(x) for x in r)) for r in copies[:nc]],
            self._query("PREFILL_TOKENS"), self._query("DECODE_TOKENS"))

    def copies_array(self) -> np.ndarray:
        """The step's copies as int64 [n][5] (the ifr_prefix_copy_jobs input)."""
        nc = self._query("NUM_COPIES")
        copies = np.zeros((max(nc, 1), 5), dtype=np.int64)
        check(lib().ifr_scheduler_export_schedule(self._h, None, 0, None, 0, _vp(copies),
                                                  copies.shape[0]))
        return copies[:nc]

    def absorb(self, emitted: Sequence[int], now: Optional[int] = None) -> None:
        e = _i32(emitted)
        check(lib().ifr_scheduler_absorb(self._h, _vp(e), e.size, _now(now)))

    def discard_step(self) -> None:
        check(lib().ifr_scheduler_discard_step(self._h))

    def fully_cancelled(self) -> bool:
        return bool(self._query("FULLY_CANCELLED"))

    def step(self, model, clock=time.perf_counter_ns) -> int:
        """scheduler.mojo:770-780: build, execute, then absorb the sampled
        tokens (or discard a fully cancelled step)."""
        if not self.build_schedule(clock()):
            return 0
        sched = self.schedule
        outs = model.execute(self, sched, self.pages)
        if self.fully_cancelled():
            self.discard_step()
        else:
            self.absorb(outs, clock())
        return len(sched.slots)


# ---------------------------------------------------------------------------
# kv_policy
# ---------------------------------------------------------------------------
@dataclass
class KVPoolMirror:
    """kv_policy.mojo:18-35: one pool's physical layout in the KV arena.
    components: (byte offset within a layer, row bytes) per cache component
    (k, v, and for the int8 format k_scale, v_scale)."""
    page_len: int
    pos_shard: int
    region_off: int
    stride: int
    layers: int
    components: List[tuple]
    spec: PagePoolSpec

    def rows_per_page(self) -> int:
        return self.page_len // self.pos_shard


def bind_pool_run_table(scheduler: ContinuousBatchScheduler, pool_id: int,
                        mirror: KVPoolMirror) -> KVRunTable:
    """kv_policy.mojo:99-123: the run table of the scheduler's current step."""
    sched = scheduler.schedule
    ns = len(sched.slots)
    cap_rows = 0
    fixed = scheduler.pages.pool_fixed_pages(pool_id)
    for s in sched.slots:
        cap_rows += fixed if fixed > 0 else (s.base_pos + s.n_tokens - 1) // mirror.page_len + 1
    runs = np.empty((max(ns, 1), 4), dtype=np.int32)
    rows = np.empty(max(cap_rows, 1), dtype=np.int32)
    nr, nb = C.c_int64(), C.c_int64()
    check(lib().ifr_bind_pool_run_table(scheduler._h, pool_id, mirror.page_len,
                                        mirror.pos_shard, _vp(runs), ns, _vp(rows),
                                        rows.size, C.byref(nr), C.byref(nb)))
    t = KVRunTable()
    t.runs = [[int(x) for x in r] for r in runs[:nr.value]]
    t.base_rows = [int(x) for x in rows[:nb.value]]
    return t


def prefix_copy_jobs(mirrors: Sequence[KVPoolMirror], copies) -> np.ndarray:
    """append_prefix_copy_jobs over a copy list (kv_policy.mojo:59-96):
    int64 [n][3] = {src_off, dst_off, byte_count} relative to the arena."""
    if isinstance(copies, np.ndarray):
        cp = np.ascontiguousarray(copies, dtype=np.int64).reshape(-1, 5)
    else:
        cp = np.ascontiguousarray(np.asarray(
            [[c.pool, c.src_page, c.dst_page, c.pos_start, c.pos_count] for c in copies],
            dtype=np.int64).reshape(-1, 5))
    mir = np.ascontiguousarray(np.asarray(
        [[m.page_len, m.pos_shard, m.region_off, m.stride, m.layers, len(m.components)]
         for m in mirrors], dtype=np.int64))
    comps = np.ascontiguousarray(np.asarray(
        [c for m in mirrors for c in m.components] or [[0, 0]], dtype=np.int64).reshape(-1, 2))
    n = C.c_int64()
    check(lib().ifr_prefix_copy_jobs(_vp(cp), cp.shape[0], _vp(mir), _vp(comps), len(mirrors),
                                     None, 0, C.byref(n)))
    jobs = np.zeros((max(n.value, 1), 3), dtype=np.int64)
    check(lib().ifr_prefix_copy_jobs(_vp(cp), cp.shape[0], _vp(mir), _vp(comps), len(mirrors),
                                     _vp(jobs), n.value, C.byref(n)))
    return jobs[:n.value]


def dispatch_prefix_copies(mirrors: Sequence[KVPoolMirror], schedule_copies, arena) -> int:
    """kv_policy.mojo:81-96: the step's copy-on-write page copies as one
    ifr_dispatch_copy_jobs launch over the arena (a device tensor).  Returns
    the number of byte jobs."""
    from .attention import dispatch_copy_jobs

    jobs = prefix_copy_jobs(mirrors, schedule_copies)
    if jobs.shape[0]:
        dispatch_copy_jobs(arena, jobs)
    return int(jobs.shape[0])


def bind_step_runs(scheduler: ContinuousBatchScheduler,
                   mirrors: Sequence[KVPoolMirror]) -> List[KVRunTable]:
    """bind_step_runs (modeling/gemma_4_moe.mojo:767-777): one run table per
    pool for the scheduler's current step, pool order as in `mirrors`."""
    return [bind_pool_run_table(scheduler, p, m) for p, m in enumerate(mirrors)]


def run_prefix_copies(scheduler: ContinuousBatchScheduler, mirrors: Sequence[KVPoolMirror],
                      arena) -> int:
    """run_prefix_copies (modeling/gemma_4_moe.mojo:763-766): the current
    step's page copies, issued before the step's appends on the same stream."""
    return dispatch_prefix_copies(mirrors, scheduler.copies_array(), arena)
