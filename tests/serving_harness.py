"""A lockstep serving loop for the GPU tests.

The product scheduler (C++, inferno_amd.host) builds each step; its run
tables, copy-on-write page copies, appends and attention run on the GPU
through libinferno_hip.so.  The oracle scheduler (oracle/host.py) and a CPU
mirror of the KV arena follow the same steps with the oracle's copy, append
and attention routines.  After every step the two schedulers' page state
must agree exactly, the appended rows and the rotated queries must match
bit for bit, and at chosen steps the attention outputs must match the
oracle within the bf16 tolerance.

K/V/Q rows are a hash of (position, token, salt), so sequences that share a
token prefix write identical rows, as a real model's layers would."""
from __future__ import annotations

from dataclasses import dataclass

import numpy as np

import oracle
import oracle.host as O
from inferno_amd import attention as A
from inferno_amd import host as P
from inferno_amd.kv import FULL, SLIDING, AttentionPlan
from tests.gpu_util import empty_dev, from_dev, to_dev
from tests.helpers import HEAD_DIM, KV_STRIDE, NUM_KV, NUM_Q, PAGE_LEN, compare_bf16

ROW_BYTES = KV_STRIDE * 2
Q_WIDTH = NUM_Q * HEAD_DIM
HALF = HEAD_DIM // 2


def hashed_bf16(pos, tok, salt: int, width: int) -> np.ndarray:
    """bf16 bits of values in [-2, 2) that depend on (position, token, salt,
    column) only."""
    p = np.asarray(pos, dtype=np.uint64)[:, None]
    t = np.asarray(tok, dtype=np.int64).astype(np.uint64)[:, None]
    c = np.arange(width, dtype=np.uint64)[None, :]
    with np.errstate(over="ignore"):
        h = (p * np.uint64(0x9E3779B97F4A7C15)) ^ (t * np.uint64(0xC2B2AE3D27D4EB4F))
        h = h ^ ((c + np.uint64(salt) * np.uint64(0x100000001B3)) * np.uint64(0x165667B19E3779F9))
        h = h ^ (h >> np.uint64(29))
        h = h * np.uint64(0xBF58476D1CE4E5B9)
        h = h ^ (h >> np.uint64(32))
    u = (h >> np.uint64(40)).astype(np.float64) / float(1 << 24)
    f = (u * 4.0 - 2.0).astype(np.float32)
    return oracle.f32_to_bf16(f.ravel()).reshape(f.shape)


class Clock:
    def __init__(self):
        self.t = 0

    def __call__(self):
        self.t += 1000
        return self.t


@dataclass
class PoolLayer:
    """One pool and the attention layer that reads it (one layer per pool)."""
    num_pages: int
    fixed_pages: int
    max_pages: int
    kind: int          # SLIDING for the ring pool, FULL for the growing pool
    window: int = 0
    page_len: int = PAGE_LEN

    @property
    def cache_size(self) -> int:
        return self.fixed_pages * self.page_len if self.kind == SLIDING else self.page_len

    @property
    def rows(self) -> int:
        return self.num_pages * self.page_len


class ServingHarness:
    def __init__(self, *, max_seqs, max_slots, max_step_tokens, pools, step_budget,
                 cap=128, max_pos=8192, seed=0, stops=(-1,), page_len=PAGE_LEN):
        import torch

        assert all(p.page_len == page_len for p in pools)
        self.pools = pools
        self.cap = cap
        self.page_len = page_len
        self.page_shift = page_len.bit_length() - 1
        pspecs = [P.PagePoolSpec(p.num_pages, p.fixed_pages, p.max_pages) for p in pools]
        ospecs = [O.PagePoolSpec(p.num_pages, p.fixed_pages, p.max_pages) for p in pools]
        self.ps = P.ContinuousBatchScheduler(
            page_len, P.BatchGeometry(max_seqs, max_slots, max_step_tokens, pspecs),
            step_budget, list(stops))
        self.os = O.ContinuousBatchScheduler(
            page_len, O.BatchGeometry(max_seqs, max_slots, max_step_tokens, ospecs),
            step_budget, list(stops))
        # Arena: per pool, the K region then the V region (bytes).
        self.k_off, self.v_off, off = [], [], 0
        for p in pools:
            self.k_off.append(off)
            off += p.rows * ROW_BYTES
            self.v_off.append(off)
            off += p.rows * ROW_BYTES
        self.arena_bytes = off
        self.arena_cpu = np.zeros(off // 2, dtype=np.uint16)
        self.arena_dev = torch.zeros(off // 2, dtype=torch.int16, device="cuda")
        self.mirrors = [P.KVPoolMirror(page_len, 1, self.k_off[i], 0, 1,
                                       [(0, ROW_BYTES), (self.v_off[i] - self.k_off[i], ROW_BYTES)],
                                       pspecs[i]) for i in range(len(pools))]
        self.omirrors = [O.KVPoolMirror(m.page_len, m.pos_shard, m.region_off, m.stride,
                                        m.layers, m.components, ospecs[i])
                         for i, m in enumerate(self.mirrors)]
        rng = np.random.default_rng(seed)
        ang = rng.uniform(-3.0, 3.0, max_pos * HALF)
        self.cos = np.cos(ang).astype(np.float32)
        self.sin = np.sin(ang).astype(np.float32)
        self.cos_dev, self.sin_dev = to_dev(self.cos), to_dev(self.sin)
        self.max_pos = max_pos
        self.pclock, self.oclock = Clock(), Clock()
        self.steps = 0
        self.checked = []
        self.copies_done = 0

    # -- views of the arena ---------------------------------------------------
    def _dev(self, off, rows):
        return self.arena_dev[off // 2: off // 2 + rows * KV_STRIDE]

    def _cpu(self, off, rows):
        return self.arena_cpu[off // 2: off // 2 + rows * KV_STRIDE]

    # -- requests ---------------------------------------------------------------
    def submit(self, tokens, max_new_tokens, no_share=False):
        a = self.ps.submit(tokens, max_new_tokens, no_share)
        b = self.os.submit(tokens, max_new_tokens, no_share)
        assert a == b
        return a

    def pending_work(self):
        a = self.ps.pending_work()
        assert a == self.os.pending_work()
        return a

    # -- one step -------------------------------------------------------------
    def step(self, check_attention=False, rng=None):
        built = self.ps.build_schedule(self.pclock())
        assert built == self.os.build_schedule(self.oclock())
        if not built:
            return None
        sched = self.ps.schedule
        osched = self.os.schedule
        assert [(s.seq_id, s.request_id, s.base_pos, s.n_tokens, s.prompt_len, s.emit)
                for s in sched.slots] == [
            (s.seq_id, s.request_id, s.base_pos, s.n_tokens, s.prompt_len, s.emit)
            for s in osched.slots]
        assert sched.tokens == osched.tokens
        assert [tuple(c.__dict__.values()) for c in sched.copies] == [
            tuple(c.__dict__.values()) for c in osched.copies]

        # Copy-on-write page copies first, as the reference's execute does.
        jobs = P.prefix_copy_jobs(self.mirrors, self.ps.copies_array())
        ojobs = []
        for c in osched.copies:
            O.append_prefix_copy_jobs(self.omirrors[c.pool], c, ojobs)
        assert jobs.tolist() == [list(j) for j in ojobs]
        if jobs.shape[0]:
            A.dispatch_copy_jobs(self.arena_dev, jobs)
            oracle.copy_jobs(self.arena_cpu, jobs)
            self.copies_done += jobs.shape[0]

        n = len(sched.tokens)
        pos = np.concatenate([np.arange(s.base_pos, s.base_pos + s.n_tokens)
                              for s in sched.slots])
        toks = np.asarray(sched.tokens, dtype=np.int64)
        assert pos.max() < self.max_pos
        tables = P.bind_step_runs(self.ps, self.mirrors)
        report = {"step": self.steps, "tokens": n, "slots": len(sched.slots),
                  "copies": int(jobs.shape[0]), "checks": []}
        for li, (layer, table) in enumerate(zip(self.pools, tables)):
            oruns, orows = O.bind_pool_run_table(osched, self.os.pages, li, self.omirrors[li])
            assert table.runs == oruns and table.base_rows == orows
            q = hashed_bf16(pos, toks, 10 * li + 1, Q_WIDTH)
            ks = hashed_bf16(pos, toks, 10 * li + 2, KV_STRIDE)
            vs = hashed_bf16(pos, toks, 10 * li + 3, KV_STRIDE)
            plan = AttentionPlan(table, n, kind=layer.kind, window=layer.window,
                                 cache_size=layer.cache_size, page_len=self.page_len,
                                 cache_rows=layer.rows, cap=self.cap, kv_row_bytes=ROW_BYTES)
            kd, vd = self._dev(self.k_off[li], layer.rows), self._dev(self.v_off[li], layer.rows)
            qd = to_dev(q)
            A.dispatch_rope_cache_write(plan, qd, to_dev(ks), to_dev(vs), kd, vd, self.cos_dev,
                                        self.sin_dev, num_q=NUM_Q, num_kv=NUM_KV, half=HALF,
                                        pair_stride=HALF, head_dim=HEAD_DIM)
            out = empty_dev(n * Q_WIDTH, np.uint16)
            partials, pstride = A.partials_buffer(plan, NUM_Q, HEAD_DIM)
            A.attention_bf16(plan, qd, kd, vd, out, partials, pstride, num_q=NUM_Q,
                             num_kv=NUM_KV, head_dim=HEAD_DIM, kv_stride=KV_STRIDE)
            # CPU mirror of the append.
            runs, rows = table.arrays()
            q_ref = q.copy()
            kc, vc = self._cpu(self.k_off[li], layer.rows), self._cpu(self.v_off[li], layer.rows)
            oracle.rope_cache_write(runs, rows, q_ref, ks, vs, kc, vc, self.cos, self.sin,
                                    num_q=NUM_Q, num_kv=NUM_KV, page_shift=self.page_shift,
                                    row_mask=self.page_len - 1,
                                    page_mask=plan.page_mask, seq_len=n, half=HALF,
                                    pair_stride=HALF, head_dim=HEAD_DIM)
            assert np.array_equal(from_dev(qd, np.uint16).ravel(), q_ref.ravel()), "rotated q"
            if check_attention:
                got = from_dev(out, np.uint16).reshape(n, Q_WIDTH)
                report["checks"].append(self._check(layer, runs, rows, q_ref.reshape(n, Q_WIDTH),
                                                    got, kc, vc, rng))
        emitted = [5000 + (self.steps * 13 + k) % 997
                   for k, s in enumerate(sched.slots) if s.emit]
        self.ps.absorb(emitted, self.pclock())
        self.os.absorb(emitted, self.oclock())
        self.compare_state()
        self.steps += 1
        return report

    def _check(self, layer, runs, rows, q_ref, got, kc, vc, rng):
        """Attention outputs of sampled tokens against the oracle on the
        CPU arena.  A pure decode step is checked whole (its route depends on
        the run count); otherwise up to 4 runs contribute 16 consecutive
        tokens each, which keeps the token-partitioned route whose per-token
        results do not depend on the other tokens of the step."""
        n = got.shape[0]
        counts = np.diff(np.append(runs[:, 0], n))
        if (counts == 1).all():
            sub_runs, sel = runs, np.arange(n)
        else:
            multi = [i for i in range(len(counts)) if counts[i] > 1]
            single = [i for i in range(len(counts)) if counts[i] == 1]
            pick = list(rng.choice(multi, size=min(3, len(multi)), replace=False))
            pick += list(rng.choice(single, size=min(1, len(single)), replace=False))
            sub, sel, buf = [], [], 0
            for i in sorted(int(x) for x in pick):
                c = int(counts[i])
                m = min(c, 16)
                o = int(rng.integers(0, c - m + 1))
                sub.append([buf, int(runs[i, 1]) + o, int(runs[i, 2]), int(runs[i, 3])])
                sel.extend(range(int(runs[i, 0]) + o, int(runs[i, 0]) + o + m))
                buf += m
            sub_runs, sel = np.asarray(sub, dtype=np.int32), np.asarray(sel)
        ref = oracle.attention(layer.kind, sub_runs, rows, np.ascontiguousarray(q_ref[sel]),
                               kc, vc, num_q=NUM_Q, num_kv=NUM_KV, head_dim=HEAD_DIM,
                               kv_stride=KV_STRIDE, window=layer.window,
                               cache_size=layer.cache_size, page_len=self.page_len,
                               seq_len=len(sel), cap=self.cap, threads=16)
        res = compare_bf16(got[sel].ravel(), ref)
        res["tokens"] = int(len(sel))
        assert res["n_fail"] == 0 and res["n_nan"] == 0, res
        self.checked.append(res)
        return res

    # -- state ------------------------------------------------------------------
    def compare_state(self):
        for p in range(len(self.pools)):
            a = [np.asarray(x).tolist() for x in self.ps.pages.export(p)]
            b = [np.asarray(x).tolist() for x in self.os.pages.export(p)]
            assert a == b, f"pool {p} page state diverged at step {self.steps}"
        reg, oreg = self.ps.registry, self.os.registry
        for sid in range(reg.max_seqs):
            assert reg.is_resident(sid) == oreg.is_resident(sid)
            assert reg.owner_of(sid) == oreg.owner_of(sid)
            assert reg.length(sid) == oreg.length(sid)
            assert self.ps.ring_floor(sid) == self.os.ring_floor(sid)
        assert self.ps.invariant_failures == self.os.invariant_failures

    def compare_arena(self):
        got = from_dev(self.arena_dev, np.uint16)
        assert np.array_equal(got, self.arena_cpu), "KV arena differs from the CPU mirror"
