"""Benchmark of the MI355X paged-KV attention path.

    python bench.py [--gpus 1] [--steps K] [--warmup W] [--config 2] [--cap C]

Headline (default): config 2 of BASELINE.json -- one layer of batched paged
decode for 64 sequences with contexts ~ U[512, 32768]: append one token per
sequence (RoPE + paged cache write), split-KV flash-decode partials over every
page, log-sum-exp merge.  --config 1, 3 and 5 run the other decode configs
(single sequence, sliding ring, butterquant int8) the same way, --config 4 the
chunked prefill.  Widening rows: --config 6 (MiniMax-M3 sparse decode), 7 and
8 (Gemma-4's full-attention layer, head_dim 512 with 16q/2kv, bf16 and bq),
9 (copy-on-write page copy), 10 (row gather), 11 (sliding-window chunked
prefill) and 12 (config 4's chunked prefill at the full-attention layer
shape).

Inputs (KV pages, queries, RoPE tables, the plan image) are resident in HBM
before the timed region; the plan is built once, as the reference binds its
run tables once per step for all layers.  Prints ONE JSON line: `value` is the
step's algorithmic bytes over its wall time (GB/s); `roofline` covers the
dominant kernel timed with HIP events on the launch stream; `cpu_baseline`
times the CPU oracle (a C restatement of the reference's algorithm) on a
bounded sample of the same batch on this host's cores.
"""
from __future__ import annotations

import argparse
import json
import os
import statistics
import sys
import time

import numpy as np

METRIC = "paged decode-attn GB/s (% HBM peak) + µs/layer, B=64 ctx≤32k bf16"
HBM_PEAK_GBS = 8000.0
NUM_Q, NUM_KV, HEAD_DIM, PAGE_LEN = 16, 8, 256, 64
HIDDEN = 2816  # Gemma 4 26B-A4B hidden size: o_proj maps 16 x 256 -> 2816
KV_STRIDE = NUM_KV * HEAD_DIM
MASK64 = (1 << 64) - 1
DEFAULT_CAP = {1: 128, 2: 512, 3: 256, 4: 16, 5: 2048, 6: 0, 7: 512, 8: 2048, 9: 0, 10: 0,
               11: 16, 12: 16}
MFMA_BF16_PEAK_TFLOPS = 2500.0
# Gemma-4's two attention layer shapes (modeling/gemma4_common.mojo:10-20):
# (num_q, num_kv, head_dim, rope_half, pair_stride).  BASELINE's configs 1-5
# are the sliding-layer shape; the five full-attention layers are 16q/2kv at
# head_dim 512 with 64 rotated pairs.
SLIDING_SHAPE = (16, 8, 256, 128, 128)
FULL_SHAPE = (16, 2, 512, 64, 256)
# The GPU box allots 16 CPUs to a one-GPU job; the CPU baselines use that many
# threads (the host may show more logical CPUs).
CPU_SHARE = 16


def host_cpu() -> dict:
    """CPU model and counts of the host the CPU baseline runs on."""
    model = "unknown"
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                if line.startswith("model name"):
                    model = line.split(":", 1)[1].strip()
                    break
    except OSError:
        pass
    try:
        avail = len(os.sched_getaffinity(0))
    except (AttributeError, OSError):
        avail = os.cpu_count() or 1
    return {"cpu_model": model, "logical_cpus": os.cpu_count(), "affinity_cpus": avail,
            "threads": max(1, min(CPU_SHARE, avail))}


# The CPU baseline's method: CPU_WARMUP untimed calls,
# then CPU_ITERS timed calls of the same sample; the median is reported.
CPU_WARMUP, CPU_ITERS = 5, 30


def cpu_oracle():
    """The oracle build the CPU baseline times: the -march=native build (AVX-512,
    with VDPBF16PS and VPDPBUSD dots where the host has AVX-512 BF16 / VNNI, as
    the reference's own kernels use them), built on this host; the portable
    x86-64-v3 build if that fails.  Returns (handle, label)."""
    import oracle

    try:
        return oracle.native_lib(), "native (-march=native)"
    except Exception as e:  # no compiler, or a host gcc cannot target
        return oracle.lib(), f"portable x86-64-v3 (native build failed: {e})"


def _same(a, b) -> bool:
    if isinstance(a, tuple):
        return all(_same(x, y) for x, y in zip(a, b))
    return a is None or np.array_equal(a, b)


def cpu_sample(make, n_max: int, cost, budget_s: float, n0: int) -> dict:
    """Size, check and time the CPU baseline's sample.

    make(n) returns a call over the first n units of the workload (sequences,
    query tokens, jobs or rows) that returns its output; cost(n) is their
    algorithmic work.  One calibration call on n0 units runs through the
    portable build and through the timed build, whose outputs must agree bit
    for bit (else the portable build is timed); the sample is then the largest
    n <= n_max whose CPU_WARMUP + CPU_ITERS calls fit budget_s at the
    calibrated rate, and its median call time is returned."""
    import oracle

    handle, label = cpu_oracle()
    fn0 = make(n0)
    ref = fn0()
    with oracle.using(handle):
        t0 = time.perf_counter()
        out = fn0()
        dt = max(time.perf_counter() - t0, 1e-6)
    identical = _same(ref, out)
    if not identical:
        handle, label = oracle.lib(), "portable x86-64-v3 (the native build's output differed)"
    rate = cost(n0) / dt
    per_call = budget_s / (CPU_WARMUP + CPU_ITERS)
    lo, hi = n0, n_max
    while lo < hi:  # the largest n whose estimated call fits per_call
        mid = (lo + hi + 1) // 2
        if cost(mid) / rate <= per_call:
            lo = mid
        else:
            hi = mid - 1
    n = lo
    fn = fn0 if n == n0 else make(n)
    del fn0
    with oracle.using(handle):
        for _ in range(CPU_WARMUP):
            fn()
        times = []
        for _ in range(CPU_ITERS):
            t0 = time.perf_counter()
            fn()
            times.append(time.perf_counter() - t0)
    return {"n": n, "median": statistics.median(times), "build": label,
            "native_bit_identical": identical, "calls": f"median of {CPU_ITERS} timed calls "
            f"after {CPU_WARMUP} warm-up calls"}


def cpu_result(hc, value, unit, cores, t, sample, **extra) -> dict:
    return {"value": value, "unit": unit, "cores": cores, "kind": "port",
            **{k: hc[k] for k in ("cpu_model", "logical_cpus", "affinity_cpus")},
            "build": t["build"], "native_bit_identical": t["native_bit_identical"],
            "sample": f"{sample}, {t['calls']}", **extra}


def splitmix64(x: int) -> int:
    z = (x + 0x9E3779B97F4A7C15) & MASK64
    z = ((z ^ (z >> 30)) * 0xBF58476D1CE4E5B9) & MASK64
    z = ((z ^ (z >> 27)) * 0x94D049BB133111EB) & MASK64
    return z ^ (z >> 31)


def uniform_ints(seed: int, n: int, lo: int, hi: int) -> list[int]:
    """n integers in [lo, hi] from the SplitMix64 counter stream."""
    return [lo + splitmix64(seed ^ splitmix64(i)) % (hi - lo + 1) for i in range(n)]


def rope_tables(max_pos: int, half: int = 128, theta: float = 10000.0):
    inv = 1.0 / theta ** (np.arange(half, dtype=np.float64) * 2 / (2 * half))
    ang = np.arange(max_pos, dtype=np.float64)[:, None] * inv[None, :]
    return np.cos(ang).astype(np.float32).reshape(-1), np.sin(ang).astype(np.float32).reshape(-1)


def layer_count(step_kv_bytes: int, limit: int = 64) -> int:
    """Layer caches to rotate through so that consecutive steps touch at least
    2 GiB of distinct K/V (8x the MI355X's 256 MB last-level cache)."""
    return max(1, min(limit, -(-(2 << 30) // max(1, step_kv_bytes))))


def _fill(t, seed, sid, outlier_every=0, scale=1.0):
    from inferno_amd._lib import check, lib

    check(lib().ifr_fill_normal_bf16(t.data_ptr(), t.numel() * t.element_size() // 2, seed,
                                     outlier_every, scale, sid))


def bq_quantize_cache(w, dev, spans, *, kind: int, cache_size: int, cache_rows: int,
                      v_is_k: bool, seed: int, chunk_tokens: int = 1 << 18) -> None:
    """Fill a butterquant cache the way the configuration produces it: every
    cached position's K and V rows, drawn N(0,1) with every 100th element x20
    (1 % outliers), go through the quantizing append (ifr_bq_attn_prep: RMS
    norm and RoPE of K, FWHT, absmax int8 codes and f32 scales;
    butterquant_kernels/attention.mojo:494-632) at their own positions.

    spans: (first position, count, page list) per sequence; the positions land
    where the page list (a ring when kind is sliding) puts them.  v_is_k: the
    full-attention layer's V is its raw K projection
    (modeling/gemma_4_moe_bq.mojo:566-573).  Untimed set-up work."""
    import torch

    from inferno_amd.kv import AttentionPlan, KVRunTable

    sid = int(torch.cuda.current_stream().cuda_stream)
    todo = [(p0, n, pages) for p0, n, pages in spans if n > 0]
    while todo:
        batch, tok = [], 0
        while todo and (not batch or tok + todo[0][1] <= chunk_tokens):
            p0, n, pages = todo.pop(0)
            if n > chunk_tokens:  # split a long span
                todo.insert(0, (p0 + chunk_tokens, n - chunk_tokens, pages))
                n = chunk_tokens
            batch.append((p0, n, pages))
            tok += n
        table = KVRunTable()
        buf = 0
        for p0, n, pages in batch:
            table.begin_run(buf, p0)
            for pg in pages:
                table.add_base_row(int(pg) * PAGE_LEN)
            buf += n
        plan = AttentionPlan(table, tok, kind=kind, window=cache_size if kind == 0 else 0,
                             cache_size=cache_size, page_len=PAGE_LEN, cache_rows=cache_rows,
                             cap=16, kv_row_bytes=w.kvs, device=dev)
        ksrc = torch.empty(tok * w.kvs, dtype=torch.int16, device=dev)
        _fill(ksrc, seed, sid, outlier_every=100, scale=20.0)
        if v_is_k:
            vsrc = ksrc
        else:
            vsrc = torch.empty_like(ksrc)
            _fill(vsrc, seed + 1, sid, outlier_every=100, scale=20.0)
        seed += 2
        qsrc = torch.zeros(tok * w.nq * w.hd, dtype=torch.int16, device=dev)
        qi = torch.empty(tok * w.nq * w.hd, dtype=torch.int8, device=dev)
        qb = torch.empty(tok * w.nq, dtype=torch.float32, device=dev)
        gain = torch.full((w.hd,), 0x3F80, dtype=torch.int16, device=dev)  # bf16 1.0
        w.A.dispatch_bq_attn_prep(plan, qsrc, ksrc, vsrc, gain, gain, qi, qb, torch.empty_like(qb),
                                  w.bq_k, w.bq_ks, w.bq_v, w.bq_vs, w.cos, w.sin, num_q=w.nq,
                                  num_kv=w.nkv, head_dim=w.hd, rope_half=w.half,
                                  pair_stride=w.pair,
                                  sqrt_n=float(np.sqrt(np.float32(w.hd))),
                                  n_eps=float(np.float32(w.hd) * np.float32(1e-6)))
        torch.cuda.synchronize()
        del ksrc, vsrc, qsrc, qi, qb, plan


class CopyStager:
    """ifr_dispatch_copy_jobs (kernels/page_copy.mojo:63-94) with a ring of
    pinned host + device staging buffers: a buffer is reused only after the
    stream has passed the call that last used it (the ws_host contract), so a
    timed loop of copies never waits on the host."""

    def __init__(self, jobs, dev, ring: int = 4):
        import torch

        from inferno_amd._lib import lib

        self.jobs = np.ascontiguousarray(jobs, dtype=np.int64).reshape(-1, 3)
        self.nbytes = int(lib().ifr_copy_jobs_bytes(self.jobs.shape[0],
                                                    int(self.jobs[:, 2].sum())))
        self.bufs = [(torch.empty(self.nbytes, dtype=torch.uint8, pin_memory=True),
                      torch.empty(self.nbytes, dtype=torch.uint8, device=dev),
                      torch.cuda.Event()) for _ in range(ring)]
        self.used = [False] * ring
        self.i = 0

    @property
    def copied_bytes(self) -> int:
        return int(self.jobs[:, 2].sum())

    def __call__(self, arena, stream) -> None:
        from inferno_amd._lib import P_I64, check, lib

        host, devb, ev = self.bufs[self.i]
        if self.used[self.i]:
            ev.synchronize()
        check(lib().ifr_dispatch_copy_jobs(
            arena.data_ptr(), self.jobs.ctypes.data_as(P_I64), self.jobs.shape[0],
            host.data_ptr(), devb.data_ptr(), self.nbytes, int(stream.cuda_stream)))
        ev.record(stream)
        self.used[self.i] = True
        self.i = (self.i + 1) % len(self.bufs)


class DecodeBf16:
    """Configs 1-3 and 7: bf16 append + split-KV decode + merge."""

    dtype = "bf16"
    phases = ("append", "partials", "merge")
    # The timed step: the append, then the attention as the host calls it
    # (ifr_attention_bf16: the partials and the merge in one call, as
    # dispatch_full_attention / dispatch_sliding_attention).
    timed_phases = ("append", "attention")
    graph = True
    dominant = "flash_partial_bf16_kernel<256,2>"

    def __init__(self, config: int, seed: int):
        self.cfg, self.seed = config, seed
        self.nq, self.nkv, self.hd, self.half, self.pair = SLIDING_SHAPE
        if config == 7:
            self.nq, self.nkv, self.hd, self.half, self.pair = FULL_SHAPE
            self.pos = uniform_ints(seed, 64, 512, 32768)
            self.kind, self.window, self.ring = 1, 0, 0
            self.extra_pages = 0
            self.dominant = "flash_partial_wide_kernel<bf16> (hd512, 8 q heads per kv head)"
            self.name = ("config7 (Gemma-4 full-attention layer): B=64 batched paged decode, "
                         "ctx ~ U[512,32768], 16q/2kv hd512 bf16, partial RoPE (64 pairs), "
                         "64-token pages, append 1 + split-KV decode + merge")
        elif config == 1:
            self.pos = [4096]
            self.kind, self.window, self.ring = 1, 0, 0
            self.extra_pages = 128 - 65
            self.name = ("config1: B=1 paged decode, ctx 4096 in a shuffled 128-page pool, "
                         "16q/8kv hd256 bf16, append 1 + split-KV decode + merge")
        elif config == 2:
            self.pos = uniform_ints(seed, 64, 512, 32768)
            self.kind, self.window, self.ring = 1, 0, 0
            self.extra_pages = 0
            self.name = ("config2: B=64 batched paged decode, ctx ~ U[512,32768], "
                         "16q/8kv hd256 bf16, 64-token pages, append 1 + split-KV decode + merge")
        else:
            self.pos = uniform_ints(seed, 64, 1023, 32767)
            self.kind, self.window, self.ring = 0, 1024, 32
            self.extra_pages = 0
            self.name = ("config3: B=64 sliding-window decode, window 1024 over 32-page rings, "
                         "positions ~ U[1023,32767], 16q/8kv hd256 bf16, append 1 + decode + merge")

    def setup(self, dev, a):
        import torch

        from inferno_amd import attention as A
        from inferno_amd.kv import AttentionPlan, KVRunTable

        self.A = A
        B = len(self.pos)
        table = KVRunTable()
        self.pages = []
        if self.ring:
            # KVPageAccountant.admit hands each sequence its fixed ring pages in
            # acquire order (continuous_batching/paging.mojo:156-170): the LIFO
            # stack starts n-1..0, so sequence s holds pages ring*s .. ring*s+ring-1.
            pool = B * self.ring
            for i, p in enumerate(self.pos):
                table.begin_run(i, p)
                pg = list(range(self.ring * i, self.ring * (i + 1)))
                self.pages.append(pg)
                for x in pg:
                    table.add_base_row(x * PAGE_LEN)
            cache_size = self.ring * PAGE_LEN
        else:
            need = [(p + 1 + PAGE_LEN - 1) // PAGE_LEN for p in self.pos]
            pool = sum(need) + self.extra_pages
            perm = np.random.default_rng(self.seed).permutation(pool)
            off = 0
            for i, p in enumerate(self.pos):
                table.begin_run(i, p)
                pg = perm[off:off + need[i]]
                off += need[i]
                self.pages.append(list(pg))
                for x in pg:
                    table.add_base_row(int(x) * PAGE_LEN)
            cache_size = PAGE_LEN
        self.pool, self.table = pool, table
        self.cache_size = cache_size
        rows = pool * PAGE_LEN
        self.kvs = self.nkv * self.hd
        self.stream = torch.cuda.current_stream()
        sid = int(self.stream.cuda_stream)
        self.k = torch.empty(rows * self.kvs, dtype=torch.int16, device=dev)
        self.v = torch.empty_like(self.k)
        self.q = torch.empty(B * self.nq * self.hd, dtype=torch.int16, device=dev)
        self.ks = torch.empty(B * self.kvs, dtype=torch.int16, device=dev)
        self.vs = torch.empty_like(self.ks)
        for i, t in enumerate((self.k, self.v, self.q, self.ks, self.vs)):
            _fill(t, self.seed * 16 + i, sid)
        # Consecutive steps run on different layers' caches, as a model's
        # decode step walks every layer before it returns to this one: a
        # configuration whose step touches less than 2 GiB of K/V would
        # otherwise find it in the 256 MB last-level cache (MALL) again.
        self.layers = layer_count(self.kv_positions() * self.kvs * 4)
        self.kl = [(self.k, self.v)]
        for j in range(1, self.layers):
            kj, vj = torch.empty_like(self.k), torch.empty_like(self.v)
            _fill(kj, self.seed * 16 + 32 * j, sid)
            _fill(vj, self.seed * 16 + 32 * j + 1, sid)
            self.kl.append((kj, vj))
        self.layer = 0
        cos, sin = rope_tables(max(self.pos) + 2, half=self.half)
        self.cos, self.sin = torch.from_numpy(cos).to(dev), torch.from_numpy(sin).to(dev)
        self.plan = AttentionPlan(table, B, kind=self.kind, window=self.window,
                                  cache_size=cache_size, page_len=PAGE_LEN, cache_rows=rows,
                                  cap=a.cap, kv_row_bytes=self.kvs * 2, device=dev)
        self.partials, self.ps = A.partials_buffer(self.plan, self.nq, self.hd)
        self.out = torch.empty(B * self.nq * self.hd, dtype=torch.int16, device=dev)
        self.q_host = self.q.cpu().numpy().view(np.uint16).copy()
        self.cap = a.cap
        self.sqrt_n = float(np.sqrt(np.float32(self.hd)))
        self.n_eps = float(np.float32(self.hd) * np.float32(1e-6))
        # Optional head RMS norm ahead of the append (dispatch_rms_norm_qkv_heads):
        # "separate" runs it as its own in-place pass, "fused" folds it into the
        # append kernel.
        self.norm = a.norm
        if self.norm != "none":
            self.qw = torch.empty(self.hd, dtype=torch.int16, device=dev)
            self.kw = torch.empty_like(self.qw)
            _fill(self.qw, self.seed * 16 + 7, sid)
            _fill(self.kw, self.seed * 16 + 8, sid)
            self.name += f", head RMS norm {self.norm}"
        if self.norm == "separate":
            self.phases = ("norm",) + DecodeBf16.phases
        # Optional o_proj after the merge (dispatch_gemm_cols, rows = HIDDEN):
        # a random bf16 weight [HIDDEN][num_q * head_dim].
        self.oproj = a.oproj
        if self.oproj:
            self.o_w = torch.empty(HIDDEN * self.nq * self.hd, dtype=torch.int16, device=dev)
            _fill(self.o_w, self.seed * 16 + 9, sid, scale=0.02)
            self.o_out = torch.empty(B * HIDDEN, dtype=torch.int16, device=dev)
            self.o_ws = A.gemm_cols_workspace(HIDDEN, self.nq * self.hd, B, device=dev)
            self.phases = self.phases + ("oproj",)
            self.name += ", o_proj bf16 GEMM"

    def launch(self, phase):
        A, p = self.A, self.plan
        if phase == self.phases[0]:
            self.layer = (self.layer + 1) % self.layers
        kc, vc = self.kl[self.layer]
        if phase == "oproj":
            A.dispatch_gemm_cols(self.out, self.o_w, self.o_out, rows=HIDDEN,
                                 cols=self.nq * self.hd, seq_len=len(self.pos),
                                 workspace=self.o_ws)
        elif phase == "norm":
            A.dispatch_rms_norm_qkv_heads(self.q, self.ks, self.vs, self.qw, self.kw,
                                          num_q=self.nq, num_kv=self.nkv,
                                          seq_len=len(self.pos), head_dim=self.hd,
                                          sqrt_n=self.sqrt_n, n_eps=self.n_eps)
        elif phase == "append" and self.norm == "fused":
            A.dispatch_rms_norm_rope_cache_write(
                p, self.q, self.ks, self.vs, kc, vc, self.qw, self.kw, self.cos,
                self.sin, num_q=self.nq, num_kv=self.nkv, half=self.half,
                pair_stride=self.pair, head_dim=self.hd, sqrt_n=self.sqrt_n,
                n_eps=self.n_eps)
        elif phase == "append":
            A.dispatch_rope_cache_write(p, self.q, self.ks, self.vs, kc, vc, self.cos,
                                        self.sin, num_q=self.nq, num_kv=self.nkv,
                                        half=self.half, pair_stride=self.pair,
                                        head_dim=self.hd)
        elif phase == "attention":
            A.attention_bf16(p, self.q, kc, vc, self.out, self.partials, self.ps,
                             num_q=self.nq, num_kv=self.nkv, head_dim=self.hd,
                             kv_stride=self.kvs)
        elif phase == "partials":
            A.flash_partials_bf16(p, self.q, kc, vc, self.partials, self.ps,
                                  num_q=self.nq, num_kv=self.nkv, head_dim=self.hd,
                                  kv_stride=self.kvs)
        else:
            A.merge_flash_partials(p, self.partials, self.out, self.ps, num_q=self.nq,
                                   head_dim=self.hd)

    def kv_positions(self, pos=None) -> int:
        pos = self.pos if pos is None else pos
        if self.kind == 0:
            return sum(min(p + 1, self.window) for p in pos)
        return sum(p + 1 for p in pos)

    def dominant_bytes(self) -> int:
        """Partial kernel: K+V of every attended position, q and the page table."""
        B = len(self.pos)
        return (self.kv_positions() * self.kvs * 4 + B * self.nq * self.hd * 2
                + 4 * len(self.table.base_rows))

    def step_bytes(self) -> int:
        """Whole step: the partial kernel's bytes, the output and the append."""
        B = len(self.pos)
        append = B * (self.kvs * 2 * 2 * 2 + self.nq * self.hd * 2 * 2)
        # o_proj: its weight, the attention output read back, the bf16 result.
        oproj = (HIDDEN * self.nq * self.hd * 2 + B * self.nq * self.hd * 2 + B * HIDDEN * 2
                 if self.oproj else 0)
        return self.dominant_bytes() + B * self.nq * self.hd * 2 + append + oproj

    def config(self) -> dict:
        return {"workload": self.name, "batch": len(self.pos),
                "attended_positions": self.kv_positions(), "pool_pages": self.pool,
                "page_len": PAGE_LEN, "num_q": self.nq, "num_kv": self.nkv,
                "head_dim": self.hd, "rope_half": self.half, "pair_stride": self.pair,
                "window": self.window or None, "cap": self.cap, "seed": self.seed,
                "plan_items": self.plan.summary.num_items, "layer_caches": self.layers}

    def cpu_baseline(self, budget_s):
        """The oracle (FlashAttentionKernel + merge_segments under the
        reference's routing, cap = worker threads) on the first n sequences of
        the batch, their pages copied into a compact host cache; n is the whole
        batch when its timed calls fit the budget."""
        import torch

        import oracle

        hc = host_cpu()
        threads = hc["threads"]
        kc, vc = self.kl[self.layer]
        B = len(self.pos)

        def make(n):
            pages = np.concatenate([np.asarray(p) for p in self.pages[:n]])
            idx = torch.from_numpy(pages.astype(np.int64)).to(kc.device)
            kp = kc.view(-1, PAGE_LEN * self.kvs).index_select(0, idx).cpu().numpy()
            vp = vc.view(-1, PAGE_LEN * self.kvs).index_select(0, idx).cpu().numpy()
            kp = np.ascontiguousarray(kp.view(np.uint16).reshape(-1))
            vp = np.ascontiguousarray(vp.view(np.uint16).reshape(-1))
            runs, rows, off = [], [], 0
            for i in range(n):
                m = len(self.pages[i])
                runs.append([i, self.pos[i], off, m])
                rows.extend((off + j) * PAGE_LEN for j in range(m))
                off += m
            runs, rows = np.asarray(runs, dtype=np.int32), np.asarray(rows, dtype=np.int32)
            q = np.ascontiguousarray(self.q_host[:n * self.nq * self.hd])
            return lambda: oracle.attention(
                self.kind, runs, rows, q, kp, vp, num_q=self.nq, num_kv=self.nkv,
                head_dim=self.hd, kv_stride=self.kvs, window=self.window,
                cache_size=self.cache_size, page_len=PAGE_LEN, seq_len=n, cap=threads,
                threads=threads)

        def cost(n):
            return self.kv_positions(self.pos[:n]) * self.kvs * 4

        t = cpu_sample(make, B, cost, budget_s, min(B, threads))
        n, med = t["n"], t["median"]
        nbytes = cost(n)
        scope = ("the whole batch" if n == B else
                 f"the first {n} of the {B} sequences, extrapolated to the batch by K/V bytes")
        return cpu_result(hc, round(nbytes / med / 1e9, 3), "GB/s", threads, t,
                          f"{scope} ({nbytes / 1e9:.3f} GB of K+V), the reference's routing "
                          f"at cap={threads} workers",
                          us_per_layer_equiv=round(med * 1e6 * cost(B) / nbytes, 1))

class DecodeBq:
    """Configs 5 and 8: butterquant int8 KV -- quantizing append + int8 decode +
    merge."""

    dtype = "int8 KV (f32 scales), f32 accumulate"
    data = ("synthetic: seeded SplitMix64/Box-Muller N(0,1) K/V with every 100th element x20 "
            "(1 % outliers), the cached positions quantized through the bq append (RMS norm, "
            "RoPE, FWHT, absmax int8 codes + f32 scales) at set-up, on device")
    phases = ("append", "attention")
    graph = True
    dominant = "bq_partial_kernel<2> + merge_kernel<256>"

    def __init__(self, config: int, seed: int):
        self.cfg, self.seed = config, seed
        self.pos = uniform_ints(seed, 128, 1024, 65536)
        if config == 8:
            self.nq, self.nkv, self.hd, self.half, self.pair = FULL_SHAPE
            self.dominant = "flash_partial_wide_kernel<int8> + merge_kernel<512>"
            self.name = ("config8 (Gemma-4 full-attention layer, bq): B=128 butterquant decode, "
                         "ctx ~ U[1024,65536], 16q/2kv hd512, int8 FWHT-512 codes + f32 scales, "
                         "partial RoPE (64 pairs), quantizing append 1 + int8 split-KV decode "
                         "+ merge")
        else:
            self.nq, self.nkv, self.hd, self.half, self.pair = SLIDING_SHAPE
            self.name = ("config5: B=128 butterquant decode, ctx ~ U[1024,65536], 16q/8kv "
                         "hd256, int8 FWHT-256 codes + f32 per-(position, kv head) scales (the "
                         "reference's bq format), quantizing append 1 + int8 split-KV decode "
                         "+ merge")
        self.kvs = self.nkv * self.hd

    def setup(self, dev, a):
        import torch

        from inferno_amd import attention as A
        from inferno_amd.kv import AttentionPlan, KVRunTable

        self.A = A
        B = len(self.pos)
        need = [(p + 1 + PAGE_LEN - 1) // PAGE_LEN for p in self.pos]
        pool = sum(need)
        perm = np.random.default_rng(self.seed).permutation(pool)
        table = KVRunTable()
        off = 0
        for i, p in enumerate(self.pos):
            table.begin_run(i, p)
            for x in perm[off:off + need[i]]:
                table.add_base_row(int(x) * PAGE_LEN)
            off += need[i]
        rows = pool * PAGE_LEN
        self.pool, self.table = pool, table
        self.pages = []
        off = 0
        for n in need:
            self.pages.append([int(x) for x in perm[off:off + n]])
            off += n
        self.stream = torch.cuda.current_stream()
        sid = int(self.stream.cuda_stream)
        self.kc = torch.zeros(rows * self.kvs, dtype=torch.int8, device=dev)
        self.vc = torch.zeros_like(self.kc)
        self.ksc = torch.zeros(rows * self.nkv, dtype=torch.float32, device=dev)
        self.vsc = torch.zeros_like(self.ksc)
        cos, sin = rope_tables(max(self.pos) + 2, half=self.half)
        self.cos, self.sin = torch.from_numpy(cos).to(dev), torch.from_numpy(sin).to(dev)
        # The cached positions 0 .. pos-1 of every sequence, quantized through
        # the append path from N(0,1) K/V with 1 % outliers x20.
        self.bq_k, self.bq_ks, self.bq_v, self.bq_vs = self.kc, self.ksc, self.vc, self.vsc
        bq_quantize_cache(self, dev, [(0, p, pg) for p, pg in zip(self.pos, self.pages)],
                          kind=1, cache_size=PAGE_LEN, cache_rows=rows, v_is_k=self.cfg == 8,
                          seed=self.seed * 16 + 1)
        self.qs = torch.empty(B * self.nq * self.hd, dtype=torch.int16, device=dev)
        self.kss = torch.empty(B * self.kvs, dtype=torch.int16, device=dev)
        self.vss = torch.empty_like(self.kss)
        for i, t in enumerate((self.qs, self.kss, self.vss)):
            _fill(t, self.seed * 16 + 3 + i, sid, outlier_every=100, scale=20.0)
        self.qn = torch.full((self.hd,), 0x3F80, dtype=torch.int16, device=dev)  # bf16 1.0
        self.kn = self.qn
        self.q_i8 = torch.empty(B * self.nq * self.hd, dtype=torch.int8, device=dev)
        self.qb = torch.empty(B * self.nq, dtype=torch.float32, device=dev)
        self.fq = torch.empty_like(self.qb)
        self.plan = AttentionPlan(table, B, kind=1, window=0, cache_size=PAGE_LEN,
                                  page_len=PAGE_LEN, cache_rows=rows, cap=a.cap,
                                  kv_row_bytes=self.kvs, device=dev)
        self.partials, self.ps = A.partials_buffer(self.plan, self.nq, self.hd)
        self.out = torch.empty(B * self.nq * self.hd, dtype=torch.int16, device=dev)
        self.cap = a.cap
        # Optional o_proj input quantisation (dispatch_bq_block_quant,
        # block = head_dim): its own pass over the output, or fused into the merge.
        self.oquant = a.oquant
        if self.oquant != "none":
            self.o_i8 = torch.empty(B * self.nq * self.hd, dtype=torch.int8, device=dev)
            self.o_sa = torch.empty(B * self.nq, dtype=torch.float32, device=dev)
            self.name += f", o_proj int8 block quant {self.oquant}"
        if self.oquant == "separate":
            self.phases = DecodeBq.phases + ("oquant",)

    def launch(self, phase):
        A, p = self.A, self.plan
        if phase == "oquant":
            A.dispatch_bq_block_quant(self.out, self.o_i8, self.o_sa, cols=self.nq * self.hd,
                                      block=self.hd, seq_len=len(self.pos))
        elif phase == "append":
            # The full layer's V is its raw K projection (gemma_4_moe_bq.mojo:566-573).
            vsrc = self.kss if self.cfg == 8 else self.vss
            A.dispatch_bq_attn_prep(p, self.qs, self.kss, vsrc, self.qn, self.kn,
                                    self.q_i8, self.qb, self.fq, self.kc, self.ksc, self.vc,
                                    self.vsc, self.cos, self.sin, num_q=self.nq,
                                    num_kv=self.nkv, head_dim=self.hd, rope_half=self.half,
                                    pair_stride=self.pair,
                                    sqrt_n=float(np.sqrt(np.float32(self.hd))),
                                    n_eps=float(np.float32(self.hd) * np.float32(1e-6)))
        else:
            fused = self.oquant == "fused"
            A.bq_attention(p, self.q_i8, self.qb, self.fq, self.kc, self.ksc, self.vc,
                           self.vsc, self.out, self.partials, self.ps, num_q=self.nq,
                           num_kv=self.nkv, head_dim=self.hd, kv_stride=self.kvs,
                           o_i8=self.o_i8 if fused else None,
                           o_sa=self.o_sa if fused else None)

    def dominant_bytes(self) -> int:
        B = len(self.pos)
        kv = sum(p + 1 for p in self.pos) * (self.kvs * 2 + self.nkv * 4 * 2)
        return (kv + B * self.nq * (self.hd + 8) + 4 * len(self.table.base_rows)
                + B * self.nq * self.hd * 2)

    def step_bytes(self) -> int:
        B = len(self.pos)
        append = B * ((self.nq + 2 * self.nkv) * self.hd * 2 +
                      (self.nq + 2 * self.nkv) * self.hd)
        # o_proj quant: int8 codes + f32 scales written; the separate pass
        # also re-reads the bf16 output.
        oquant = {"none": 0, "fused": B * self.nq * (self.hd + 4),
                  "separate": B * self.nq * (3 * self.hd + 4)}[self.oquant]
        return self.dominant_bytes() + append + oquant

    def config(self) -> dict:
        return {"workload": self.name, "batch": len(self.pos),
                "attended_positions": sum(p + 1 for p in self.pos), "pool_pages": self.pool,
                "page_len": PAGE_LEN, "num_q": self.nq, "num_kv": self.nkv,
                "head_dim": self.hd, "rope_half": self.half, "pair_stride": self.pair,
                "cap": self.cap, "seed": self.seed, "plan_items": self.plan.summary.num_items}

    def cpu_baseline(self, budget_s):
        """The oracle's bq attention (bq_process_kv_tile and the merge, the
        reference's routing) on the first n sequences of the batch, n the whole
        batch when its timed calls fit the budget."""
        import torch

        import oracle

        hc = host_cpu()
        threads = hc["threads"]
        B = len(self.pos)

        def make(n):
            pages = np.concatenate([np.asarray(p) for p in self.pages[:n]])
            idx = torch.from_numpy(pages.astype(np.int64)).to(self.kc.device)

            def sel(t, per_row):
                return np.ascontiguousarray(
                    t.view(-1, PAGE_LEN * per_row).index_select(0, idx).cpu().numpy()
                ).reshape(-1)

            kp, vp = sel(self.kc, self.kvs), sel(self.vc, self.kvs)
            ksp, vsp = sel(self.ksc, self.nkv), sel(self.vsc, self.nkv)
            runs, rows, off = [], [], 0
            for i in range(n):
                m = len(self.pages[i])
                runs.append([i, self.pos[i], off, m])
                rows.extend((off + j) * PAGE_LEN for j in range(m))
                off += m
            runs, rows = np.asarray(runs, dtype=np.int32), np.asarray(rows, dtype=np.int32)
            nq = n * self.nq
            q_i8 = np.ascontiguousarray(self.q_i8.cpu().numpy()[:nq * self.hd])
            qb = np.ascontiguousarray(self.qb.cpu().numpy()[:nq])
            fq = np.ascontiguousarray(self.fq.cpu().numpy()[:nq])
            return lambda: oracle.bq_attention(
                1, runs, rows, q_i8, qb, fq, kp, ksp, vp, vsp, num_q=self.nq,
                num_kv=self.nkv, head_dim=self.hd, kv_stride=self.kvs, window=0,
                cache_size=PAGE_LEN, page_len=PAGE_LEN, seq_len=n, cap=threads,
                threads=threads)

        def cost(n):
            return sum(p + 1 for p in self.pos[:n]) * (self.kvs * 2 + self.nkv * 8)

        t = cpu_sample(make, B, cost, budget_s, min(B, threads))
        n, med = t["n"], t["median"]
        nbytes = cost(n)
        scope = ("the whole batch" if n == B else
                 f"the first {n} of the {B} sequences, extrapolated to the batch by bytes")
        return cpu_result(hc, round(nbytes / med / 1e9, 3), "GB/s", threads, t,
                          f"{scope} ({nbytes / 1e9:.3f} GB of int8 K+V and scales), the "
                          f"reference's bq routing at cap={threads} workers",
                          us_per_layer_equiv=round(med * 1e6 * cost(B) / nbytes, 1))

class SparseM3:
    """Config 6 (widening row, no BASELINE counterpart): MiniMax-M3 block-sparse
    decode -- lightning indexer (block scores over every cached position + top-16
    blocks per index head) then block-sparse attention over the selected blocks
    (prototypes/benchmark_sparse_attention.mojo's decode sweep, batched)."""

    dtype = "bf16 (indexer VDPBF16PS-order f32 dots; attention MFMA QK, f32 PV)"
    phases = ("indexer", "sparse")
    dominant = "index_scores_kernel + select_blocks_kernel"
    dominant_phase = "indexer"
    NQ, NKV, HD, IH, BLOCK, TOPK, PLEN = 64, 4, 128, 4, 128, 16, 128

    def __init__(self, seed: int):
        self.seed = seed
        self.pos = uniform_ints(seed, 64, 1024, 131071)
        self.name = ("config6: MiniMax-M3 block-sparse decode, B=64, ctx ~ U[1024,131072], "
                     "lightning indexer (4 heads x 128, 128-position blocks, top 16) + sparse "
                     "attention 64q/4kv hd128 bf16, 128-token pages")

    def setup(self, dev, a):
        import torch

        from inferno_amd import attention as A
        from inferno_amd.kv import AttentionPlan, KVRunTable

        self.A = A
        B, P = len(self.pos), self.PLEN
        need = [(p + 1 + P - 1) // P for p in self.pos]
        pool = sum(need)
        perm = np.random.default_rng(self.seed).permutation(pool)
        table = KVRunTable()
        off = 0
        self.pages = []
        for i, p in enumerate(self.pos):
            table.begin_run(i, p)
            pg = [int(x) for x in perm[off:off + need[i]]]
            self.pages.append(pg)
            for x in pg:
                table.add_base_row(x * P)
            off += need[i]
        rows = pool * P
        self.pool, self.table, self.rows = pool, table, rows
        self.stream = torch.cuda.current_stream()
        sid = int(self.stream.cuda_stream)
        kvs = self.NKV * self.HD
        self.index_k = torch.empty(rows * self.HD, dtype=torch.int16, device=dev)
        self.index_q = torch.empty(B * self.IH * self.HD, dtype=torch.int16, device=dev)
        self.kv = a.kv
        elt = torch.int8 if self.kv == "bq" else torch.int16
        self.k = torch.empty(rows * kvs, dtype=elt, device=dev)
        self.v = torch.empty_like(self.k)
        self.q = torch.empty(B * self.NQ * self.HD, dtype=elt, device=dev)
        _fill(self.index_k, self.seed * 16 + 1, sid)
        _fill(self.index_q, self.seed * 16 + 2, sid)
        _fill(self.k, self.seed * 16 + 3, sid)
        _fill(self.v, self.seed * 16 + 4, sid)
        _fill(self.q, self.seed * 16 + 5, sid, scale=float(1.0 / np.sqrt(self.HD)))
        if self.kv == "bq":
            # int8 codes (random bytes) with f32 scales, as ifr_bq_attn_prep lays them out.
            gen = torch.Generator(device=dev)
            gen.manual_seed(self.seed)
            self.ksc = torch.rand(rows * self.NKV, device=dev, generator=gen) * 4 + 0.5
            self.vsc = torch.rand(rows * self.NKV, device=dev, generator=gen) * 4 + 0.5
            self.qb = torch.zeros(B * self.NQ, dtype=torch.float32, device=dev)
            self.fq = torch.full((B * self.NQ,), 0.01, dtype=torch.float32, device=dev)
            self.dtype = "int8 KV (f32 scales); indexer bf16"
            self.name = self.name.replace("sparse attention 64q/4kv hd128 bf16",
                                          "bq int8 sparse attention 64q/4kv hd128")
        self.plan = AttentionPlan(table, B, kind=1, window=0, cache_size=P, page_len=P,
                                  cache_rows=rows, cap=16, kv_row_bytes=kvs * 2, device=dev)
        self.scores = A.index_scores_buffer(self.plan, self.IH, self.BLOCK, device=dev)
        self.block_idx = torch.empty(B * self.IH * self.TOPK, dtype=torch.int32, device=dev)
        self.out = torch.empty(B * self.NQ * self.HD, dtype=torch.int16, device=dev)
        self.cap = 0
        # Layer caches rotated per step, as in the dense decode: the selected
        # blocks are the same every step, and a model would read every other
        # layer's index keys and K/V before this layer's again.
        self.layers = layer_count(self.step_bytes(), limit=4)
        bq = self.kv == "bq"
        self.kl = [(self.index_k, self.k, self.v, self.ksc if bq else None,
                    self.vsc if bq else None)]
        for j in range(1, self.layers):
            ik, kj, vj = (torch.empty_like(self.index_k), torch.empty_like(self.k),
                          torch.empty_like(self.v))
            for i, t in enumerate((ik, kj, vj)):
                _fill(t, self.seed * 16 + 32 * j + i, sid)
            ks = vs = None
            if bq:
                ks = torch.rand(rows * self.NKV, device=dev, generator=gen) * 4 + 0.5
                vs = torch.rand(rows * self.NKV, device=dev, generator=gen) * 4 + 0.5
            self.kl.append((ik, kj, vj, ks, vs))
        self.layer = 0

    def launch(self, phase):
        A, p = self.A, self.plan
        if phase == self.phases[0]:
            self.layer = (self.layer + 1) % self.layers
        ik, kc, vc, ks, vs = self.kl[self.layer]
        if phase == "indexer":
            A.dispatch_lightning_indexer(p, self.index_q, ik, self.block_idx, self.scores)
        elif self.kv == "bq":
            A.dispatch_bq_block_sparse_attention(p, self.q, self.qb, self.fq, kc, ks, vc, vs,
                                                 self.block_idx, self.out, cap=128)
        else:
            A.dispatch_block_sparse_attention(p, self.q, kc, vc, self.block_idx, self.out)

    def dominant_bytes(self) -> int:
        """Indexer: every cached position's index key, the queries, the score
        rows written and read back, the page table."""
        B = len(self.pos)
        return (sum(p + 1 for p in self.pos) * self.HD * 2 + B * self.IH * self.HD * 2
                + 2 * self.scores.numel() * 4 + 4 * len(self.table.base_rows))

    def attended(self) -> int:
        """Positions the sparse attention reads per kv head: the local block and
        15 full blocks (every context here has more than 16 blocks)."""
        return sum(min(self.TOPK - 1, p // self.BLOCK) * self.BLOCK + p % self.BLOCK + 1
                   for p in self.pos)

    def step_bytes(self) -> int:
        B = len(self.pos)
        if self.kv == "bq":  # int8 codes + two f32 scales per position and kv head
            attn = (self.attended() * self.NKV * (self.HD * 2 + 8) + B * self.NQ * self.HD * 3
                    + B * self.NQ * 8 + B * self.IH * self.TOPK * 4)
        else:
            attn = (self.attended() * self.NKV * self.HD * 2 * 2
                    + B * self.NQ * self.HD * 2 * 2 + B * self.IH * self.TOPK * 4)
        return self.dominant_bytes() + attn

    def config(self) -> dict:
        return {"workload": self.name, "batch": len(self.pos),
                "indexed_positions": sum(p + 1 for p in self.pos),
                "attended_positions_per_kv_head": self.attended(), "pool_pages": self.pool,
                "page_len": self.PLEN, "num_q": self.NQ, "num_kv": self.NKV,
                "head_dim": self.HD, "index_heads": self.IH, "block": self.BLOCK,
                "topk_blocks": self.TOPK, "kv": self.kv, "seed": self.seed,
                "layer_caches": self.layers}

    def cpu_baseline(self, budget_s):
        """The oracle's indexer + block-sparse attention (one thread: the
        prototypes run them as single kernels) on the first n sequences of the
        batch (bf16 KV), n sized to the budget."""
        import torch

        if self.kv == "bq":
            return None

        import oracle

        hc = host_cpu()
        P, kvs = self.PLEN, self.NKV * self.HD
        scale = float(np.float32(1.0) / np.sqrt(np.float32(self.HD)))
        B = len(self.pos)

        def make(n):
            pages = np.concatenate([np.asarray(p) for p in self.pages[:n]])
            idx = torch.from_numpy(pages.astype(np.int64)).to(self.k.device)
            ik = self.index_k.view(-1, P * self.HD).index_select(0, idx).cpu().numpy()
            kp = self.k.view(-1, P * kvs).index_select(0, idx).cpu().numpy()
            vp = self.v.view(-1, P * kvs).index_select(0, idx).cpu().numpy()
            ik, kp, vp = (np.ascontiguousarray(x.view(np.uint16).reshape(-1))
                          for x in (ik, kp, vp))
            runs, rows, off = [], [], 0
            for i in range(n):
                m = len(self.pages[i])
                runs.append([i, self.pos[i], off, m])
                rows.extend((off + j) * P for j in range(m))
                off += m
            runs, rows = np.asarray(runs, dtype=np.int32), np.asarray(rows, dtype=np.int32)
            iq = self.index_q.cpu().numpy().view(np.uint16)[:n * self.IH * self.HD].copy()
            q = self.q.cpu().numpy().view(np.uint16)[:n * self.NQ * self.HD].copy()

            def call():
                bi, _ = oracle.lightning_indexer(runs, rows, iq, ik, num_heads=self.IH,
                                                 head_dim=self.HD, block_size=self.BLOCK,
                                                 topk=self.TOPK, local_blocks=1,
                                                 init_blocks=0, scale=scale, page_len=P,
                                                 seq_len=n)
                return bi, oracle.block_sparse_attention(
                    runs, rows, q, kp, vp, bi, num_q=self.NQ, num_kv=self.NKV,
                    head_dim=self.HD, kv_stride=kvs, block_size=self.BLOCK, topk=self.TOPK,
                    page_len=P, seq_len=n)
            return call

        def cost(n):
            return self.step_bytes() * sum(self.pos[:n]) / sum(self.pos)

        t = cpu_sample(make, B, cost, budget_s, 1)
        n, med = t["n"], t["median"]
        nbytes = cost(n)
        return cpu_result(hc, round(nbytes / med / 1e9, 3), "GB/s", 1, t,
                          f"first {n} of the {B} sequences ({n / B:.3f} of the batch by "
                          f"count, extrapolated by cached positions), indexer + sparse "
                          f"attention, one thread",
                          us_per_layer_equiv=round(med * 1e6 * sum(self.pos) /
                                                   sum(self.pos[:n]), 1))


class PrefillBf16:
    """Config 4: chunked prefill -- 8 sequences append 2048 tokens each onto
    prefixes ~ U[0, 16384]; sequences 2k and 2k+1 share one prefix, its sealed
    pages by reference and its partial last page by a copy-on-write page copy
    (ContinuousBatchScheduler.fork_prefix, continuous_batching/scheduler.mojo:
    395-466, copies at :427-436).  A step: the COW copies, the append (RoPE +
    cache write), then causal full-attention prefill over the paged prefix +
    chunk (MFMA).  Config 12 (widening): the same at Gemma-4's full-attention
    layer shape (16 q / 2 kv heads x 512, partial RoPE over 64 pairs at
    pair_stride 256; modeling/gemma4_common.mojo:14-20).  --kv bq: butterquant
    int8 KV (BqFlashPrefillFullKernel, butterquant_kernels/attention.mojo:
    267-351), the append being bq prep and the copy-on-write moving codes
    and scales."""

    phases = ("cow", "append", "attention")
    dominant_phase = "attention"
    bound = "mfma"

    def __init__(self, seed: int, config: int = 4, kv: str = "bf16"):
        self.seed, self.cfg, self.bq = seed, config, kv == "bq"
        self.dtype = ("int8 KV (f32 scales): int8 MFMA scores, bf16 MFMA P.V, f32 accumulate"
                      if self.bq else "bf16 (MFMA bf16 in, f32 accumulate)")
        shared = uniform_ints(seed, 4, 0, 16384)
        self.prefix = [p for p in shared for _ in range(2)]
        self.new = 2048
        if config == 12:
            self.nq, self.nkv, self.hd, self.half, self.pair = 16, 2, 512, 64, 256
            self.dominant = "prefill_wide_mfma_kernel"
            label = ("config12 (widening, Gemma-4 full-attention layer): chunked prefill, "
                     "8 sequences x 2048 new tokens on prefixes ~ U[0,16384] shared by "
                     "sequence pairs (sealed pages shared, the partial page copied on "
                     "write), 16q/2kv hd512 bf16, partial RoPE (half 64, pair_stride 256)")
        else:
            self.nq, self.nkv, self.hd, self.half, self.pair = 16, 8, 256, 128, 128
            self.dominant = "prefill_full_mfma_kernel"
            label = ("config4: chunked prefill, 8 sequences x 2048 new tokens on prefixes "
                     "~ U[0,16384] shared by sequence pairs (sealed pages shared, the partial "
                     "page copied on write), 16q/8kv hd256 bf16")
        self.kvs = self.nkv * self.hd
        if self.bq:
            self.dominant += "<bq>"
            label = label.replace(" bf16", " butterquant int8 KV (f32 scales)")
        self.name = label + (", 64-token pages, COW copy + append + causal MFMA prefill "
                             "over the paged prefix and chunk")

    def setup(self, dev, a):
        import torch

        from inferno_amd import attention as A
        from inferno_amd.kv import AttentionPlan, KVRunTable

        self.A = A
        n_seq = len(self.prefix)
        # Page ordinals per sequence; the second of a pair takes the first's
        # sealed prefix pages and owns the rest (its partial prefix page is the
        # COW copy).
        rng = np.random.default_rng(self.seed)
        owned, tables = [], []
        for i, p in enumerate(self.prefix):
            n_ord = (p + self.new + PAGE_LEN - 1) // PAGE_LEN
            n_shared = p // PAGE_LEN if i % 2 == 1 else 0
            owned.append(n_ord - n_shared)
            tables.append([None] * n_shared + [0] * (n_ord - n_shared))
        pool = sum(owned)
        perm = [int(x) for x in rng.permutation(pool)]
        off = 0
        for i in range(n_seq):
            t = tables[i]
            for o in range(len(t)):
                if t[o] is None:
                    t[o] = tables[i - 1][o]
                else:
                    t[o] = perm[off]
                    off += 1
        table = KVRunTable()
        for i, p in enumerate(self.prefix):
            table.begin_run(i * self.new, p)
            for pg in tables[i]:
                table.add_base_row(pg * PAGE_LEN)
        n = n_seq * self.new
        rows = pool * PAGE_LEN
        self.pool, self.table, self.n, self.tables = pool, table, n, tables
        self.stream = torch.cuda.current_stream()
        sid = int(self.stream.cuda_stream)
        # K and V share one arena, as the reference's KV mirror lays the
        # components out, so the copy jobs address both with byte offsets.
        cdt = torch.int8 if self.bq else torch.int16
        self.arena = torch.empty(2 * rows * self.kvs, dtype=cdt, device=dev)
        self.k = self.arena[:rows * self.kvs]
        self.v = self.arena[rows * self.kvs:]
        if self.bq:
            # Scales [row][kv head] of K then V, one arena for their COW copies.
            gen = torch.Generator(device=dev)
            gen.manual_seed(self.seed)
            self.sarena = torch.rand(2 * rows * self.nkv, device=dev, generator=gen) * 4 + 0.5
            self.ksc = self.sarena[:rows * self.nkv]
            self.vsc = self.sarena[rows * self.nkv:]
            self.gain = torch.full((self.hd,), 0x3F80, dtype=torch.int16, device=dev)
            self.q_i8 = torch.empty(n * self.nq * self.hd, dtype=torch.int8, device=dev)
            self.qb = torch.empty(n * self.nq, dtype=torch.float32, device=dev)
            self.fq = torch.empty_like(self.qb)
        self.q = torch.empty(n * self.nq * self.hd, dtype=torch.int16, device=dev)
        self.ks = torch.empty(n * self.kvs, dtype=torch.int16, device=dev)
        self.vs = torch.empty_like(self.ks)
        for i, t in enumerate((self.k, self.v, self.q, self.ks, self.vs)):
            _fill(t, self.seed * 16 + i, sid)
        # COW jobs: rows [0, p % 64) of the first's partial prefix page into the
        # second's own page at the same ordinal, for K and V
        # (append_prefix_copy_jobs, modeling/kv_policy.mojo:59-78).
        row_bytes = self.kvs * (1 if self.bq else 2)
        v_base = rows * row_bytes
        jobs, sjobs = [], []
        for i in range(1, n_seq, 2):
            p = self.prefix[i]
            if p % PAGE_LEN == 0:
                continue
            o = p // PAGE_LEN
            src, dst = tables[i - 1][o] * PAGE_LEN, tables[i][o] * PAGE_LEN
            nb = (p % PAGE_LEN) * row_bytes
            for base in (0, v_base):
                jobs.append([base + src * row_bytes, base + dst * row_bytes, nb])
            if self.bq:
                sb = self.nkv * 4
                for base in (0, rows * sb):
                    sjobs.append([base + src * sb, base + dst * sb, (p % PAGE_LEN) * sb])
        self.jobs = np.asarray(jobs + sjobs, dtype=np.int64).reshape(-1, 3)
        self.cow = CopyStager(np.asarray(jobs, dtype=np.int64).reshape(-1, 3), dev) \
            if len(jobs) else None
        self.scow = CopyStager(np.asarray(sjobs, dtype=np.int64).reshape(-1, 3), dev) \
            if len(sjobs) else None
        cos, sin = rope_tables(max(self.prefix) + self.new + 1, self.half)
        self.cos, self.sin = torch.from_numpy(cos).to(dev), torch.from_numpy(sin).to(dev)
        if self.bq:
            # The cached prefixes as the configuration produces them: N(0,1) K/V
            # with 1 % outliers x20 through the quantizing append.  A pair's
            # second sequence reads the first's sealed pages and the copy of its
            # partial page, so the first sequence of each pair is filled.
            self.data = DecodeBq.data
            self.bq_k, self.bq_ks, self.bq_v, self.bq_vs = self.k, self.ksc, self.v, self.vsc
            bq_quantize_cache(self, dev, [(0, self.prefix[i], tables[i])
                                          for i in range(0, n_seq, 2)],
                              kind=1, cache_size=PAGE_LEN, cache_rows=rows,
                              v_is_k=self.cfg == 12, seed=self.seed * 16 + 8)
        self.plan = AttentionPlan(table, n, kind=1, window=0, cache_size=PAGE_LEN,
                                  page_len=PAGE_LEN, cache_rows=rows, cap=a.cap,
                                  kv_row_bytes=self.kvs * (1 if self.bq else 2), device=dev)
        self.partials, self.ps = A.partials_buffer(self.plan, self.nq, self.hd)
        self.out = torch.empty(n * self.nq * self.hd, dtype=torch.int16, device=dev)
        self.cap = a.cap

    def launch(self, phase):
        A, p = self.A, self.plan
        if phase == "cow":
            if self.cow is not None:
                self.cow(self.arena, self.stream)
            if self.bq and self.scow is not None:
                self.scow(self.sarena, self.stream)
        elif self.bq and phase == "append":
            # The full layer's V is its raw K projection (gemma_4_moe_bq.mojo:566-573).
            vsrc = self.ks if self.cfg == 12 else self.vs
            A.dispatch_bq_attn_prep(p, self.q, self.ks, vsrc, self.gain, self.gain, self.q_i8,
                                    self.qb, self.fq, self.k, self.ksc, self.v, self.vsc,
                                    self.cos, self.sin, num_q=self.nq, num_kv=self.nkv,
                                    head_dim=self.hd, rope_half=self.half,
                                    pair_stride=self.pair,
                                    sqrt_n=float(np.sqrt(np.float32(self.hd))),
                                    n_eps=float(np.float32(self.hd) * np.float32(1e-6)))
        elif self.bq:
            A.bq_attention(p, self.q_i8, self.qb, self.fq, self.k, self.ksc, self.v, self.vsc,
                           self.out, self.partials, self.ps, num_q=self.nq, num_kv=self.nkv,
                           head_dim=self.hd, kv_stride=self.kvs)
        elif phase == "append":
            A.dispatch_rope_cache_write(p, self.q, self.ks, self.vs, self.k, self.v, self.cos,
                                        self.sin, num_q=self.nq, num_kv=self.nkv,
                                        half=self.half, pair_stride=self.pair, head_dim=self.hd)
        else:
            A.attention_bf16(p, self.q, self.k, self.v, self.out, self.partials, self.ps,
                             num_q=self.nq, num_kv=self.nkv, head_dim=self.hd,
                             kv_stride=self.kvs)

    def flops(self) -> int:
        """4 * D * Hq * sum over query tokens of attended keys (QK^T + PV)."""
        keys = sum(sum(p + t + 1 for t in range(self.new)) for p in self.prefix)
        return 4 * self.hd * self.nq * keys

    def step_bytes(self) -> int:
        cow = 2 * int(self.jobs[:, 2].sum()) if self.jobs.size else 0
        if self.bq:  # bf16 q/k/v in, codes out; bf16 output
            return self.n * ((self.nq + 2 * self.nkv) * self.hd * 3 +
                             self.nq * self.hd * 2) + cow
        return self.n * (self.kvs * 2 * 2 * 2 + self.nq * self.hd * 2 * 3) + cow

    def dominant_bytes(self) -> int:
        return 0

    def config(self) -> dict:
        return {"workload": self.name, "sequences": len(self.prefix), "new_tokens": self.new,
                "prefixes": self.prefix, "pool_pages": self.pool, "page_len": PAGE_LEN,
                "shared_pages": sum(p // PAGE_LEN for p in self.prefix[1::2]),
                "cow_jobs": int(self.jobs.shape[0]),
                "cow_bytes": int(self.jobs[:, 2].sum()) if self.jobs.size else 0,
                "num_q": self.nq, "num_kv": self.nkv, "head_dim": self.hd, "cap": self.cap,
                "seed": self.seed, "query_blocks": int(self.plan.info[14]),
                "algorithmic_tflop": round(self.flops() / 1e12, 3)}

    def cpu_baseline(self, budget_s):
        """The oracle's token route (FlashPrefillFullKernel + PrefillMergeKernel,
        or BqFlashPrefillFullKernel) over the last n query tokens of the longest
        sequence (the most keys per token), n sized to the budget."""
        import torch

        import oracle

        hc = host_cpu()
        threads = hc["threads"]
        i = int(np.argmax(self.prefix))
        p0 = self.prefix[i]
        pages = np.asarray(self.tables[i], dtype=np.int64)
        npage = pages.size
        idx = torch.from_numpy(pages).to(self.k.device)

        def sel(t, per_row):
            return np.ascontiguousarray(
                t.view(-1, PAGE_LEN * per_row).index_select(0, idx).cpu().numpy()).reshape(-1)

        kp, vp = sel(self.k, self.kvs), sel(self.v, self.kvs)
        if self.bq:
            ksp, vsp = sel(self.ksc, self.nkv), sel(self.vsc, self.nkv)
        else:
            kp, vp = kp.view(np.uint16), vp.view(np.uint16)
        base = np.arange(npage, dtype=np.int32) * PAGE_LEN

        def make(n):
            first = self.new - n
            runs = np.asarray([[0, p0 + first, 0, npage]], dtype=np.int32)
            t0_, t1_ = i * self.new + first, (i + 1) * self.new
            if not self.bq:
                qh = np.ascontiguousarray(self.q.view(-1, self.nq * self.hd)[t0_:t1_].cpu()
                                          .numpy().view(np.uint16).reshape(-1))
                return lambda: oracle.attention(
                    1, runs, base, qh, kp, vp, num_q=self.nq, num_kv=self.nkv,
                    head_dim=self.hd, kv_stride=self.kvs, window=0, cache_size=PAGE_LEN,
                    page_len=PAGE_LEN, seq_len=n, cap=threads, threads=threads)
            qh = np.ascontiguousarray(
                self.q_i8.view(-1, self.nq * self.hd)[t0_:t1_].cpu().numpy()).reshape(-1)
            qb = np.ascontiguousarray(self.qb.view(-1, self.nq)[t0_:t1_].cpu().numpy())
            fq = np.ascontiguousarray(self.fq.view(-1, self.nq)[t0_:t1_].cpu().numpy())
            return lambda: oracle.bq_attention(
                1, runs, base, qh, qb.reshape(-1), fq.reshape(-1), kp, ksp, vp, vsp,
                num_q=self.nq, num_kv=self.nkv, head_dim=self.hd, kv_stride=self.kvs,
                window=0, cache_size=PAGE_LEN, page_len=PAGE_LEN, seq_len=n, cap=threads,
                threads=threads)

        def cost(n):
            first = self.new - n
            return 4 * self.hd * self.nq * sum(p0 + first + t + 1 for t in range(n))

        t = cpu_sample(make, self.new, cost, budget_s, 16)
        n, med = t["n"], t["median"]
        fl = cost(n)
        route = "bq token route" if self.bq else "token route"
        return cpu_result(hc, round(fl / med / 1e12, 5), "TFLOP/s", threads, t,
                          f"last {n} query tokens of the longest sequence "
                          f"({fl // (4 * self.hd * self.nq)} query-key pairs), the reference's "
                          f"{route} at cap={threads} workers",
                          us_per_layer_equiv=round(med * 1e6 * self.flops() / fl, 1))

class PrefillSliding:
    """Config 11 (widening): chunked prefill of a sliding-window layer --
    8 sequences append 2048 tokens each onto prefixes ~ U[0, 16384], each
    sequence on its own 64-page ring (4096 positions, enough for the chunk
    and its window), then the sliding prefill over window 1024
    (FlashPrefillSlidingKernel, kernels/flash_attention_prefill.mojo:18-114),
    on MFMA when the window is a multiple of 16.  --kv bq: the butterquant
    layer (BqFlashPrefillSlidingKernel, butterquant_kernels/attention.mojo:
    170-264), the append being bq prep (codes and scales of the chunk into
    the ring, q codes)."""

    phases = ("append", "attention")
    dominant_phase = "attention"
    bound = "mfma"
    RING = 64

    def __init__(self, seed: int, window: int, kv: str = "bf16"):
        self.seed, self.window, self.bq = seed, window, kv == "bq"
        self.nq, self.nkv, self.hd, self.half, self.pair = NUM_Q, NUM_KV, HEAD_DIM, 128, 128
        self.kvs = KV_STRIDE
        self.prefix = uniform_ints(seed, 8, 0, 16384)
        self.new = 2048
        if self.bq:
            self.dtype = "int8 KV (f32 scales): int8 MFMA scores, bf16 MFMA P.V, f32 accumulate"
            self.dominant = "prefill_sliding_mfma_kernel<bq>"
            kind = ("butterquant int8 KV (f32 scales per position and kv head), bq prep + "
                    "causal sliding prefill")
        else:
            self.dtype = "bf16 (MFMA bf16 in, f32 accumulate)"
            self.dominant = "prefill_sliding_mfma_kernel"
            kind = "bf16, append + causal sliding prefill"
        self.name = (f"config11 (widening): sliding-window chunked prefill, 8 sequences x 2048 "
                     f"new tokens on prefixes ~ U[0,16384], window {window}, 64-page rings of "
                     f"64-token pages, 16q/8kv hd256 {kind}")

    def setup(self, dev, a):
        import torch

        from inferno_amd import attention as A
        from inferno_amd.kv import AttentionPlan, KVRunTable

        self.A = A
        n_seq = len(self.prefix)
        perm = np.random.default_rng(self.seed).permutation(n_seq * self.RING)
        table = KVRunTable()
        for i, p in enumerate(self.prefix):
            table.begin_run(i * self.new, p)
            for x in perm[i * self.RING:(i + 1) * self.RING]:
                table.add_base_row(int(x) * PAGE_LEN)
        n = n_seq * self.new
        rows = n_seq * self.RING * PAGE_LEN
        self.table, self.n = table, n
        self.stream = torch.cuda.current_stream()
        sid = int(self.stream.cuda_stream)
        cdt = torch.int8 if self.bq else torch.int16
        self.k = torch.empty(rows * KV_STRIDE, dtype=cdt, device=dev)
        self.v = torch.empty_like(self.k)
        self.q = torch.empty(n * NUM_Q * HEAD_DIM, dtype=torch.int16, device=dev)
        self.ks = torch.empty(n * KV_STRIDE, dtype=torch.int16, device=dev)
        self.vs = torch.empty_like(self.ks)
        for i, t in enumerate((self.k, self.v, self.q, self.ks, self.vs)):
            _fill(t, self.seed * 16 + i, sid)
        if self.bq:
            gen = torch.Generator(device=dev)
            gen.manual_seed(self.seed)
            self.ksc = torch.rand(rows * NUM_KV, device=dev, generator=gen) * 4 + 0.5
            self.vsc = torch.rand(rows * NUM_KV, device=dev, generator=gen) * 4 + 0.5
            self.gain = torch.full((HEAD_DIM,), 0x3F80, dtype=torch.int16, device=dev)
            self.q_i8 = torch.empty(n * NUM_Q * HEAD_DIM, dtype=torch.int8, device=dev)
            self.qb = torch.empty(n * NUM_Q, dtype=torch.float32, device=dev)
            self.fq = torch.empty_like(self.qb)
        cos, sin = rope_tables(max(self.prefix) + self.new + 1)
        self.cos, self.sin = torch.from_numpy(cos).to(dev), torch.from_numpy(sin).to(dev)
        if self.bq:
            # The ring positions the chunk's windows reach back to, quantized
            # from N(0,1) K/V with 1 % outliers x20 through the append path.
            self.data = DecodeBq.data
            self.bq_k, self.bq_ks, self.bq_v, self.bq_vs = self.k, self.ksc, self.v, self.vsc
            rings = [perm[i * self.RING:(i + 1) * self.RING] for i in range(n_seq)]
            bq_quantize_cache(self, dev, [(max(0, p - self.new), p - max(0, p - self.new), rg)
                                          for p, rg in zip(self.prefix, rings)],
                              kind=0, cache_size=self.RING * PAGE_LEN, cache_rows=rows,
                              v_is_k=False, seed=self.seed * 16 + 8)
        self.plan = AttentionPlan(table, n, kind=0, window=self.window,
                                  cache_size=self.RING * PAGE_LEN, page_len=PAGE_LEN,
                                  cache_rows=rows, cap=a.cap,
                                  kv_row_bytes=KV_STRIDE * (1 if self.bq else 2), device=dev)
        self.partials, self.ps = A.partials_buffer(self.plan, NUM_Q, HEAD_DIM)
        self.out = torch.empty(n * NUM_Q * HEAD_DIM, dtype=torch.int16, device=dev)
        self.cap = a.cap
        if int(self.plan.info[14]) == 0:
            self.dominant = ("bq_partial_kernel (token route) + merge_kernel" if self.bq else
                             "flash_partial_bf16_kernel (token route) + merge_kernel")

    def launch(self, phase):
        A, p = self.A, self.plan
        if self.bq and phase == "append":
            A.dispatch_bq_attn_prep(p, self.q, self.ks, self.vs, self.gain, self.gain,
                                    self.q_i8, self.qb, self.fq, self.k, self.ksc, self.v,
                                    self.vsc, self.cos, self.sin, num_q=NUM_Q, num_kv=NUM_KV,
                                    head_dim=HEAD_DIM, rope_half=128, pair_stride=128,
                                    sqrt_n=float(np.sqrt(np.float32(HEAD_DIM))),
                                    n_eps=float(np.float32(HEAD_DIM) * np.float32(1e-6)))
        elif self.bq:
            A.bq_attention(p, self.q_i8, self.qb, self.fq, self.k, self.ksc, self.v, self.vsc,
                           self.out, self.partials, self.ps, num_q=NUM_Q, num_kv=NUM_KV,
                           head_dim=HEAD_DIM, kv_stride=KV_STRIDE)
        elif phase == "append":
            A.dispatch_rope_cache_write(p, self.q, self.ks, self.vs, self.k, self.v, self.cos,
                                        self.sin, num_q=NUM_Q, num_kv=NUM_KV, half=128,
                                        pair_stride=128, head_dim=HEAD_DIM)
        else:
            A.attention_bf16(p, self.q, self.k, self.v, self.out, self.partials, self.ps,
                             num_q=NUM_Q, num_kv=NUM_KV, head_dim=HEAD_DIM,
                             kv_stride=KV_STRIDE)

    def flops(self) -> int:
        """4 * D * Hq * sum over query tokens of attended keys (QK^T + PV)."""
        keys = sum(sum(min(p + t + 1, self.window) for t in range(self.new))
                   for p in self.prefix)
        return 4 * HEAD_DIM * NUM_Q * keys

    def step_bytes(self) -> int:
        if self.bq:  # bf16 q/k/v in, codes out; bf16 output
            return self.n * ((NUM_Q + 2 * NUM_KV) * HEAD_DIM * 3 + NUM_Q * HEAD_DIM * 2)
        return self.n * (KV_STRIDE * 2 * 2 * 2 + NUM_Q * HEAD_DIM * 2 * 3)

    def dominant_bytes(self) -> int:
        return 0

    def config(self) -> dict:
        return {"workload": self.name, "sequences": len(self.prefix), "new_tokens": self.new,
                "prefixes": self.prefix, "window": self.window, "ring_pages": self.RING,
                "page_len": PAGE_LEN, "num_q": NUM_Q, "num_kv": NUM_KV, "head_dim": HEAD_DIM,
                "cap": self.cap, "seed": self.seed, "query_blocks": int(self.plan.info[14]),
                "algorithmic_tflop": round(self.flops() / 1e12, 3)}

    def cpu_baseline(self, budget_s):
        """The oracle's sliding token route (FlashPrefillSlidingKernel, or
        BqFlashPrefillSlidingKernel) over the last n query tokens of the first
        sequence, n sized to the budget."""
        import torch

        import oracle

        hc = host_cpu()
        threads = hc["threads"]
        p0 = self.prefix[0]
        pages = np.asarray(self.table.base_rows[:self.RING], dtype=np.int64) // PAGE_LEN
        idx = torch.from_numpy(pages).to(self.k.device)

        def sel(t, per_row):
            return np.ascontiguousarray(
                t.view(-1, PAGE_LEN * per_row).index_select(0, idx).cpu().numpy()).reshape(-1)

        kp, vp = sel(self.k, KV_STRIDE), sel(self.v, KV_STRIDE)
        if self.bq:
            ksp, vsp = sel(self.ksc, NUM_KV), sel(self.vsc, NUM_KV)
        else:
            kp, vp = kp.view(np.uint16), vp.view(np.uint16)
        base = np.arange(self.RING, dtype=np.int32) * PAGE_LEN
        geo = dict(num_q=NUM_Q, num_kv=NUM_KV, head_dim=HEAD_DIM, kv_stride=KV_STRIDE,
                   window=self.window, cache_size=self.RING * PAGE_LEN, page_len=PAGE_LEN,
                   cap=threads, threads=threads)

        def make(n):
            first = self.new - n
            runs = np.asarray([[0, p0 + first, 0, self.RING]], dtype=np.int32)
            if not self.bq:
                qh = np.ascontiguousarray(self.q.view(-1, NUM_Q * HEAD_DIM)[first:self.new]
                                          .cpu().numpy().view(np.uint16).reshape(-1))
                return lambda: oracle.attention(0, runs, base, qh, kp, vp, seq_len=n, **geo)
            qh = np.ascontiguousarray(
                self.q_i8.view(-1, NUM_Q * HEAD_DIM)[first:self.new].cpu().numpy()).reshape(-1)
            qb = np.ascontiguousarray(self.qb.view(-1, NUM_Q)[first:self.new].cpu().numpy())
            fq = np.ascontiguousarray(self.fq.view(-1, NUM_Q)[first:self.new].cpu().numpy())
            return lambda: oracle.bq_attention(0, runs, base, qh, qb.reshape(-1),
                                               fq.reshape(-1), kp, ksp, vp, vsp, seq_len=n,
                                               **geo)

        def cost(n):
            first = self.new - n
            return 4 * HEAD_DIM * NUM_Q * sum(min(p0 + first + t + 1, self.window)
                                              for t in range(n))

        t = cpu_sample(make, self.new, cost, budget_s, 16)
        n, med = t["n"], t["median"]
        fl = cost(n)
        route = "bq sliding token route" if self.bq else "sliding token route"
        return cpu_result(hc, round(fl / med / 1e12, 5), "TFLOP/s", threads, t,
                          f"last {n} query tokens of the first sequence "
                          f"({fl // (4 * HEAD_DIM * NUM_Q)} query-key pairs), the reference's "
                          f"{route} at cap={threads} workers",
                          us_per_layer_equiv=round(med * 1e6 * self.flops() / fl, 1))

class PageCopyBench:
    """Config 9 (widening): dispatch_copy_jobs (kernels/page_copy.mojo:63-94) as
    copy-on-write of bf16 pages of the 16q/8kv hd256 cache: 2048 page copies
    per component (K and V) between shuffled pages of one arena, every fourth a
    partial page of 1-63 rows (a fork's divergent page).  The timed dispatch
    includes the job list's upload."""

    dtype = "bytes"
    phases = ("copy",)
    dominant = "copy dispatch (job-list upload + copy_chunks_kernel)"
    dominant_phase = "copy"

    def __init__(self, seed: int):
        self.seed = seed
        self.copies = 2048
        self.name = ("config9 (widening): copy-on-write page copy, 2048 page copies per K/V "
                     "component of a 16q/8kv hd256 bf16 cache (256 KiB pages), every 4th a "
                     "partial page of 1-63 rows, shuffled source/destination pages of one "
                     "arena, dispatch_copy_jobs")

    def setup(self, dev, a):
        import torch

        rng = np.random.default_rng(self.seed)
        row_bytes = KV_STRIDE * 2
        page_bytes = PAGE_LEN * row_bytes
        pages = 2 * self.copies  # per component: sources, then destinations
        comp = pages * page_bytes
        self.stream = torch.cuda.current_stream()
        self.arena = torch.empty(2 * comp, dtype=torch.uint8, device=dev)
        _fill(self.arena, self.seed * 16 + 1, int(self.stream.cuda_stream))
        src = rng.permutation(self.copies)
        dst = self.copies + rng.permutation(self.copies)
        nrows = np.where(np.arange(self.copies) % 4 == 3,
                         rng.integers(1, PAGE_LEN, self.copies), PAGE_LEN)
        jobs = []
        for c in range(2):
            for j in range(self.copies):
                jobs.append([c * comp + int(src[j]) * page_bytes,
                             c * comp + int(dst[j]) * page_bytes, int(nrows[j]) * row_bytes])
        self.jobs = np.asarray(jobs, dtype=np.int64)
        self.stager = CopyStager(self.jobs, dev)
        self.cap = 0

    def launch(self, phase):
        self.stager(self.arena, self.stream)

    def dominant_bytes(self) -> int:
        return 2 * self.stager.copied_bytes  # read + write

    def step_bytes(self) -> int:
        return self.dominant_bytes()

    def config(self) -> dict:
        return {"workload": self.name, "jobs": int(self.jobs.shape[0]),
                "copied_bytes": self.stager.copied_bytes, "page_len": PAGE_LEN,
                "row_bytes": KV_STRIDE * 2, "seed": self.seed}

    def cpu_baseline(self, budget_s):
        """The oracle's fanned-out copy (dispatch_copy_jobs: 64-byte aligned
        worker shares of the concatenated jobs, one PageCopyKernel per worker)
        over the first n jobs remapped into a compact host arena, on the worker
        threads; n is every job when the timed calls fit the budget."""
        import oracle

        hc = host_cpu()
        threads = hc["threads"]
        total = self.jobs.shape[0]
        page_bytes = PAGE_LEN * KV_STRIDE * 2

        def make(n):
            jobs = np.empty((n, 3), dtype=np.int64)
            jobs[:, 0] = np.arange(n) * page_bytes
            jobs[:, 1] = (n + np.arange(n)) * page_bytes
            jobs[:, 2] = self.jobs[:n, 2]
            arena = np.ones(2 * n * page_bytes, dtype=np.uint8)

            def call():
                oracle.copy_jobs_workers(arena, jobs, threads, threads)
                return None
            call()  # first touch of every page
            return call

        def cost(n):
            return 2 * int(self.jobs[:n, 2].sum())

        t = cpu_sample(make, total, cost, budget_s, min(total, 64))
        n, med = t["n"], t["median"]
        nbytes = cost(n)
        return cpu_result(hc, round(nbytes / med / 1e9, 3), "GB/s", threads, t,
                          f"{'all' if n == total else 'the first'} {n} of the {total} jobs "
                          f"({nbytes / 2e6:.1f} MB copied) in a compact host arena, "
                          f"{threads} worker shares on {threads} threads")

class GatherBench:
    """Config 10 (widening): dispatch_gather_rows (kernels/gather.mojo:30-55)
    of bf16 hidden rows (cols = Gemma-4's 2816): 16384 of 65536 rows in a
    seeded random order."""

    dtype = "bytes"
    phases = ("gather",)
    dominant = "gather_rows_kernel"
    dominant_phase = "gather"
    SRC_ROWS, ROWS, COLS = 65536, 16384, HIDDEN

    def __init__(self, seed: int):
        self.seed = seed
        self.name = ("config10 (widening): row gather, 16384 of 65536 bf16 hidden rows "
                     "(cols 2816, the emit-row gather of stage_sampling_inputs at prefill "
                     "scale), seeded random order, dispatch_gather_rows")

    def setup(self, dev, a):
        import torch

        from inferno_amd import attention as A

        self.A = A
        self.stream = torch.cuda.current_stream()
        self.src = torch.empty(self.SRC_ROWS * self.COLS, dtype=torch.int16, device=dev)
        _fill(self.src, self.seed * 16 + 1, int(self.stream.cuda_stream))
        rows = np.random.default_rng(self.seed).choice(self.SRC_ROWS, self.ROWS, replace=False)
        self.rows_host = rows.astype(np.int32)
        self.rows = torch.from_numpy(self.rows_host).to(dev)
        self.dst = torch.empty(self.ROWS * self.COLS, dtype=torch.int16, device=dev)
        self.cap = 0

    def launch(self, phase):
        self.A.dispatch_gather_rows(self.src, self.dst, self.rows, self.ROWS, self.COLS)

    def dominant_bytes(self) -> int:
        return 2 * self.ROWS * self.COLS * 2 + 4 * self.ROWS

    def step_bytes(self) -> int:
        return self.dominant_bytes()

    def config(self) -> dict:
        return {"workload": self.name, "rows": self.ROWS, "source_rows": self.SRC_ROWS,
                "cols": self.COLS, "seed": self.seed}

    def cpu_baseline(self, budget_s):
        """The oracle's fanned-out gather (dispatch_gather_rows: worker_range
        shares of the rows) of the first n rows on the worker threads, n every
        row when the timed calls fit the budget."""
        import oracle

        hc = host_cpu()
        threads = hc["threads"]
        src = self.src.cpu().numpy().view(np.uint16)

        def make(n):
            rows = np.ascontiguousarray(self.rows_host[:n])
            dst = np.zeros(n * self.COLS, dtype=np.uint16)
            return lambda: oracle.gather_rows_workers(src, rows, self.COLS, threads, threads,
                                                      dst=dst)

        def cost(n):
            return 2 * n * self.COLS * 2

        t = cpu_sample(make, self.ROWS, cost, budget_s, min(self.ROWS, 1024))
        n, med = t["n"], t["median"]
        nbytes = cost(n)
        return cpu_result(hc, round(nbytes / med / 1e9, 3), "GB/s", threads, t,
                          f"{'all' if n == self.ROWS else 'the first'} {n} of the {self.ROWS} "
                          f"rows, {threads} worker shares on {threads} threads")

class PhaseEvents:
    """HIP timing events created with hipEventDisableSystemFence, recorded on
    the launch stream.  A default event (torch.cuda.Event) ends with a
    system-scope fence whose cache writeback and invalidation slow the kernel
    that follows it (config 11's sliding prefill: about 800 instead of 700 us
    after an event, 700 us when launched right after the append, as rocprofv3
    shows for both); these events time the phases as they run back to back.
    The runtime is the HIP library torch has loaded (one per process)."""

    DISABLE_SYSTEM_FENCE = 0x20000000

    def __init__(self, stream):
        import ctypes

        self.ct = ctypes
        self.hip = ctypes.CDLL("libamdhip64.so.7")
        self.stream = ctypes.c_void_p(int(stream.cuda_stream))
        self.events = []

    def _check(self, rc, what):
        if rc != 0:
            raise RuntimeError(f"{what} failed with hipError {rc}")

    def record(self):
        ev = self.ct.c_void_p()
        self._check(self.hip.hipEventCreateWithFlags(self.ct.byref(ev),
                                                     self.ct.c_uint(self.DISABLE_SYSTEM_FENCE)),
                    "hipEventCreateWithFlags")
        self._check(self.hip.hipEventRecord(ev, self.stream), "hipEventRecord")
        self.events.append(ev)
        return ev

    def elapsed_us(self, a, b) -> float:
        ms = self.ct.c_float()
        self._check(self.hip.hipEventElapsedTime(self.ct.byref(ms), a, b), "hipEventElapsedTime")
        return ms.value * 1e3

    def close(self):
        for ev in self.events:
            self.hip.hipEventDestroy(ev)
        self.events = []


def measure(w, steps: int, warmup: int, graph: bool):
    """Returns the wall time of K eager steps, of K steps replayed from a HIP
    graph (None unless graph), and per-phase HIP-event times."""
    import torch

    stream = w.stream
    timed = getattr(w, "timed_phases", w.phases)

    def step():
        for ph in timed:
            w.launch(ph)

    for _ in range(warmup):
        step()
    torch.cuda.synchronize()
    # Past the W warmup steps, keep stepping (untimed) until at least 0.2 s of
    # work has run, so that a step of a few microseconds (config 1) is timed
    # at steady clocks rather than on a GPU still leaving its idle state.
    t_warm = time.perf_counter()
    while time.perf_counter() - t_warm < 0.2:
        for _ in range(8):
            step()
        torch.cuda.synchronize()
    # Timed region 1: wall clock over K steps, nothing but the step's launches
    # (each a C-ABI call from Python).
    t0 = time.perf_counter()
    for _ in range(steps):
        step()
    torch.cuda.synchronize()
    wall = time.perf_counter() - t0
    # Timed region 2: the same K steps captured once in a HIP graph (the same
    # C-ABI calls, recorded on torch's capture stream) and replayed: the GPU
    # time of the step without the host's per-launch cost, as a serving loop
    # that captures a layer's decode runs it.
    wall_graph = None
    if graph:
        g = torch.cuda.CUDAGraph()
        with torch.cuda.graph(g):
            for _ in range(steps):
                step()
        for _ in range(2):
            g.replay()
        torch.cuda.synchronize()
        t0 = time.perf_counter()
        g.replay()
        torch.cuda.synchronize()
        wall_graph = time.perf_counter() - t0
        del g
    # Timed region 3: K steps phase by phase with HIP events between them
    # (events without the system-scope fence; see PhaseEvents).
    n = len(w.phases)
    pe = PhaseEvents(stream)
    torch.cuda.synchronize()
    evs = []
    for i in range(steps):
        row = [pe.record()]
        for ph in w.phases:
            w.launch(ph)
            row.append(pe.record())
        evs.append(row)
    torch.cuda.synchronize()
    per = {ph: statistics.mean(pe.elapsed_us(e[j], e[j + 1]) for e in evs)
           for j, ph in enumerate(w.phases)}
    per["step"] = statistics.mean(pe.elapsed_us(e[0], e[n]) for e in evs)
    pe.close()
    return wall, wall_graph, per


def copy_calibration(dev) -> None:
    import torch

    n = 1 << 30
    src = torch.ones(n, dtype=torch.uint8, device=dev)
    dst = torch.empty_like(src)
    torch.cuda.synchronize()
    dst.copy_(src)
    torch.cuda.synchronize()
    print(json.dumps({"copy_calibration_bytes": n, "read_kib": n // 1024,
                      "write_kib": n // 1024}))


def main() -> None:
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=50)
    ap.add_argument("--warmup", type=int, default=5)
    ap.add_argument("--config", type=int, default=2, choices=tuple(range(1, 13)))
    ap.add_argument("--window", type=int, default=1024,
                    help="config 11: sliding window (a multiple of 16 takes the MFMA kernel)")
    ap.add_argument("--cap", type=int, default=0, help="worker capacity (0: per-config default)")
    ap.add_argument("--seed", type=int, default=20241)
    ap.add_argument("--cpu-budget", type=float, default=20.0)
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--norm", choices=("none", "separate", "fused"), default="none",
                    help="configs 1-3: head RMS norm of q/k/v ahead of the append, as its "
                         "own pass or fused into the append kernel")
    ap.add_argument("--kv", choices=("bf16", "bq"), default="bf16",
                    help="configs 4, 6, 11 and 12: bf16 or butterquant int8 KV")
    ap.add_argument("--oproj", action="store_true",
                    help="configs 1-3: the bf16 o_proj GEMM after the merge")
    ap.add_argument("--oquant", choices=("none", "separate", "fused"), default="none",
                    help="config 5: int8 block quant of the attention output for o_proj, "
                         "as its own pass or fused into the merge")
    ap.add_argument("--launch", choices=("graph", "eager"), default="graph",
                    help="decode configs: time the K steps replayed from a HIP graph "
                         "(default; the eager per-call figure is reported beside it) or "
                         "as eager C-ABI calls")
    ap.add_argument("--copy-calibration", action="store_true",
                    help="one 1 GiB device-to-device copy (torch's copy kernel): the "
                         "known-size reference for scaling rocprofv3 FETCH_SIZE/WRITE_SIZE")
    a = ap.parse_args()
    if a.gpus != 1:
        print(f"bench.py measures one GPU: every GPU box in this build has one MI355X, "
              f"so --gpus {a.gpus} is not run (the path shards by sequence; see DESIGN.md).",
              file=sys.stderr)
        sys.exit(2)
    import torch

    dev = torch.device("cuda:0")
    torch.cuda.set_device(dev)
    if a.copy_calibration:
        copy_calibration(dev)
        return
    if a.cap <= 0 and DEFAULT_CAP[a.config] > 0:
        a.cap = DEFAULT_CAP[a.config]
    if a.config == 6:
        w = SparseM3(a.seed)
    elif a.config in (5, 8):
        w = DecodeBq(a.config, a.seed)
    elif a.config in (4, 12):
        w = PrefillBf16(a.seed, a.config, a.kv)
    elif a.config == 9:
        w = PageCopyBench(a.seed)
    elif a.config == 10:
        w = GatherBench(a.seed)
    elif a.config == 11:
        w = PrefillSliding(a.seed, a.window, a.kv)
    else:
        w = DecodeBf16(a.config, a.seed)
    w.setup(dev, a)
    torch.cuda.synchronize()
    use_graph = a.launch == "graph" and getattr(w, "graph", False)
    wall_eager, wall_graph, per = measure(w, a.steps, a.warmup, use_graph)
    wall = wall_graph if use_graph else wall_eager
    ms_per_step = wall / a.steps * 1e3
    value = w.step_bytes() / (wall / a.steps) / 1e9
    dom_us = per[getattr(w, "dominant_phase", "partials" if "partials" in per else "attention")]
    if getattr(w, "bound", "hbm") == "mfma":
        tflops = w.flops() / (dom_us * 1e-6) / 1e12
        roof = {"bound": "mfma", "kernel": w.dominant, "achieved": round(tflops, 1),
                "peak": MFMA_BF16_PEAK_TFLOPS, "unit": "TFLOP/s",
                "frac": round(tflops / MFMA_BF16_PEAK_TFLOPS, 4), "traffic": None,
                "flops_per_launch": w.flops()}
        value_override = round(w.flops() / (wall / a.steps) / 1e12, 2)
    else:
        achieved = w.dominant_bytes() / (dom_us * 1e-6) / 1e9
        roof = {"bound": "hbm", "kernel": w.dominant, "achieved": round(achieved, 1),
                "peak": HBM_PEAK_GBS, "unit": "GB/s",
                "frac": round(achieved / HBM_PEAK_GBS, 4), "traffic": None,
                "bytes_per_launch": w.dominant_bytes()}
        value_override = None
    res = {
        "metric": METRIC,
        "value": round(value, 1),
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": a.steps,
        "warmup": a.warmup,
        "ms_per_step": round(ms_per_step, 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": w.dtype,
        "data": getattr(w, "data", "synthetic (seeded SplitMix64/Box-Muller N(0,1) on device)"),
        "config": w.config(),
        "pct_hbm_peak": round(100 * value / HBM_PEAK_GBS, 2),
        "us_per_layer": round(ms_per_step * 1e3, 2),
        "launch": ("hip graph: the K steps' C-ABI calls captured once and replayed"
                   if use_graph else "eager C-ABI calls from Python"),
        "eager_us_per_layer": round(wall_eager / a.steps * 1e6, 2),
        "us_breakdown_events": {k: round(v, 2) for k, v in per.items()},
        "step_bytes": w.step_bytes(),
        "roofline": roof,
    }
    if value_override is not None:
        # Prefill is MFMA-bound: report TFLOP/s of the step (append + prefill).
        res["value"] = value_override
        res["unit"] = "TFLOP/s"
        res["pct_hbm_peak"] = None
        res["pct_mfma_peak"] = round(100 * value_override / MFMA_BF16_PEAK_TFLOPS, 2)
    traffic_file = os.path.join(os.path.dirname(os.path.abspath(__file__)), "profiles",
                                "traffic.json")
    key = f"config{a.config}_cap{a.cap}" + ("_bq" if a.kv == "bq" and a.config in (4, 6, 11, 12)
                                            else "")
    if os.path.exists(traffic_file):
        with open(traffic_file) as f:
            measured = json.load(f).get(key)
        if measured:
            res["roofline"]["traffic"] = measured["traffic"]
            res["roofline"]["traffic_source"] = measured["source"]
    if not a.no_cpu:
        cb = w.cpu_baseline(a.cpu_budget)
        if cb is not None:
            res["cpu_baseline"] = cb
    print(json.dumps(res), flush=True)


if __name__ == "__main__":
    main()
