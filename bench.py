"""Benchmark of the MI355X paged-KV decode path (headline: config 2).

    python bench.py [--gpus 1] [--steps K] [--warmup W] [--cap C] [--config 2]

One step = one layer of batched paged decode: append one token per sequence
(RoPE + paged cache write), split-KV flash-decode partials over every page of
every sequence, and the log-sum-exp merge.  Inputs (KV cache pages, queries,
RoPE tables, plan image) are resident in HBM before the timed region; the
plan is built once, as the reference binds its run tables once per step for
all layers.

Prints ONE JSON line.  `value` is the whole step's algorithmic bytes divided
by its wall time (GB/s); `roofline` covers the dominant kernel (the split-KV
partial kernel) timed with HIP events on the launch stream; `cpu_baseline`
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
KV_STRIDE = NUM_KV * HEAD_DIM
MASK64 = (1 << 64) - 1


def splitmix64(x: int) -> int:
    z = (x + 0x9E3779B97F4A7C15) & MASK64
    z = ((z ^ (z >> 30)) * 0xBF58476D1CE4E5B9) & MASK64
    z = ((z ^ (z >> 27)) * 0x94D049BB133111EB) & MASK64
    return z ^ (z >> 31)


def config_contexts(config: int, seed: int) -> tuple[list[int], str]:
    """Context lengths of the configured batch (SplitMix64 counter stream)."""
    if config == 1:
        return [4096], "config1: B=1, ctx 4096, 128-page pool, append 1 + decode"
    if config == 2:
        ctx = [512 + splitmix64(seed ^ splitmix64(i)) % 32257 for i in range(64)]
        return ctx, ("config2: B=64 batched paged decode, ctx ~ U[512,32768], "
                     "16q/8kv hd256 bf16, 64-token pages, append 1 + split-KV decode + merge")
    raise SystemExit(f"unknown --config {config}")


def build_case(ctx: list[int], seed: int, extra_pages: int = 0):
    """Pages per sequence after the append, drawn from a seeded permutation of
    one shared pool; the run table of the step (one token per sequence)."""
    from inferno_amd.kv import KVRunTable

    need = [(c + 1 + PAGE_LEN - 1) // PAGE_LEN for c in ctx]
    pool = sum(need) + extra_pages
    rng = np.random.default_rng(seed)
    perm = rng.permutation(pool)
    table = KVRunTable()
    off = 0
    pages = []
    for i, c in enumerate(ctx):
        table.begin_run(i, c)
        pg = perm[off:off + need[i]]
        off += need[i]
        pages.append(pg)
        for p in pg:
            table.add_base_row(int(p) * PAGE_LEN)
    return table, pool, pages


def rope_tables(max_pos: int, half: int = 128, theta: float = 10000.0):
    inv = 1.0 / theta ** (np.arange(half, dtype=np.float64) * 2 / (2 * half))
    ang = np.arange(max_pos, dtype=np.float64)[:, None] * inv[None, :]
    return np.cos(ang).astype(np.float32).reshape(-1), np.sin(ang).astype(np.float32).reshape(-1)


def step_bytes(ctx: list[int], pages: int) -> dict:
    B = len(ctx)
    kv = sum(c + 1 for c in ctx) * KV_STRIDE * 2 * 2
    q = B * NUM_Q * HEAD_DIM * 2
    out = q
    table = 4 * pages
    append = B * (KV_STRIDE * 2 * 2 * 2 + NUM_Q * HEAD_DIM * 2 * 2)
    return {"kv": kv, "q": q, "out": out, "table": table, "append": append,
            "decode": kv + q + out + table, "step": kv + q + out + table + append,
            "partials_kernel": kv + q + table}


def cpu_baseline(ctx, pages_list, k_dev, v_dev, q_host, cap_unused, budget_s: float):
    """Times the CPU oracle on a bounded sample of the batch (the first
    sequences, their pages copied from HBM into a compact host cache)."""
    import torch

    import oracle

    threads = min(16, os.cpu_count() or 1)
    n_seq = min(len(ctx), max(threads, 8))
    sample_ctx = ctx[:n_seq]
    pages = np.concatenate([np.asarray(p) for p in pages_list[:n_seq]])
    idx = torch.from_numpy(pages.astype(np.int64)).to(k_dev.device)
    kp = k_dev.view(-1, PAGE_LEN * KV_STRIDE).index_select(0, idx).cpu().numpy().view(np.uint16)
    vp = v_dev.view(-1, PAGE_LEN * KV_STRIDE).index_select(0, idx).cpu().numpy().view(np.uint16)
    runs, rows, off = [], [], 0
    for i, c in enumerate(sample_ctx):
        n = len(pages_list[i])
        runs.append([i, c, off, n])
        rows.extend((off + j) * PAGE_LEN for j in range(n))
        off += n
    runs = np.asarray(runs, dtype=np.int32)
    rows = np.asarray(rows, dtype=np.int32)
    q = np.ascontiguousarray(q_host[:n_seq * NUM_Q * HEAD_DIM])
    kp, vp = np.ascontiguousarray(kp.reshape(-1)), np.ascontiguousarray(vp.reshape(-1))
    nbytes = sum(c + 1 for c in sample_ctx) * KV_STRIDE * 2 * 2
    times = []
    t_end = time.perf_counter() + budget_s
    while len(times) < 5 and (not times or time.perf_counter() < t_end):
        t0 = time.perf_counter()
        oracle.attention(1, runs, rows, q, kp, vp, num_q=NUM_Q, num_kv=NUM_KV,
                         head_dim=HEAD_DIM, kv_stride=KV_STRIDE, window=0,
                         cache_size=PAGE_LEN, page_len=PAGE_LEN, seq_len=n_seq,
                         cap=threads, threads=threads)
        times.append(time.perf_counter() - t0)
    med = statistics.median(times)
    return {"value": round(nbytes / med / 1e9, 3), "unit": "GB/s", "cores": threads,
            "kind": "port",
            "sample": (f"first {n_seq} of the {len(ctx)} sequences ({nbytes / 1e9:.2f} GB of K+V), "
                       f"reference routing at cap={threads} workers, median of {len(times)}"),
            "us_per_layer_equiv": round(med * 1e6 * sum(c + 1 for c in ctx)
                                        / sum(c + 1 for c in sample_ctx), 1)}


def main() -> None:
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=50)
    ap.add_argument("--warmup", type=int, default=5)
    ap.add_argument("--cap", type=int, default=512)
    ap.add_argument("--config", type=int, default=2)
    ap.add_argument("--seed", type=int, default=20241)
    ap.add_argument("--cpu-budget", type=float, default=15.0)
    ap.add_argument("--no-cpu", action="store_true")
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

    from inferno_amd import attention as A
    from inferno_amd._lib import check, lib
    from inferno_amd.kv import FULL, AttentionPlan

    dev = torch.device("cuda:0")
    torch.cuda.set_device(dev)
    if a.copy_calibration:
        n = 1 << 30
        src = torch.ones(n, dtype=torch.uint8, device=dev)
        dst = torch.empty_like(src)
        torch.cuda.synchronize()
        dst.copy_(src)
        torch.cuda.synchronize()
        print(json.dumps({"copy_calibration_bytes": n, "read_kib": n // 1024,
                          "write_kib": n // 1024}))
        return
    ctx, workload = config_contexts(a.config, a.seed)
    extra = 128 - 65 if a.config == 1 else 0
    table, pool, pages = build_case(ctx, a.seed, extra)
    B = len(ctx)
    rows_cache = pool * PAGE_LEN
    stream = torch.cuda.current_stream()
    sid = int(stream.cuda_stream)

    k_cache = torch.empty(rows_cache * KV_STRIDE, dtype=torch.int16, device=dev)
    v_cache = torch.empty_like(k_cache)
    q = torch.empty(B * NUM_Q * HEAD_DIM, dtype=torch.int16, device=dev)
    k_src = torch.empty(B * KV_STRIDE, dtype=torch.int16, device=dev)
    v_src = torch.empty_like(k_src)
    for i, t in enumerate((k_cache, v_cache, q, k_src, v_src)):
        check(lib().ifr_fill_normal_bf16(t.data_ptr(), t.numel(), a.seed * 16 + i, 0, 1.0, sid))
    cos, sin = rope_tables(max(ctx) + 2)
    cos_d, sin_d = torch.from_numpy(cos).to(dev), torch.from_numpy(sin).to(dev)
    plan = AttentionPlan(table, B, kind=FULL, window=0, cache_size=PAGE_LEN,
                         page_len=PAGE_LEN, cache_rows=rows_cache, cap=a.cap,
                         kv_row_bytes=KV_STRIDE * 2, device=dev)
    partials, ps = A.partials_buffer(plan, NUM_Q, HEAD_DIM)
    out = torch.empty(B * NUM_Q * HEAD_DIM, dtype=torch.int16, device=dev)
    q_host = q.cpu().numpy().view(np.uint16).copy()
    torch.cuda.synchronize()

    def step(ev=None):
        if ev is not None:
            ev[0].record(stream)
        A.dispatch_rope_cache_write(plan, q, k_src, v_src, k_cache, v_cache, cos_d, sin_d,
                                    num_q=NUM_Q, num_kv=NUM_KV, half=128, pair_stride=128,
                                    head_dim=HEAD_DIM)
        if ev is not None:
            ev[1].record(stream)
        A.flash_partials_bf16(plan, q, k_cache, v_cache, partials, ps, num_q=NUM_Q,
                              num_kv=NUM_KV, head_dim=HEAD_DIM, kv_stride=KV_STRIDE)
        if ev is not None:
            ev[2].record(stream)
        A.merge_flash_partials(plan, partials, out, ps, num_q=NUM_Q, head_dim=HEAD_DIM)
        if ev is not None:
            ev[3].record(stream)

    for _ in range(a.warmup):
        step()
    torch.cuda.synchronize()

    # Timed region 1: wall clock over K steps, nothing but the step's launches.
    t0 = time.perf_counter()
    for _ in range(a.steps):
        step()
    torch.cuda.synchronize()
    wall = time.perf_counter() - t0

    # Timed region 2: the same K steps with HIP events between the kernels.
    evs = [[torch.cuda.Event(enable_timing=True) for _ in range(4)] for _ in range(a.steps)]
    torch.cuda.synchronize()
    for i in range(a.steps):
        step(evs[i])
    torch.cuda.synchronize()
    t_app = [e[0].elapsed_time(e[1]) * 1e3 for e in evs]
    t_par = [e[1].elapsed_time(e[2]) * 1e3 for e in evs]
    t_mrg = [e[2].elapsed_time(e[3]) * 1e3 for e in evs]
    t_all = [e[0].elapsed_time(e[3]) * 1e3 for e in evs]

    nb = step_bytes(ctx, len(table.base_rows))
    ms_per_step = wall / a.steps * 1e3
    value = nb["step"] / (wall / a.steps) / 1e9
    par_us = statistics.mean(t_par)
    achieved = nb["partials_kernel"] / (par_us * 1e-6) / 1e9
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
        "dtype": "bf16",
        "data": "synthetic (seeded SplitMix64/Box-Muller N(0,1) bf16 on device)",
        "config": {"workload": workload, "batch": B, "context_tokens": int(sum(ctx)),
                   "pool_pages": pool, "page_len": PAGE_LEN, "num_q": NUM_Q,
                   "num_kv": NUM_KV, "head_dim": HEAD_DIM, "cap": a.cap,
                   "seed": a.seed, "plan_items": plan.summary.num_items},
        "pct_hbm_peak": round(100 * value / HBM_PEAK_GBS, 2),
        "us_per_layer": round(ms_per_step * 1e3, 2),
        "us_breakdown_events": {"append": round(statistics.mean(t_app), 2),
                                "partials": round(par_us, 2),
                                "merge": round(statistics.mean(t_mrg), 2),
                                "step": round(statistics.mean(t_all), 2)},
        "step_bytes": nb["step"],
        "roofline": {"bound": "hbm", "kernel": "flash_partial_bf16_kernel<256,2>",
                     "achieved": round(achieved, 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                     "frac": round(achieved / HBM_PEAK_GBS, 4), "traffic": None,
                     "bytes_per_launch": nb["partials_kernel"]},
    }
    traffic_file = os.path.join(os.path.dirname(os.path.abspath(__file__)), "profiles",
                                "traffic.json")
    key = f"config{a.config}_cap{a.cap}"
    if os.path.exists(traffic_file):
        with open(traffic_file) as f:
            measured = json.load(f).get(key)
        if measured:
            res["roofline"]["traffic"] = measured["traffic"]
            res["roofline"]["traffic_source"] = measured["source"]
    if not a.no_cpu:
        res["cpu_baseline"] = cpu_baseline(ctx, pages, k_cache, v_cache, q_host, a.cap,
                                           a.cpu_budget)
    print(json.dumps(res), flush=True)


if __name__ == "__main__":
    main()
