"""ctypes binding of the CPU oracle (oracle/liboracle.so).

TEST INFRASTRUCTURE ONLY: imported by tests/, __graft_entry__.smoke() and
bench.py's cpu_baseline leg, as the checker or the timed CPU baseline.  The
product package (inferno_amd) never imports it.
"""
from __future__ import annotations

import ctypes as C
import subprocess
from pathlib import Path

import numpy as np

HERE = Path(__file__).resolve().parent
LIB_PATH = HERE / "liboracle.so"

I64, F32, U64, VP = C.c_int64, C.c_float, C.c_uint64, C.c_void_p

_SIG = {
    "ifo_bf16_to_f32": (F32, [C.c_uint16]),
    "ifo_f32_to_bf16": (C.c_uint16, [F32]),
    "ifo_fexp": (F32, [F32]),
    "ifo_fexp_array": (None, [VP, VP, I64]),
    "ifo_splitmix64": (U64, [U64]),
    "ifo_rng_uniform": (F32, [U64, U64]),
    "ifo_fill_normal_bf16": (None, [VP, I64, U64, U64]),
    "ifo_tree_sum16": (F32, [VP]),
    "ifo_pow2_shift": (I64, [I64]),
    "ifo_flash_partial_stride": (I64, [I64, I64]),
    "ifo_paged_slot": (I64, [VP, I64, I64, I64, I64, I64]),
    "ifo_worker_range": (None, [I64, I64, I64, I64, VP]),
    "ifo_recommended_workers": (I64, [I64, I64]),
    "ifo_sliding_valid_len": (I64, [I64, I64]),
    "ifo_full_local_kv_count": (I64, [I64, I64, I64]),
    "ifo_plan_run_splits": (None, [VP, VP, I64, I64, I64, VP]),
    "ifo_flash_partial": (None, [VP, I64, I64, I64, VP, VP, VP, VP, I64, I64, I64, I64,
                                 I64, I64, I64]),
    "ifo_finalize_head": (None, [VP, VP, I64, I64, I64, I64, I64]),
    "ifo_attention": (C.c_int, [I64, VP, I64, VP, VP, VP, VP, VP, I64, I64, I64, I64, I64,
                                I64, I64, I64, I64, I64]),
    "ifo_rope_cache_write": (None, [VP, I64, VP, VP, VP, VP, VP, VP, VP, VP, I64, I64, I64,
                                    I64, I64, I64, I64, I64, I64, I64, I64]),
    "ifo_rms_norm_qkv_heads": (None, [VP, VP, VP, VP, VP, I64, I64, I64, I64, F32, F32]),
    "ifo_copy_jobs": (None, [VP, VP, I64]),
    "ifo_gather_rows": (None, [VP, VP, VP, I64, I64]),
    "ifo_copy_jobs_workers": (None, [VP, VP, I64, I64, I64]),
    "ifo_gather_rows_workers": (None, [VP, VP, VP, I64, I64, I64, I64]),
    "ifo_fwht": (None, [VP, I64]),
    "ifo_head_inv_rms": (F32, [VP, I64, F32, F32]),
    "ifo_absmax_quantize": (F32, [VP, I64, VP, VP]),
    "ifo_bq_block_quant": (None, [VP, VP, VP, I64, I64, I64]),
    "ifo_gemm_cols": (None, [VP, VP, VP, I64, I64, I64]),
    "ifo_bq_block_sparse_attention": (C.c_int, [VP, I64, VP, VP, VP, VP, VP, VP, VP, VP, VP,
                                                VP, I64, I64, I64, I64, I64, I64, I64, I64,
                                                I64]),
    "ifo_index_block_scores": (None, [VP, I64, VP, VP, VP, VP, I64, I64, I64, I64, F32, I64,
                                      I64]),
    "ifo_select_blocks": (None, [VP, I64, I64, I64, I64, VP]),
    "ifo_lightning_indexer": (None, [VP, I64, VP, VP, VP, VP, VP, I64, I64, I64, I64, I64,
                                     I64, I64, F32, I64, I64]),
    "ifo_block_sparse_attention": (C.c_int, [VP, I64, VP, VP, VP, VP, VP, VP, I64, I64, I64,
                                             I64, I64, I64, I64, I64]),
    "ifo_bq_attn_prep": (None, [VP, I64, VP, VP, VP, VP, VP, VP, VP, VP, VP, VP, VP, VP,
                                VP, VP, VP, I64, I64, I64, I64, I64, I64, I64, I64, I64,
                                I64, I64, F32, F32]),
    "ifo_bq_attention": (C.c_int, [I64, VP, I64, VP, VP, VP, VP, VP, VP, VP, VP, VP, I64,
                                   I64, I64, I64, I64, I64, I64, I64, I64, I64]),
}

_LIB = None
_ACTIVE = None
NATIVE_PATH = HERE / "_native" / "liboracle.so"


def build() -> Path:
    subprocess.run(["make", "-s", "-C", str(HERE)], check=True)
    return LIB_PATH


def build_native() -> Path:
    """The same source built with -march=native for this host (AVX-512, and the
    VDPBF16PS / VPDPBUSD dots where the host has them): the timed CPU baseline."""
    subprocess.run(["make", "-s", "-C", str(HERE), "native"], check=True)
    return NATIVE_PATH


def _load(path: Path):
    h = C.CDLL(str(path))
    for name, (res, args) in _SIG.items():
        fn = getattr(h, name)
        fn.restype = res
        fn.argtypes = args
    return h


def native_lib():
    """Handle of the -march=native build (built on first use)."""
    if not NATIVE_PATH.exists():
        build_native()
    return _load(NATIVE_PATH)


class using:
    """Route this module's calls through another build of the oracle inside
    a with-block: `with oracle.using(oracle.native_lib()): ...`."""

    def __init__(self, handle):
        self.handle, self.prev = handle, None

    def __enter__(self):
        global _ACTIVE
        self.prev, _ACTIVE = _ACTIVE, self.handle
        return self.handle

    def __exit__(self, *exc):
        global _ACTIVE
        _ACTIVE = self.prev
        return False


def lib():
    global _LIB
    if _ACTIVE is not None:
        return _ACTIVE
    if _LIB is None:
        if not LIB_PATH.exists():
            build()
        _LIB = _load(LIB_PATH)
    return _LIB


def _p(a: np.ndarray | None):
    return None if a is None else a.ctypes.data


# ---- numerics --------------------------------------------------------------

def fexp(x) -> np.ndarray:
    shape = np.shape(x)
    x = np.ascontiguousarray(x, dtype=np.float32).reshape(-1)
    y = np.empty_like(x)
    lib().ifo_fexp_array(_p(x), _p(y), x.size)
    return y.reshape(shape)


def splitmix64(x: int) -> int:
    return int(lib().ifo_splitmix64(x))


def bf16_to_f32(b: np.ndarray) -> np.ndarray:
    return (np.asarray(b, dtype=np.uint16).astype(np.uint32) << 16).view(np.float32)


def f32_to_bf16(f: np.ndarray) -> np.ndarray:
    u = np.ascontiguousarray(f, dtype=np.float32).view(np.uint32).astype(np.uint64)
    return ((u + ((u >> 16) & 1) + 0x7FFF) >> 16).astype(np.uint16)


def normal_bf16(n: int, seed: int, counter0: int = 0) -> np.ndarray:
    out = np.empty(n, dtype=np.uint16)
    lib().ifo_fill_normal_bf16(_p(out), n, seed, counter0)
    return out


# ---- planning --------------------------------------------------------------

def plan_run_splits(kv_lens, buf_starts, cap: int, min_split: int = 16) -> np.ndarray:
    kv = np.ascontiguousarray(kv_lens, dtype=np.int64)
    bs = np.ascontiguousarray(buf_starts, dtype=np.int64)
    out = np.zeros((kv.size, 3), dtype=np.int64)
    lib().ifo_plan_run_splits(_p(kv), _p(bs), kv.size, cap, min_split, _p(out))
    return out


def worker_range(total: int, nw: int, w: int, base: int = 0) -> tuple[int, int]:
    out = np.zeros(2, dtype=np.int64)
    lib().ifo_worker_range(total, nw, w, base, _p(out))
    return int(out[0]), int(out[1])


def recommended_workers(data_bytes: int, capacity: int) -> int:
    return int(lib().ifo_recommended_workers(data_bytes, capacity))


def paged_slot(base_rows, shift, row_mask, page_mask, start_pos, pos_t) -> int:
    rows = np.ascontiguousarray(base_rows, dtype=np.int32)
    return int(lib().ifo_paged_slot(_p(rows), shift, row_mask, page_mask, start_pos, pos_t))


def flash_partial_stride(num_q: int, head_dim: int) -> int:
    return int(lib().ifo_flash_partial_stride(num_q, head_dim))


# ---- kernels -----------------------------------------------------------------

def attention(kind, runs, base_rows, q, k, v, *, num_q, num_kv, head_dim, kv_stride,
              window, cache_size, page_len, seq_len, cap, threads=1,
              out=None) -> np.ndarray:
    """dispatch_sliding_attention (kind 0) / dispatch_full_attention (kind 1)."""
    runs = np.ascontiguousarray(runs, dtype=np.int32)
    rows = np.ascontiguousarray(base_rows, dtype=np.int32)
    if out is None:
        out = np.zeros(seq_len * num_q * head_dim, dtype=np.uint16)
    st = lib().ifo_attention(kind, _p(runs), runs.shape[0], _p(rows), _p(q), _p(k), _p(v),
                             _p(out), num_q, num_kv, head_dim, kv_stride, window,
                             cache_size, page_len, seq_len, cap, threads)
    if st != 0:
        raise ValueError(f"oracle attention rejected the arguments ({st})")
    return out


def rope_cache_write(runs, base_rows, q, k_src, v_src, k_cache, v_cache, cos, sin, *,
                     num_q, num_kv, page_shift, row_mask, page_mask, seq_len, half,
                     pair_stride, head_dim) -> None:
    runs = np.ascontiguousarray(runs, dtype=np.int32)
    rows = np.ascontiguousarray(base_rows, dtype=np.int32)
    lib().ifo_rope_cache_write(_p(runs), runs.shape[0], _p(rows), _p(q), _p(k_src),
                               _p(v_src), _p(k_cache), _p(v_cache), _p(cos), _p(sin),
                               num_q, num_kv, 1, 0, page_shift, row_mask, page_mask,
                               seq_len, half, pair_stride, head_dim)


def rms_norm_qkv_heads(q, k, v, q_weight, k_weight, *, num_q, num_kv, seq_len, head_dim,
                       sqrt_n, n_eps) -> None:
    """dispatch_rms_norm_qkv_heads (kernels/rmsnorm.mojo:168-215), in place."""
    lib().ifo_rms_norm_qkv_heads(_p(q), _p(k), _p(v), _p(q_weight), _p(k_weight), num_q,
                                 num_kv, seq_len, head_dim, sqrt_n, n_eps)


def copy_jobs(arena: np.ndarray, jobs) -> None:
    j = np.ascontiguousarray(jobs, dtype=np.int64)
    lib().ifo_copy_jobs(_p(arena), _p(j), j.shape[0])


def gather_rows(src, rows, cols) -> np.ndarray:
    rows = np.ascontiguousarray(rows, dtype=np.int32)
    dst = np.zeros(rows.size * cols, dtype=np.uint16)
    lib().ifo_gather_rows(_p(src), _p(dst), _p(rows), rows.size, cols)
    return dst


def copy_jobs_workers(arena: np.ndarray, jobs, workers: int, threads: int) -> None:
    """dispatch_copy_jobs' fan-out: 64-byte aligned worker shares of the
    concatenated jobs, run on `threads` threads."""
    j = np.ascontiguousarray(jobs, dtype=np.int64)
    lib().ifo_copy_jobs_workers(_p(arena), _p(j), j.shape[0], workers, threads)


def gather_rows_workers(src, rows, cols, workers: int, threads: int,
                        dst: np.ndarray | None = None) -> np.ndarray:
    """dispatch_gather_rows' fan-out: worker_range shares of the rows."""
    rows = np.ascontiguousarray(rows, dtype=np.int32)
    if dst is None:
        dst = np.zeros(rows.size * cols, dtype=np.uint16)
    lib().ifo_gather_rows_workers(_p(src), _p(dst), _p(rows), rows.size, cols, workers,
                                  threads)
    return dst


def fwht(v) -> np.ndarray:
    x = np.array(v, dtype=np.float32, copy=True)
    lib().ifo_fwht(_p(x), x.size)
    return x


def absmax_quantize(x) -> tuple[np.ndarray, float, int]:
    x = np.ascontiguousarray(x, dtype=np.float32)
    q = np.zeros(x.size, dtype=np.int8)
    qs = np.zeros(1, dtype=np.int32)
    amax = lib().ifo_absmax_quantize(_p(x), x.size, _p(q), _p(qs))
    return q, float(amax), int(qs[0])


def index_block_stride(runs, seq_len: int, block_size: int) -> int:
    """Blocks per (token, head) score row: the largest position's block count,
    rounded up to 16 (lightning_indexer.mojo:420-422 for one run)."""
    runs = np.asarray(runs, dtype=np.int64).reshape(-1, 4)
    last = 0
    for i, r in enumerate(runs):
        end = runs[i + 1][0] if i + 1 < len(runs) else seq_len
        last = max(last, int(r[1]) + int(end - r[0]) - 1)
    return (last // block_size + 1 + 15) // 16 * 16


def index_block_scores(runs, base_rows, index_q, index_k, *, num_heads, head_dim,
                       block_size, scale, page_len, seq_len) -> np.ndarray:
    runs = np.ascontiguousarray(runs, dtype=np.int32)
    rows = np.ascontiguousarray(base_rows, dtype=np.int32)
    bs = index_block_stride(runs, seq_len, block_size)
    scores = np.full(seq_len * num_heads * bs, np.nan, dtype=np.float32)
    lib().ifo_index_block_scores(_p(runs), runs.shape[0], _p(rows), _p(index_q), _p(index_k),
                                 _p(scores), bs, num_heads, head_dim, block_size,
                                 np.float32(scale), page_len, seq_len)
    return scores.reshape(seq_len, num_heads, bs)


def select_blocks(row_scores, num_blocks: int, *, topk: int, local_blocks: int,
                  init_blocks: int) -> np.ndarray:
    row = np.ascontiguousarray(row_scores, dtype=np.float32)
    out = np.zeros(topk, dtype=np.int32)
    lib().ifo_select_blocks(_p(row), num_blocks, topk, local_blocks, init_blocks, _p(out))
    return out


def lightning_indexer(runs, base_rows, index_q, index_k, *, num_heads, head_dim, block_size,
                      topk, local_blocks, init_blocks, scale, page_len, seq_len):
    """Returns (block_idx [seq][heads][topk] int32, scores [seq][heads][stride])."""
    runs = np.ascontiguousarray(runs, dtype=np.int32)
    rows = np.ascontiguousarray(base_rows, dtype=np.int32)
    bs = index_block_stride(runs, seq_len, block_size)
    scores = np.full(seq_len * num_heads * bs, np.nan, dtype=np.float32)
    idx = np.full(seq_len * num_heads * topk, -2, dtype=np.int32)
    lib().ifo_lightning_indexer(_p(runs), runs.shape[0], _p(rows), _p(index_q), _p(index_k),
                                _p(idx), _p(scores), bs, num_heads, head_dim, block_size, topk,
                                local_blocks, init_blocks, np.float32(scale), page_len,
                                seq_len)
    return idx.reshape(seq_len, num_heads, topk), scores.reshape(seq_len, num_heads, bs)


def block_sparse_attention(runs, base_rows, q, k, v, block_idx, *, num_q, num_kv, head_dim,
                           kv_stride, block_size, topk, page_len, seq_len) -> np.ndarray:
    runs = np.ascontiguousarray(runs, dtype=np.int32)
    rows = np.ascontiguousarray(base_rows, dtype=np.int32)
    bi = np.ascontiguousarray(block_idx, dtype=np.int32)
    out = np.zeros(seq_len * num_q * head_dim, dtype=np.uint16)
    st = lib().ifo_block_sparse_attention(_p(runs), runs.shape[0], _p(rows), _p(q), _p(k),
                                          _p(v), _p(bi), _p(out), num_q, num_kv, head_dim,
                                          kv_stride, block_size, topk, page_len, seq_len)
    if st != 0:
        raise ValueError(f"oracle sparse attention rejected the arguments ({st})")
    return out


def bq_block_sparse_attention(runs, base_rows, q_i8, qi_bias, f_q, k_cache, k_scale, v_cache,
                              v_scale, block_idx, *, num_q, num_kv, head_dim, kv_stride,
                              block_size, topk, page_len, seq_len, cap) -> np.ndarray:
    runs = np.ascontiguousarray(runs, dtype=np.int32)
    rows = np.ascontiguousarray(base_rows, dtype=np.int32)
    bi = np.ascontiguousarray(block_idx, dtype=np.int32)
    out = np.zeros(seq_len * num_q * head_dim, dtype=np.uint16)
    st = lib().ifo_bq_block_sparse_attention(
        _p(runs), runs.shape[0], _p(rows), _p(q_i8), _p(qi_bias), _p(f_q), _p(k_cache),
        _p(k_scale), _p(v_cache), _p(v_scale), _p(bi), _p(out), num_q, num_kv, head_dim,
        kv_stride, block_size, topk, page_len, seq_len, cap)
    if st != 0:
        raise ValueError(f"oracle bq sparse attention rejected the arguments ({st})")
    return out


def gemm_cols(x, w, *, rows: int, cols: int) -> np.ndarray:
    """o_proj: bf16 [seq][rows] = x [seq][cols] . w [rows][cols]^T (bf16 bits)."""
    x = np.ascontiguousarray(x, dtype=np.uint16).reshape(-1, cols)
    w = np.ascontiguousarray(w, dtype=np.uint16).reshape(rows, cols)
    out = np.zeros((x.shape[0], rows), dtype=np.uint16)
    lib().ifo_gemm_cols(_p(x), _p(w), _p(out), rows, cols, x.shape[0])
    return out


def bq_block_quant(src, cols: int, block: int) -> tuple[np.ndarray, np.ndarray]:
    """Per-block absmax int8 of bf16 rows: (codes [rows][cols], scales [rows][cols/block])."""
    src = np.ascontiguousarray(src, dtype=np.uint16).reshape(-1, cols)
    rows = src.shape[0]
    x_i8 = np.zeros((rows, cols), dtype=np.int8)
    x_sa = np.zeros((rows, cols // block), dtype=np.float32)
    lib().ifo_bq_block_quant(_p(src), _p(x_i8), _p(x_sa), cols, block, rows)
    return x_i8, x_sa


def head_inv_rms(x, sqrt_n, n_eps) -> float:
    x = np.ascontiguousarray(x, dtype=np.float32)
    return float(lib().ifo_head_inv_rms(_p(x), x.size, sqrt_n, n_eps))


def bq_attn_prep(runs, base_rows, q_src, k_src, v_src, q_norm, k_norm, q_i8, qi_bias, f_q,
                 k_cache, k_scale, v_cache, v_scale, cos, sin, *, num_q, num_kv,
                 page_shift, row_mask, page_mask, seq_len, head_dim, rope_half,
                 pair_stride, sqrt_n, n_eps) -> None:
    runs = np.ascontiguousarray(runs, dtype=np.int32)
    rows = np.ascontiguousarray(base_rows, dtype=np.int32)
    lib().ifo_bq_attn_prep(_p(runs), runs.shape[0], _p(rows), _p(q_src), _p(k_src),
                           _p(v_src), _p(q_norm), _p(k_norm), _p(q_i8), _p(qi_bias),
                           _p(f_q), _p(k_cache), _p(k_scale), _p(v_cache), _p(v_scale),
                           _p(cos), _p(sin), num_q, num_kv, 1, 0, page_shift, row_mask,
                           page_mask, seq_len, head_dim, rope_half, pair_stride,
                           sqrt_n, n_eps)


def bq_attention(kind, runs, base_rows, q_i8, qi_bias, f_q, k_cache, k_scale, v_cache,
                 v_scale, *, num_q, num_kv, head_dim, kv_stride, window, cache_size,
                 page_len, seq_len, cap, threads=1) -> np.ndarray:
    runs = np.ascontiguousarray(runs, dtype=np.int32)
    rows = np.ascontiguousarray(base_rows, dtype=np.int32)
    out = np.zeros(seq_len * num_q * head_dim, dtype=np.uint16)
    st = lib().ifo_bq_attention(kind, _p(runs), runs.shape[0], _p(rows), _p(q_i8),
                                _p(qi_bias), _p(f_q), _p(k_cache), _p(k_scale),
                                _p(v_cache), _p(v_scale), _p(out), num_q, num_kv,
                                head_dim, kv_stride, window, cache_size, page_len,
                                seq_len, cap, threads)
    if st != 0:
        raise ValueError(f"oracle bq attention rejected the arguments ({st})")
    return out
