"""Reference-named dispatch functions over libinferno_hip.so.

Each function keeps the name and argument meaning of the reference dispatcher
it stands in for (cited per function) and launches the HIP kernels on the
current torch stream.  Buffers are torch tensors on the GPU; nothing here
computes on the host beyond planning.
"""
from __future__ import annotations

import ctypes as C

import numpy as np

from ._lib import P_I64, check, lib
from .kv import FULL, SLIDING, AttentionPlan, KVRunTable, flash_partial_stride


def _stream() -> int:
    """The current HIP stream of the current device (torch's capture stream
    under graph capture), as the raw handle the C ABI takes."""
    import torch

    raw = getattr(torch._C, "_cuda_getCurrentRawStream", None)
    if raw is not None:
        return int(raw(torch.cuda.current_device()))
    return int(torch.cuda.current_stream().cuda_stream)


def _ptr(t) -> int:
    return int(t.data_ptr())


def partials_buffer(plan: AttentionPlan, num_q: int, head_dim: int):
    """Float32 partials sized for the plan's stripes (flash_partial_stride)."""
    import torch

    ps = flash_partial_stride(num_q, head_dim)
    n = max(plan.summary.num_stripes, 1) * ps
    return torch.empty(n, dtype=torch.float32, device=plan.image.device), ps


def dispatch_rope_cache_write(plan: AttentionPlan, q, k_src, v_src, k_cache, v_cache,
                              cos_table, sin_table, *, num_q: int, num_kv: int,
                              half: int, pair_stride: int, head_dim: int) -> None:
    """dispatch_rope_cache_write (kernels/rope.mojo:128-171), cache_degree 1."""
    check(lib().ifr_rope_cache_write(
        _ptr(plan.image), plan.info_ptr, _ptr(q), _ptr(k_src), _ptr(v_src),
        _ptr(k_cache), _ptr(v_cache), _ptr(cos_table), _ptr(sin_table),
        num_q, num_kv, plan.page_shift, plan.page_len - 1, plan.page_mask,
        plan.seq_len, half, pair_stride, head_dim, _stream()))


def dispatch_rms_norm_qkv_heads(q, k, v, q_weight, k_weight, *, num_q: int, num_kv: int,
                                seq_len: int, head_dim: int, sqrt_n: float,
                                n_eps: float) -> None:
    """dispatch_rms_norm_qkv_heads (kernels/rmsnorm.mojo:168-215), in place."""
    check(lib().ifr_rms_norm_qkv_heads(_ptr(q), _ptr(k), _ptr(v), _ptr(q_weight),
                                       _ptr(k_weight), num_q, num_kv, seq_len, head_dim,
                                       sqrt_n, n_eps, _stream()))


def dispatch_rms_norm_rope_cache_write(plan: AttentionPlan, q, k_src, v_src, k_cache, v_cache,
                                       q_weight, k_weight, cos_table, sin_table, *,
                                       num_q: int, num_kv: int, half: int, pair_stride: int,
                                       head_dim: int, sqrt_n: float, n_eps: float) -> None:
    """dispatch_rms_norm_qkv_heads fused ahead of dispatch_rope_cache_write
    (kernels/rmsnorm.mojo:168-215, kernels/rope.mojo:128-171); k_src and
    v_src are only read."""
    check(lib().ifr_rms_norm_rope_cache_write(
        _ptr(plan.image), plan.info_ptr, _ptr(q), _ptr(k_src), _ptr(v_src), _ptr(k_cache),
        _ptr(v_cache), _ptr(q_weight), _ptr(k_weight), _ptr(cos_table), _ptr(sin_table),
        num_q, num_kv, plan.page_shift, plan.page_len - 1, plan.page_mask, plan.seq_len,
        half, pair_stride, head_dim, sqrt_n, n_eps, _stream()))


def attention_bf16(plan: AttentionPlan, q, k_base, v_base, output, partials,
                   partial_stride: int, *, num_q: int, num_kv: int, head_dim: int,
                   kv_stride: int) -> None:
    """Paged flash attention + merge on an uploaded plan
    (kernels/flash_attention.mojo, kernels/logsum_merge.mojo)."""
    check(lib().ifr_attention_bf16(
        _ptr(plan.image), plan.info_ptr, _ptr(q), _ptr(k_base), _ptr(v_base),
        _ptr(output), _ptr(partials), partials.numel() * 4, num_q, num_kv, head_dim,
        partial_stride, kv_stride, plan.page_len, plan.page_mask, _stream()))


def flash_partials_bf16(plan: AttentionPlan, q, k_base, v_base, partials,
                        partial_stride: int, *, num_q: int, num_kv: int, head_dim: int,
                        kv_stride: int) -> None:
    """The split-KV partial phase alone (FlashAttentionKernel fan-out)."""
    check(lib().ifr_flash_partials_bf16(
        _ptr(plan.image), plan.info_ptr, _ptr(q), _ptr(k_base), _ptr(v_base),
        _ptr(partials), partials.numel() * 4, num_q, num_kv, head_dim, partial_stride,
        kv_stride, plan.page_len, plan.page_mask, _stream()))


def merge_flash_partials(plan: AttentionPlan, partials, output, partial_stride: int, *,
                         num_q: int, head_dim: int) -> None:
    """dispatch_merge_batched_flash_partials (kernels/logsum_merge.mojo:331-365)
    and the other merge/finalise routes, on the plan's merge units."""
    check(lib().ifr_merge_flash_partials(
        _ptr(plan.image), plan.info_ptr, _ptr(partials), partials.numel() * 4,
        _ptr(output), num_q, head_dim, partial_stride, _stream()))


def dispatch_sliding_attention(q, k_base, v_base, output, table: KVRunTable, *,
                               num_q: int, kv_stride: int, seq_len: int,
                               head_dim: int, gqa_ratio: int, window: int,
                               cache_size: int, page_len: int, cache_rows: int,
                               cap: int) -> None:
    """dispatch_sliding_attention (kernels/attention_dispatch_kernels.mojo:302-363)
    through the one-call C entry point (plan, upload, launch)."""
    _dispatch(0, q, k_base, v_base, output, table, num_q=num_q, kv_stride=kv_stride,
              seq_len=seq_len, head_dim=head_dim, gqa_ratio=gqa_ratio, window=window,
              cache_size=cache_size, page_len=page_len, cache_rows=cache_rows, cap=cap)


def dispatch_full_attention(q, k_base, v_base, output, table: KVRunTable, *,
                            num_q: int, kv_stride: int, seq_len: int, head_dim: int,
                            gqa_ratio: int, page_len: int, cache_rows: int,
                            cap: int) -> None:
    """dispatch_full_attention (kernels/attention_dispatch_kernels.mojo:366-426)
    at context degree 1."""
    _dispatch(1, q, k_base, v_base, output, table, num_q=num_q, kv_stride=kv_stride,
              seq_len=seq_len, head_dim=head_dim, gqa_ratio=gqa_ratio, window=0,
              cache_size=page_len, page_len=page_len, cache_rows=cache_rows, cap=cap)


class _Staging:
    """Pinned host + device plan staging reused across one-call dispatches."""

    def __init__(self) -> None:
        self.nbytes = 0
        self.host = None
        self.dev = None

    def get(self, nbytes: int, device):
        import torch

        if nbytes > self.nbytes:
            torch.cuda.synchronize()
            self.host = torch.empty(nbytes, dtype=torch.uint8, pin_memory=True)
            self.dev = torch.empty(nbytes, dtype=torch.uint8, device=device)
            self.nbytes = nbytes
        return self.host, self.dev


_STAGING = _Staging()


def _dispatch(kind, q, k_base, v_base, output, table, *, num_q, kv_stride, seq_len,
              head_dim, gqa_ratio, window, cache_size, page_len, cache_rows, cap):
    import torch

    runs, rows = table.arrays()
    nbytes = int(lib().ifr_plan_bytes(runs.shape[0], rows.shape[0], seq_len, cap))
    torch.cuda.current_stream().synchronize()  # staging reuse
    host, dev = _STAGING.get(nbytes, q.device)
    ps = flash_partial_stride(num_q, head_dim)
    stripes = max(cap, seq_len, 1)
    partials = torch.empty(stripes * ps, dtype=torch.float32, device=q.device)
    args = [_ptr(q), _ptr(k_base), _ptr(v_base), _ptr(output), _ptr(partials),
            partials.numel() * 4, runs.ctypes.data_as(C.POINTER(C.c_int32)),
            runs.shape[0], rows.ctypes.data_as(C.POINTER(C.c_int32)), rows.shape[0],
            num_q, ps, kv_stride, seq_len, head_dim, gqa_ratio]
    if kind == 0:
        args += [window, cache_size, page_len, cache_rows, cap]
        fn = lib().ifr_dispatch_sliding_attention
    else:
        args += [page_len, cache_rows, cap]
        fn = lib().ifr_dispatch_full_attention
    args += [_ptr(host), _ptr(dev), nbytes, _stream()]
    check(fn(*args))


def dispatch_copy_jobs(arena, jobs: np.ndarray) -> None:
    """dispatch_copy_jobs (kernels/page_copy.mojo:63-94); jobs int64 [n][3] =
    {src_off, dst_off, byte_count} relative to `arena` (a device tensor)."""
    import torch

    jobs = np.ascontiguousarray(jobs, dtype=np.int64).reshape(-1, 3)
    if jobs.shape[0] == 0:
        return
    nbytes = int(lib().ifr_copy_jobs_bytes(jobs.shape[0], int(jobs[:, 2].sum())))
    torch.cuda.current_stream().synchronize()
    host, dev = _STAGING.get(nbytes, arena.device)
    check(lib().ifr_dispatch_copy_jobs(
        _ptr(arena), jobs.ctypes.data_as(P_I64), jobs.shape[0], _ptr(host), _ptr(dev),
        nbytes, _stream()))


def dispatch_gather_rows(src, dst, rows, num_rows: int, cols: int) -> None:
    """dispatch_gather_rows (kernels/gather.mojo:30-55); rows is a device int32
    tensor."""
    check(lib().ifr_dispatch_gather_rows(_ptr(src), _ptr(dst), _ptr(rows), num_rows,
                                         cols, _stream()))


def dispatch_bq_attn_prep(plan: AttentionPlan, q_src, k_src, v_src, q_norm, k_norm,
                          q_i8, qi_bias, f_q, k_cache, k_scale, v_cache, v_scale,
                          cos_table, sin_table, *, num_q: int, num_kv: int,
                          head_dim: int, rope_half: int, pair_stride: int,
                          sqrt_n: float, n_eps: float) -> None:
    """dispatch_bq_attn_prep (butterquant_kernels/attention.mojo:585-632)."""
    check(lib().ifr_bq_attn_prep(
        _ptr(plan.image), plan.info_ptr, _ptr(q_src), _ptr(k_src), _ptr(v_src),
        _ptr(q_norm), _ptr(k_norm), _ptr(q_i8), _ptr(qi_bias), _ptr(f_q), _ptr(k_cache),
        _ptr(k_scale), _ptr(v_cache), _ptr(v_scale), _ptr(cos_table), _ptr(sin_table),
        num_q, num_kv, plan.page_shift, plan.page_len - 1, plan.page_mask,
        plan.seq_len, head_dim, rope_half, pair_stride, sqrt_n, n_eps, _stream()))


def bq_attention(plan: AttentionPlan, q_i8, qi_bias, f_q, k_base, k_scale, v_base,
                 v_scale, output, partials, partial_stride: int, *, num_q: int,
                 num_kv: int, head_dim: int, kv_stride: int, o_i8=None, o_sa=None) -> None:
    """dispatch_bq_sliding_attention / dispatch_bq_full_attention
    (butterquant_kernels/attention.mojo:354-491) on an uploaded plan.

    With o_i8/o_sa, the o_proj input quantisation that follows it
    (dispatch_bq_block_quant[block=head_dim], modeling/gemma_4_moe_bq.mojo:
    515-517) is fused into the merge."""
    args = (_ptr(plan.image), plan.info_ptr, _ptr(q_i8), _ptr(qi_bias), _ptr(f_q),
            _ptr(k_base), _ptr(k_scale), _ptr(v_base), _ptr(v_scale), _ptr(output),
            _ptr(partials), partials.numel() * 4, num_q, num_kv, head_dim, partial_stride,
            kv_stride, plan.page_len, plan.page_mask)
    if o_i8 is None and o_sa is None:
        check(lib().ifr_bq_attention(*args, _stream()))
    else:
        check(lib().ifr_bq_attention_block_quant(*args, _ptr(o_i8), _ptr(o_sa), _stream()))


def index_scores_buffer(plan: AttentionPlan, num_index_heads: int, block_size: int,
                        device="cuda"):
    """f32 scratch for the indexer's block scores at this plan."""
    import torch

    n = lib().ifr_index_scores_bytes(plan.info_ptr, num_index_heads, block_size)
    if n < 0:
        raise ValueError("bad indexer shape")
    return torch.empty(max(n // 4, 1), dtype=torch.float32, device=device)


def dispatch_lightning_indexer(plan: AttentionPlan, index_q, index_k, block_idx, scores, *,
                               num_index_heads: int = 4, index_head_dim: int = 128,
                               block_size: int = 128, topk_blocks: int = 16,
                               local_blocks: int = 1, init_blocks: int = 0,
                               scale: float | None = None) -> None:
    """dispatch_lightning_indexer (prototypes/lightning_indexer.mojo:399-443),
    defaults of dispatch_minimax_m3_indexer (:454-477)."""
    import numpy as np

    if scale is None:
        scale = float(np.float32(1.0) / np.sqrt(np.float32(index_head_dim)))
    check(lib().ifr_lightning_indexer(
        _ptr(plan.image), plan.info_ptr, _ptr(index_q), _ptr(index_k), _ptr(block_idx),
        _ptr(scores), scores.numel() * 4, num_index_heads, index_head_dim, block_size,
        topk_blocks, local_blocks, init_blocks, scale, plan.page_len, _stream()))


def dispatch_block_sparse_attention(plan: AttentionPlan, q, k_base, v_base, block_idx, output, *,
                                    num_q: int = 64, num_kv: int = 4, head_dim: int = 128,
                                    kv_stride: int = 512, block_size: int = 128,
                                    topk_blocks: int = 16) -> None:
    """dispatch_block_sparse_attention (prototypes/sparse_attention.mojo:184-222),
    defaults of dispatch_minimax_m3_sparse_attention (:231-253)."""
    check(lib().ifr_block_sparse_attention(
        _ptr(plan.image), plan.info_ptr, _ptr(q), _ptr(k_base), _ptr(v_base), _ptr(block_idx),
        _ptr(output), num_q, num_kv, head_dim, kv_stride, block_size, topk_blocks,
        plan.page_len, _stream()))


def dispatch_bq_block_sparse_attention(plan: AttentionPlan, q_i8, qi_bias, f_q, k_base,
                                       k_scale, v_base, v_scale, block_idx, output, *,
                                       cap: int, num_q: int = 64, num_kv: int = 4,
                                       head_dim: int = 128, kv_stride: int = 512,
                                       block_size: int = 128, topk_blocks: int = 16,
                                       partials=None) -> None:
    """dispatch_bq_block_sparse_attention (prototypes/bq_sparse_attention.mojo:
    366-451), defaults of dispatch_bq_minimax_m3_sparse_attention (:460-486).
    `cap` is the reference's worker capacity (it bands a decode step's blocks)."""
    import torch

    n = lib().ifr_bq_sparse_partials_bytes(plan.info_ptr, num_q, num_kv, head_dim, block_size,
                                          topk_blocks, cap)
    if n < 0:
        raise ValueError("bad bq sparse shape")
    if partials is None and n > 0:
        partials = torch.empty(n // 4, dtype=torch.float32, device=output.device)
    pbytes = partials.numel() * 4 if partials is not None else 0
    check(lib().ifr_bq_block_sparse_attention(
        _ptr(plan.image), plan.info_ptr, _ptr(q_i8), _ptr(qi_bias), _ptr(f_q), _ptr(k_base),
        _ptr(k_scale), _ptr(v_base), _ptr(v_scale), _ptr(block_idx), _ptr(output),
        _ptr(partials) if partials is not None else None, pbytes, num_q, num_kv, head_dim,
        kv_stride, block_size, topk_blocks, plan.page_len, cap, _stream()))


def gemm_cols_workspace(rows: int, cols: int, seq_len: int, device="cuda"):
    """f32 workspace for dispatch_gemm_cols at this shape (None if unneeded)."""
    import torch

    n = lib().ifr_gemm_cols_workspace_bytes(rows, cols, seq_len)
    if n < 0:
        raise ValueError("bad gemm_cols shape")
    return torch.empty(max(n // 4, 1), dtype=torch.float32, device=device) if n else None


def dispatch_gemm_cols(x, weight, output, *, rows: int, cols: int, seq_len: int,
                       workspace=None) -> None:
    """dispatch_gemm_cols[rows] (kernels/gemm.mojo:198-225): the o_proj after the
    attention, output[m][n] = bf16(sum_k x[m][k] * weight[n][k])."""
    ws_bytes = workspace.numel() * workspace.element_size() if workspace is not None else 0
    check(lib().ifr_dispatch_gemm_cols(_ptr(x), _ptr(weight), _ptr(output), rows, cols,
                                       seq_len, _ptr(workspace) if workspace is not None
                                       else None, ws_bytes, _stream()))


def dispatch_bq_block_quant(src, x_i8, x_sa, *, cols: int, block: int, seq_len: int) -> None:
    """dispatch_bq_block_quant[apply_fwht=False] (butterquant_kernels/linear.mojo:
    182-206): per-block absmax int8 of seq_len bf16 rows."""
    check(lib().ifr_bq_block_quant(_ptr(src), _ptr(x_i8), _ptr(x_sa), cols, block, seq_len,
                                   _stream()))


__all__ = [
    "SLIDING", "FULL", "KVRunTable", "AttentionPlan", "partials_buffer",
    "dispatch_rope_cache_write", "attention_bf16", "flash_partials_bf16",
    "merge_flash_partials", "dispatch_sliding_attention",
    "dispatch_full_attention", "dispatch_copy_jobs", "dispatch_gather_rows",
    "dispatch_bq_attn_prep", "bq_attention", "dispatch_bq_block_quant",
    "gemm_cols_workspace", "dispatch_gemm_cols", "index_scores_buffer",
    "dispatch_lightning_indexer", "dispatch_block_sparse_attention",
    "dispatch_bq_block_sparse_attention",
]
