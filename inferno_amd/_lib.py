"""ctypes binding of libinferno_hip.so (declared in include/inferno_hip.h).

Loading fails loudly when the library has not been built: there is no CPU
fallback for any entry point.
"""
from __future__ import annotations

import ctypes as C
from pathlib import Path

LIB_PATH = Path(__file__).resolve().parent / "libinferno_hip.so"

I32, I64, U64, F32, VP = C.c_int32, C.c_int64, C.c_uint64, C.c_float, C.c_void_p
P_I32 = C.POINTER(C.c_int32)
P_I64 = C.POINTER(C.c_int64)
P_F32 = C.POINTER(C.c_float)

INFO_LEN = 16
PLAN_SPLIT_MERGE, PLAN_TOKEN_DIRECT, PLAN_TOKEN_MERGE = 0, 1, 2

# name -> (restype, argtypes)
SIGNATURES: dict[str, tuple[object, list[object]]] = {
    "ifr_abi_version": (I32, []),
    "ifr_last_error": (I32, [C.c_char_p, I64]),
    "ifr_device_count": (I32, [P_I64]),
    "ifr_set_device": (I32, [I64]),
    "ifr_malloc": (I32, [C.POINTER(VP), I64]),
    "ifr_free": (I32, [VP]),
    "ifr_host_alloc": (I32, [C.POINTER(VP), I64]),
    "ifr_host_free": (I32, [VP]),
    "ifr_memcpy_h2d": (I32, [VP, VP, I64, U64]),
    "ifr_memcpy_d2h": (I32, [VP, VP, I64, U64]),
    "ifr_memcpy_d2d": (I32, [VP, VP, I64, U64]),
    "ifr_memset": (I32, [VP, I32, I64, U64]),
    "ifr_stream_create": (I32, [C.POINTER(U64)]),
    "ifr_stream_destroy": (I32, [U64]),
    "ifr_stream_sync": (I32, [U64]),
    "ifr_fill_normal_bf16": (I32, [VP, I64, U64, I64, F32, U64]),
    "ifr_flash_partial_stride": (I64, [I64, I64]),
    "ifr_plan_bytes": (I64, [I64, I64, I64, I64]),
    "ifr_plan_attention": (I32, [VP, I64, P_I32, I64, P_I32, I64, I64, I64, I64,
                                 I64, I64, I64, I64, I64, P_I64]),
    "ifr_rope_cache_write": (I32, [VP, P_I64, VP, VP, VP, VP, VP, VP, VP, I64, I64,
                                   I64, I64, I64, I64, I64, I64, I64, U64]),
    "ifr_rms_norm_qkv_heads": (I32, [VP, VP, VP, VP, VP, I64, I64, I64, I64, F32, F32, U64]),
    "ifr_rms_norm_rope_cache_write": (I32, [VP, P_I64, VP, VP, VP, VP, VP, VP, VP, VP, VP,
                                            I64, I64, I64, I64, I64, I64, I64, I64, I64,
                                            F32, F32, U64]),
    "ifr_attention_bf16": (I32, [VP, P_I64, VP, VP, VP, VP, VP, I64, I64, I64, I64,
                                 I64, I64, I64, I64, U64]),
    "ifr_attention_bf16_noalloc": (I32, [VP, P_I64, VP, VP, VP, VP, I64, I64, I64, I64,
                                         I64, I64, U64]),
    "ifr_flash_partials_bf16": (I32, [VP, P_I64, VP, VP, VP, VP, I64, I64, I64, I64, I64,
                                      I64, I64, I64, U64]),
    "ifr_merge_flash_partials": (I32, [VP, P_I64, VP, I64, VP, I64, I64, I64, U64]),
    "ifr_dispatch_sliding_attention": (I32, [VP, VP, VP, VP, VP, I64, P_I32, I64, P_I32,
                                             I64, I64, I64, I64, I64, I64, I64, I64, I64,
                                             I64, I64, I64, VP, VP, I64, U64]),
    "ifr_dispatch_full_attention": (I32, [VP, VP, VP, VP, VP, I64, P_I32, I64, P_I32,
                                          I64, I64, I64, I64, I64, I64, I64, I64, I64,
                                          I64, VP, VP, I64, U64]),
    "ifr_copy_jobs_bytes": (I64, [I64, I64]),
    "ifr_dispatch_copy_jobs": (I32, [VP, P_I64, I64, VP, VP, I64, U64]),
    "ifr_dispatch_gather_rows": (I32, [VP, VP, VP, I64, I64, U64]),
    "ifr_bq_attn_prep": (I32, [VP, P_I64, VP, VP, VP, VP, VP, VP, VP, VP, VP, VP, VP, VP,
                               VP, VP, I64, I64, I64, I64, I64, I64, I64, I64, I64, F32,
                               F32, U64]),
    "ifr_bq_attention": (I32, [VP, P_I64, VP, VP, VP, VP, VP, VP, VP, VP, VP, I64, I64,
                               I64, I64, I64, I64, I64, I64, U64]),
    "ifr_bq_attention_block_quant": (I32, [VP, P_I64, VP, VP, VP, VP, VP, VP, VP, VP, VP,
                                           I64, I64, I64, I64, I64, I64, I64, I64, VP, VP,
                                           U64]),
    "ifr_bq_block_quant": (I32, [VP, VP, VP, I64, I64, I64, U64]),
    "ifr_index_scores_bytes": (I64, [P_I64, I64, I64]),
    "ifr_lightning_indexer": (I32, [VP, P_I64, VP, VP, VP, VP, I64, I64, I64, I64, I64, I64,
                                    I64, F32, I64, U64]),
    "ifr_block_sparse_attention": (I32, [VP, P_I64, VP, VP, VP, VP, VP, I64, I64, I64, I64,
                                         I64, I64, I64, U64]),
    "ifr_bq_sparse_partials_bytes": (I64, [P_I64, I64, I64, I64, I64, I64, I64]),
    "ifr_bq_block_sparse_attention": (I32, [VP, P_I64, VP, VP, VP, VP, VP, VP, VP, VP, VP, VP,
                                            I64, I64, I64, I64, I64, I64, I64, I64, I64,
                                            U64]),
    "ifr_gemm_cols_workspace_bytes": (I64, [I64, I64, I64]),
    "ifr_dispatch_gemm_cols": (I32, [VP, VP, VP, I64, I64, I64, VP, I64, U64]),
    # ---- host-side page state (include/inferno_host.h) ----
    "ifr_splitmix64": (U64, [U64]),
    "ifr_hash_token_block": (U64, [VP, I64, I64]),
    "ifr_chain_link": (U64, [U64, U64]),
    "ifr_refresh_chain": (I64, [VP, I64, I64, VP, I64, I64]),
    "ifr_hashed_prefix_len": (I64, [I64, VP, I64, VP, I64, VP, I64, VP, I64]),
    "ifr_pages_create": (I32, [I64, VP, I64, C.POINTER(VP)]),
    "ifr_pages_destroy": (None, [VP]),
    "ifr_pages_admit": (I32, [VP, P_I64]),
    "ifr_pages_release": (I32, [VP, I64]),
    "ifr_pages_share": (I32, [VP, I64, I64, I64, I64]),
    "ifr_pages_truncate": (I32, [VP, I64, I64]),
    "ifr_pages_replace_with_private": (I32, [VP, I64, I64, I64, P_I64]),
    "ifr_pages_pages_needed": (I32, [VP, I64, I64, VP]),
    "ifr_pages_fits": (I32, [VP, VP, P_I64]),
    "ifr_pages_reserve": (I32, [VP, I64, I64, P_I64]),
    "ifr_pages_retain_page": (I32, [VP, I64, I64]),
    "ifr_pages_release_page": (I32, [VP, I64, I64]),
    "ifr_pages_query": (I64, [VP, I64, I64, I64, I64]),
    "ifr_pages_export": (I32, [VP, I64, VP, VP, VP, P_I64]),
    "ifr_registry_create": (I32, [I64, I64, C.POINTER(VP)]),
    "ifr_registry_destroy": (None, [VP]),
    "ifr_registry_open": (I32, [VP, I64, I64, U64]),
    "ifr_registry_adopt": (I32, [VP, I64, I64, U64]),
    "ifr_registry_extend": (I32, [VP, I64, VP, I64, I64, I64, I64, U64]),
    "ifr_registry_seed": (I32, [VP, I64, VP, I64, I64, U64]),
    "ifr_registry_set_warm": (I32, [VP, I64]),
    "ifr_registry_close": (I32, [VP, I64]),
    "ifr_registry_prefix_len": (I64, [VP, I64, VP, I64, VP, I64]),
    "ifr_registry_exact_prefix_len": (I64, [VP, I64, VP, I64]),
    "ifr_registry_lru_victim": (I64, [VP]),
    "ifr_registry_query": (I64, [VP, I64, I64]),
    "ifr_registry_export": (I32, [VP, I64, VP, I64, VP, I64]),
    "ifr_scheduler_create": (I32, [I64, I64, I64, I64, VP, I64, I64, VP, I64, I64,
                                   C.POINTER(VP)]),
    "ifr_scheduler_destroy": (None, [VP]),
    "ifr_scheduler_pages": (VP, [VP]),
    "ifr_scheduler_registry": (VP, [VP]),
    "ifr_scheduler_submit": (I32, [VP, VP, I64, I64, I64, P_I64]),
    "ifr_scheduler_cancel": (I32, [VP, I64]),
    "ifr_scheduler_retire": (I32, [VP, I64, P_I64]),
    "ifr_scheduler_evict_warm": (I32, [VP, P_I64]),
    "ifr_scheduler_build_schedule": (I32, [VP, U64, P_I64]),
    "ifr_scheduler_absorb": (I32, [VP, VP, I64, U64]),
    "ifr_scheduler_discard_step": (I32, [VP]),
    "ifr_scheduler_query": (I64, [VP, I64, I64]),
    "ifr_scheduler_export_schedule": (I32, [VP, VP, I64, VP, I64, VP, I64]),
    "ifr_scheduler_export_request": (I32, [VP, I64, VP, I64, VP, I64]),
    "ifr_scheduler_export_pending": (I32, [VP, VP, I64, P_I64]),
    "ifr_bind_pool_run_table": (I32, [VP, I64, I64, I64, VP, I64, VP, I64, P_I64, P_I64]),
    "ifr_prefix_copy_jobs": (I32, [VP, I64, VP, VP, I64, VP, I64, P_I64]),
}

QUERY_ERROR = -(1 << 63)


class InfernoHipError(RuntimeError):
    def __init__(self, status: int, message: str):
        super().__init__(f"inferno_hip status {status}: {message}")
        self.status = status


_LIB: C.CDLL | None = None


def lib() -> C.CDLL:
    """Returns the loaded library; raises if it is not built."""
    global _LIB
    if _LIB is None:
        if not LIB_PATH.exists():
            raise FileNotFoundError(
                f"{LIB_PATH} is missing: build it with `python -m inferno_amd.build`")
        # The library and torch must share one HIP runtime: device pointers and
        # stream handles cross between them.  torch ships its own libamdhip64
        # (same soname, loaded under another name), so it has to be loaded
        # first; the library's dependency then resolves to it.  Without torch
        # (e.g. under the Mojo host) the system runtime is used.
        try:
            import torch  # noqa: F401
        except ImportError:
            pass
        handle = C.CDLL(str(LIB_PATH))
        for name, (res, args) in SIGNATURES.items():
            fn = getattr(handle, name)
            fn.restype = res
            fn.argtypes = args
        _LIB = handle
    return _LIB


def last_error() -> str:
    buf = C.create_string_buffer(1024)
    lib().ifr_last_error(buf, len(buf))
    return buf.value.decode(errors="replace")


def check(status: int) -> None:
    if status != 0:
        raise InfernoHipError(status, last_error())


def exported_symbols() -> list[str]:
    return list(SIGNATURES)
