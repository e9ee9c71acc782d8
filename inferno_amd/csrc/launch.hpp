// Internal launch interface between the C ABI layer (api.hip) and the kernel
// translation units.  Nothing here is exported.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace ifr {

struct PagedGeom {
  int shift;      // log2(page_len)
  int row_mask;   // page_len - 1
  int page_mask;  // ring pages - 1, or -1 for an unbounded page table
};

// Split-KV partials for every work item of the plan, then the merge units.
hipError_t launch_attention_bf16(const int32_t* image_dev, int num_items,
                                 int num_units, int mode, const void* q,
                                 const void* k_base, const void* v_base,
                                 void* output, float* partials,
                                 int64_t partial_stride, int num_q, int num_kv,
                                 int head_dim, int64_t kv_stride,
                                 PagedGeom geom, hipStream_t stream);

// The partial phase alone (no merge).
hipError_t launch_partials_bf16(const int32_t* image_dev, int num_items,
                                const void* q, const void* k_base,
                                const void* v_base, float* partials,
                                int64_t partial_stride, int num_q, int num_kv,
                                int head_dim, int64_t kv_stride, PagedGeom geom,
                                hipStream_t stream);

// The partials of Gemma-4's full-attention shape (head_dim 512, 8 q heads per
// kv head), bf16 and butterquant int8 KV (attention_wide.hip).
hipError_t launch_partials_wide_bf16(const int32_t* image, int num_items, const void* q,
                                     const void* k, const void* v, float* partials,
                                     int64_t ps, int num_q, int num_kv, int64_t kv_stride,
                                     PagedGeom geom, hipStream_t stream);
hipError_t launch_partials_wide_bq(const int32_t* image, int num_items, const void* q_i8,
                                   const float* qi_bias, const float* f_q, const void* k,
                                   const float* k_scale, const void* v, const float* v_scale,
                                   float* partials, int64_t ps, int num_q, int num_kv,
                                   int64_t kv_stride, PagedGeom geom, hipStream_t stream);

// MFMA chunked prefill, full attention, head_dim 256, gqa 2: writes the
// finalised output of every query block of a token plan.
hipError_t launch_prefill_full_mfma(const int32_t* image_dev, int num_qblocks,
                                    const void* q, const void* k_base,
                                    const void* v_base, void* output, int num_q,
                                    int num_kv, int64_t kv_stride, PagedGeom geom,
                                    hipStream_t stream);
// The same over butterquant int8 KV (f32 scales per row and kv head).
hipError_t launch_prefill_full_mfma_bq(const int32_t* image, int num_qblocks, const void* q_i8,
                                       const float* qi_bias, const float* f_q, const void* k,
                                       const float* k_scale, const void* v,
                                       const float* v_scale, void* output, int num_q,
                                       int num_kv, int64_t kv_stride, PagedGeom geom,
                                       hipStream_t stream);
// The same for head_dim 512 / 8 q heads per kv head (prefill_wide.hip).
hipError_t launch_prefill_wide_mfma_bq(const int32_t* image, int num_qblocks, const void* q_i8,
                                       const float* qi_bias, const float* f_q, const void* k,
                                       const float* k_scale, const void* v,
                                       const float* v_scale, void* output, int num_q,
                                       int num_kv, int64_t kv_stride, PagedGeom geom,
                                       hipStream_t stream);
hipError_t launch_prefill_wide_mfma(const int32_t* image, int num_qblocks, const void* q,
                                    const void* k, const void* v, void* output, int num_q,
                                    int num_kv, int64_t kv_stride, PagedGeom geom,
                                    hipStream_t stream);

// MFMA chunked prefill, sliding window (head_dim 256, gqa 2): the finalised
// output of every query block.
hipError_t launch_prefill_sliding_mfma(const int32_t* image_dev, int num_qblocks,
                                       const void* q, const void* k_base, const void* v_base,
                                       void* output, int num_q, int num_kv, int64_t kv_stride,
                                       PagedGeom geom, int window, hipStream_t stream);
// The same over butterquant int8 KV (f32 scales per row and kv head).
hipError_t launch_prefill_sliding_mfma_bq(const int32_t* image_dev, int num_qblocks,
                                          const void* q_i8, const float* qi_bias,
                                          const float* f_q, const void* k_base,
                                          const float* k_scale, const void* v_base,
                                          const float* v_scale, void* output, int num_q,
                                          int num_kv, int64_t kv_stride, PagedGeom geom,
                                          int window, hipStream_t stream);

hipError_t launch_bq_attention(const int32_t* image_dev, int num_items,
                               int num_units, int mode, const void* q_i8,
                               const float* qi_bias, const float* f_q,
                               const void* k_base, const float* k_scale,
                               const void* v_base, const float* v_scale,
                               void* output, float* partials,
                               int64_t partial_stride, int num_q, int num_kv,
                               int head_dim, int64_t kv_stride, PagedGeom geom,
                               hipStream_t stream, int8_t* q_out = nullptr,
                               float* q_scale = nullptr);

// dispatch_bq_block_quant[apply_fwht=False]: per-block absmax int8 of bf16
// rows [seq_len][cols]; cols a multiple of block.
hipError_t launch_bq_block_quant(const void* src, void* x_i8, float* x_sa, int64_t cols,
                                 int block, int64_t seq_len, hipStream_t stream);

// dispatch_gemm_cols: out[m][n] = bf16(sum_k x[m][k] * w[n][k]); N % 16 == 0,
// K % 128 == 0.  k splits (and with them the workspace) depend on the shape.
int gemm_cols_splits(int64_t M, int64_t N, int64_t K);
int64_t gemm_cols_workspace_bytes(int64_t M, int64_t N, int64_t K);
hipError_t launch_gemm_cols(const void* x, const void* w, void* out, float* workspace,
                            int64_t M, int64_t N, int64_t K, hipStream_t stream);

// MiniMax-M3 lightning indexer (block scores + top-k) and block-sparse
// attention over a full-attention plan image.
int index_block_stride(int64_t max_pos, int64_t block_size);
int select_bank_cap(int topk);
hipError_t launch_lightning_indexer(const int32_t* image, int seq_len, const void* index_q,
                                    const void* index_k, int32_t* block_idx, float* scores,
                                    int block_stride, int num_heads, int head_dim,
                                    int block_size, int topk, int local_blocks,
                                    int init_blocks, float scale, int shift, int row_mask,
                                    hipStream_t stream);
hipError_t launch_block_sparse_attention(const int32_t* image, int seq_len, const void* q,
                                         const void* k_base, const void* v_base,
                                         const int32_t* block_idx, void* output,
                                         int64_t kv_stride, int num_q, int num_kv,
                                         int block_size, int topk, int shift, int row_mask,
                                         hipStream_t stream);

// write_finalized_head for every head of one output row over stripes
// [0, n_stripes) of head_dim 128 partials (no plan image).
hipError_t launch_merge_stripes(const float* partials, void* output, int64_t ps,
                                int n_stripes, int num_q, hipStream_t stream);
hipError_t launch_bq_block_sparse_attention(
    const int32_t* image, int seq_len, const void* q_i8, const float* qi_bias,
    const float* f_q, const void* k_base, const float* k_scale, const void* v_base,
    const float* v_scale, const int32_t* block_idx, void* output, float* partials,
    int64_t partial_stride, int64_t kv_stride, int num_q, int num_kv, int block_size,
    int topk, int decode_slots, int decode_workers, int shift, int row_mask,
    hipStream_t stream);

// num_stripes: partial stripes of the plan (one per split).  q_out / q_scale
// (optional): per-head absmax int8 of the merged outputs, fused.
hipError_t launch_merge(const int32_t* image_dev, int num_units, int num_stripes, int mode,
                        const float* partials, void* output,
                        int64_t partial_stride, int num_q, int head_dim,
                        hipStream_t stream, int8_t* q_out = nullptr,
                        float* q_scale = nullptr);

hipError_t launch_rope_cache_write(const int32_t* image_dev, int seq_len,
                                   void* q, const void* k_src,
                                   const void* v_src, void* k_cache,
                                   void* v_cache, const float* cos_table,
                                   const float* sin_table, int num_q,
                                   int num_kv, PagedGeom geom, int half,
                                   int pair_stride, int head_dim,
                                   hipStream_t stream);

// In-place head RMS norm of q, k (with gains) and v.
hipError_t launch_rms_norm_qkv(void* q, void* k, void* v, const void* q_w, const void* k_w,
                               int seq_len, int num_q, int num_kv, int head_dim, float sqrt_n,
                               float n_eps, hipStream_t stream);

// The head RMS norm fused ahead of rope_cache_write.
hipError_t launch_rms_rope_cache_write(const int32_t* image_dev, int seq_len, void* q,
                                       const void* k_src, const void* v_src, void* k_cache,
                                       void* v_cache, const void* q_w, const void* k_w,
                                       const float* cos_table, const float* sin_table,
                                       int num_q, int num_kv, PagedGeom geom, int half,
                                       int pair_stride, int head_dim, float sqrt_n,
                                       float n_eps, hipStream_t stream);

hipError_t launch_bq_attn_prep(const int32_t* image_dev, int seq_len,
                               const void* q_src, const void* k_src,
                               const void* v_src, const void* q_norm,
                               const void* k_norm, void* q_i8, float* qi_bias,
                               float* f_q, void* k_cache, float* k_scale,
                               void* v_cache, float* v_scale,
                               const float* cos_table, const float* sin_table,
                               int num_q, int num_kv, PagedGeom geom,
                               int head_dim, int rope_half, int pair_stride,
                               float sqrt_n, float n_eps, hipStream_t stream);

// Copy chunks: int64 [n][4] = {src_off, dst_off, bytes, 0}.
hipError_t launch_copy_chunks(void* arena, const int64_t* chunks_dev, int num_chunks,
                              hipStream_t stream);

hipError_t launch_gather_rows(const void* src, void* dst, const int32_t* rows,
                              int num_rows, int cols, hipStream_t stream);

hipError_t launch_fill_normal_bf16(void* dst, int64_t n, uint64_t seed,
                                   int64_t outlier_every, float outlier_scale,
                                   hipStream_t stream);

// Head-dim / GQA pairs the attention kernels are compiled for.
bool attention_shape_supported(int head_dim, int gqa);

}  // namespace ifr
