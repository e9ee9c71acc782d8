/*
 * CPU oracle for the Inferno paged-KV attention path.
 *
 * TEST INFRASTRUCTURE ONLY.  This library restates, in plain C, the
 * reference's Mojo kernels for the paged-KV attention path so that the HIP
 * path in inferno_amd/ can be checked against it.  Only tests/,
 * __graft_entry__.smoke() and bench.py's cpu_baseline leg may load it, and
 * only as the checker (or, in bench.py, as the timed CPU baseline).  The
 * product library never links, loads or calls it; there is no CPU fallback.
 *
 * Conventions
 *   - bf16 values are passed as uint16_t bit patterns.
 *   - A run table is int32 [num_runs][4] = {buf_start, base_pos, rows_off,
 *     page_count} (reference KVRun, kernels/attention_ops.mojo:54-59) plus a
 *     flat int32 base_rows[] array (KVRunTable.base_rows, :62-89).
 *   - All functions are single-rank (degree 1, cache_degree 1) unless an
 *     argument says otherwise.
 *   - Floating point follows the reference's operation order, with no FMA
 *     contraction except where the reference calls fma() explicitly.  The
 *     library is compiled with -ffp-contract=off.
 *   - `cap` is the reference's worker capacity (min(max_worker_count,
 *     pool.get_capacity()), kernels/helpers.mojo:195-203).  The split plan,
 *     and therefore the bits of every attention output, is a function of it.
 *
 * Parity pins (what checks each function against something other than
 * itself) are listed in the header comment of oracle.c, function by function.
 */
#ifndef INFERNO_ORACLE_H
#define INFERNO_ORACLE_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* ---- numeric primitives ---------------------------------------------- */
float    ifo_bf16_to_f32(uint16_t b);
uint16_t ifo_f32_to_bf16(float f);
float    ifo_fexp(float x);
void     ifo_fexp_array(const float* x, float* y, int64_t n);
uint64_t ifo_splitmix64(uint64_t x);
float    ifo_rng_uniform(uint64_t seed, uint64_t counter);
void     ifo_fill_normal_bf16(uint16_t* dst, int64_t n, uint64_t seed,
                              uint64_t counter0);
float    ifo_tree_sum16(const float* v);

/* ---- geometry and planning ------------------------------------------- */
int64_t ifo_pow2_shift(int64_t value);
int64_t ifo_flash_partial_stride(int64_t num_q, int64_t head_dim);
int64_t ifo_paged_slot(const int32_t* base_rows, int64_t shift,
                       int64_t row_mask, int64_t page_mask,
                       int64_t start_pos, int64_t pos_t);
void    ifo_worker_range(int64_t total, int64_t num_workers,
                         int64_t worker_id, int64_t base, int64_t* out2);
int64_t ifo_recommended_workers(int64_t data_bytes, int64_t capacity);
int64_t ifo_sliding_valid_len(int64_t pos, int64_t window);
int64_t ifo_full_local_kv_count(int64_t rank, int64_t abs_pos,
                                int64_t degree);
void    ifo_plan_run_splits(const int64_t* kv_lens, const int64_t* buf_starts,
                            int64_t num_runs, int64_t cap, int64_t min_split,
                            int64_t* bands /* [num_runs][3] */);

/* ---- bf16 attention ---------------------------------------------------- */
void ifo_flash_partial(const int32_t* base_rows, int64_t shift,
                       int64_t row_mask, int64_t page_mask,
                       const uint16_t* q, const uint16_t* k_base,
                       const uint16_t* v_base, float* partial,
                       int64_t num_q, int64_t head_dim, int64_t gqa_ratio,
                       int64_t kv_stride, int64_t start_pos, int64_t start,
                       int64_t end);
void ifo_finalize_head(uint16_t* dst, const float* seg_base,
                       int64_t seg_stride, int64_t seg_n, int64_t num_q,
                       int64_t head_dim, int64_t h);

/* kind: 0 = sliding (dispatch_sliding_attention), 1 = full
 * (dispatch_full_attention).  window/cache_size are used by sliding only.
 * Returns 0, or a negative value on invalid arguments. */
int ifo_attention(int64_t kind, const int32_t* runs, int64_t num_runs,
                  const int32_t* base_rows, const uint16_t* q,
                  const uint16_t* k_base, const uint16_t* v_base,
                  uint16_t* out, int64_t num_q, int64_t num_kv,
                  int64_t head_dim, int64_t kv_stride, int64_t window,
                  int64_t cache_size, int64_t page_len, int64_t seq_len,
                  int64_t cap, int64_t threads);

/* ---- append, page copy, gather ---------------------------------------- */
void ifo_rms_norm_qkv_heads(uint16_t* q, uint16_t* k, uint16_t* v,
                            const uint16_t* q_weight, const uint16_t* k_weight,
                            int64_t num_q, int64_t num_kv, int64_t seq_len,
                            int64_t head_dim, float sqrt_n, float n_eps);
void ifo_rope_cache_write(const int32_t* runs, int64_t num_runs,
                          const int32_t* base_rows, uint16_t* q,
                          const uint16_t* k_src, const uint16_t* v_src,
                          uint16_t* k_cache, uint16_t* v_cache,
                          const float* cos_table, const float* sin_table,
                          int64_t num_q, int64_t num_kv, int64_t cache_degree,
                          int64_t rank, int64_t page_shift, int64_t row_mask,
                          int64_t page_mask, int64_t seq_len, int64_t half,
                          int64_t pair_stride, int64_t head_dim);
void ifo_copy_jobs(uint8_t* arena, const int64_t* jobs /* [n][3] */,
                   int64_t num_jobs);
void ifo_gather_rows(const uint16_t* src, uint16_t* dst, const int32_t* rows,
                     int64_t num_rows, int64_t cols);
void ifo_copy_jobs_workers(uint8_t* arena, const int64_t* jobs, int64_t num_jobs,
                           int64_t workers, int64_t threads);
void ifo_gather_rows_workers(const uint16_t* src, uint16_t* dst, const int32_t* rows,
                             int64_t num_rows, int64_t cols, int64_t workers,
                             int64_t threads);

/* ---- MiniMax-M3 block-sparse attention (degree 1) ---------------------- */
void ifo_index_block_scores(const int32_t* runs, int64_t num_runs,
                            const int32_t* base_rows, const uint16_t* index_q,
                            const uint16_t* index_k, float* scores,
                            int64_t block_stride, int64_t num_heads,
                            int64_t head_dim, int64_t block_size, float scale,
                            int64_t page_len, int64_t seq_len);
void ifo_select_blocks(const float* row_scores, int64_t num_blocks, int64_t topk,
                       int64_t local_blocks, int64_t init_blocks, int32_t* out_row);
void ifo_lightning_indexer(const int32_t* runs, int64_t num_runs,
                           const int32_t* base_rows, const uint16_t* index_q,
                           const uint16_t* index_k, int32_t* block_idx,
                           float* scores, int64_t block_stride, int64_t num_heads,
                           int64_t head_dim, int64_t block_size, int64_t topk,
                           int64_t local_blocks, int64_t init_blocks, float scale,
                           int64_t page_len, int64_t seq_len);
int ifo_block_sparse_attention(const int32_t* runs, int64_t num_runs,
                               const int32_t* base_rows, const uint16_t* q,
                               const uint16_t* k_base, const uint16_t* v_base,
                               const int32_t* block_idx, uint16_t* out,
                               int64_t num_q, int64_t num_kv, int64_t head_dim,
                               int64_t kv_stride, int64_t block_size, int64_t topk,
                               int64_t page_len, int64_t seq_len);

int ifo_bq_block_sparse_attention(const int32_t* runs, int64_t num_runs,
                                  const int32_t* base_rows, const int8_t* q_i8,
                                  const float* qi_bias, const float* f_q,
                                  const int8_t* k_base, const float* k_scale,
                                  const int8_t* v_base, const float* v_scale,
                                  const int32_t* block_idx, uint16_t* out,
                                  int64_t num_q, int64_t num_kv, int64_t head_dim,
                                  int64_t kv_stride, int64_t block_size, int64_t topk,
                                  int64_t page_len, int64_t seq_len, int64_t cap);

void ifo_gemm_cols(const uint16_t* x, const uint16_t* w, uint16_t* out,
                   int64_t rows, int64_t cols, int64_t seq_len);

/* ---- butterquant int8 KV ------------------------------------------------ */
void  ifo_fwht(float* v, int64_t n);
float ifo_head_inv_rms(const float* x, int64_t n, float sqrt_n, float n_eps);
float ifo_absmax_quantize(const float* x, int64_t n, int8_t* out,
                          int32_t* qsum);
void  ifo_bq_block_quant(const uint16_t* src, int8_t* x_i8, float* x_sa,
                         int64_t cols, int64_t block, int64_t seq_len);
void ifo_bq_attn_prep(const int32_t* runs, int64_t num_runs,
                      const int32_t* base_rows, const uint16_t* q_src,
                      const uint16_t* k_src, const uint16_t* v_src,
                      const uint16_t* q_norm, const uint16_t* k_norm,
                      int8_t* q_i8, float* qi_bias, float* f_q,
                      int8_t* k_cache, float* k_scale, int8_t* v_cache,
                      float* v_scale, const float* cos_table,
                      const float* sin_table, int64_t num_q, int64_t num_kv,
                      int64_t cache_degree, int64_t rank, int64_t page_shift,
                      int64_t row_mask, int64_t page_mask, int64_t seq_len,
                      int64_t head_dim, int64_t rope_half,
                      int64_t pair_stride, float sqrt_n, float n_eps);
int ifo_bq_attention(int64_t kind, const int32_t* runs, int64_t num_runs,
                     const int32_t* base_rows, const int8_t* q_i8,
                     const float* qi_bias, const float* f_q,
                     const int8_t* k_base, const float* k_scale,
                     const int8_t* v_base, const float* v_scale,
                     uint16_t* out, int64_t num_q, int64_t num_kv,
                     int64_t head_dim, int64_t kv_stride, int64_t window,
                     int64_t cache_size, int64_t page_len, int64_t seq_len,
                     int64_t cap, int64_t threads);

#ifdef __cplusplus
}
#endif

#endif /* INFERNO_ORACLE_H */
