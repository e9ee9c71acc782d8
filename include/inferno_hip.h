/*
 * inferno_hip.h -- C ABI of libinferno_hip.so, the MI355X (gfx950) paged-KV
 * attention path for Inferno.
 *
 * Every entry point takes plain pointers, int64 sizes and a HIP stream passed
 * as uint64_t (0 = the default stream), so the reference's Mojo host can bind
 * them with `external_call` exactly as it binds its other native entry points
 * (the reference's precedent passes Int64s: butterquant/amx_tiles.mojo:44-51).
 * No torch type, C++ type or handle object crosses the boundary.
 *
 * Status: every function returning int32_t returns IFR_OK (0) or a negative
 * IFR_E* code; ifr_last_error() returns the calling thread's message.  The
 * library never aborts: the reference's debug_asserts and aborts on contract
 * violations (continuous_batching/paging.mojo:36-47,
 * kernels/attention_dispatch_kernels.mojo:60-61) become argument checks here.
 *
 * Ownership: the caller owns every buffer (KV caches, partials, outputs,
 * plan images and staging).  The library keeps no pointer beyond a call and
 * allocates no device memory inside any dispatch.  Calls are asynchronous on
 * the given stream; results are ready when the stream is synchronised
 * (ifr_stream_sync), which replaces the reference's join_all
 * (kernels/helpers.mojo:158-160).
 *
 * Run tables: the reference's KVRunTable (kernels/attention_ops.mojo:54-89)
 * is a host object read by its CPU workers.  Here a run table crosses as
 *     int32 runs[num_runs][4] = {buf_start, base_pos, rows_off, page_count}
 *     int32 base_rows[num_rows]
 * in host memory.  ifr_plan_attention() turns it, together with the split
 * plan the reference's dispatcher would choose for a worker capacity `cap`,
 * into a flat int32 "plan image" the caller uploads once per step and every
 * layer reuses.  The ifr_dispatch_* wrappers do plan + upload + launch in one
 * call, with the reference's argument lists.
 *
 * `cap` is the reference's worker capacity, min(max_worker_count,
 * pool.get_capacity()) (kernels/helpers.mojo:195-203).  The reference's
 * attention output depends on it bit for bit, because the split plan fixes
 * where the online softmax's tiles start and the biased exp
 * (simd_math/exponential.mojo:177-194) rescales every earlier tile by
 * fexp(0) != 1.  The same cap reproduces the reference's result.
 */
#ifndef INFERNO_HIP_H
#define INFERNO_HIP_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define IFR_OK 0
#define IFR_EINVAL (-1)        /* invalid argument */
#define IFR_EUNSUPPORTED (-2)  /* shape outside the compiled kernel set */
#define IFR_EHIP (-3)          /* HIP runtime error */
#define IFR_ESPACE (-4)        /* caller-provided buffer too small */

#define IFR_ABI_VERSION 1

/* Plan modes reported in info[2] by ifr_plan_attention. */
#define IFR_PLAN_SPLIT_MERGE 0   /* split-KV partials + log-sum-exp merge   */
#define IFR_PLAN_TOKEN_DIRECT 1  /* one item per token, finalised as acc/l */
#define IFR_PLAN_TOKEN_MERGE 2   /* one item per token, one-segment merge  */

/* ---- status, version ---------------------------------------------------- */
int32_t ifr_abi_version(void);
/* Copies the calling thread's last error message into buf (NUL-terminated,
 * truncated to len).  Returns the last status code. */
int32_t ifr_last_error(char* buf, int64_t len);

/* ---- device plumbing (the Mojo host has no HIP runtime of its own) ------ */
int32_t ifr_device_count(int64_t* out);
int32_t ifr_set_device(int64_t device);
int32_t ifr_malloc(void** out, int64_t bytes);
int32_t ifr_free(void* ptr);
int32_t ifr_host_alloc(void** out, int64_t bytes);   /* pinned host memory */
int32_t ifr_host_free(void* ptr);
int32_t ifr_memcpy_h2d(void* dst, const void* src, int64_t bytes, uint64_t stream);
int32_t ifr_memcpy_d2h(void* dst, const void* src, int64_t bytes, uint64_t stream);
int32_t ifr_memcpy_d2d(void* dst, const void* src, int64_t bytes, uint64_t stream);
int32_t ifr_memset(void* dst, int32_t value, int64_t bytes, uint64_t stream);
int32_t ifr_stream_create(uint64_t* out);
int32_t ifr_stream_destroy(uint64_t stream);
int32_t ifr_stream_sync(uint64_t stream);
/* Fills n bf16 values with seeded N(0,1) samples (SplitMix64 counter stream,
 * Box-Muller, RNE to bf16), then, if outlier_every > 0, multiplies every
 * element whose hashed index falls in a 1/outlier_every class by
 * outlier_scale.  Synthetic-input generator for benchmarks and tests. */
int32_t ifr_fill_normal_bf16(void* dst, int64_t n, uint64_t seed,
                             int64_t outlier_every, float outlier_scale,
                             uint64_t stream);

/* ---- geometry ---------------------------------------------------------- */
/* flash_partial_stride (kernels/attention_ops.mojo:140-142), in floats. */
int64_t ifr_flash_partial_stride(int64_t num_q, int64_t head_dim);
/* Upper bound of the plan image size for a run table of num_runs runs and
 * num_rows base rows, seq_len tokens and worker capacity cap. */
int64_t ifr_plan_bytes(int64_t num_runs, int64_t num_rows, int64_t seq_len,
                       int64_t cap);

/* ---- planning (host only; no HIP call) ------------------------------------
 * Replaces the routing of dispatch_flash_sliding / dispatch_flash_full
 * (kernels/attention_dispatch_kernels.mojo:36-299) and plan_run_splits
 * (kernels/attention_ops.mojo:99-137).  kind: 0 = sliding, 1 = full.
 * window and cache_size (ring size in positions) are used by sliding only.
 * cache_rows is the number of rows of the KV cache allocation: every page a
 * run references, at every position the append and attention kernels will
 * touch, must lie inside it (the GPU has no bounds check of its own).
 * kv_row_bytes = kv_stride * element bytes
 * (2 for bf16, 1 for butterquant int8) feeds the single-token worker heuristic
 * (recommended_workers, kernels/helpers.mojo:206-219).
 * Writes the plan image into `image` (host memory of image_bytes) and fills
 * info[IFR_INFO_LEN]:
 *   info[0] = number of work items       info[1] = number of merge units
 *   info[2] = plan mode (IFR_PLAN_*)      info[3] = partial stripes needed
 *   info[4] = image bytes used            info[5] = seq_len
 *   info[6] = num_runs                    info[7] = page shift
 *   info[8] = row mask                    info[9] = page mask (-1 = full)
 *   info[10] = cache_rows                 info[11] = kind
 *   info[12] = window                     info[13] = highest token position
 *   info[14] = MFMA prefill query blocks (token plans of full attention)
 *   info[15] = 0
 * Every launch entry point below takes the same info and refuses a page
 * geometry other than the one the plan was validated for. */
#define IFR_INFO_LEN 16
int32_t ifr_plan_attention(void* image, int64_t image_bytes,
                           const int32_t* runs, int64_t num_runs,
                           const int32_t* base_rows, int64_t num_rows,
                           int64_t seq_len, int64_t kind, int64_t window,
                           int64_t cache_size, int64_t page_len,
                           int64_t cache_rows, int64_t cap,
                           int64_t kv_row_bytes, int64_t* info);

/* ---- KV append ------------------------------------------------------------
 * dispatch_rope_cache_write (kernels/rope.mojo:128-171), one rank
 * (cache_degree 1).  RoPE of q in place; RoPE of k_src into k_cache at the
 * paged slot; copy of v_src into v_cache.  image_dev is an uploaded plan
 * image of the step's run table (its token -> run map is used).
 * half, pair_stride, head_dim are the reference's comptime parameters. */
int32_t ifr_rope_cache_write(const void* image_dev, const int64_t* info,
                             void* q, const void* k_src, const void* v_src,
                             void* k_cache, void* v_cache,
                             const float* cos_table, const float* sin_table,
                             int64_t num_q, int64_t num_kv,
                             int64_t page_shift, int64_t row_mask,
                             int64_t page_mask, int64_t seq_len, int64_t half,
                             int64_t pair_stride, int64_t head_dim,
                             uint64_t stream);
/* dispatch_rms_norm_qkv_heads (kernels/rmsnorm.mojo:168-215), in place: every
 * q head scaled by q_weight, every k head by k_weight, every v head unscaled,
 * each as rms_norm_row (:37-48): sum of squares in the reference's
 * VDPBF16PS/accumulator/halving-tree order, inv = sqrt_n / sqrt(ssq + n_eps),
 * y = bf16((x * inv) * w).  q, k, v: [seq_len][heads][head_dim] bf16;
 * weights: [head_dim] bf16. */
int32_t ifr_rms_norm_qkv_heads(void* q, void* k, void* v, const void* q_weight,
                               const void* k_weight, int64_t num_q, int64_t num_kv,
                               int64_t seq_len, int64_t head_dim, float sqrt_n,
                               float n_eps, uint64_t stream);
/* dispatch_rms_norm_qkv_heads followed by dispatch_rope_cache_write
 * (kernels/rope.mojo:128-171), fused: one pass reads q/k/v once.  q ends
 * normalised and rotated (as after the two reference calls); the k and v
 * cache rows receive the normalised (k: rotated) rows.  Unlike the reference,
 * k_src and v_src are left as passed (the reference normalises them in place
 * and nothing reads them afterwards). */
int32_t ifr_rms_norm_rope_cache_write(const void* image_dev, const int64_t* info,
                                      void* q, const void* k_src, const void* v_src,
                                      void* k_cache, void* v_cache,
                                      const void* q_weight, const void* k_weight,
                                      const float* cos_table, const float* sin_table,
                                      int64_t num_q, int64_t num_kv,
                                      int64_t page_shift, int64_t row_mask,
                                      int64_t page_mask, int64_t seq_len,
                                      int64_t half, int64_t pair_stride,
                                      int64_t head_dim, float sqrt_n, float n_eps,
                                      uint64_t stream);

/* ---- bf16 paged attention (plan already uploaded) --------------------------
 * FlashAttentionKernel / FlashPrefill*Kernel (kernels/flash_attention.mojo,
 * kernels/flash_attention_prefill.mojo) followed by the log-sum-exp merge
 * (kernels/logsum_merge.mojo:28-122, 295-328).  page_mask is
 * cache_size/page_len - 1 for a sliding ring and -1 for a full cache.
 * partials holds partial_stride floats per stripe (info[3] stripes). */
int32_t ifr_attention_bf16(const void* image_dev, const int64_t* info,
                           const void* q, const void* k_base,
                           const void* v_base, void* output, void* partials,
                           int64_t partials_bytes, int64_t num_q,
                           int64_t num_kv, int64_t head_dim,
                           int64_t partial_stride, int64_t kv_stride,
                           int64_t page_len, int64_t page_mask,
                           uint64_t stream);

/* ifr_attention_bf16 without a partials argument: the partials live in a
 * library-owned device array of IFR_STATIC_SCRATCH_BYTES per GPU (held from
 * the library's first call on that GPU until the process ends), so the call
 * allocates nothing, for callers that cannot allocate (code under HIP graph
 * capture, tight serving loops, harnesses that forbid hipMalloc).  No
 * counterpart in the reference.  partial_stride is ifr_flash_partial_stride(
 * num_q, head_dim); a plan whose info[3] stripes need more than the array
 * returns IFR_ESPACE.  Every call on one GPU shares that GPU's array: calls
 * that overlap on one GPU (two streams, or two host threads) race. */
#define IFR_STATIC_SCRATCH_BYTES (32LL << 20)
int32_t ifr_attention_bf16_noalloc(const void* image_dev, const int64_t* info,
                                   const void* q, const void* k_base,
                                   const void* v_base, void* output, int64_t num_q,
                                   int64_t num_kv, int64_t head_dim,
                                   int64_t kv_stride, int64_t page_len,
                                   int64_t page_mask, uint64_t stream);

/* The two phases of ifr_attention_bf16 as separate launches: the split-KV
 * partials (the FlashAttentionKernel fan-out of dispatch_flash_sliding /
 * dispatch_flash_full, kernels/attention_dispatch_kernels.mojo:116-134) and
 * the merge (dispatch_merge_flash_partials / dispatch_merge_batched_flash_
 * partials, kernels/logsum_merge.mojo:205-248,331-365; with a token plan,
 * the finalisation of kernels/flash_attention_prefill.mojo:95-106,251-286).
 * The merge reads only the partials, so it serves the bf16 and the
 * butterquant partials alike. */
int32_t ifr_flash_partials_bf16(const void* image_dev, const int64_t* info,
                                const void* q, const void* k_base,
                                const void* v_base, void* partials,
                                int64_t partials_bytes, int64_t num_q,
                                int64_t num_kv, int64_t head_dim,
                                int64_t partial_stride, int64_t kv_stride,
                                int64_t page_len, int64_t page_mask,
                                uint64_t stream);
int32_t ifr_merge_flash_partials(const void* image_dev, const int64_t* info,
                                 const void* partials, int64_t partials_bytes,
                                 void* output, int64_t num_q, int64_t head_dim,
                                 int64_t partial_stride, uint64_t stream);

/* dispatch_sliding_attention (kernels/attention_dispatch_kernels.mojo:302-363)
 * with its argument list, plus the plan staging the GPU needs: the run table
 * is read from host memory, planned for `cap`, written to ws_host (pinned,
 * ws_bytes >= ifr_plan_bytes) and copied to ws_dev on `stream`.  ws_host must
 * not be reused until the stream has passed this call. */
int32_t ifr_dispatch_sliding_attention(
    const void* q, const void* k_base, const void* v_base, void* output,
    void* partials, int64_t partials_bytes, const int32_t* runs,
    int64_t num_runs, const int32_t* base_rows, int64_t num_rows,
    int64_t num_q, int64_t partial_stride, int64_t kv_stride,
    int64_t seq_len, int64_t head_dim, int64_t gqa_ratio, int64_t window,
    int64_t cache_size, int64_t page_len, int64_t cache_rows, int64_t cap,
    void* ws_host, void* ws_dev, int64_t ws_bytes, uint64_t stream);

/* dispatch_full_attention (kernels/attention_dispatch_kernels.mojo:366-426)
 * at context degree 1 (local_num_q == num_q). */
int32_t ifr_dispatch_full_attention(
    const void* q, const void* k_base, const void* v_base, void* output,
    void* partials, int64_t partials_bytes, const int32_t* runs,
    int64_t num_runs, const int32_t* base_rows, int64_t num_rows,
    int64_t num_q, int64_t partial_stride, int64_t kv_stride,
    int64_t seq_len, int64_t head_dim, int64_t gqa_ratio, int64_t page_len,
    int64_t cache_rows, int64_t cap, void* ws_host, void* ws_dev,
    int64_t ws_bytes, uint64_t stream);

/* ---- page copy and row gather ---------------------------------------------
 * dispatch_copy_jobs (kernels/page_copy.mojo:63-94): jobs are int64
 * [num_jobs][3] = {src_off, dst_off, byte_count} relative to arena (device).
 * The job list is staged through ws_host -> ws_dev like a plan image
 * (ws_bytes >= ifr_copy_jobs_bytes(num_jobs, total_bytes)). */
int64_t ifr_copy_jobs_bytes(int64_t num_jobs, int64_t total_bytes);
int32_t ifr_dispatch_copy_jobs(void* arena, const int64_t* jobs,
                               int64_t num_jobs, void* ws_host, void* ws_dev,
                               int64_t ws_bytes, uint64_t stream);
/* dispatch_gather_rows (kernels/gather.mojo:30-55): dst[j] = src[rows[j]]
 * for bf16 rows of `cols` elements; rows is a device int32 array. */
int32_t ifr_dispatch_gather_rows(const void* src, void* dst,
                                 const int32_t* rows, int64_t num_rows,
                                 int64_t cols, uint64_t stream);

/* ---- MiniMax-M3 block-sparse attention (prototypes/, degree 1) -------------
 * Both calls read a full-attention plan image of the step (kind 1,
 * ifr_plan_attention): its run table, page table and token->run map.
 *
 * dispatch_lightning_indexer (prototypes/lightning_indexer.mojo:399-443):
 * block scores (IndexBlockScoreKernel :129-209: per token and index head, the
 * max over each block's causal positions of scale * dot(index_q, index_k)),
 * then top-k block selection (IndexTopkMergeKernel :253-303 over
 * stream_select_blocks :48-126).  index_q [seq][4][128] bf16, index_k
 * [rows][128] bf16 paged like the plan, block_idx [seq][4][topk] int32
 * ascending with -1 padding, scores scratch of ifr_index_scores_bytes.
 * The reference's top-k pass takes positions from the first run only
 * (:420 and :278, a one-sequence prototype); here each token's run gives its
 * position, which is the same for one run. */
int64_t ifr_index_scores_bytes(const int64_t* info, int64_t num_index_heads,
                               int64_t block_size);
int32_t ifr_lightning_indexer(const void* image_dev, const int64_t* info,
                              const void* index_q, const void* index_k,
                              int32_t* block_idx, float* scores, int64_t scores_bytes,
                              int64_t num_index_heads, int64_t index_head_dim,
                              int64_t block_size, int64_t topk_blocks,
                              int64_t local_blocks, int64_t init_blocks, float scale,
                              int64_t page_len, uint64_t stream);
/* dispatch_block_sparse_attention (prototypes/sparse_attention.mojo:184-222):
 * BlockSparseFlashKernel (:41-136) over each (token, kv head)'s block list in
 * order, then the one-stripe PrefillMergeKernel finalisation
 * (kernels/flash_attention_prefill.mojo:208-248).  head_dim 128, 16 q heads
 * per kv head; output [seq][num_q][128] bf16. */
int32_t ifr_block_sparse_attention(const void* image_dev, const int64_t* info,
                                   const void* q, const void* k_base, const void* v_base,
                                   const int32_t* block_idx, void* output, int64_t num_q,
                                   int64_t num_kv, int64_t head_dim, int64_t kv_stride,
                                   int64_t block_size, int64_t topk_blocks,
                                   int64_t page_len, uint64_t stream);

/* dispatch_bq_block_sparse_attention (prototypes/bq_sparse_attention.mojo:
 * 366-451): the int8 KV variant (codes and f32 scales as ifr_bq_attn_prep
 * writes them, q codes with qi_bias and f_q).  seq_len > 1:
 * BqBlockSparseFlashKernel (:94-200) per (token, kv head), blocks in order,
 * -1 ends the list.  seq_len == 1: BqBlockSparseFlashDecodeKernel (:254-364):
 * the num_kv * min(topk, causal blocks) (kv head, slot) units are banded over
 * min(cap, units) workers (cap: the reference's worker capacity, which fixes
 * the result as in ifr_plan_attention), -1 slots skipped, and the workers'
 * partial stripes merged per head; partials of ifr_bq_sparse_partials_bytes
 * (0 bytes for seq_len > 1). */
int64_t ifr_bq_sparse_partials_bytes(const int64_t* info, int64_t num_q, int64_t num_kv,
                                     int64_t head_dim, int64_t block_size,
                                     int64_t topk_blocks, int64_t cap);
int32_t ifr_bq_block_sparse_attention(
    const void* image_dev, const int64_t* info, const void* q_i8, const float* qi_bias,
    const float* f_q, const void* k_base, const float* k_scale, const void* v_base,
    const float* v_scale, const int32_t* block_idx, void* output, void* partials,
    int64_t partials_bytes, int64_t num_q, int64_t num_kv, int64_t head_dim,
    int64_t kv_stride, int64_t block_size, int64_t topk_blocks, int64_t page_len,
    int64_t cap, uint64_t stream);

/* ---- o_proj (the step after the attention) ----------------------------------
 * dispatch_gemm_cols[rows] (kernels/gemm.mojo:198-225; called at
 * modeling/gemma_4_moe.mojo:387-392 and :485-490 with rows = HIDDEN):
 * output[m][n] = bf16(sum_k x[m][k] * weight[n][k]) for bf16 x [seq_len][cols],
 * weight [rows][cols], f32 accumulation.  rows % 16 == 0, cols % 128 == 0
 * (the reference also takes a scalar tail of cols % 32; not provided).  Small
 * seq_len splits the contraction over workgroups into f32 partials in
 * `workspace` (ifr_gemm_cols_workspace_bytes; 0 means none is needed). */
int64_t ifr_gemm_cols_workspace_bytes(int64_t rows, int64_t cols, int64_t seq_len);
int32_t ifr_dispatch_gemm_cols(const void* x, const void* weight, void* output,
                               int64_t rows, int64_t cols, int64_t seq_len,
                               void* workspace, int64_t workspace_bytes,
                               uint64_t stream);

/* ---- butterquant int8 KV ----------------------------------------------------
 * dispatch_bq_attn_prep (butterquant_kernels/attention.mojo:585-632): RMS
 * norm, gain, RoPE, FWHT over head_dim and absmax int8 for q and k, FWHT and
 * absmax int8 for v; k/v codes and f32 scales written at the paged slot. */
int32_t ifr_bq_attn_prep(const void* image_dev, const int64_t* info,
                         const void* q_src, const void* k_src,
                         const void* v_src, const void* q_norm,
                         const void* k_norm, void* q_i8, float* qi_bias,
                         float* f_q, void* k_cache, float* k_scale,
                         void* v_cache, float* v_scale,
                         const float* cos_table, const float* sin_table,
                         int64_t num_q, int64_t num_kv, int64_t page_shift,
                         int64_t row_mask, int64_t page_mask, int64_t seq_len,
                         int64_t head_dim, int64_t rope_half,
                         int64_t pair_stride, float sqrt_n, float n_eps,
                         uint64_t stream);
/* BqFlashAttentionKernel / BqFlashPrefill*Kernel + merge
 * (butterquant_kernels/attention.mojo:27-351) on an uploaded plan image. */
int32_t ifr_bq_attention(const void* image_dev, const int64_t* info,
                         const void* q_i8, const float* qi_bias,
                         const float* f_q, const void* k_base,
                         const float* k_scale, const void* v_base,
                         const float* v_scale, void* output, void* partials,
                         int64_t partials_bytes, int64_t num_q,
                         int64_t num_kv, int64_t head_dim,
                         int64_t partial_stride, int64_t kv_stride,
                         int64_t page_len, int64_t page_mask, uint64_t stream);
/* ifr_bq_attention followed by the o_proj input quantisation
 * dispatch_bq_block_quant[block=head_dim, apply_fwht=False]
 * (butterquant_kernels/linear.mojo:182-206, called at
 * modeling/gemma_4_moe_bq.mojo:515-517 and :618-620), fused into the merge:
 * o_i8[row][h*head_dim + d] and o_sa[row][h] = amax of head h of the bf16
 * output row (quant_segment[store_divided=False], butterquant/kernels.mojo:
 * 83-92).  `output` is written as by ifr_bq_attention. */
int32_t ifr_bq_attention_block_quant(const void* image_dev, const int64_t* info,
                                     const void* q_i8, const float* qi_bias,
                                     const float* f_q, const void* k_base,
                                     const float* k_scale, const void* v_base,
                                     const float* v_scale, void* output, void* partials,
                                     int64_t partials_bytes, int64_t num_q,
                                     int64_t num_kv, int64_t head_dim,
                                     int64_t partial_stride, int64_t kv_stride,
                                     int64_t page_len, int64_t page_mask, void* o_i8,
                                     float* o_sa, uint64_t stream);
/* dispatch_bq_block_quant[apply_fwht=False] (butterquant_kernels/linear.mojo:
 * 182-206, prepare_block_activation butterquant/runtime.mojo:63-80): for each
 * of seq_len bf16 rows of `cols` elements and each block of `block` columns,
 * x_sa[row][b] = amax and x_i8 = clamp(roundeven(x * 127/amax), -128, 127)
 * (0 when amax is 0).  The FWHT variant (apply_fwht=True) is not provided. */
int32_t ifr_bq_block_quant(const void* src, void* x_i8, float* x_sa, int64_t cols,
                           int64_t block, int64_t seq_len, uint64_t stream);

#ifdef __cplusplus
}
#endif

#endif /* INFERNO_HIP_H */
