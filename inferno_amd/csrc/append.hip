// KV append: RoPE + paged cache write (RopeCacheWriteKernel,
// kernels/rope.mojo:53-125) for gfx950.  One workgroup per token.  The
// token's run comes from the plan image's token -> run map, its slot from the
// run's base rows (PagedKV.slot, kernels/attention_ops.mojo:47-51).  Each
// thread owns whole rotation pairs (j, pair_stride + j), so the in-place
// rotation of q has no read/write overlap between threads.
#include "common.hpp"
#include "launch.hpp"

namespace ifr {
namespace {

__global__ __launch_bounds__(256) void rope_cache_write_kernel(
    const int32_t* __restrict__ image, uint16_t* __restrict__ q,
    const uint16_t* __restrict__ k_src, const uint16_t* __restrict__ v_src,
    uint16_t* __restrict__ k_cache, uint16_t* __restrict__ v_cache,
    const float* __restrict__ cos_table, const float* __restrict__ sin_table,
    int num_q, int num_kv, int shift, int row_mask, int page_mask, int half,
    int pair_stride, int head_dim) {
  const int tok = blockIdx.x;
  const int run = image[image[kHdrOffTokRun] + tok];
  const int32_t* rp = image + image[kHdrOffRuns] + run * 4;
  const int pos = rp[1] + (tok - rp[0]);
  const int32_t* rows = image + image[kHdrOffRows] + rp[2];
  const float* cos_row = cos_table + static_cast<int64_t>(pos) * half;
  const float* sin_row = sin_table + static_cast<int64_t>(pos) * half;
  const int64_t q_stride = static_cast<int64_t>(num_q) * head_dim;
  const int64_t kv_stride = static_cast<int64_t>(num_kv) * head_dim;

  // rotate_pair_to on every q head, in place (kernels/rope.mojo:16-35).
  uint16_t* q_tok = q + tok * q_stride;
  for (int idx = threadIdx.x; idx < num_q * half; idx += blockDim.x) {
    const int h = idx / half, j = idx - h * half;
    uint16_t* qh = q_tok + static_cast<int64_t>(h) * head_dim;
    const float x_lo = bf16_to_f32(qh[j]);
    const float x_hi = bf16_to_f32(qh[pair_stride + j]);
    const float cv = cos_row[j], sv = sin_row[j];
    const float a = x_lo * cv, b = x_hi * sv;
    const float c = x_hi * cv, d = x_lo * sv;
    qh[j] = static_cast<uint16_t>(f32_to_bf16_bits(a - b));
    qh[pair_stride + j] = static_cast<uint16_t>(f32_to_bf16_bits(c + d));
  }

  // rope_head_to for k into the cache slot, then memcpy of v
  // (kernels/rope.mojo:38-50,108-120).  cache_degree is 1.
  const int64_t slot =
      static_cast<int64_t>(rows[(pos >> shift) & page_mask]) + (pos & row_mask);
  const uint16_t* k_tok = k_src + tok * kv_stride;
  uint16_t* k_dst = k_cache + slot * kv_stride;
  for (int idx = threadIdx.x; idx < num_kv * head_dim; idx += blockDim.x) {
    const int h = idx / head_dim, e = idx - h * head_dim;
    const uint16_t* s = k_tok + static_cast<int64_t>(h) * head_dim;
    uint16_t* d = k_dst + static_cast<int64_t>(h) * head_dim;
    if (e < half) {
      const float x_lo = bf16_to_f32(s[e]);
      const float x_hi = bf16_to_f32(s[pair_stride + e]);
      const float cv = cos_row[e], sv = sin_row[e];
      const float a = x_lo * cv, b = x_hi * sv;
      d[e] = static_cast<uint16_t>(f32_to_bf16_bits(a - b));
    } else if (e >= pair_stride && e < pair_stride + half) {
      const int j = e - pair_stride;
      const float x_lo = bf16_to_f32(s[j]);
      const float x_hi = bf16_to_f32(s[e]);
      const float cv = cos_row[j], sv = sin_row[j];
      const float c = x_hi * cv, dd = x_lo * sv;
      d[e] = static_cast<uint16_t>(f32_to_bf16_bits(c + dd));
    } else {
      d[e] = s[e];
    }
  }
  const uint16_t* v_tok = v_src + tok * kv_stride;
  uint16_t* v_dst = v_cache + slot * kv_stride;
  if ((kv_stride & 7) == 0) {
    const uint4* vs = reinterpret_cast<const uint4*>(v_tok);
    uint4* vd = reinterpret_cast<uint4*>(v_dst);
    for (int64_t i = threadIdx.x; i < kv_stride / 8; i += blockDim.x) vd[i] = vs[i];
  } else {
    for (int64_t i = threadIdx.x; i < kv_stride; i += blockDim.x) v_dst[i] = v_tok[i];
  }
}

}  // namespace

hipError_t launch_rope_cache_write(const int32_t* image, int seq_len, void* q,
                                   const void* k_src, const void* v_src,
                                   void* k_cache, void* v_cache,
                                   const float* cos_table,
                                   const float* sin_table, int num_q,
                                   int num_kv, PagedGeom geom, int half,
                                   int pair_stride, int head_dim,
                                   hipStream_t stream) {
  if (seq_len <= 0) return hipSuccess;
  hipLaunchKernelGGL(rope_cache_write_kernel, dim3(seq_len), dim3(256), 0,
                     stream, image, static_cast<uint16_t*>(q),
                     static_cast<const uint16_t*>(k_src),
                     static_cast<const uint16_t*>(v_src),
                     static_cast<uint16_t*>(k_cache),
                     static_cast<uint16_t*>(v_cache), cos_table, sin_table,
                     num_q, num_kv, geom.shift, geom.row_mask, geom.page_mask,
                     half, pair_stride, head_dim);
  return hipGetLastError();
}

}  // namespace ifr
