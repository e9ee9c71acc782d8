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

// ---------------------------------------------------------------------------
// Head RMS norm (dispatch_rms_norm_qkv_heads, kernels/rmsnorm.mojo:168-215),
// alone or fused ahead of the append.  Per head row: the reference's
// dot_to_scalar(x, x) (kernels/dot_products.mojo:181-191) -- VDPBF16PS into
// pu accumulators of 16 lanes (odd product, then even, per lane), the
// accumulators added in order, then the halving-tree reduce over the 16
// lanes -- then inv = sqrt_n / sqrt(ssq + n_eps) and y = bf16((x*inv)*w)
// for q and k heads, bf16(x*inv) for v heads.  16 lanes compute one row's
// sum, so a 256-thread block covers 16 rows per pass.
// ---------------------------------------------------------------------------
constexpr int kMaxNormHeads = 192;  // num_q + 2 * num_kv

__device__ __forceinline__ const uint16_t* head_row(const uint16_t* q_tok,
                                                    const uint16_t* k_tok,
                                                    const uint16_t* v_tok, int r, int num_q,
                                                    int num_kv, int head_dim) {
  if (r < num_q) return q_tok + static_cast<int64_t>(r) * head_dim;
  if (r < num_q + num_kv) return k_tok + static_cast<int64_t>(r - num_q) * head_dim;
  return v_tok + static_cast<int64_t>(r - num_q - num_kv) * head_dim;
}

// Fills inv[r] for the token's num_q + 2*num_kv head rows.  Ends with a
// barrier.
__device__ void head_inv_rms_rows(const uint16_t* q_tok, const uint16_t* k_tok,
                                  const uint16_t* v_tok, int num_q, int num_kv, int head_dim,
                                  int pu, float sqrt_n, float n_eps, float* inv) {
  const int rows = num_q + 2 * num_kv;
  const int j = threadIdx.x & 15;
  const int stride = 32 * pu;
  for (int r0 = 0; r0 < rows; r0 += blockDim.x / 16) {
    const int r = r0 + (threadIdx.x >> 4);
    const bool live = r < rows;  // uniform per 16-lane group
    const uint16_t* row = head_row(q_tok, k_tok, v_tok, live ? r : 0, num_q, num_kv, head_dim);
    float acc[8] = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
    for (int i = 0; i < head_dim / stride; ++i) {
#pragma unroll
      for (int p = 0; p < 8; ++p) {
        if (p >= pu) break;
        const uint32_t pair =
            *reinterpret_cast<const uint32_t*>(row + i * stride + 32 * p + 2 * j);
        const float xe = bf16_lo(pair), xo = bf16_hi(pair);
        float a = acc[p];
        a = a + xo * xo;
        a = a + xe * xe;
        acc[p] = a;
      }
    }
    float sum = 0.0f;
#pragma unroll
    for (int p = 0; p < 8; ++p)
      if (p < pu) sum = sum + acc[p];
    // Halving tree over the 16 lanes: every lane of the group ends with the
    // bits of lane 0's ((s0+s8)+(s4+s12)) + ... (each step pairs lanes
    // symmetrically, so all lanes agree).
    sum = sum + shfl_xor_f32(sum, 8);
    sum = sum + shfl_xor_f32(sum, 4);
    sum = sum + shfl_xor_f32(sum, 2);
    sum = sum + shfl_xor_f32(sum, 1);
    if (live && j == 0) inv[r] = sqrt_n / sqrtf(sum + n_eps);
  }
  __syncthreads();
}

__device__ __forceinline__ float norm_elem(const uint16_t* row, float inv, const uint16_t* w,
                                           int e) {
  float y = bf16_to_f32(row[e]) * inv;
  if (w) y = y * bf16_to_f32(w[e]);
  return bf16_to_f32(static_cast<uint16_t>(f32_to_bf16_bits(y)));
}

// In-place norm of every head of each token (one block per token).
__global__ __launch_bounds__(256) void rms_norm_qkv_kernel(
    uint16_t* __restrict__ q, uint16_t* __restrict__ k, uint16_t* __restrict__ v,
    const uint16_t* __restrict__ q_w, const uint16_t* __restrict__ k_w, int num_q, int num_kv,
    int head_dim, int pu, float sqrt_n, float n_eps) {
  __shared__ float inv[kMaxNormHeads];
  const int64_t tok = blockIdx.x;
  uint16_t* q_tok = q + tok * num_q * head_dim;
  uint16_t* k_tok = k + tok * num_kv * head_dim;
  uint16_t* v_tok = v + tok * num_kv * head_dim;
  head_inv_rms_rows(q_tok, k_tok, v_tok, num_q, num_kv, head_dim, pu, sqrt_n, n_eps, inv);
  const int rows = num_q + 2 * num_kv;
  for (int idx = threadIdx.x; idx < rows * head_dim; idx += blockDim.x) {
    const int r = idx / head_dim, e = idx - r * head_dim;
    uint16_t* row = const_cast<uint16_t*>(head_row(q_tok, k_tok, v_tok, r, num_q, num_kv,
                                                   head_dim));
    const uint16_t* w = r < num_q ? q_w : (r < num_q + num_kv ? k_w : nullptr);
    float y = bf16_to_f32(row[e]) * inv[r];
    if (w) y = y * bf16_to_f32(w[e]);
    row[e] = static_cast<uint16_t>(f32_to_bf16_bits(y));
  }
}

// Norm fused ahead of the append: q normalised and rotated in place, k
// normalised, rotated and written to its cache slot, v normalised into its
// slot.  k_src and v_src are only read.
__global__ __launch_bounds__(256) void rms_rope_cache_write_kernel(
    const int32_t* __restrict__ image, uint16_t* __restrict__ q,
    const uint16_t* __restrict__ k_src, const uint16_t* __restrict__ v_src,
    uint16_t* __restrict__ k_cache, uint16_t* __restrict__ v_cache,
    const uint16_t* __restrict__ q_w, const uint16_t* __restrict__ k_w,
    const float* __restrict__ cos_table, const float* __restrict__ sin_table, int num_q,
    int num_kv, int shift, int row_mask, int page_mask, int half, int pair_stride,
    int head_dim, int pu, float sqrt_n, float n_eps) {
  __shared__ float inv[kMaxNormHeads];
  const int tok = blockIdx.x;
  const int run = image[image[kHdrOffTokRun] + tok];
  const int32_t* rp = image + image[kHdrOffRuns] + run * 4;
  const int pos = rp[1] + (tok - rp[0]);
  const int32_t* rows = image + image[kHdrOffRows] + rp[2];
  const float* cos_row = cos_table + static_cast<int64_t>(pos) * half;
  const float* sin_row = sin_table + static_cast<int64_t>(pos) * half;
  const int64_t q_stride = static_cast<int64_t>(num_q) * head_dim;
  const int64_t kv_stride = static_cast<int64_t>(num_kv) * head_dim;
  uint16_t* q_tok = q + tok * q_stride;
  const uint16_t* k_tok = k_src + tok * kv_stride;
  const uint16_t* v_tok = v_src + tok * kv_stride;
  head_inv_rms_rows(q_tok, k_tok, v_tok, num_q, num_kv, head_dim, pu, sqrt_n, n_eps, inv);

  // q: units of one rotation pair (j, pair_stride + j) or one unrotated
  // element, so no thread reads an element another thread writes.
  const int units = head_dim - half;
  const int gap = pair_stride - half;  // unrotated elements between the halves
  for (int idx = threadIdx.x; idx < num_q * units; idx += blockDim.x) {
    const int h = idx / units, u = idx - h * units;
    uint16_t* qh = q_tok + static_cast<int64_t>(h) * head_dim;
    const float iv = inv[h];
    if (u < half) {
      const float x_lo = norm_elem(qh, iv, q_w, u);
      const float x_hi = norm_elem(qh, iv, q_w, pair_stride + u);
      const float cv = cos_row[u], sv = sin_row[u];
      const float a = x_lo * cv, b = x_hi * sv;
      const float c = x_hi * cv, d = x_lo * sv;
      qh[u] = static_cast<uint16_t>(f32_to_bf16_bits(a - b));
      qh[pair_stride + u] = static_cast<uint16_t>(f32_to_bf16_bits(c + d));
    } else {
      const int v = u - half;
      const int e = v < gap ? half + v : pair_stride + half + (v - gap);
      qh[e] = static_cast<uint16_t>(f32_to_bf16_bits(norm_elem(qh, iv, q_w, e)));
    }
  }

  const int64_t slot =
      static_cast<int64_t>(rows[(pos >> shift) & page_mask]) + (pos & row_mask);
  uint16_t* k_dst = k_cache + slot * kv_stride;
  for (int idx = threadIdx.x; idx < num_kv * head_dim; idx += blockDim.x) {
    const int h = idx / head_dim, e = idx - h * head_dim;
    const uint16_t* s = k_tok + static_cast<int64_t>(h) * head_dim;
    uint16_t* d = k_dst + static_cast<int64_t>(h) * head_dim;
    const float iv = inv[num_q + h];
    if (e < half) {
      const float x_lo = norm_elem(s, iv, k_w, e);
      const float x_hi = norm_elem(s, iv, k_w, pair_stride + e);
      const float cv = cos_row[e], sv = sin_row[e];
      const float a = x_lo * cv, b = x_hi * sv;
      d[e] = static_cast<uint16_t>(f32_to_bf16_bits(a - b));
    } else if (e >= pair_stride && e < pair_stride + half) {
      const int jj = e - pair_stride;
      const float x_lo = norm_elem(s, iv, k_w, jj);
      const float x_hi = norm_elem(s, iv, k_w, e);
      const float cv = cos_row[jj], sv = sin_row[jj];
      const float c = x_hi * cv, dd = x_lo * sv;
      d[e] = static_cast<uint16_t>(f32_to_bf16_bits(c + dd));
    } else {
      d[e] = static_cast<uint16_t>(f32_to_bf16_bits(norm_elem(s, iv, k_w, e)));
    }
  }
  uint16_t* v_dst = v_cache + slot * kv_stride;
  for (int idx = threadIdx.x; idx < num_kv * head_dim; idx += blockDim.x) {
    const int h = idx / head_dim, e = idx - h * head_dim;
    const uint16_t* s = v_tok + static_cast<int64_t>(h) * head_dim;
    v_dst[static_cast<int64_t>(h) * head_dim + e] = static_cast<uint16_t>(
        f32_to_bf16_bits(norm_elem(s, inv[num_q + num_kv + h], nullptr, e)));
  }
}

int port_unroll_for(int head_dim) {  // pick_port_unroll[32, head_dim]
  for (int pu = 8; pu > 1; pu >>= 1)
    if (head_dim % (32 * pu) == 0) return pu;
  return 1;
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

namespace ifr {

hipError_t launch_rms_norm_qkv(void* q, void* k, void* v, const void* q_w, const void* k_w,
                               int seq_len, int num_q, int num_kv, int head_dim, float sqrt_n,
                               float n_eps, hipStream_t stream) {
  if (seq_len <= 0) return hipSuccess;
  hipLaunchKernelGGL(rms_norm_qkv_kernel, dim3(seq_len), dim3(256), 0, stream,
                     static_cast<uint16_t*>(q), static_cast<uint16_t*>(k),
                     static_cast<uint16_t*>(v), static_cast<const uint16_t*>(q_w),
                     static_cast<const uint16_t*>(k_w), num_q, num_kv, head_dim,
                     port_unroll_for(head_dim), sqrt_n, n_eps);
  return hipGetLastError();
}

hipError_t launch_rms_rope_cache_write(const int32_t* image, int seq_len, void* q,
                                       const void* k_src, const void* v_src, void* k_cache,
                                       void* v_cache, const void* q_w, const void* k_w,
                                       const float* cos_table, const float* sin_table,
                                       int num_q, int num_kv, PagedGeom geom, int half,
                                       int pair_stride, int head_dim, float sqrt_n,
                                       float n_eps, hipStream_t stream) {
  if (seq_len <= 0) return hipSuccess;
  hipLaunchKernelGGL(rms_rope_cache_write_kernel, dim3(seq_len), dim3(256), 0, stream, image,
                     static_cast<uint16_t*>(q), static_cast<const uint16_t*>(k_src),
                     static_cast<const uint16_t*>(v_src), static_cast<uint16_t*>(k_cache),
                     static_cast<uint16_t*>(v_cache), static_cast<const uint16_t*>(q_w),
                     static_cast<const uint16_t*>(k_w), cos_table, sin_table, num_q, num_kv,
                     geom.shift, geom.row_mask, geom.page_mask, half, pair_stride, head_dim,
                     port_unroll_for(head_dim), sqrt_n, n_eps);
  return hipGetLastError();
}

}  // namespace ifr
