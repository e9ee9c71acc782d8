// KV append for gfx950: RoPE + paged cache write (RopeCacheWriteKernel,
// kernels/rope.mojo:53-125), optionally preceded by the head RMS norm of
// dispatch_rms_norm_qkv_heads (kernels/rmsnorm.mojo:168-215), and the norm on
// its own.
//
// Grid: (tokens, head groups).  A head group is up to 8 heads of one kind --
// the q heads first, then the k heads, then the v heads -- so one token's
// append spreads over several CUs.  The token's run comes from the plan
// image's token -> run map, its slot from the run's base rows (PagedKV.slot,
// kernels/attention_ops.mojo:47-51).  q is rotated in place by work units
// that own whole rotation pairs (j, pair_stride + j) (and, with the norm,
// single unrotated elements), so no thread reads an element another writes.
#include "common.hpp"
#include "launch.hpp"

namespace ifr {
namespace {

constexpr int kGroupHeads = 8;

struct HeadGroup {
  int kind;    // 0: q heads, 1: k heads, 2: v heads
  int h0, h1;  // head range [h0, h1) of that kind
};

__host__ __device__ inline int groups_of(int heads) {
  return (heads + kGroupHeads - 1) / kGroupHeads;
}
__host__ __device__ inline int num_head_groups(int num_q, int num_kv) {
  return groups_of(num_q) + 2 * groups_of(num_kv);
}
__device__ inline HeadGroup head_group(int y, int num_q, int num_kv) {
  const int nq = groups_of(num_q), nk = groups_of(num_kv);
  if (y < nq) return {0, kGroupHeads * y, min(num_q, kGroupHeads * (y + 1))};
  y -= nq;
  if (y < nk) return {1, kGroupHeads * y, min(num_kv, kGroupHeads * (y + 1))};
  y -= nk;
  return {2, kGroupHeads * y, min(num_kv, kGroupHeads * (y + 1))};
}

// ---------------------------------------------------------------------------
// Head RMS norm (rms_norm_row, kernels/rmsnorm.mojo:37-48, applied per head
// row by ScaledNormKernel :130-153): sum of squares as the reference's
// dot_to_scalar(x, x) (kernels/dot_products.mojo:181-191) -- VDPBF16PS into
// pu accumulators of 16 lanes (odd product, then even, per lane), the
// accumulators added in order, then the halving-tree reduce over the 16
// lanes -- then inv = sqrt_n / sqrt(ssq + n_eps) and y = bf16((x*inv)*w)
// for q and k heads, bf16(x*inv) for v heads.  16 lanes compute one row's
// sum, so a 256-thread block covers a whole head group in one pass.
// ---------------------------------------------------------------------------
__device__ void group_inv_rms(const uint16_t* rows0, int n_rows, int head_dim, int pu,
                              float sqrt_n, float n_eps, float* inv) {
  const int j = threadIdx.x & 15;
  const int r = threadIdx.x >> 4;
  const int stride = 32 * pu;
  const bool live = r < n_rows;  // uniform per 16-lane group
  const uint16_t* row = rows0 + static_cast<int64_t>(live ? r : 0) * head_dim;
  float acc[8] = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
  for (int i = 0; i < head_dim / stride; ++i) {
#pragma unroll
    for (int p = 0; p < 8; ++p) {
      if (p >= pu) break;
      const uint32_t pair = *reinterpret_cast<const uint32_t*>(row + i * stride + 32 * p + 2 * j);
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
  // Halving tree over the 16 lanes: each step pairs lanes symmetrically,
  // so every lane ends with the bits of ((s0+s8)+(s4+s12)) + ... of lane 0.
  sum = sum + shfl_xor_f32(sum, 8);
  sum = sum + shfl_xor_f32(sum, 4);
  sum = sum + shfl_xor_f32(sum, 2);
  sum = sum + shfl_xor_f32(sum, 1);
  if (live && j == 0) inv[r] = sqrt_n / sqrtf(sum + n_eps);
  __syncthreads();
}

// One element after the norm, as the bf16 value the reference stores.
__device__ __forceinline__ float norm_elem(const uint16_t* row, float inv, const uint16_t* w,
                                           int e) {
  float y = bf16_to_f32(row[e]) * inv;
  if (w) y = y * bf16_to_f32(w[e]);
  return bf16_to_f32(static_cast<uint16_t>(f32_to_bf16_bits(y)));
}

// rotate_pair_to / rope_head_to (kernels/rope.mojo:16-50) on one pair.
__device__ __forceinline__ void rotate(float x_lo, float x_hi, float cv, float sv, float& lo,
                                       float& hi) {
  const float a = x_lo * cv, b = x_hi * sv;
  const float c = x_hi * cv, d = x_lo * sv;
  lo = a - b;
  hi = c + d;
}

template <bool kNorm>
__global__ __launch_bounds__(256) void append_kernel(
    const int32_t* __restrict__ image, uint16_t* __restrict__ q,
    const uint16_t* __restrict__ k_src, const uint16_t* __restrict__ v_src,
    uint16_t* __restrict__ k_cache, uint16_t* __restrict__ v_cache,
    const uint16_t* __restrict__ q_w, const uint16_t* __restrict__ k_w,
    const float* __restrict__ cos_table, const float* __restrict__ sin_table, int num_q,
    int num_kv, int shift, int row_mask, int page_mask, int half, int pair_stride,
    int head_dim, int pu, float sqrt_n, float n_eps) {
  __shared__ float inv[kGroupHeads];
  const int tok = blockIdx.x;
  const HeadGroup grp = head_group(blockIdx.y, num_q, num_kv);
  const int run = image[image[kHdrOffTokRun] + tok];
  const int32_t* rp = image + image[kHdrOffRuns] + run * 4;
  const int pos = rp[1] + (tok - rp[0]);
  const int32_t* rows = image + image[kHdrOffRows] + rp[2];
  const float* cos_row = cos_table + static_cast<int64_t>(pos) * half;
  const float* sin_row = sin_table + static_cast<int64_t>(pos) * half;
  const int64_t q_stride = static_cast<int64_t>(num_q) * head_dim;
  const int64_t kv_stride = static_cast<int64_t>(num_kv) * head_dim;
  const int n_heads = grp.h1 - grp.h0;

  if (grp.kind == 0) {
    uint16_t* qg = q + tok * q_stride + static_cast<int64_t>(grp.h0) * head_dim;
    if (kNorm) group_inv_rms(qg, n_heads, head_dim, pu, sqrt_n, n_eps, inv);
    // Units: rotation pairs, plus (with the norm) the unrotated elements.
    const int units = kNorm ? head_dim - half : half;
    const int gap = pair_stride - half;
    for (int idx = threadIdx.x; idx < n_heads * units; idx += blockDim.x) {
      const int h = idx / units, u = idx - h * units;
      uint16_t* qh = qg + static_cast<int64_t>(h) * head_dim;
      if (u < half) {
        const float x_lo = kNorm ? norm_elem(qh, inv[h], q_w, u) : bf16_to_f32(qh[u]);
        const float x_hi = kNorm ? norm_elem(qh, inv[h], q_w, pair_stride + u)
                                 : bf16_to_f32(qh[pair_stride + u]);
        float lo, hi;
        rotate(x_lo, x_hi, cos_row[u], sin_row[u], lo, hi);
        qh[u] = static_cast<uint16_t>(f32_to_bf16_bits(lo));
        qh[pair_stride + u] = static_cast<uint16_t>(f32_to_bf16_bits(hi));
      } else {
        const int v = u - half;
        const int e = v < gap ? half + v : pair_stride + half + (v - gap);
        qh[e] = static_cast<uint16_t>(f32_to_bf16_bits(norm_elem(qh, inv[h], q_w, e)));
      }
    }
    return;
  }

  const int64_t slot =
      static_cast<int64_t>(rows[(pos >> shift) & page_mask]) + (pos & row_mask);
  const int64_t g_off = static_cast<int64_t>(grp.h0) * head_dim;
  if (grp.kind == 1) {
    const uint16_t* kg = k_src + tok * kv_stride + g_off;
    uint16_t* dg = k_cache + slot * kv_stride + g_off;
    if (kNorm) group_inv_rms(kg, n_heads, head_dim, pu, sqrt_n, n_eps, inv);
    for (int idx = threadIdx.x; idx < n_heads * head_dim; idx += blockDim.x) {
      const int h = idx / head_dim, e = idx - h * head_dim;
      const uint16_t* s = kg + static_cast<int64_t>(h) * head_dim;
      uint16_t* d = dg + static_cast<int64_t>(h) * head_dim;
      const float iv = kNorm ? inv[h] : 0.0f;
      auto x = [&](int i) { return kNorm ? norm_elem(s, iv, k_w, i) : bf16_to_f32(s[i]); };
      if (e < half) {
        float lo, hi;
        rotate(x(e), x(pair_stride + e), cos_row[e], sin_row[e], lo, hi);
        d[e] = static_cast<uint16_t>(f32_to_bf16_bits(lo));
      } else if (e >= pair_stride && e < pair_stride + half) {
        const int jj = e - pair_stride;
        float lo, hi;
        rotate(x(jj), x(e), cos_row[jj], sin_row[jj], lo, hi);
        d[e] = static_cast<uint16_t>(f32_to_bf16_bits(hi));
      } else {
        d[e] = kNorm ? static_cast<uint16_t>(f32_to_bf16_bits(x(e))) : s[e];
      }
    }
    return;
  }

  const uint16_t* vg = v_src + tok * kv_stride + g_off;
  uint16_t* dg = v_cache + slot * kv_stride + g_off;
  const int n_elem = n_heads * head_dim;
  if (kNorm) {
    group_inv_rms(vg, n_heads, head_dim, pu, sqrt_n, n_eps, inv);
    for (int idx = threadIdx.x; idx < n_elem; idx += blockDim.x) {
      const int h = idx / head_dim, e = idx - h * head_dim;
      dg[idx] = static_cast<uint16_t>(
          f32_to_bf16_bits(norm_elem(vg + static_cast<int64_t>(h) * head_dim, inv[h], nullptr, e)));
    }
  } else if ((n_elem & 7) == 0 && ((reinterpret_cast<uintptr_t>(vg) |
                                     reinterpret_cast<uintptr_t>(dg)) & 15) == 0) {
    const uint4* vs = reinterpret_cast<const uint4*>(vg);
    uint4* vd = reinterpret_cast<uint4*>(dg);
    for (int i = threadIdx.x; i < n_elem / 8; i += blockDim.x) vd[i] = vs[i];
  } else {
    for (int i = threadIdx.x; i < n_elem; i += blockDim.x) dg[i] = vg[i];
  }
}

// The append without the norm on 16-byte vectors.  A q unit owns 8
// consecutive rotation pairs (j .. j+7 with their partners at pair_stride +
// j), a k unit 8 rotation pairs or 8 unrotated elements, a v unit 8
// elements, so every source element is read once and every output element
// written once, all with 16-byte loads and stores; each unit issues its
// loads before any of its math.  The rotation of every pair is rotate()'s, so
// the bits equal append_kernel<false>'s.  Requires half, pair_stride and
// head_dim to be multiples of 8 and every base 16-byte aligned (checked by
// the launcher).
__device__ __forceinline__ void unpack8_bf16(const uint4& w, float* f) {
  const uint32_t x[4] = {w.x, w.y, w.z, w.w};
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    f[2 * i] = bf16_lo(x[i]);
    f[2 * i + 1] = bf16_hi(x[i]);
  }
}
__device__ __forceinline__ uint32_t pack2_bf16(float a, float b) {
  return f32_to_bf16_bits(a) | (f32_to_bf16_bits(b) << 16);
}
__device__ __forceinline__ void rotate8(const uint4& lo_in, const uint4& hi_in, const float4& c0,
                                        const float4& c1, const float4& s0, const float4& s1,
                                        uint4& lo_out, uint4& hi_out) {
  float xl[8], xh[8], lo[8], hi[8];
  unpack8_bf16(lo_in, xl);
  unpack8_bf16(hi_in, xh);
  const float c[8] = {c0.x, c0.y, c0.z, c0.w, c1.x, c1.y, c1.z, c1.w};
  const float sn[8] = {s0.x, s0.y, s0.z, s0.w, s1.x, s1.y, s1.z, s1.w};
#pragma unroll
  for (int i = 0; i < 8; ++i) rotate(xl[i], xh[i], c[i], sn[i], lo[i], hi[i]);
  lo_out = make_uint4(pack2_bf16(lo[0], lo[1]), pack2_bf16(lo[2], lo[3]),
                      pack2_bf16(lo[4], lo[5]), pack2_bf16(lo[6], lo[7]));
  hi_out = make_uint4(pack2_bf16(hi[0], hi[1]), pack2_bf16(hi[2], hi[3]),
                      pack2_bf16(hi[4], hi[5]), pack2_bf16(hi[6], hi[7]));
}

__global__ __launch_bounds__(128) void append_vec_kernel(
    const int32_t* __restrict__ image, uint16_t* __restrict__ q,
    const uint16_t* __restrict__ k_src, const uint16_t* __restrict__ v_src,
    uint16_t* __restrict__ k_cache, uint16_t* __restrict__ v_cache,
    const float* __restrict__ cos_table, const float* __restrict__ sin_table, int num_q,
    int num_kv, int shift, int row_mask, int page_mask, int half, int pair_stride,
    int head_dim) {
  const int tok = blockIdx.x;
  const HeadGroup grp = head_group(blockIdx.y, num_q, num_kv);
  const int n_heads = grp.h1 - grp.h0;
  const int pairs8 = half >> 3;
  const int gap = pair_stride - half;
  const int units_k = pairs8 + ((head_dim - 2 * half) >> 3);
  const int64_t q_stride = static_cast<int64_t>(num_q) * head_dim;
  const int64_t kv_stride = static_cast<int64_t>(num_kv) * head_dim;
  const int64_t g_off = static_cast<int64_t>(grp.h0) * head_dim;
  const int run = image[image[kHdrOffTokRun] + tok];
  const int32_t* rp = image + image[kHdrOffRuns] + run * 4;
  const int pos = rp[1] + (tok - rp[0]);
  const float* cos_row = cos_table + static_cast<int64_t>(pos) * half;
  const float* sin_row = sin_table + static_cast<int64_t>(pos) * half;

  if (grp.kind == 0) {
    uint16_t* qg = q + tok * q_stride + g_off;
    for (int u = threadIdx.x; u < n_heads * pairs8; u += blockDim.x) {
      const int h = u / pairs8, j = (u - h * pairs8) * 8;
      uint16_t* qh = qg + static_cast<int64_t>(h) * head_dim;
      const uint4 xl = *reinterpret_cast<const uint4*>(qh + j);
      const uint4 xh = *reinterpret_cast<const uint4*>(qh + pair_stride + j);
      const float4 c0 = *reinterpret_cast<const float4*>(cos_row + j);
      const float4 c1 = *reinterpret_cast<const float4*>(cos_row + j + 4);
      const float4 s0 = *reinterpret_cast<const float4*>(sin_row + j);
      const float4 s1 = *reinterpret_cast<const float4*>(sin_row + j + 4);
      uint4 lo, hi;
      rotate8(xl, xh, c0, c1, s0, s1, lo, hi);
      *reinterpret_cast<uint4*>(qh + j) = lo;
      *reinterpret_cast<uint4*>(qh + pair_stride + j) = hi;
    }
    return;
  }

  const int32_t* rows = image + image[kHdrOffRows] + rp[2];
  const int64_t slot =
      static_cast<int64_t>(rows[(pos >> shift) & page_mask]) + (pos & row_mask);
  if (grp.kind == 1) {
    const uint16_t* kg = k_src + tok * kv_stride + g_off;
    uint16_t* dg = k_cache + slot * kv_stride + g_off;
    for (int u = threadIdx.x; u < n_heads * units_k; u += blockDim.x) {
      const int h = u / units_k, r = u - h * units_k;
      const uint16_t* sh = kg + static_cast<int64_t>(h) * head_dim;
      uint16_t* dh = dg + static_cast<int64_t>(h) * head_dim;
      if (r < pairs8) {
        const int j = r * 8;
        const uint4 xl = *reinterpret_cast<const uint4*>(sh + j);
        const uint4 xh = *reinterpret_cast<const uint4*>(sh + pair_stride + j);
        const float4 c0 = *reinterpret_cast<const float4*>(cos_row + j);
        const float4 c1 = *reinterpret_cast<const float4*>(cos_row + j + 4);
        const float4 s0 = *reinterpret_cast<const float4*>(sin_row + j);
        const float4 s1 = *reinterpret_cast<const float4*>(sin_row + j + 4);
        uint4 lo, hi;
        rotate8(xl, xh, c0, c1, s0, s1, lo, hi);
        *reinterpret_cast<uint4*>(dh + j) = lo;
        *reinterpret_cast<uint4*>(dh + pair_stride + j) = hi;
      } else {
        const int v = (r - pairs8) * 8;
        const int e = v < gap ? half + v : pair_stride + half + (v - gap);
        *reinterpret_cast<uint4*>(dh + e) = *reinterpret_cast<const uint4*>(sh + e);
      }
    }
    return;
  }

  const uint4* vs = reinterpret_cast<const uint4*>(v_src + tok * kv_stride + g_off);
  uint4* vd = reinterpret_cast<uint4*>(v_cache + slot * kv_stride + g_off);
  for (int i = threadIdx.x; i < (n_heads * head_dim) >> 3; i += blockDim.x) vd[i] = vs[i];
}

// In-place head RMS norm of q, k and v (one block per token and head group).
__global__ __launch_bounds__(256) void rms_norm_qkv_kernel(
    uint16_t* __restrict__ q, uint16_t* __restrict__ k, uint16_t* __restrict__ v,
    const uint16_t* __restrict__ q_w, const uint16_t* __restrict__ k_w, int num_q, int num_kv,
    int head_dim, int pu, float sqrt_n, float n_eps) {
  __shared__ float inv[kGroupHeads];
  const int64_t tok = blockIdx.x;
  const HeadGroup grp = head_group(blockIdx.y, num_q, num_kv);
  const int heads = grp.kind == 0 ? num_q : num_kv;
  uint16_t* base = grp.kind == 0 ? q : (grp.kind == 1 ? k : v);
  const uint16_t* w = grp.kind == 0 ? q_w : (grp.kind == 1 ? k_w : nullptr);
  uint16_t* rows0 = base + (tok * heads + grp.h0) * head_dim;
  const int n_heads = grp.h1 - grp.h0;
  group_inv_rms(rows0, n_heads, head_dim, pu, sqrt_n, n_eps, inv);
  for (int idx = threadIdx.x; idx < n_heads * head_dim; idx += blockDim.x) {
    const int h = idx / head_dim, e = idx - h * head_dim;
    uint16_t* row = rows0 + static_cast<int64_t>(h) * head_dim;
    float y = bf16_to_f32(row[e]) * inv[h];
    if (w) y = y * bf16_to_f32(w[e]);
    row[e] = static_cast<uint16_t>(f32_to_bf16_bits(y));
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
  const uintptr_t bases = reinterpret_cast<uintptr_t>(q) | reinterpret_cast<uintptr_t>(k_src) |
                          reinterpret_cast<uintptr_t>(v_src) |
                          reinterpret_cast<uintptr_t>(k_cache) |
                          reinterpret_cast<uintptr_t>(v_cache) |
                          reinterpret_cast<uintptr_t>(cos_table) |
                          reinterpret_cast<uintptr_t>(sin_table);
  if ((bases & 15) == 0 && half % 8 == 0 && pair_stride % 8 == 0 && head_dim % 8 == 0) {
    hipLaunchKernelGGL(append_vec_kernel, dim3(seq_len, num_head_groups(num_q, num_kv)),
                       dim3(128), 0, stream, image, static_cast<uint16_t*>(q),
                       static_cast<const uint16_t*>(k_src), static_cast<const uint16_t*>(v_src),
                       static_cast<uint16_t*>(k_cache), static_cast<uint16_t*>(v_cache),
                       cos_table, sin_table, num_q, num_kv, geom.shift, geom.row_mask,
                       geom.page_mask, half, pair_stride, head_dim);
    return hipGetLastError();
  }
  hipLaunchKernelGGL(append_kernel<false>, dim3(seq_len, num_head_groups(num_q, num_kv)),
                     dim3(256), 0, stream, image, static_cast<uint16_t*>(q),
                     static_cast<const uint16_t*>(k_src), static_cast<const uint16_t*>(v_src),
                     static_cast<uint16_t*>(k_cache), static_cast<uint16_t*>(v_cache), nullptr,
                     nullptr, cos_table, sin_table, num_q, num_kv, geom.shift, geom.row_mask,
                     geom.page_mask, half, pair_stride, head_dim, 1, 0.0f, 0.0f);
  return hipGetLastError();
}

hipError_t launch_rms_norm_qkv(void* q, void* k, void* v, const void* q_w, const void* k_w,
                               int seq_len, int num_q, int num_kv, int head_dim, float sqrt_n,
                               float n_eps, hipStream_t stream) {
  if (seq_len <= 0) return hipSuccess;
  hipLaunchKernelGGL(rms_norm_qkv_kernel, dim3(seq_len, num_head_groups(num_q, num_kv)),
                     dim3(256), 0, stream, static_cast<uint16_t*>(q), static_cast<uint16_t*>(k),
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
  hipLaunchKernelGGL(append_kernel<true>, dim3(seq_len, num_head_groups(num_q, num_kv)),
                     dim3(256), 0, stream, image, static_cast<uint16_t*>(q),
                     static_cast<const uint16_t*>(k_src), static_cast<const uint16_t*>(v_src),
                     static_cast<uint16_t*>(k_cache), static_cast<uint16_t*>(v_cache),
                     static_cast<const uint16_t*>(q_w), static_cast<const uint16_t*>(k_w),
                     cos_table, sin_table, num_q, num_kv, geom.shift, geom.row_mask,
                     geom.page_mask, half, pair_stride, head_dim, port_unroll_for(head_dim),
                     sqrt_n, n_eps);
  return hipGetLastError();
}

}  // namespace ifr
