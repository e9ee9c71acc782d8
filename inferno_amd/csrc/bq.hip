// Butterquant int8 KV for gfx950: the quantizing KV append (BqAttnPrepKernel,
// butterquant_kernels/attention.mojo:494-582) and the int8 paged split-KV
// attention (bq_process_kv_tile / BqFlashAttentionKernel, :27-167), whose
// partials feed the shared log-sum-exp merge.
//
// Prep (bq_prep_rows_kernel: 16 lanes per head, four heads per wave, for the
// Gemma-4 layer shapes; bq_prep_kernel below, one wave per head, for any
// other RoPE split).  One wave per head (D = 256 or 512, lane L owns elements
// EPL*L .. EPL*L + EPL - 1, EPL = D/64):
//   RMS     the reference's lane-wise chain over 16 AVX-512 lanes
//           (butterquant/head_prep.mojo:9-16) is replayed exactly: lane
//           j < 16 runs ssq_j = x_j^2, then fma(x_{16ri+j}, x_{16ri+j}, ssq_j)
//           for ri = 1 .. D/16 - 1, and the 16 partial sums are tree-reduced.
//   RoPE    partner elements arrive with ds_bpermute; no FMA contraction.
//   FWHT    strides below EPL inside the lane, the rest across lanes (xor 1..32);
//           the lower element of each pair becomes a+b, the upper a-b, in the
//           reference's stage order (butterquant/fwht.mojo:20-57), so the
//           rotated values -- and with them the int8 codes -- are the
//           reference's bit for bit.
//   absmax  wave max, 127/amax, round-to-nearest-even, clamp [-128, 127].
// Attention (head_dim 256, gqa 2; head_dim 512 with gqa 8 runs the kernel of
// attention_wide.hip), one wave per (work item, kv head): 4 lanes per position, 16
// positions per pass (one tile); integer scores with v_dot4_i32_i8 (exact),
// scaled as (((float)dot * f_q) * k_scale) / 127^2 like the reference; PV with
// lane L owning output dims 4L..4L+3 and fma in position order.
#include <type_traits>

#include "common.hpp"
#include "launch.hpp"

namespace ifr {
namespace {

constexpr int kBqD = 256;  // head_dim of bq_partial_kernel

__device__ __forceinline__ float bpermute_f32(float v, int src_lane) {
  return __int_as_float(__builtin_amdgcn_ds_bpermute(src_lane << 2, __float_as_int(v)));
}

// v[lane ^ M] for M = 1 .. 32 on the VALU: DPP inside 16-lane rows (xor 4 as
// the rotate by 12 or by 4, picked by lane bit 2), the gfx950 lane swaps
// across rows (with v as both operands the results are the pair's lower and
// upper members).
constexpr int kDppRowRor12 = 0x12C;  // lane i <- (i-12)%16 = (i+4)%16 within 16 lanes
template <int M>
__device__ __forceinline__ uint32_t xor_lane_u32(uint32_t v, int lane) {
  if constexpr (M == 1) {
    return __builtin_amdgcn_update_dpp(0, v, kDppXor1, 0xF, 0xF, true);
  } else if constexpr (M == 2) {
    return __builtin_amdgcn_update_dpp(0, v, kDppXor2, 0xF, 0xF, true);
  } else if constexpr (M == 4) {
    // row_ror:n gives lane i the value of lane (i - n) mod 16.
    const uint32_t a = __builtin_amdgcn_update_dpp(0, v, kDppRowRor4, 0xF, 0xF, true);
    const uint32_t b = __builtin_amdgcn_update_dpp(0, v, kDppRowRor12, 0xF, 0xF, true);
    return (lane & 4) ? a : b;
  } else if constexpr (M == 8) {
    return __builtin_amdgcn_update_dpp(0, v, kDppRowRor8, 0xF, 0xF, true);
  } else if constexpr (M == 16) {
    const auto r = __builtin_amdgcn_permlane16_swap(v, v, false, false);
    return (lane & 16) ? r[0] : r[1];
  } else {
    const auto r = __builtin_amdgcn_permlane32_swap(v, v, false, false);
    return (lane & 32) ? r[0] : r[1];
  }
}
template <int M>
__device__ __forceinline__ float xor_lane_f32(float v, int lane) {
  return __uint_as_float(xor_lane_u32<M>(__float_as_uint(v), lane));
}
template <int M>
__device__ __forceinline__ int xor_lane_i32(int v, int lane) {
  return static_cast<int>(xor_lane_u32<M>(static_cast<uint32_t>(v), lane));
}
// f(x, x[lane ^ M]) for M = 1, 2, 4, .., 32 in that order.
template <typename T, typename F>
__device__ __forceinline__ T butterfly_all(T x, int lane, F f) {
  if constexpr (std::is_same<T, float>::value) {
    x = f(x, xor_lane_f32<1>(x, lane));
    x = f(x, xor_lane_f32<2>(x, lane));
    x = f(x, xor_lane_f32<4>(x, lane));
    x = f(x, xor_lane_f32<8>(x, lane));
    x = f(x, xor_lane_f32<16>(x, lane));
    return f(x, xor_lane_f32<32>(x, lane));
  } else {
    x = f(x, xor_lane_i32<1>(x, lane));
    x = f(x, xor_lane_i32<2>(x, lane));
    x = f(x, xor_lane_i32<4>(x, lane));
    x = f(x, xor_lane_i32<8>(x, lane));
    x = f(x, xor_lane_i32<16>(x, lane));
    return f(x, xor_lane_i32<32>(x, lane));
  }
}

// Absmax int8 quantisation of the wave's 64 * EPL values (EPL per lane);
// returns amax and writes the lane's EPL codes packed little-endian into
// codes[EPL / 4].
template <int EPL>
__device__ __forceinline__ float absmax_quantize(const float* r, uint32_t* codes,
                                                 int* qsum) {
  float vmax = 0.0f;
#pragma unroll
  for (int e = 0; e < EPL; ++e) {
    const float a = fabsf(r[e]);
    vmax = a > vmax ? a : vmax;
  }
  const int lane = __lane_id();
  vmax = butterfly_all(vmax, lane, [](float a, float o) { return o > a ? o : a; });
  float amax = vmax;
  if (amax < 1e-10f) amax = 1e-10f;
  const float inv = 127.0f / amax;
  int s = 0;
#pragma unroll
  for (int w = 0; w < EPL / 4; ++w) {
    uint32_t packed = 0;
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      float v = rintf(r[4 * w + e] * inv);
      v = v < -128.0f ? -128.0f : v;
      v = v > 127.0f ? 127.0f : v;
      const int qi = static_cast<int>(v);
      s += qi;
      packed |= (static_cast<uint32_t>(qi) & 0xFFu) << (8 * e);
    }
    codes[w] = packed;
  }
  s = butterfly_all(s, lane, [](int a, int o) { return a + o; });
  *qsum = s;
  return amax;
}

// fwht_apply over 64 * EPL values held EPL per lane (element EPL*lane + e):
// strides below EPL inside the lane, the rest across lanes (xor 1 .. 32), in
// the reference's stage order; the lower element of each pair becomes a + b,
// the upper a - b.
template <int EPL>
__device__ __forceinline__ void fwht_wave(float* r, int lane) {
#pragma unroll
  for (int st = 1; st < EPL; st <<= 1) {
#pragma unroll
    for (int e = 0; e < EPL; ++e) {
      if (e & st) continue;
      const float a = r[e], b = r[e + st];
      r[e] = a + b;
      r[e + st] = a - b;
    }
  }
  // Strides EPL .. 32 * EPL: lane bit m; the lower lane of a pair takes
  // a + b, the upper a - b (a the lower lane's value), on the VALU.
  auto stage = [&](auto mc) {
    constexpr int m = decltype(mc)::value;
    const bool upper = (lane & m) != 0;
#pragma unroll
    for (int e = 0; e < EPL; ++e) {
      const float p = xor_lane_f32<m>(r[e], lane);
      r[e] = upper ? (p - r[e]) : (r[e] + p);
    }
  };
  stage(std::integral_constant<int, 1>{});
  stage(std::integral_constant<int, 2>{});
  stage(std::integral_constant<int, 4>{});
  stage(std::integral_constant<int, 8>{});
  stage(std::integral_constant<int, 16>{});
  stage(std::integral_constant<int, 32>{});
  const float sc = static_cast<float>(1.0 / static_cast<double>(sqrtf(64.0f * EPL)));
#pragma unroll
  for (int e = 0; e < EPL; ++e) r[e] = r[e] * sc;
}

// One wave per head; head_dim D = 64 * EPL, lane L owns elements
// EPL*L .. EPL*L + EPL - 1.
template <int EPL>
__global__ __launch_bounds__(256) void bq_prep_kernel(
    const int32_t* __restrict__ image, const uint16_t* __restrict__ q_src,
    const uint16_t* __restrict__ k_src, const uint16_t* __restrict__ v_src,
    const uint16_t* __restrict__ q_norm, const uint16_t* __restrict__ k_norm,
    int8_t* __restrict__ q_i8, float* __restrict__ qi_bias,
    float* __restrict__ f_q, int8_t* __restrict__ k_cache,
    float* __restrict__ k_scale, int8_t* __restrict__ v_cache,
    float* __restrict__ v_scale, const float* __restrict__ cos_table,
    const float* __restrict__ sin_table, int num_q, int num_kv, int shift,
    int row_mask, int page_mask, int rope_half, int pair_stride, float sqrt_n,
    float n_eps) {
  constexpr int D = 64 * EPL;
  using Raw = typename std::conditional<EPL == 4, uint2, uint4>::type;
  const int wave = threadIdx.x >> 6;
  const int lane = threadIdx.x & 63;
  const int tok = blockIdx.x;
  const int run = image[image[kHdrOffTokRun] + tok];
  const int32_t* rp = image + image[kHdrOffRuns] + run * 4;
  const int pos = rp[1] + (tok - rp[0]);
  const int32_t* rows = image + image[kHdrOffRows] + rp[2];
  const float* cos_row = cos_table + static_cast<int64_t>(pos) * rope_half;
  const float* sin_row = sin_table + static_cast<int64_t>(pos) * rope_half;
  const int64_t slot =
      static_cast<int64_t>(rows[(pos >> shift) & page_mask]) + (pos & row_mask);
  const int64_t kv_stride = static_cast<int64_t>(num_kv) * D;
  const float inv_sqrt_n = 1.0f / sqrt_n;
  const int n_heads = num_q + 2 * num_kv;

  for (int hh = wave; hh < n_heads; hh += 4) {
    const bool is_q = hh < num_q;
    const bool is_k = !is_q && hh < num_q + num_kv;
    const int h = is_q ? hh : (is_k ? hh - num_q : hh - num_q - num_kv);
    const uint16_t* src =
        is_q ? q_src + (static_cast<int64_t>(tok) * num_q + h) * D
             : (is_k ? k_src : v_src) + (static_cast<int64_t>(tok) * num_kv + h) * D;
    float r[EPL];
    {
      const Raw raw = *reinterpret_cast<const Raw*>(src + EPL * lane);
      const uint32_t* w = reinterpret_cast<const uint32_t*>(&raw);
#pragma unroll
      for (int i = 0; i < EPL / 2; ++i) {
        r[2 * i] = bf16_lo(w[i]);
        r[2 * i + 1] = bf16_hi(w[i]);
      }
    }

    if (is_q || is_k) {
      // head_inv_rms: lane j < 16 replays the reference's 16-lane register
      // chain over elements 16*ri + j, reading the bf16 row again (cached).
      float ssq = 0.0f;
      if (lane < 16) {
        const float x0 = bf16_to_f32(src[lane]);
        ssq = x0 * x0;
#pragma unroll
        for (int ri = 1; ri < D / 16; ++ri) {
          const float x = bf16_to_f32(src[16 * ri + lane]);
          ssq = fmaf(x, x, ssq);
        }
      }
      ssq = ssq + xor_lane_f32<8>(ssq, lane);
      ssq = ssq + xor_lane_f32<4>(ssq, lane);
      ssq = ssq + xor_lane_f32<2>(ssq, lane);
      ssq = ssq + xor_lane_f32<1>(ssq, lane);
      const float total = readlane_f32(ssq, 0);
      const float inv_rms = sqrt_n / sqrtf(total + n_eps);
      const uint16_t* gamma = is_q ? q_norm : k_norm;
#pragma unroll
      for (int e = 0; e < EPL; ++e) {
        const float g = bf16_to_f32(gamma[EPL * lane + e]);
        const float t = r[e] * inv_rms;
        r[e] = t * g;
      }
      // RoPE pairs (j, pair_stride + j), j < rope_half (both multiples of EPL,
      // so a lane's elements are all rotated or all passed through).
      const int e0 = EPL * lane;
      int partner = lane;
      if (e0 < rope_half) partner = (e0 + pair_stride) / EPL;
      else if (e0 >= pair_stride && e0 < pair_stride + rope_half) partner = (e0 - pair_stride) / EPL;
      float pv[EPL];
#pragma unroll
      for (int e = 0; e < EPL; ++e) pv[e] = bpermute_f32(r[e], partner);
      if (e0 < rope_half) {
#pragma unroll
        for (int e = 0; e < EPL; ++e) {
          const float cv = cos_row[e0 + e], sv = sin_row[e0 + e];
          const float a = r[e] * cv, b = pv[e] * sv;
          r[e] = a - b;
        }
      } else if (e0 >= pair_stride && e0 < pair_stride + rope_half) {
#pragma unroll
        for (int e = 0; e < EPL; ++e) {
          const int j = e0 - pair_stride + e;
          const float cv = cos_row[j], sv = sin_row[j];
          const float c = r[e] * cv, d = pv[e] * sv;
          r[e] = c + d;
        }
      }
    }

    fwht_wave<EPL>(r, lane);
    uint32_t codes[EPL / 4];
    int qsum;
    const float amax = absmax_quantize<EPL>(r, codes, &qsum);
    int8_t* dst;
    if (is_q) {
      dst = q_i8 + (static_cast<int64_t>(tok) * num_q + h) * D;
      if (lane == 0) {
        qi_bias[static_cast<int64_t>(tok) * num_q + h] = static_cast<float>(qsum) * 128.0f;
        f_q[static_cast<int64_t>(tok) * num_q + h] = amax * inv_sqrt_n;
      }
    } else if (is_k) {
      dst = k_cache + slot * kv_stride + h * D;
      if (lane == 0) k_scale[slot * num_kv + h] = amax;
    } else {
      dst = v_cache + slot * kv_stride + h * D;
      if (lane == 0) v_scale[slot * num_kv + h] = amax;
    }
    if constexpr (EPL == 4) {
      *reinterpret_cast<uint32_t*>(dst + 4 * lane) = codes[0];
    } else {
      *reinterpret_cast<uint2*>(dst + 8 * lane) = make_uint2(codes[0], codes[1]);
    }
  }
}

// The same prep with 16 lanes per head and four heads per wave: lane j of a
// head's 16-lane row owns elements 16*i + j (i < E = D/16), so
//   RMS     lane j's chain over elements 16*i + j is the reference's register
//           chain of SIMD lane j, in the lane's own registers, and the 16
//           partial sums take the xor 8, 4, 2, 1 tree of bq_prep_kernel;
//   RoPE    the partner of element 16*i + j (pair_stride away, a multiple of
//           16) is the lane's own element i + pair_stride/16;
//   FWHT    strides 1 .. 8 are DPP lane exchanges inside the row and strides
//           16 .. D/2 pairs of the lane's registers, in the reference's stage
//           order with the same operand pairs;
//   absmax  lane max, then the row's xor 1 .. 8 exchanges.
// Every instruction serves four heads, about half the VALU work per head of
// one wave per head.  The int8 codes go to LDS byte by byte and leave as
// 16-byte rows.  Needs (num_q + 2 num_kv) % 4 == 0; a row's lanes share one
// head, so the q/k-only steps branch per row.  RoPE's rope_half and
// pair_stride are template constants (kRopeHalf, kPairStride: multiples of 16).
template <int D, int kRopeHalf, int kPairStride>
__global__ __launch_bounds__(512) void bq_prep_rows_kernel(
    const int32_t* __restrict__ image, const uint16_t* __restrict__ q_src,
    const uint16_t* __restrict__ k_src, const uint16_t* __restrict__ v_src,
    const uint16_t* __restrict__ q_norm, const uint16_t* __restrict__ k_norm,
    int8_t* __restrict__ q_i8, float* __restrict__ qi_bias,
    float* __restrict__ f_q, int8_t* __restrict__ k_cache,
    float* __restrict__ k_scale, int8_t* __restrict__ v_cache,
    float* __restrict__ v_scale, const float* __restrict__ cos_table,
    const float* __restrict__ sin_table, int num_q, int num_kv, int shift,
    int row_mask, int page_mask, int rope_half, int pair_stride, float sqrt_n,
    float n_eps) {
  constexpr int E = D / 16;
  constexpr int kMaxWaves = 512 / 64;
  __shared__ __align__(16) uint8_t cbuf[kMaxWaves][4 * D];
  const int wave = threadIdx.x >> 6;
  const int lane = threadIdx.x & 63;
  const int j = lane & 15;
  const int tok = blockIdx.x;
  const int run = image[image[kHdrOffTokRun] + tok];
  const int32_t* rp = image + image[kHdrOffRuns] + run * 4;
  const int pos = rp[1] + (tok - rp[0]);
  const int32_t* rows = image + image[kHdrOffRows] + rp[2];
  const float* cos_row = cos_table + static_cast<int64_t>(pos) * rope_half;
  const float* sin_row = sin_table + static_cast<int64_t>(pos) * rope_half;
  const int64_t slot =
      static_cast<int64_t>(rows[(pos >> shift) & page_mask]) + (pos & row_mask);
  const int64_t kv_stride = static_cast<int64_t>(num_kv) * D;
  const float inv_sqrt_n = 1.0f / sqrt_n;

  // Head of a 16-lane row: q heads, then k heads, then v heads.
  auto head_of = [&](int hh, bool& is_q, bool& is_k) {
    is_q = hh < num_q;
    is_k = !is_q && hh < num_q + num_kv;
    return is_q ? hh : (is_k ? hh - num_q : hh - num_q - num_kv);
  };
  bool is_q, is_k;
  const int hh = 4 * wave + (lane >> 4);
  const int h = head_of(hh, is_q, is_k);
  const uint16_t* src =
      (is_q ? q_src + (static_cast<int64_t>(tok) * num_q + h) * D
            : (is_k ? k_src : v_src) + (static_cast<int64_t>(tok) * num_kv + h) * D) + j;
  float r[E];
#pragma unroll
  for (int i = 0; i < E; ++i) r[i] = bf16_to_f32(src[16 * i]);

  if (is_q || is_k) {  // uniform over the row
    // head_inv_rms: the chain of SIMD lane j, then the 16-lane tree.
    float ssq = r[0] * r[0];
#pragma unroll
    for (int i = 1; i < E; ++i) ssq = fmaf(r[i], r[i], ssq);
    ssq = ssq + xor_lane_f32<8>(ssq, lane);
    ssq = ssq + xor_lane_f32<4>(ssq, lane);
    ssq = ssq + xor_lane_f32<2>(ssq, lane);
    ssq = ssq + xor_lane_f32<1>(ssq, lane);
    const float inv_rms = sqrt_n / sqrtf(ssq + n_eps);
    const uint16_t* gamma = (is_q ? q_norm : k_norm) + j;
#pragma unroll
    for (int i = 0; i < E; ++i) {
      const float g = bf16_to_f32(gamma[16 * i]);
      const float t = r[i] * inv_rms;
      r[i] = t * g;
    }
    // RoPE pairs (e, pair_stride + e), e < rope_half: element 16*i + j with
    // i < rope_half/16 and its partner i + pair_stride/16, both this lane's.
    constexpr int kNr = kRopeHalf / 16, kPs = kPairStride / 16;
    static_assert(kRopeHalf % 16 == 0 && kPairStride % 16 == 0 && kNr <= kPs &&
                      kPs + kNr <= E,
                  "RoPE pairs inside the head");
#pragma unroll
    for (int i = 0; i < kNr; ++i) {
      const float lo = r[i], hi = r[i + kPs];
      const float cv = cos_row[16 * i + j], sv = sin_row[16 * i + j];
      const float a = lo * cv, b = hi * sv;
      const float c = hi * cv, d = lo * sv;
      r[i] = a - b;
      r[i + kPs] = c + d;
    }
  }

  // fwht_apply: strides 1 .. 8 across the row's lanes (the lower lane of a
  // pair takes a + b, the upper a - b, a the lower lane's value), strides
  // 16 .. D/2 inside the lane.  fma(+-1, own, partner) is that sum or
  // difference with its single rounding, one instruction for both halves.
  // x[lane ^ 4] is taken as (x[lane ^ 7])[lane ^ 3]: two DPP moves.
  auto stage = [&](auto mc) {
    constexpr int m = decltype(mc)::value;
    const float sg = (lane & m) != 0 ? -1.0f : 1.0f;
#pragma unroll
    for (int i = 0; i < E; ++i) {
      float p;
      if constexpr (m == 4) {
        p = dpp_f32<kDppQuadReverse>(dpp_f32<kDppHalfMirror>(r[i]));
      } else {
        p = xor_lane_f32<m>(r[i], lane);
      }
      r[i] = __builtin_fmaf(sg, r[i], p);
    }
  };
  stage(std::integral_constant<int, 1>{});
  stage(std::integral_constant<int, 2>{});
  stage(std::integral_constant<int, 4>{});
  stage(std::integral_constant<int, 8>{});
#pragma unroll
  for (int st = 1; st < E; st <<= 1) {
#pragma unroll
    for (int i = 0; i < E; ++i) {
      if (i & st) continue;
      const float a = r[i], b = r[i + st];
      r[i] = a + b;
      r[i + st] = a - b;
    }
  }
  const float sc = static_cast<float>(1.0 / static_cast<double>(sqrtf(static_cast<float>(D))));
#pragma unroll
  for (int i = 0; i < E; ++i) r[i] = r[i] * sc;

  // absmax_quantize over the row.
  float vmax = 0.0f;
#pragma unroll
  for (int i = 0; i < E; ++i) {
    const float a = fabsf(r[i]);
    vmax = a > vmax ? a : vmax;
  }
  {
    float o = xor_lane_f32<1>(vmax, lane);
    vmax = o > vmax ? o : vmax;
    o = xor_lane_f32<2>(vmax, lane);
    vmax = o > vmax ? o : vmax;
    o = xor_lane_f32<4>(vmax, lane);
    vmax = o > vmax ? o : vmax;
    o = xor_lane_f32<8>(vmax, lane);
    vmax = o > vmax ? o : vmax;
  }
  float amax = vmax;
  if (amax < 1e-10f) amax = 1e-10f;
  const float inv = 127.0f / amax;
  uint8_t* crow = &cbuf[wave][(lane >> 4) * D + j];
  int s = 0;
#pragma unroll
  for (int i = 0; i < E; ++i) {
    // clamp(roundeven(x * 127/amax), -128, 127) as one med3 (finite x).
    const float v = __builtin_amdgcn_fmed3f(rintf(r[i] * inv), -128.0f, 127.0f);
    const int qi = static_cast<int>(v);
    s += qi;
    crow[16 * i] = static_cast<uint8_t>(qi & 0xFF);
  }
  s = s + xor_lane_i32<1>(s, lane);
  s = s + xor_lane_i32<2>(s, lane);
  s = s + xor_lane_i32<4>(s, lane);
  s = s + xor_lane_i32<8>(s, lane);
  if (j == 0) {
    if (is_q) {
      qi_bias[static_cast<int64_t>(tok) * num_q + h] = static_cast<float>(s) * 128.0f;
      f_q[static_cast<int64_t>(tok) * num_q + h] = amax * inv_sqrt_n;
    } else if (is_k) {
      k_scale[slot * num_kv + h] = amax;
    } else {
      v_scale[slot * num_kv + h] = amax;
    }
  }
  // The wave's 4 rows of codes leave LDS 16 bytes per lane (the wave's own
  // LDS bytes: its writes land before its reads).
  __builtin_amdgcn_s_waitcnt(0xC07F);  // lgkmcnt(0)
#pragma unroll
  for (int c = lane; c < 4 * D / 16; c += 64) {
    bool cq, ck;
    const int ch = head_of(4 * wave + c / (D / 16), cq, ck);
    const int off = 16 * (c % (D / 16));
    int8_t* dst = cq ? q_i8 + (static_cast<int64_t>(tok) * num_q + ch) * D
                     : (ck ? k_cache : v_cache) + slot * kv_stride + ch * D;
    *reinterpret_cast<uint4*>(dst + off) =
        *reinterpret_cast<const uint4*>(&cbuf[wave][16 * c]);
  }
}

typedef unsigned int bq_u32x4_t __attribute__((ext_vector_type(4)));

// Codes are streamed once per step: non-temporal loads, as for the bf16
// cache, keep them from displacing the reused plan image, queries and scales.
__device__ __forceinline__ uint4 load_codes16(const int8_t* p) {
  const bq_u32x4_t v =
      __builtin_nontemporal_load(reinterpret_cast<const bq_u32x4_t*>(p));
  return make_uint4(v.x, v.y, v.z, v.w);
}
__device__ __forceinline__ uint32_t load_codes4(const int8_t* p) {
  return __builtin_nontemporal_load(reinterpret_cast<const uint32_t*>(p));
}

__device__ __forceinline__ void unpack_i8x4(uint32_t w, float* f) {
  f[0] = static_cast<float>(static_cast<int8_t>(w & 0xFFu));
  f[1] = static_cast<float>(static_cast<int8_t>((w >> 8) & 0xFFu));
  f[2] = static_cast<float>(static_cast<int8_t>((w >> 16) & 0xFFu));
  f[3] = static_cast<float>(static_cast<int8_t>(w >> 24));
}

template <int G, bool kTwoPages>
__global__ __launch_bounds__(256) void bq_partial_kernel(
    const int32_t* __restrict__ image, const int8_t* __restrict__ q_i8,
    const float* __restrict__ qi_bias, const float* __restrict__ f_q,
    const int8_t* __restrict__ kc,
    const float* __restrict__ k_scale, const int8_t* __restrict__ vc,
    const float* __restrict__ v_scale, float* __restrict__ partials,
    int64_t partial_stride, int num_q, int num_kv, int64_t kv_stride,
    int shift, int row_mask, int page_mask) {
  constexpr int D = kBqD;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);  // wave-uniform
  const int lane = threadIdx.x & 63;
  const int g = blockIdx.x * 4 + wave;
  if (g >= num_kv) return;
  const int32_t* item = image + image[kHdrOffItems] + blockIdx.y * kItemWords;
  const int q_row = item[0];
  const int start_pos = item[2];
  const int start = item[3];
  const int end = item[4];
  const int stripe = item[5];
  const int32_t* rows = image + item[kItemRowsOff];
  const float inv127 = 1.0f / 127.0f;
  const float inv127sq = inv127 * inv127;

  const int tk = lane >> 2;  // position within the tile
  const int c = lane & 3;
  uint4 qv[G][4];
  float fq[G], qb[G];
  int qsum128[G];
#pragma unroll
  for (int r = 0; r < G; ++r) {
    const int8_t* qr = q_i8 + (static_cast<int64_t>(q_row) * num_q + g * G + r) * D + 16 * c;
#pragma unroll
    for (int i = 0; i < 4; ++i) qv[r][i] = *reinterpret_cast<const uint4*>(qr + 64 * i);
    fq[r] = f_q[static_cast<int64_t>(q_row) * num_q + g * G + r];
    qb[r] = qi_bias[static_cast<int64_t>(q_row) * num_q + g * G + r];
    // The reference's VNNI dot reads (k ^ 0x80) as unsigned: raw = dot +
    // 128 * sum(q).  Sum the lane's 64 codes, then the 4 lanes of a group.
    int qs = 0;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      qs = __builtin_amdgcn_sdot4(static_cast<int>(qv[r][i].x), 0x01010101, qs, false);
      qs = __builtin_amdgcn_sdot4(static_cast<int>(qv[r][i].y), 0x01010101, qs, false);
      qs = __builtin_amdgcn_sdot4(static_cast<int>(qv[r][i].z), 0x01010101, qs, false);
      qs = __builtin_amdgcn_sdot4(static_cast<int>(qv[r][i].w), 0x01010101, qs, false);
    }
    qs = qs + dpp_i32<kDppXor1>(qs);
    qs = qs + dpp_i32<kDppXor2>(qs);
    qsum128[r] = 128 * qs;
  }
  const int8_t* kh = kc + static_cast<int64_t>(g) * D + 16 * c;
  const int8_t* vh = vc + static_cast<int64_t>(g) * D + 4 * lane;

  float m[G], l[G], acc[G][4];
#pragma unroll
  for (int r = 0; r < G; ++r) {
    m[r] = kNegBig;
    l[r] = 0.0f;
#pragma unroll
    for (int e = 0; e < 4; ++e) acc[r][e] = 0.0f;
  }

  // One tile's loads: the lane's 64 key bytes of position tk and its scale,
  // then the 4 value bytes (dims 4*lane..) of every position and the
  // positions' value scales.  Positions past the tile's end load the tile's
  // last position (in bounds) and are masked below.  kTwoPages (pages of
  // >= 16 positions): a tile spans at most two pages, whose rows come from
  // two scalar loads, and the value scales are scalar loads too, so no
  // vector load waits on another.
  struct BqDecodeTile {
    uint4 k[4];
    float ks;
    uint32_t v[kTile];
    float vs[kTile];
  };
  struct TileRows {
    int p0, pg0, len;
    int64_t ra, rb;
  };
  auto tile_rows = [&](int pos0) {
    TileRows r;
    r.p0 = start_pos + pos0;
    r.pg0 = r.p0 >> shift;
    r.len = min(kTile, end - pos0);
    r.ra = r.rb = 0;
    if constexpr (kTwoPages) {
      const int pg1 = (r.p0 + r.len - 1) >> shift;
      r.ra = sload(rows + (r.pg0 & page_mask));
      r.rb = pg1 != r.pg0 ? sload(rows + (pg1 & page_mask)) : r.ra;
    }
    return r;
  };
  auto slot_of = [&](const TileRows& r, int t) -> int64_t {
    const int p = r.p0 + min(t, r.len - 1);
    if constexpr (kTwoPages) {
      return ((p >> shift) == r.pg0 ? r.ra : r.rb) + (p & row_mask);
    } else {
      return static_cast<int64_t>(rows[(p >> shift) & page_mask]) + (p & row_mask);
    }
  };
  auto load_k = [&](BqDecodeTile& d, const TileRows& r) {
    const int64_t kslot = slot_of(r, tk);
    const int8_t* kr = kh + kslot * kv_stride;
#pragma unroll
    for (int i = 0; i < 4; ++i) d.k[i] = load_codes16(kr + 64 * i);
    d.ks = k_scale[kslot * num_kv + g];
  };
  auto load_v = [&](BqDecodeTile& d, const TileRows& r) {
#pragma unroll
    for (int t = 0; t < kTile; ++t) {
      const int64_t vslot = slot_of(r, t);
      d.v[t] = load_codes4(vh + vslot * kv_stride);
      if constexpr (kTwoPages) {
        d.vs[t] = __int_as_float(sload(reinterpret_cast<const int32_t*>(v_scale) +
                                       vslot * num_kv + g));
      } else {
        d.vs[t] = v_scale[vslot * num_kv + g];
      }
    }
  };

  // Software-pipelined in the tile's own registers: the next tile's key
  // loads are issued once the scores have read this tile's keys and run
  // under the softmax and P.V; its value loads are issued after the P.V and
  // run under the next scores.  The loads are unconditional (after the
  // item's last tile they all read that tile's first row, in bounds, cached
  // and unused), so each wait covers only older loads.
  BqDecodeTile cur;
  TileRows rc = {0, 0, 0, 0, 0};
  if (start < end) {
    rc = tile_rows(start);
    load_k(cur, rc);
    __builtin_amdgcn_sched_barrier(0);  // keys before values, as in the loop
    load_v(cur, rc);
    __builtin_amdgcn_sched_barrier(0);
  }
  for (int pos0 = start; pos0 < end; pos0 += kTile) {
    const int tile_len = rc.len;
    const bool valid = tk < tile_len;
    TileRows rn = rc;
    if (pos0 + kTile < end)
      rn = tile_rows(pos0 + kTile);
    else
      rn.len = 1;  // every load of the dummy tile reads the last tile's first row
    float s[G];
    {
      const float ks = cur.ks;
#pragma unroll
      for (int r = 0; r < G; ++r) {
        int a = 0;
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          a = __builtin_amdgcn_sdot4(static_cast<int>(cur.k[i].x), static_cast<int>(qv[r][i].x), a, false);
          a = __builtin_amdgcn_sdot4(static_cast<int>(cur.k[i].y), static_cast<int>(qv[r][i].y), a, false);
          a = __builtin_amdgcn_sdot4(static_cast<int>(cur.k[i].z), static_cast<int>(qv[r][i].z), a, false);
          a = __builtin_amdgcn_sdot4(static_cast<int>(cur.k[i].w), static_cast<int>(qv[r][i].w), a, false);
        }
        a = a + dpp_i32<kDppXor1>(a);
        a = a + dpp_i32<kDppXor2>(a);
        float sc = static_cast<float>(a + qsum128[r]) - qb[r];
        sc = sc * fq[r];
        sc = sc * ks;
        sc = sc * inv127sq;
        s[r] = valid ? sc : kNegBig;
      }
    }
    __builtin_amdgcn_sched_barrier(0);
    load_k(cur, rn);
    __builtin_amdgcn_sched_barrier(0);

    float w[G];
#pragma unroll
    for (int r = 0; r < G; ++r) {
      float mx = s[r];
      mx = max_ref(mx, dpp_f32<kDppHalfMirror>(mx));  // position ^ 1
      mx = max_ref(mx, dpp_f32<kDppRowRor8>(mx));     // position ^ 2
      mx = pair_max32(pair_max16(mx));                // position ^ 4, ^ 8
      const float m_new = mx > m[r] ? mx : m[r];
      const float corr = fexp(max_ref(-87.0f, m[r] - m_new));
      w[r] = fexp(max_ref(-87.0f, s[r] - m_new));
      // Halving tree over positions: ^8, ^4, ^2, ^1 = lane ^32, ^16, ^8, ^4.
      float ts = w[r];
      ts = pair_sum16(pair_sum32(ts));
      ts = ts + dpp_f32<kDppRowRor8>(ts);
      ts = ts + dpp_f32<kDppHalfMirror>(ts);
      const float lc = l[r] * corr;
      l[r] = lc + ts;
      m[r] = m_new;
#pragma unroll
      for (int e = 0; e < 4; ++e) acc[r][e] = acc[r][e] * corr;
    }

    // Every position's weights first: a v_readlane result read by the very
    // next VALU instruction costs wait states.
    float wtl[kTile][G];
#pragma unroll
    for (int t = 0; t < kTile; ++t)
#pragma unroll
      for (int r = 0; r < G; ++r) wtl[t][r] = readlane_f32(w[r], 4 * t);
    __builtin_amdgcn_sched_barrier(0);
#pragma unroll
    for (int t = 0; t < kTile; ++t) {
      if (t < tile_len) {  // wave-uniform
        float vf[4];
        unpack_i8x4(cur.v[t], vf);
#pragma unroll
        for (int r = 0; r < G; ++r) {
          const float wt = wtl[t][r];
          const float a = wt * cur.vs[t];
          const float wts = a * inv127;
#pragma unroll
          for (int e = 0; e < 4; ++e) acc[r][e] = fmaf(vf[e], wts, acc[r][e]);
        }
      }
    }
    __builtin_amdgcn_sched_barrier(0);
    load_v(cur, rn);
    __builtin_amdgcn_sched_barrier(0);
    rc = rn;
  }

  float* part = partials + static_cast<int64_t>(stripe) * partial_stride;
#pragma unroll
  for (int r = 0; r < G; ++r) {
    float* dst = part + static_cast<int64_t>(g * G + r) * D + 4 * lane;
    *reinterpret_cast<float4*>(dst) = make_float4(acc[r][0], acc[r][1], acc[r][2], acc[r][3]);
  }
  if (lane == 0) {
#pragma unroll
    for (int r = 0; r < G; ++r) {
      part[num_q * D + g * G + r] = m[r];
      part[num_q * D + num_q + g * G + r] = l[r];
    }
  }
}

}  // namespace

hipError_t launch_bq_attn_prep(const int32_t* image, int seq_len, const void* q_src,
                               const void* k_src, const void* v_src, const void* q_norm,
                               const void* k_norm, void* q_i8, float* qi_bias, float* f_q,
                               void* k_cache, float* k_scale, void* v_cache,
                               float* v_scale, const float* cos_table,
                               const float* sin_table, int num_q, int num_kv,
                               PagedGeom geom, int head_dim, int rope_half,
                               int pair_stride, float sqrt_n, float n_eps,
                               hipStream_t stream) {
  if (seq_len <= 0) return hipSuccess;
  const int n_heads = num_q + 2 * num_kv;
  const bool rows_form = n_heads % 4 == 0 && n_heads / 4 <= 8 &&
                         ((head_dim == 256 && rope_half == 128 && pair_stride == 128) ||
                          (head_dim == 512 && rope_half == 64 && pair_stride == 256));
  if (rows_form) {
    auto kernel = head_dim == 512 ? bq_prep_rows_kernel<512, 64, 256>
                                  : bq_prep_rows_kernel<256, 128, 128>;
    hipLaunchKernelGGL(kernel, dim3(seq_len), dim3(16 * n_heads), 0, stream, image,
                       static_cast<const uint16_t*>(q_src),
                       static_cast<const uint16_t*>(k_src),
                       static_cast<const uint16_t*>(v_src),
                       static_cast<const uint16_t*>(q_norm),
                       static_cast<const uint16_t*>(k_norm), static_cast<int8_t*>(q_i8),
                       qi_bias, f_q, static_cast<int8_t*>(k_cache), k_scale,
                       static_cast<int8_t*>(v_cache), v_scale, cos_table, sin_table, num_q,
                       num_kv, geom.shift, geom.row_mask, geom.page_mask, rope_half,
                       pair_stride, sqrt_n, n_eps);
    return hipGetLastError();
  }
  auto kernel = head_dim == 512 ? bq_prep_kernel<8> : bq_prep_kernel<4>;
  hipLaunchKernelGGL(kernel, dim3(seq_len), dim3(256), 0, stream, image,
                     static_cast<const uint16_t*>(q_src), static_cast<const uint16_t*>(k_src),
                     static_cast<const uint16_t*>(v_src), static_cast<const uint16_t*>(q_norm),
                     static_cast<const uint16_t*>(k_norm), static_cast<int8_t*>(q_i8),
                     qi_bias, f_q, static_cast<int8_t*>(k_cache), k_scale,
                     static_cast<int8_t*>(v_cache), v_scale, cos_table, sin_table, num_q,
                     num_kv, geom.shift, geom.row_mask, geom.page_mask, rope_half,
                     pair_stride, sqrt_n, n_eps);
  return hipGetLastError();
}

hipError_t launch_bq_attention(const int32_t* image, int num_items, int num_units,
                               int mode, const void* q_i8, const float* qi_bias,
                               const float* f_q, const void* k_base, const float* k_scale,
                               const void* v_base, const float* v_scale, void* output,
                               float* partials, int64_t ps, int num_q, int num_kv,
                               int head_dim, int64_t kv_stride, PagedGeom geom,
                               hipStream_t stream, int8_t* q_out, float* q_scale) {
  if (num_items > 0 && head_dim == 512) {
    hipError_t err = launch_partials_wide_bq(image, num_items, q_i8, qi_bias, f_q, k_base,
                                             k_scale, v_base, v_scale, partials, ps, num_q,
                                             num_kv, kv_stride, geom, stream);
    if (err != hipSuccess) return err;
  } else if (num_items > 0) {
    // kv-head groups of an item side by side, as in the bf16 decode.
    dim3 grid((num_kv + 3) / 4, num_items);
    if (geom.row_mask + 1 >= kTile)
      hipLaunchKernelGGL((bq_partial_kernel<2, true>), grid, dim3(256), 0, stream, image,
                         static_cast<const int8_t*>(q_i8), qi_bias, f_q,
                         static_cast<const int8_t*>(k_base), k_scale,
                         static_cast<const int8_t*>(v_base), v_scale, partials, ps, num_q,
                         num_kv, kv_stride, geom.shift, geom.row_mask, geom.page_mask);
    else
      hipLaunchKernelGGL((bq_partial_kernel<2, false>), grid, dim3(256), 0, stream, image,
                         static_cast<const int8_t*>(q_i8), qi_bias, f_q,
                         static_cast<const int8_t*>(k_base), k_scale,
                         static_cast<const int8_t*>(v_base), v_scale, partials, ps, num_q,
                         num_kv, kv_stride, geom.shift, geom.row_mask, geom.page_mask);
    hipError_t err = hipGetLastError();
    if (err != hipSuccess) return err;
  }
  return launch_merge(image, num_units, num_items, mode, partials, output, ps, num_q, head_dim,
                      stream, q_out, q_scale);
}

namespace {
// quant_segment[store_divided=False] (butterquant/kernels.mojo:83-92) on one
// block of one token: sa = amax, inv = 127/amax (0 if amax is 0), codes =
// clamp(roundeven(x * inv), -128, 127).  One wave per (token, block).
__global__ __launch_bounds__(256) void bq_block_quant_kernel(
    const uint16_t* __restrict__ src, int8_t* __restrict__ x_i8, float* __restrict__ x_sa,
    int64_t cols, int block, int64_t n_pairs) {
  const int wave = threadIdx.x >> 6;
  const int lane = threadIdx.x & 63;
  const int64_t pair = static_cast<int64_t>(blockIdx.x) * 4 + wave;  // (token, block)
  if (pair >= n_pairs) return;
  const int64_t base = pair * block;  // blocks tile each row: token*cols + b*block
  const uint16_t* s = src + base;
  float amax = 0.0f;
  for (int i = lane; i < block; i += 64) amax = fmaxf(amax, fabsf(bf16_to_f32(s[i])));
  amax = butterfly_all(amax, lane, [](float a, float o) { return fmaxf(a, o); });
  const float inv = amax > 0.0f ? 127.0f / amax : 0.0f;
  int8_t* d = x_i8 + base;
  for (int i = lane; i < block; i += 64) {
    const float r = fminf(fmaxf(rintf(bf16_to_f32(s[i]) * inv), -128.0f), 127.0f);
    d[i] = static_cast<int8_t>(static_cast<int32_t>(r));
  }
  if (lane == 0) x_sa[pair] = amax;
}
}  // namespace

hipError_t launch_bq_block_quant(const void* src, void* x_i8, float* x_sa, int64_t cols,
                                 int block, int64_t seq_len, hipStream_t stream) {
  if (seq_len <= 0) return hipSuccess;
  const int64_t pairs = static_cast<int64_t>(seq_len) * (cols / block);
  hipLaunchKernelGGL(bq_block_quant_kernel, dim3(static_cast<unsigned>((pairs + 3) / 4)),
                     dim3(256), 0, stream, static_cast<const uint16_t*>(src),
                     static_cast<int8_t*>(x_i8), x_sa, cols, block, pairs);
  return hipGetLastError();
}

}  // namespace ifr
