// Paged split-KV flash attention (bf16 KV) and the log-sum-exp merge for
// gfx950.
//
// One wave64 owns one (work item, kv head): it walks the item's positions in
// tiles of 16 consecutive positions starting at the item's first position,
// exactly as FlashAttentionKernel walks its worker range
// (kernels/flash_attention.mojo:44-54), and applies the online softmax of
// process_kv_tile (kernels/attention_ops.mojo:193-253) once per tile per q
// head.  Matching the tile boundaries matters: the reference's biased exp
// returns fexp(0) = 0.99963, so every tile rescales all earlier tiles and the
// output depends on where tiles start.
//
// Lane layouts (D = head_dim):
//   QK:  8 lanes per position, 8 positions per pass, two passes per tile.
//        Lane (tk, c) holds bf16 elements {8c + 64i .. 8c + 64i + 7} of K and
//        of each GQA query head, so one pass loads 8 rows x 128 contiguous
//        bytes per 16-byte load.  Scores use v_dot2_f32_bf16 and a 3-step DPP
//        reduction inside each 8-lane group.
//   PV:  lane L owns output dims {DPL*L .. DPL*L + DPL-1}, DPL = D/64, and
//        accumulates positions in order with fma(v, w, acc), the reference's
//        per-element order.  Weights are broadcast with v_readlane.
// The tile max is a wave-wide max (exact in any order); the tile weight sum
// follows the halving tree of SIMD.reduce_add over the 16 positions.
#include "common.hpp"
#include "launch.hpp"

namespace ifr {
namespace {

typedef __bf16 bf16x2_t __attribute__((ext_vector_type(2)));

__device__ __forceinline__ float dot2_bf16(uint32_t a, uint32_t b, float c) {
  return __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(bf16x2_t, a),
                                         __builtin_bit_cast(bf16x2_t, b), c,
                                         false);
}

template <int DPL>
struct VecOf;
template <>
struct VecOf<4> {
  using T = uint2;
  __device__ static void unpack(const uint2& v, float* f) {
    f[0] = bf16_lo(v.x);
    f[1] = bf16_hi(v.x);
    f[2] = bf16_lo(v.y);
    f[3] = bf16_hi(v.y);
  }
};
template <>
struct VecOf<8> {
  using T = uint4;
  __device__ static void unpack(const uint4& v, float* f) {
    f[0] = bf16_lo(v.x);
    f[1] = bf16_hi(v.x);
    f[2] = bf16_lo(v.y);
    f[3] = bf16_hi(v.y);
    f[4] = bf16_lo(v.z);
    f[5] = bf16_hi(v.z);
    f[6] = bf16_lo(v.w);
    f[7] = bf16_hi(v.w);
  }
};

// Waves per workgroup; each wave owns one kv head of the work item.
constexpr int kDecodeWaves = 4;

typedef unsigned int u32x4_t __attribute__((ext_vector_type(4)));
typedef unsigned int u32x2_t __attribute__((ext_vector_type(2)));

// K/V pages are streamed once per step: non-temporal loads keep them from
// displacing reusable lines (plan image, queries, partials) and lift the
// achievable read bandwidth on gfx950 (about 7.1 vs 6.3 TB/s for a plain
// streaming read measured on the same box).
__device__ __forceinline__ uint4 load_kv(const uint4* p) {
  const u32x4_t v = __builtin_nontemporal_load(reinterpret_cast<const u32x4_t*>(p));
  return make_uint4(v.x, v.y, v.z, v.w);
}
__device__ __forceinline__ uint2 load_kv(const uint2* p) {
  const u32x2_t v = __builtin_nontemporal_load(reinterpret_cast<const u32x2_t*>(p));
  return make_uint2(v.x, v.y);
}

template <int D, int G, bool kTwoPages, bool kShort>
__global__ __launch_bounds__(64 * kDecodeWaves) void flash_partial_bf16_kernel(
    const int32_t* __restrict__ image, const uint16_t* __restrict__ q,
    const uint16_t* __restrict__ kc, const uint16_t* __restrict__ vc,
    float* __restrict__ partials, int64_t partial_stride, int num_q,
    int num_kv, int64_t kv_stride, int shift, int row_mask, int page_mask) {
  constexpr int NCH = D / 64;  // 16-byte K chunks per lane per position
  constexpr int DPL = D / 64;  // PV output dims per lane
  using V = VecOf<DPL>;
  using VT = typename V::T;

  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);  // wave-uniform
  const int lane = threadIdx.x & 63;
  const int g = blockIdx.x * kDecodeWaves + wave;
  if (g >= num_kv) return;

  const int32_t* item = image + kItemsOff + blockIdx.y * kItemWords;
  const int q_row = item[0];
  const int start_pos = item[2];
  const int start = item[3];
  const int end = item[4];
  const int stripe = item[5];
  const int32_t* rows = image + item[kItemRowsOff];

  const int tk = lane >> 3;
  const int c = lane & 7;

  uint4 qv[G][NCH];
#pragma unroll
  for (int r = 0; r < G; ++r) {
    const uint16_t* qr =
        q + (static_cast<int64_t>(q_row) * num_q + g * G + r) * D + 8 * c;
#pragma unroll
    for (int i = 0; i < NCH; ++i)
      qv[r][i] = *reinterpret_cast<const uint4*>(qr + 64 * i);
  }

  const uint16_t* kh = kc + static_cast<int64_t>(g) * D + 8 * c;
  const uint16_t* vg = vc + static_cast<int64_t>(g) * D;  // + lane's dims at load

  float m[G], l[G], acc[G][DPL];
#pragma unroll
  for (int r = 0; r < G; ++r) {
    m[r] = kNegBig;
    l[r] = 0.0f;
#pragma unroll
    for (int e = 0; e < DPL; ++e) acc[r][e] = 0.0f;
  }

  // Loads of one tile: K for the two passes of 8 positions (lane's position
  // tk and tk + 8) and V for all 16 positions (wave-uniform slots).
  // kTwoPages (pages of >= 16 positions): a tile spans at most two pages,
  // whose rows come from two scalar loads, so no K/V load waits behind a
  // page-table vector load (vmcnt counts in order).
  auto load_tile = [&](uint4 (&kbuf)[2][NCH], VT (&vbuf)[kTile], int pos0) {
    const int tile_len = min(kTile, end - pos0);
    const int p0 = start_pos + pos0;
    const int pg0 = p0 >> shift;
    int64_t ra = 0, rb = 0;
    if constexpr (kTwoPages) {
      const int pg1 = (p0 + tile_len - 1) >> shift;
      ra = sload(rows + (pg0 & page_mask));
      rb = pg1 != pg0 ? sload(rows + (pg1 & page_mask)) : ra;
    }
    auto slot_of = [&](int p) -> int64_t {
      if constexpr (kTwoPages) {
        return ((p >> shift) == pg0 ? ra : rb) + (p & row_mask);
      } else {
        return static_cast<int64_t>(rows[(p >> shift) & page_mask]) + (p & row_mask);
      }
    };
    // Branch-free: a position past the tile reloads the tile's first row
    // (its score is masked and its value skipped), so every load of the tile
    // issues back to back.
#pragma unroll
    for (int b = 0; b < 2; ++b) {
      const int t = 8 * b + tk;
      const int64_t slot = slot_of(p0 + (t < tile_len ? t : 0));
      const uint16_t* kr = kh + slot * kv_stride;
#pragma unroll
      for (int i = 0; i < NCH; ++i)
        kbuf[b][i] = load_kv(reinterpret_cast<const uint4*>(kr + 64 * i));
    }
#pragma unroll
    for (int t = 0; t < kTile; ++t) {
      const int64_t slot = slot_of(p0 + (t < tile_len ? t : 0));
      vbuf[t] = load_kv(reinterpret_cast<const VT*>(vg + slot * kv_stride) + lane);
    }
    // Keep the V loads ahead of the score math: one memory round trip a tile.
    __builtin_amdgcn_sched_barrier(0);
  };

  auto process = [&](const uint4 (&kv4s)[2][NCH], const VT (&vv)[kTile], int pos0) {
    const int tile_len = min(kTile, end - pos0);

    // ---- scores for the tile's 16 positions (two passes of 8) ----
    float s[2][G];
#pragma unroll
    for (int b = 0; b < 2; ++b) {
      const bool valid = 8 * b + tk < tile_len;
#pragma unroll
      for (int r = 0; r < G; ++r) {
        float a = 0.0f;
#pragma unroll
        for (int i = 0; i < NCH; ++i) {
          a = dot2_bf16(kv4s[b][i].x, qv[r][i].x, a);
          a = dot2_bf16(kv4s[b][i].y, qv[r][i].y, a);
          a = dot2_bf16(kv4s[b][i].z, qv[r][i].z, a);
          a = dot2_bf16(kv4s[b][i].w, qv[r][i].w, a);
        }
        a = a + dpp_f32<kDppXor1>(a);
        a = a + dpp_f32<kDppXor2>(a);
        a = a + dpp_f32<kDppHalfMirror>(a);
        s[b][r] = valid ? a : kNegBig;
      }
    }

    // ---- online softmax, once per tile per q head ----
    float w[2][G];
#pragma unroll
    for (int r = 0; r < G; ++r) {
      float mx = max_ref(s[0][r], s[1][r]);
      mx = max_ref(mx, dpp_f32<kDppRowRor8>(mx));
      mx = pair_max32(pair_max16(mx));
      const float m_new = mx > m[r] ? mx : m[r];
      const float corr = fexp(max_ref(-87.0f, m[r] - m_new));
      w[0][r] = fexp(max_ref(-87.0f, s[0][r] - m_new));
      w[1][r] = fexp(max_ref(-87.0f, s[1][r] - m_new));
      // Halving tree over positions t = 8b + tk: (t, t+8) in-lane, then
      // tk ^ 4, tk ^ 2, tk ^ 1 = lane ^ 32, ^ 16, ^ 8.
      float ts = w[0][r] + w[1][r];
      ts = pair_sum16(pair_sum32(ts));
      ts = ts + dpp_f32<kDppRowRor8>(ts);
      const float lc = l[r] * corr;
      l[r] = lc + ts;
      m[r] = m_new;
#pragma unroll
      for (int e = 0; e < DPL; ++e) acc[r][e] = acc[r][e] * corr;
    }

    // ---- PV in position order ----
#pragma unroll
    for (int t = 0; t < kTile; ++t) {
      if (t < tile_len) {
        float wr[G];
#pragma unroll
        for (int r = 0; r < G; ++r) wr[r] = readlane_f32(w[t >> 3][r], 8 * (t & 7));
        float vf[DPL];
        V::unpack(vv[t], vf);
#pragma unroll
        for (int e = 0; e < DPL; ++e)
#pragma unroll
          for (int r = 0; r < G; ++r) acc[r][e] = fmaf(vf[e], wr[r], acc[r][e]);
      }
    }
    };

  uint4 kbuf[2][NCH];
  VT vbuf[kTile];
  const int n_tiles = (end - start + kTile - 1) / kTile;
  if (kShort && n_tiles <= 3) {
    // Items of at most three tiles (one sequence over many splits, about
    // one wave per SIMD): straight-line code with the loads of the first two
    // tiles issued together and the third's issued while the second is
    // processed.  Every load is unconditional (a missing tile rereads the
    // previous one, never used), so each wait covers only older loads.
    uint4 kbuf2[2][NCH];
    VT vbuf2[kTile];
    const int p1 = n_tiles > 1 ? start + kTile : start;
    const int p2 = n_tiles > 2 ? start + 2 * kTile : p1;
    load_tile(kbuf, vbuf, start);
    load_tile(kbuf2, vbuf2, p1);
    process(kbuf, vbuf, start);
    load_tile(kbuf, vbuf, p2);
    if (n_tiles > 1) process(kbuf2, vbuf2, p1);
    if (n_tiles > 2) process(kbuf, vbuf, p2);
  } else {
    for (int pos0 = start; pos0 < end; pos0 += kTile) {
      load_tile(kbuf, vbuf, pos0);
      process(kbuf, vbuf, pos0);
    }
  }

  float* part = partials + static_cast<int64_t>(stripe) * partial_stride;
#pragma unroll
  for (int r = 0; r < G; ++r) {
    float* dst = part + static_cast<int64_t>(g * G + r) * D + DPL * lane;
#pragma unroll
    for (int e = 0; e < DPL; e += 4)
      *reinterpret_cast<float4*>(dst + e) =
          make_float4(acc[r][e], acc[r][e + 1], acc[r][e + 2], acc[r][e + 3]);
  }
  if (lane == 0) {
#pragma unroll
    for (int r = 0; r < G; ++r) {
      part[num_q * D + g * G + r] = m[r];
      part[num_q * D + num_q + g * G + r] = l[r];
    }
  }
}

// merge_segments + write_finalized_head (kernels/logsum_merge.mojo:28-122)
// for one merge unit and one q head per wave; mode IFR_PLAN_TOKEN_DIRECT
// finalises as acc * (1/l) like the sliding prefill kernels
// (kernels/flash_attention_prefill.mojo:95-106).  The order of operations is
// the reference's: global max, 16-wide batches of corrections summed by the
// halving tree, acc initialised by the first live segment, then fma in split
// order.
template <int D>
__global__ __launch_bounds__(256) void merge_kernel(
    const int32_t* __restrict__ image, const float* __restrict__ partials,
    uint16_t* __restrict__ out, int64_t partial_stride, int num_q, int mode,
    int8_t* __restrict__ q_out, float* __restrict__ q_scale) {
  constexpr int DPL = D / 64;
  const int wave = threadIdx.x >> 6;
  const int lane = threadIdx.x & 63;
  const int h = blockIdx.y * 4 + wave;
  if (h >= num_q) return;
  const int32_t* unit = image + image[kHdrOffUnits] + blockIdx.x * kUnitWords;
  const int out_row = unit[0];
  const int stripe_base = unit[1];
  const int n = unit[2];
  const float* base = partials + static_cast<int64_t>(stripe_base) * partial_stride;
  const int m_off = num_q * D;
  const int l_off = m_off + num_q;
  float acc[DPL];
#pragma unroll
  for (int e = 0; e < DPL; ++e) acc[e] = 0.0f;
  float inv_l = 0.0f;
  bool live = false;

  if (mode == 1) {
    const float lv = base[l_off + h];
    if (lv > 0.0f) {
      live = true;
      inv_l = 1.0f / lv;
      const float* src = base + static_cast<int64_t>(h) * D + DPL * lane;
#pragma unroll
      for (int e = 0; e < DPL; ++e) acc[e] = src[e];
    }
  } else {
    // Lanes own splits.  Global max: wave max per 64-split chunk (exact in any
    // order).  Corrections and L: the reference sums the splits in batches
    // of 16, each batch by the halving tree (lane ^ 8, ^ 4, ^ 2, ^ 1 inside
    // 16-lane groups), batches in order.  acc: the splits in order, loads
    // issued eight at a time ahead of the fma chain.
    float gm = kNegBig;
    for (int s0 = 0; s0 < n; s0 += 64) {
      float sm = kNegBig;
      if (s0 + lane < n)
        sm = base[static_cast<int64_t>(s0 + lane) * partial_stride + m_off + h];
      sm = wave_max_ref(sm);
      gm = max_ref(gm, sm);
    }
    float gl = 0.0f;
    bool first = true;
    for (int s0 = 0; s0 < n; s0 += 64) {
      float delta = kNegBig, ls = 0.0f;
      if (s0 + lane < n) {
        const float* sp = base + static_cast<int64_t>(s0 + lane) * partial_stride;
        delta = sp[m_off + h] - gm;
        ls = sp[l_off + h];
      }
      float cv = fexp(max_ref(-87.0f, delta));
      cv = ls > 0.0f ? cv : 0.0f;
      float prod = ls * cv;
      prod = tree16_sum(prod);
      const int cnt = min(64, n - s0);
      for (int b = 0; b * 16 < cnt; ++b) gl = gl + readlane_f32(prod, 16 * b);
      for (int j = 0; j < cnt; j += 8) {
        float src[8][DPL];
        float c8[8];
#pragma unroll
        for (int u = 0; u < 8; ++u) {
          c8[u] = 0.0f;
          if (j + u < cnt) {
            c8[u] = readlane_f32(cv, j + u);
            const float* sp = base + static_cast<int64_t>(s0 + j + u) * partial_stride +
                              static_cast<int64_t>(h) * D + DPL * lane;
#pragma unroll
            for (int e = 0; e < DPL; e += 4) {
              const float4 v4 = *reinterpret_cast<const float4*>(sp + e);
              src[u][e] = v4.x;
              src[u][e + 1] = v4.y;
              src[u][e + 2] = v4.z;
              src[u][e + 3] = v4.w;
            }
          }
        }
#pragma unroll
        for (int u = 0; u < 8; ++u) {
          if (c8[u] <= 0.0f) continue;
          if (first) {
#pragma unroll
            for (int e = 0; e < DPL; ++e) acc[e] = src[u][e] * c8[u];
            first = false;
          } else {
#pragma unroll
            for (int e = 0; e < DPL; ++e) acc[e] = fmaf(src[u][e], c8[u], acc[e]);
          }
        }
      }
    }
    if (gl > 0.0f) {
      live = true;
      inv_l = 1.0f / gl;
    }
  }

  uint16_t* dst = out + (static_cast<int64_t>(out_row) * num_q + h) * D + DPL * lane;
  uint32_t packed[DPL / 2];
#pragma unroll
  for (int e = 0; e < DPL; e += 2) {
    uint32_t lo = live ? f32_to_bf16_bits(acc[e] * inv_l) : 0u;
    uint32_t hi = live ? f32_to_bf16_bits(acc[e + 1] * inv_l) : 0u;
    packed[e / 2] = lo | (hi << 16);
  }
  if constexpr (DPL == 4) {
    *reinterpret_cast<uint2*>(dst) = make_uint2(packed[0], packed[1]);
  } else {
    *reinterpret_cast<uint4*>(dst) =
        make_uint4(packed[0], packed[1], packed[2], packed[3]);
  }
  if (q_out) {
    // The o_proj input step fused in: per-head absmax int8 of the bf16
    // outputs just stored (dispatch_bq_block_quant[block=head_dim,
    // apply_fwht=False], butterquant_kernels/linear.mojo:182-206; quant_segment,
    // butterquant/kernels.mojo:83-92).
    float vals[DPL];
    float amax = 0.0f;
#pragma unroll
    for (int e = 0; e < DPL; e += 2) {
      vals[e] = bf16_lo(packed[e / 2]);
      vals[e + 1] = bf16_hi(packed[e / 2]);
      amax = fmaxf(amax, fmaxf(fabsf(vals[e]), fabsf(vals[e + 1])));
    }
#pragma unroll
    for (int msk = 1; msk < 64; msk <<= 1) amax = fmaxf(amax, shfl_xor_f32(amax, msk));
    const float inv = amax > 0.0f ? 127.0f / amax : 0.0f;
    uint32_t codes[DPL / 4];
#pragma unroll
    for (int c = 0; c < DPL / 4; ++c) {
      uint32_t word = 0;
#pragma unroll
      for (int b = 0; b < 4; ++b) {
        const float r = fminf(fmaxf(rintf(vals[4 * c + b] * inv), -128.0f), 127.0f);
        word |= (static_cast<uint32_t>(static_cast<int32_t>(r)) & 0xFFu) << (8 * b);
      }
      codes[c] = word;
    }
    int8_t* qd = q_out + (static_cast<int64_t>(out_row) * num_q + h) * D + DPL * lane;
    if constexpr (DPL == 4) {
      *reinterpret_cast<uint32_t*>(qd) = codes[0];
    } else {
      *reinterpret_cast<uint2*>(qd) = make_uint2(codes[0], codes[1]);
    }
    if (lane == 0) q_scale[static_cast<int64_t>(out_row) * num_q + h] = amax;
  }
}

// The merge for units with many splits (single-sequence decode): a block
// owns one (unit, q head, 64-dim slice), a lane one dim.  The four waves
// load 32 splits each of every 128-split group into LDS, so a wave has at
// most 34 loads in flight and the group costs one memory round trip; wave 0
// then runs the operations of merge_kernel in the same order: the global
// max, per 64-split chunk the corrections and the halving-tree sums of L in
// batches of 16, and the acc chain over the splits in order.
template <int D>
__global__ __launch_bounds__(256) void merge_staged_kernel(
    const int32_t* __restrict__ image, const float* __restrict__ partials,
    uint16_t* __restrict__ out, int64_t partial_stride, int num_q, int direct_n) {
  constexpr int kGroup = 128;  // splits staged per round, 32 per wave
  __shared__ float stage[kGroup][64];
  __shared__ float coef[64];
  const int wave = threadIdx.x >> 6;
  const int lane = threadIdx.x & 63;
  const int h = blockIdx.y;
  const int dim = 64 * blockIdx.z + lane;
  // direct_n > 0: one output row 0 over stripes [0, direct_n), no plan image.
  int out_row = 0, stripe_base = 0, n = direct_n;
  if (direct_n <= 0) {
    const int32_t* unit = image + image[kHdrOffUnits] + blockIdx.x * kUnitWords;
    out_row = unit[0];
    stripe_base = unit[1];
    n = unit[2];
  }
  const float* base = partials + static_cast<int64_t>(stripe_base) * partial_stride;
  const int m_off = num_q * D;
  const int l_off = m_off + num_q;
  const float* col = base + static_cast<int64_t>(h) * D + dim;

  float gm = kNegBig;
  if (wave == 0 && n > kGroup) {
    for (int s0 = 0; s0 < n; s0 += 64) {
      float sm = kNegBig;
      if (s0 + lane < n)
        sm = base[static_cast<int64_t>(s0 + lane) * partial_stride + m_off + h];
      gm = max_ref(gm, wave_max_ref(sm));
    }
  }
  float acc = 0.0f, gl = 0.0f;
  bool first = true;
  for (int g0 = 0; g0 < n; g0 += kGroup) {
    // All 32 loads issue before the first LDS write (a split past n rereads
    // split n - 1; the chain never uses it).
    float ld[32];
#pragma unroll
    for (int j = 0; j < 32; ++j)
      ld[j] = col[static_cast<int64_t>(min(g0 + 32 * wave + j, n - 1)) * partial_stride];
#pragma unroll
    for (int j = 0; j < 32; ++j) stage[32 * wave + j][lane] = ld[j];
    float mv[2], lv[2];
    if (wave == 0) {
#pragma unroll
      for (int c = 0; c < 2; ++c) {
        const int sp = g0 + 64 * c + lane;
        mv[c] = kNegBig;
        lv[c] = 0.0f;
        if (sp < n) {
          const float* p = base + static_cast<int64_t>(sp) * partial_stride;
          mv[c] = p[m_off + h];
          lv[c] = p[l_off + h];
        }
      }
      if (n <= kGroup) gm = max_ref(wave_max_ref(mv[0]), wave_max_ref(mv[1]));
    }
    __syncthreads();
    if (wave == 0) {
#pragma unroll
      for (int c = 0; c < 2; ++c) {
        const int c0 = g0 + 64 * c;
        if (c0 >= n) break;
        const float delta = c0 + lane < n ? mv[c] - gm : kNegBig;
        float cv = fexp(max_ref(-87.0f, delta));
        cv = lv[c] > 0.0f ? cv : 0.0f;
        float prod = lv[c] * cv;
        prod = tree16_sum(prod);
        const int cnt = min(64, n - c0);
        for (int b = 0; b * 16 < cnt; ++b) gl = gl + readlane_f32(prod, 16 * b);
        float x[64];
#pragma unroll
        for (int u = 0; u < 64; ++u) x[u] = stage[64 * c + u][lane];
        if (cnt == 64 && __builtin_amdgcn_ballot_w64(cv > 0.0f) == ~0ull) {
          // Every split of the chunk live (the normal case): the same
          // operations as below without a test per split, the corrections
          // broadcast from LDS so that each step waits only on the last fma.
          coef[lane] = cv;
          float cb[64];
#pragma unroll
          for (int u = 0; u < 64; ++u) cb[u] = coef[u];
          acc = first ? x[0] * cb[0] : fmaf(x[0], cb[0], acc);
          first = false;
#pragma unroll
          for (int u = 1; u < 64; ++u) acc = fmaf(x[u], cb[u], acc);
        } else {
#pragma unroll
          for (int u = 0; u < 64; ++u) {
            const float cu = u < cnt ? readlane_f32(cv, u) : 0.0f;  // cv is 0 past n
            if (cu <= 0.0f) continue;
            if (first) {
              acc = x[u] * cu;
              first = false;
            } else {
              acc = fmaf(x[u], cu, acc);
            }
          }
        }
      }
    }
    __syncthreads();
  }
  if (wave == 0) {
    const bool live = gl > 0.0f;
    const float inv_l = live ? 1.0f / gl : 0.0f;
    uint16_t* dst = out + (static_cast<int64_t>(out_row) * num_q + h) * D + dim;
    *dst = static_cast<uint16_t>(live ? f32_to_bf16_bits(acc * inv_l) : 0u);
  }
}

template <int D, int G>
hipError_t launch_partials(const int32_t* image, int num_items, const void* q,
                           const void* k, const void* v, float* partials,
                           int64_t ps, int num_q, int num_kv, int64_t kv_stride,
                           PagedGeom geom, hipStream_t stream) {
  // The kv-head groups of an item are the fast grid dimension: the blocks
  // reading the two halves of each K/V row run side by side (config 3:
  // 5.83 -> 6.02 TB/s; items keep their longest-first order).
  dim3 grid((num_kv + kDecodeWaves - 1) / kDecodeWaves, num_items);
  const auto* qp = static_cast<const uint16_t*>(q);
  const auto* kp = static_cast<const uint16_t*>(k);
  const auto* vp = static_cast<const uint16_t*>(v);
  // Grids of at most one wave per SIMD (256 CUs x 4 SIMDs) take the
  // straight-line path for short items; larger grids keep 4 waves per SIMD.
  const bool small = static_cast<int64_t>(grid.x) * grid.y * kDecodeWaves <= 1024;
  auto go = [&](auto kernel) {
    hipLaunchKernelGGL(kernel, grid, dim3(64 * kDecodeWaves), 0, stream, image, qp, kp, vp,
                       partials, ps, num_q, num_kv, kv_stride, geom.shift, geom.row_mask,
                       geom.page_mask);
  };
  const bool two_pages = geom.row_mask + 1 >= kTile;
  if (two_pages && small) go(flash_partial_bf16_kernel<D, G, true, true>);
  else if (two_pages) go(flash_partial_bf16_kernel<D, G, true, false>);
  else if (small) go(flash_partial_bf16_kernel<D, G, false, true>);
  else go(flash_partial_bf16_kernel<D, G, false, false>);
  return hipGetLastError();
}

}  // namespace

bool attention_shape_supported(int head_dim, int gqa) {
  return ((head_dim == 256 || head_dim == 512) && (gqa == 1 || gqa == 2)) ||
         (head_dim == 512 && gqa == 8);
}

hipError_t launch_merge_stripes(const float* partials, void* output, int64_t ps,
                                int n_stripes, int num_q, hipStream_t stream) {
  if (n_stripes <= 0) return hipSuccess;
  dim3 grid(1, num_q, 128 / 64);
  hipLaunchKernelGGL(merge_staged_kernel<128>, grid, dim3(256), 0, stream, nullptr, partials,
                     static_cast<uint16_t*>(output), ps, num_q, n_stripes);
  return hipGetLastError();
}

hipError_t launch_merge(const int32_t* image, int num_units, int num_stripes, int mode,
                        const float* partials, void* output, int64_t ps,
                        int num_q, int head_dim, hipStream_t stream, int8_t* q_out,
                        float* q_scale) {
  if (num_units <= 0) return hipSuccess;
  // Measured on MI355X: units with many splits (single-sequence decode)
  // merge fastest staged through LDS by one block per (unit, head, 64-dim
  // slice); with 8-16 splits per unit (batched decode) the one-wave-per-head
  // kernel is faster.  The fused int8 epilogue needs a whole head per wave.
  const bool staged = mode != 1 && num_stripes >= 32 * num_units && q_out == nullptr;
  uint16_t* o = static_cast<uint16_t*>(output);
  if (staged) {
    dim3 grid(num_units, num_q, head_dim / 64);
    if (head_dim == 256)
      hipLaunchKernelGGL(merge_staged_kernel<256>, grid, dim3(256), 0, stream, image,
                         partials, o, ps, num_q, 0);
    else
      hipLaunchKernelGGL(merge_staged_kernel<512>, grid, dim3(256), 0, stream, image,
                         partials, o, ps, num_q, 0);
    return hipGetLastError();
  }
  dim3 grid(num_units, (num_q + 3) / 4, 1);
  if (head_dim == 256)
    hipLaunchKernelGGL(merge_kernel<256>, grid, dim3(256), 0, stream, image, partials, o, ps,
                       num_q, mode, q_out, q_scale);
  else
    hipLaunchKernelGGL(merge_kernel<512>, grid, dim3(256), 0, stream, image, partials, o, ps,
                       num_q, mode, q_out, q_scale);
  return hipGetLastError();
}

hipError_t launch_partials_bf16(const int32_t* image, int num_items,
                                const void* q, const void* k, const void* v,
                                float* partials, int64_t ps, int num_q,
                                int num_kv, int head_dim, int64_t kv_stride,
                                PagedGeom geom, hipStream_t stream) {
  if (num_items <= 0) return hipSuccess;
  const int gqa = num_q / num_kv;
  if (head_dim == 512 && gqa == 8)
    return launch_partials_wide_bf16(image, num_items, q, k, v, partials, ps, num_q, num_kv,
                                     kv_stride, geom, stream);
  if (head_dim == 256 && gqa == 2)
    return launch_partials<256, 2>(image, num_items, q, k, v, partials, ps,
                                   num_q, num_kv, kv_stride, geom, stream);
  if (head_dim == 256 && gqa == 1)
    return launch_partials<256, 1>(image, num_items, q, k, v, partials, ps,
                                   num_q, num_kv, kv_stride, geom, stream);
  if (head_dim == 512 && gqa == 2)
    return launch_partials<512, 2>(image, num_items, q, k, v, partials, ps,
                                   num_q, num_kv, kv_stride, geom, stream);
  return launch_partials<512, 1>(image, num_items, q, k, v, partials, ps,
                                 num_q, num_kv, kv_stride, geom, stream);
}

hipError_t launch_attention_bf16(const int32_t* image, int num_items,
                                 int num_units, int mode, const void* q,
                                 const void* k, const void* v, void* output,
                                 float* partials, int64_t ps, int num_q,
                                 int num_kv, int head_dim, int64_t kv_stride,
                                 PagedGeom geom, hipStream_t stream) {
  hipError_t err = launch_partials_bf16(image, num_items, q, k, v, partials, ps,
                                        num_q, num_kv, head_dim, kv_stride,
                                        geom, stream);
  if (err != hipSuccess) return err;
  return launch_merge(image, num_units, num_items, mode, partials, output, ps, num_q,
                      head_dim, stream);
}

}  // namespace ifr
