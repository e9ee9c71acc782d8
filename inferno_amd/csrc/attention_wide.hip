// Split-KV partials for Gemma-4's full-attention layers: head_dim 512 with 8 q
// heads per kv head (16 q / 2 kv heads, modeling/gemma4_common.mojo:14-20,
// called through dispatch_full_attention and dispatch_bq_full_attention at
// modeling/gemma_4_moe.mojo:470-476 and modeling/gemma_4_moe_bq.mojo:593-601),
// for bf16 and butterquant int8 KV.
//
// One wave owns one (work item, kv head) and walks the item in the
// reference's 16-position tiles from its first position (FlashAttentionKernel,
// kernels/flash_attention.mojo:44-54; BqFlashAttentionKernel,
// butterquant_kernels/attention.mojo:128-161), one online-softmax update per
// tile per q head (process_kv_tile, kernels/attention_ops.mojo:193-253;
// bq_process_kv_tile, butterquant_kernels/attention.mojo:27-102).
//
// Eight q heads share every K and V load:
//   Scores  S (16 positions x 16 columns) = K . Q^T on MFMA, columns 8..15
//           repeating heads 0..7.  bf16: v_mfma_f32_16x16x32_bf16, 16 steps
//           over the 512 dims (products exact in f32).  int8:
//           v_mfma_i32_16x16x64_i8, 8 steps; sum k*q is exact, and with
//           128 * sum q it is the reference's VNNI raw dot, so the bq scores
//           are the reference's bit for bit.  Lane l holds S[position
//           4*(l/16) + j][head l%16], j = 0..3; the A operand of step s is
//           16 bytes of the key row of position l%16 at byte 64*s + 16*(l/16),
//           so one load instruction reads 64 contiguous bytes of 16 rows.
//   Softmax per head in that layout: the tile max over the lane's 4 values
//           and the lane ^ 16 / ^ 32 swaps; the weight sum in the halving tree
//           of SIMD.reduce_add over positions (t, t+8) = lane ^ 32, (t, t+4) =
//           lane ^ 16, then (j, j+2), (j, j+1) in the lane.
//   P.V     on VALU: lane L owns output dims 8L..8L+7 of all 8 heads (64
//           accumulators) and adds fma(v, w, acc) in position order, the
//           reference's per-element order; each position's weights reach
//           every lane as two broadcast LDS reads.  The V row of a position
//           (1 KiB bf16 or 512 B int8) is one load instruction.
// Loads are software-pipelined in the tile's own registers (no second tile
// buffer): the next tile's K loads are issued once the score MFMAs have read
// K and run under the softmax and P.V; its V loads are issued after the P.V
// and run under the next scores and softmax.  A wave thus always has about
// one tile in flight (about 220 VGPRs for bf16, 185-190 for int8: two waves
// per SIMD).
#include <type_traits>

#include "common.hpp"
#include "launch.hpp"

namespace ifr {
namespace {

constexpr int kWD = 512;                // head_dim
constexpr int kWG = 8;                  // q heads per kv head
constexpr int kWQPitch = 2 * kWD + 16;  // bytes per staged bf16 q row in LDS
constexpr int kWQPitchBq = kWD + 16;    // bytes per staged int8 q row in LDS

typedef __bf16 wbf16x8_t __attribute__((ext_vector_type(8)));
typedef float wf32x4_t __attribute__((ext_vector_type(4)));
typedef int wi32x4_t __attribute__((ext_vector_type(4)));
typedef unsigned int wu32x4_t __attribute__((ext_vector_type(4)));
typedef unsigned int wu32x2_t __attribute__((ext_vector_type(2)));

// K/V are streamed once per step (non-temporal, as in the other decode
// kernels).
__device__ __forceinline__ uint4 wide_load16(const uint8_t* p) {
  const wu32x4_t v = __builtin_nontemporal_load(reinterpret_cast<const wu32x4_t*>(p));
  return make_uint4(v.x, v.y, v.z, v.w);
}
__device__ __forceinline__ uint2 wide_load8(const uint8_t* p) {
  const wu32x2_t v = __builtin_nontemporal_load(reinterpret_cast<const wu32x2_t*>(p));
  return make_uint2(v.x, v.y);
}

typedef __attribute__((address_space(1))) const uint8_t gu8_t;  // global memory

template <bool kBq>
struct WideTile {
  static constexpr int kRow = kBq ? kWD : 2 * kWD;  // bytes of one head's row
  static constexpr int kSteps = kRow / 64;          // MFMA k-steps, 16 B per lane
  using VT = typename std::conditional<kBq, uint2, uint4>::type;
  uint4 k[kSteps];
  VT v[kTile];
  float ks, vs;  // bq: the scales of position l % 16 (the lane's K row)
};

__device__ __forceinline__ void unpack8(const uint4& w, float* f) {
  f[0] = bf16_lo(w.x);
  f[1] = bf16_hi(w.x);
  f[2] = bf16_lo(w.y);
  f[3] = bf16_hi(w.y);
  f[4] = bf16_lo(w.z);
  f[5] = bf16_hi(w.z);
  f[6] = bf16_lo(w.w);
  f[7] = bf16_hi(w.w);
}
__device__ __forceinline__ void unpack8(const uint2& w, float* f) {
#pragma unroll
  for (int b = 0; b < 4; ++b) {
    f[b] = static_cast<float>(static_cast<int8_t>(w.x >> (8 * b)));
    f[4 + b] = static_cast<float>(static_cast<int8_t>(w.y >> (8 * b)));
  }
}

template <bool kBq, bool kTwoPages>
__global__ __launch_bounds__(64) void flash_partial_wide_kernel(
    const int32_t* __restrict__ image, const uint8_t* __restrict__ q,
    const float* __restrict__ qi_bias, const float* __restrict__ f_q,
    const uint8_t* __restrict__ kc, const float* __restrict__ k_scale,
    const uint8_t* __restrict__ vc, const float* __restrict__ v_scale,
    float* __restrict__ partials, int64_t partial_stride, int num_q, int num_kv,
    int64_t row_bytes, int shift, int row_mask, int page_mask) {
  using Tile = WideTile<kBq>;
  constexpr int kRow = Tile::kRow;
  constexpr int kSteps = Tile::kSteps;
  constexpr int kVB = kRow / 64;  // value bytes per lane per position
  using VT = typename Tile::VT;
  __shared__ __align__(16) uint8_t qs[kWG * (kBq ? kWQPitchBq : kWQPitch)];
  // The tile's weights, [position][q head]: each position's 8 weights reach
  // every lane as two broadcast LDS reads (LDS instructions, where 8
  // v_readlanes per position were VALU work in a VALU-bound loop).
  __shared__ __align__(16) float wl[kTile * kWG];
  // bq: the tile's K and V scales, lane l's at [l] (position l % 16, four
  // copies), so a lane reads positions 4*(l/16) .. +3 as one float4: one
  // scale load per lane and tile instead of four, each with its own row
  // lookup.
  __shared__ __align__(16) float scl[2][kBq ? 64 : 1];
  // The tile's corrections of the 8 heads (lane h writes head h's), read
  // back by every lane as two broadcast LDS reads instead of 8 v_readlanes.
  __shared__ __align__(16) float cl[kWG];

  const int lane = threadIdx.x;
  const int g = blockIdx.x;
  const int32_t* item = image + sload(image + kHdrOffItems) + blockIdx.y * kItemWords;
  const int q_row = sload(item);
  const int start_pos = sload(item + 2);
  const int start = sload(item + 3);
  const int end = sload(item + 4);
  const int stripe = sload(item + 5);
  const int32_t* rows = image + sload(item + kItemRowsOff);

  const int r16 = lane & 15;
  const int qd = lane >> 4;
  const int hq = r16 & (kWG - 1);  // q head of the lane's score column
  const int64_t qh = static_cast<int64_t>(q_row) * num_q + g * kWG + hq;

  // ---- the B operand of the scores ----
  // Both kinds stage the group's 8 q rows in LDS (lane (head lane/8, chunks
  // lane%8 + 8i) copies 16 bytes at a time), so the operands take no
  // registers across the tile loop; each score MFMA reads its 16 bytes.
  int qsum128 = 0;
  float qbias = 0.0f, fq = 0.0f;
  if constexpr (kBq) {
    const uint8_t* qg = q + (static_cast<int64_t>(q_row) * num_q + g * kWG) * kWD;
    const int sh = lane >> 3;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int c = (lane & 7) + 8 * i;
      *reinterpret_cast<uint4*>(qs + sh * kWQPitchBq + 16 * c) =
          *reinterpret_cast<const uint4*>(qg + sh * kWD + 16 * c);
    }
    __syncthreads();
    int qs4 = 0;
#pragma unroll
    for (int s = 0; s < kSteps; ++s) {
      const uint4 qc = *reinterpret_cast<const uint4*>(qs + hq * kWQPitchBq + 64 * s + 16 * qd);
      qs4 = __builtin_amdgcn_sdot4(static_cast<int>(qc.x), 0x01010101, qs4, false);
      qs4 = __builtin_amdgcn_sdot4(static_cast<int>(qc.y), 0x01010101, qs4, false);
      qs4 = __builtin_amdgcn_sdot4(static_cast<int>(qc.z), 0x01010101, qs4, false);
      qs4 = __builtin_amdgcn_sdot4(static_cast<int>(qc.w), 0x01010101, qs4, false);
    }
    // The four lane groups hold disjoint quarters of the head's codes.
    qs4 = qs4 + __shfl_xor(qs4, 16);
    qs4 = qs4 + __shfl_xor(qs4, 32);
    qsum128 = 128 * qs4;
    qbias = qi_bias[qh];
    fq = f_q[qh];
  } else {
    const uint8_t* qg = q + (static_cast<int64_t>(q_row) * num_q + g * kWG) * (2 * kWD);
    const int sh = lane >> 3;
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      const int c = (lane & 7) + 8 * i;
      *reinterpret_cast<uint4*>(qs + sh * kWQPitch + 16 * c) =
          *reinterpret_cast<const uint4*>(qg + sh * (2 * kWD) + 16 * c);
    }
    __syncthreads();
  }
  const float inv127 = 1.0f / 127.0f;
  const float inv127sq = inv127 * inv127;

  // Row addresses: slots are page-table rows (int32) and row_bytes is
  // below 2^31 (checked at launch), so slot * row_bytes is one 32 x 32 ->
  // 64-bit multiply (v_mad_u64_u32) instead of a 64-bit product.  A V row's
  // address is wave-uniform: its base stays in SGPRs and the load adds the
  // lane's 32-bit offset (global_load's saddr form, no VALU address work).
  const uint32_t rb32 = static_cast<uint32_t>(row_bytes);
  auto row_off = [&](int64_t slot) -> uint64_t {
    return static_cast<uint64_t>(static_cast<uint32_t>(slot)) * rb32;
  };
  auto scale_idx = [&](int64_t slot) -> uint64_t {
    return static_cast<uint64_t>(static_cast<uint32_t>(slot)) * static_cast<uint32_t>(num_kv) +
           static_cast<uint32_t>(g);
  };
  const uint8_t* kh = kc + static_cast<int64_t>(g) * kRow + 16 * qd;
  const uint8_t* vg = vc + static_cast<int64_t>(g) * kRow;
  const uint32_t v_lane = kVB * lane;

  float m = kNegBig;  // state of head hq (the same in the lanes of a column)
  float lsum = 0.0f;
  float acc[kWG][8];
#pragma unroll
  for (int h = 0; h < kWG; ++h)
#pragma unroll
    for (int e = 0; e < 8; ++e) acc[h][e] = 0.0f;

  // A tile's row lookups and loads, branch-free: a position past the tile
  // reloads the tile's first row (its score is masked, its value skipped).
  // kTwoPages (pages of >= 16 positions): a tile spans at most two pages,
  // whose rows come from two scalar loads.
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
    const int p = r.p0 + (t < r.len ? t : 0);
    if constexpr (kTwoPages) {
      return ((p >> shift) == r.pg0 ? r.ra : r.rb) + (p & row_mask);
    } else {
      return static_cast<int64_t>(rows[(p >> shift) & page_mask]) + (p & row_mask);
    }
  };
  auto load_k = [&](Tile& d, const TileRows& r) {
    const uint8_t* kr = kh + row_off(slot_of(r, r16));
#pragma unroll
    for (int s = 0; s < kSteps; ++s) d.k[s] = wide_load16(kr + 64 * s);
    if constexpr (kBq) d.ks = k_scale[scale_idx(slot_of(r, r16))];
  };
  // The V scale first: the softmax then waits for it alone, not for the
  // tile's V rows, which only the P.V needs.
  auto load_v = [&](Tile& d, const TileRows& r) {
    if constexpr (kBq) d.vs = v_scale[scale_idx(slot_of(r, r16))];
#pragma unroll
    for (int t = 0; t < kTile; ++t) {
      const gu8_t* vrow = (const gu8_t*)(vg + row_off(slot_of(r, t)));
      asm("" : "+s"(vrow));
      const uint8_t* vr = (const uint8_t*)(vrow + v_lane);
      if constexpr (kBq) {
        d.v[t] = wide_load8(vr);
      } else {
        d.v[t] = wide_load16(vr);
      }
    }
  };

  Tile d;
  // One tile: scores, online softmax, P.V.  kFlat: the P.V visits all
  // kTile positions without branches, a position past the tile with weight
  // 0 (its V row is the tile's first row, so fma(v, 0, acc) leaves acc as
  // it is: the accumulators start at +0 and never become -0 by addition).
  // Otherwise positions past the tile are skipped.  kNext: the loads of
  // tile rn are issued into the tile's registers as soon as this tile is
  // done with them (K after the score MFMAs, V after the P.V).  kFull: the
  // tile holds kTile positions, so no score is masked and no position
  // skipped (the same operations as the general form on such a tile).
  auto step = [&](auto flat_c, auto next_c, auto full_c, const TileRows& r,
                  const TileRows& rn) {
    constexpr bool kFlat = decltype(flat_c)::value;
    constexpr bool kNext = decltype(next_c)::value;
    constexpr bool kFull = decltype(full_c)::value;
    const int tile_len = kFull ? kTile : r.len;

    // ---- scores: lane holds positions 4*qd + j of head hq ----
    float sj[4];
    if constexpr (kBq) {
      wi32x4_t si = {0, 0, 0, 0};
#pragma unroll
      for (int s = 0; s < kSteps; ++s) {
        const uint4 qf =
            *reinterpret_cast<const uint4*>(qs + hq * kWQPitchBq + 64 * s + 16 * qd);
        si = __builtin_amdgcn_mfma_i32_16x16x64_i8(__builtin_bit_cast(wi32x4_t, d.k[s]),
                                                    __builtin_bit_cast(wi32x4_t, qf), si,
                                                    0, 0, 0);
      }
      // The K scales of the lane's positions 4*qd + j from the lanes that
      // loaded them (the wave's own LDS: its write lands before its read).
      scl[0][lane] = d.ks;
      const float4 ks4 = *reinterpret_cast<const float4*>(&scl[0][4 * qd]);
      const float ksj[4] = {ks4.x, ks4.y, ks4.z, ks4.w};
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        float sc = static_cast<float>(si[j] + qsum128) - qbias;
        sc = sc * fq;
        sc = sc * ksj[j];
        sc = sc * inv127sq;
        sj[j] = (kFull || 4 * qd + j < tile_len) ? sc : kNegBig;
      }
    } else {
      wf32x4_t sc = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
      for (int s = 0; s < kSteps; ++s) {
        const uint4 qf = *reinterpret_cast<const uint4*>(qs + hq * kWQPitch + 64 * s + 16 * qd);
        sc = __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(wbf16x8_t, d.k[s]),
                                                     __builtin_bit_cast(wbf16x8_t, qf), sc, 0,
                                                     0, 0);
      }
#pragma unroll
      for (int j = 0; j < 4; ++j) sj[j] = (kFull || 4 * qd + j < tile_len) ? sc[j] : kNegBig;
    }
    if constexpr (kNext) {
      __builtin_amdgcn_sched_barrier(0);
      load_k(d, rn);
      __builtin_amdgcn_sched_barrier(0);
    }

    // ---- online softmax of head hq (online_softmax_tile) ----
    float mx = max_ref(max_ref(sj[0], sj[1]), max_ref(sj[2], sj[3]));
    mx = pair_max32(pair_max16(mx));
    const float m_new = mx > m ? mx : m;
    const float corr = fexp(max_ref(-87.0f, m - m_new));
    float w[4];
#pragma unroll
    for (int j = 0; j < 4; ++j) w[j] = fexp(max_ref(-87.0f, sj[j] - m_new));
    float ws[4];
#pragma unroll
    for (int j = 0; j < 4; ++j) ws[j] = pair_sum16(pair_sum32(w[j]));
    const float wsum = (ws[0] + ws[2]) + (ws[1] + ws[3]);
    const float lc = lsum * corr;
    lsum = lc + wsum;
    m = m_new;
    if constexpr (kBq) {
      // bq_process_kv_tile's value weights: (w * v_scale) / 127.
      scl[1][lane] = d.vs;
      const float4 vs4 = *reinterpret_cast<const float4*>(&scl[1][4 * qd]);
      const float vsj[4] = {vs4.x, vs4.y, vs4.z, vs4.w};
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        const float a = w[j] * vsj[j];
        w[j] = a * inv127;
      }
    }

    if constexpr (kFlat && !kFull) {
#pragma unroll
      for (int j = 0; j < 4; ++j) w[j] = 4 * qd + j < tile_len ? w[j] : 0.0f;
    }

    // Lanes of columns 0..7 publish their weights (the wave's own LDS: its
    // writes land before its reads, and the previous tile's reads are done).
    if ((lane & 15) < kWG) {
#pragma unroll
      for (int j = 0; j < 4; ++j) wl[(4 * qd + j) * kWG + (lane & (kWG - 1))] = w[j];
    }

    // ---- scale_unrolled, then P.V in position order ----
    if (lane < kWG) cl[lane] = corr;  // lane h: column h, head h
    const float4 ca = *reinterpret_cast<const float4*>(&cl[0]);
    const float4 cb = *reinterpret_cast<const float4*>(&cl[4]);
    const float chs[kWG] = {ca.x, ca.y, ca.z, ca.w, cb.x, cb.y, cb.z, cb.w};
#pragma unroll
    for (int h = 0; h < kWG; ++h) {
#pragma unroll
      for (int e = 0; e < 8; ++e) acc[h][e] = acc[h][e] * chs[h];
    }
#pragma unroll
    for (int t = 0; t < kTile; ++t) {
      if (kFlat || kFull || t < tile_len) {  // wave-uniform
        float vf[8];
        unpack8(d.v[t], vf);
        const float4 wa = *reinterpret_cast<const float4*>(&wl[t * kWG]);
        const float4 wb = *reinterpret_cast<const float4*>(&wl[t * kWG + 4]);
        const float wt[kWG] = {wa.x, wa.y, wa.z, wa.w, wb.x, wb.y, wb.z, wb.w};
#pragma unroll
        for (int h = 0; h < kWG; ++h)
#pragma unroll
          for (int e = 0; e < 8; ++e) acc[h][e] = fmaf(vf[e], wt[h], acc[h][e]);
      }
      // One position at a time (unpacking every V row ahead of its FMAs
      // would not fit the registers).
      if constexpr (kFlat) __builtin_amdgcn_sched_barrier(0);
    }
    if constexpr (kNext) {
      __builtin_amdgcn_sched_barrier(0);
      load_v(d, rn);
      __builtin_amdgcn_sched_barrier(0);
    }
  };
  const std::true_type yes{};
  const std::false_type no{};

  if (start < end) {
    // Software-pipelined in the tile's own registers: the next tile's K
    // loads run under this tile's softmax and P.V, its V loads under the
    // next tile's scores and softmax.  After the last tile the loads go on
    // (in bounds, unused: all of them read the last tile's first row, which
    // the caches hold), so every iteration leaves the same loads in flight
    // and the waits stay exact.
    TileRows r = tile_rows(start);
    load_k(d, r);
    __builtin_amdgcn_sched_barrier(0);  // K before V, as in the loop
    load_v(d, r);
    __builtin_amdgcn_sched_barrier(0);
    // The item's full tiles run without masks, in a loop of their own; a
    // last partial tile takes the general form.
    int pos0 = start;
    auto tile = [&](auto full_c) {
      const int nxt = pos0 + kTile;
      TileRows rn = r;
      if (nxt < end)
        rn = tile_rows(nxt);
      else
        rn.len = 1;  // every load of the dummy tile reads the last tile's first row
      // bf16 with flat P.V; int8 skips positions past the tile (its
      // outputs are compared bit for bit).
      if constexpr (kBq)
        step(no, yes, full_c, r, rn);
      else
        step(yes, yes, full_c, r, rn);
      r = rn;
      pos0 = nxt;
    };
    const int n_full = (end - start) / kTile;
    for (int i = 0; i < n_full; ++i) tile(yes);
    if (pos0 < end) tile(no);
  }

  float* part = partials + static_cast<int64_t>(stripe) * partial_stride;
#pragma unroll
  for (int h = 0; h < kWG; ++h) {
    float* dst = part + static_cast<int64_t>(g * kWG + h) * kWD + 8 * lane;
    *reinterpret_cast<float4*>(dst) = make_float4(acc[h][0], acc[h][1], acc[h][2], acc[h][3]);
    *reinterpret_cast<float4*>(dst + 4) =
        make_float4(acc[h][4], acc[h][5], acc[h][6], acc[h][7]);
  }
  if (lane < kWG) {
    part[num_q * kWD + g * kWG + lane] = m;
    part[num_q * kWD + num_q + g * kWG + lane] = lsum;
  }
}

template <bool kBq>
hipError_t launch_wide(const int32_t* image, int num_items, const void* q,
                       const float* qi_bias, const float* f_q, const void* k,
                       const float* k_scale, const void* v, const float* v_scale,
                       float* partials, int64_t ps, int num_q, int num_kv,
                       int64_t kv_stride, PagedGeom geom, hipStream_t stream) {
  if (num_items <= 0) return hipSuccess;
  const int64_t row_bytes = kv_stride * (kBq ? 1 : 2);
  if (row_bytes <= 0 || row_bytes > INT32_MAX) return hipErrorInvalidValue;  // 32-bit row math
  dim3 grid(num_kv, num_items);  // an item's kv heads side by side
  const auto* qp = static_cast<const uint8_t*>(q);
  const auto* kp = static_cast<const uint8_t*>(k);
  const auto* vp = static_cast<const uint8_t*>(v);
  if (geom.row_mask + 1 >= kTile) {
    hipLaunchKernelGGL((flash_partial_wide_kernel<kBq, true>), grid, dim3(64), 0, stream,
                       image, qp, qi_bias, f_q, kp, k_scale, vp, v_scale, partials, ps,
                       num_q, num_kv, row_bytes, geom.shift, geom.row_mask, geom.page_mask);
  } else {
    hipLaunchKernelGGL((flash_partial_wide_kernel<kBq, false>), grid, dim3(64), 0, stream,
                       image, qp, qi_bias, f_q, kp, k_scale, vp, v_scale, partials, ps,
                       num_q, num_kv, row_bytes, geom.shift, geom.row_mask, geom.page_mask);
  }
  return hipGetLastError();
}

}  // namespace

hipError_t launch_partials_wide_bf16(const int32_t* image, int num_items, const void* q,
                                     const void* k, const void* v, float* partials,
                                     int64_t ps, int num_q, int num_kv, int64_t kv_stride,
                                     PagedGeom geom, hipStream_t stream) {
  return launch_wide<false>(image, num_items, q, nullptr, nullptr, k, nullptr, v, nullptr,
                            partials, ps, num_q, num_kv, kv_stride, geom, stream);
}

hipError_t launch_partials_wide_bq(const int32_t* image, int num_items, const void* q_i8,
                                   const float* qi_bias, const float* f_q, const void* k,
                                   const float* k_scale, const void* v, const float* v_scale,
                                   float* partials, int64_t ps, int num_q, int num_kv,
                                   int64_t kv_stride, PagedGeom geom, hipStream_t stream) {
  return launch_wide<true>(image, num_items, q_i8, qi_bias, f_q, k, k_scale, v, v_scale,
                           partials, ps, num_q, num_kv, kv_stride, geom, stream);
}

}  // namespace ifr
