// Shared device helpers and the plan-image layout for libinferno_hip.so.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace ifr {

// ---------------------------------------------------------------------------
// Plan image layout (int32 words).  Built on the host by ifr_plan_attention,
// uploaded once per step, read by the append, attention and merge kernels.
// ---------------------------------------------------------------------------
constexpr int32_t kPlanMagic = 0x49465231;  // "IFR1"
enum PlanHeader : int {
  kHdrMagic = 0,
  kHdrNumRuns,
  kHdrNumRows,
  kHdrSeqLen,
  kHdrNumItems,
  kHdrNumUnits,
  kHdrMode,
  kHdrNumStripes,
  kHdrOffRuns,
  kHdrOffRows,
  kHdrOffTokRun,
  kHdrOffItems,
  kHdrOffUnits,
  kHdrTotalWords,
  kHdrOffQBlocks,
  kHdrNumQBlocks,
  kHdrWords = 16
};
// A work item: one contiguous position range of one run, for every kv head.
// {q_row, run, start_pos, start, end, stripe, rows_off, 0}; rows_off is the
// image word offset of the run's row table.
constexpr int kItemRowsOff = 6;
constexpr int kItemWords = 8;
// The items start right after the header (the planner reserves room for
// its largest item count there), so a decode wave reaches its item in one
// load instead of a header load followed by the item load.
constexpr int kItemsOff = kHdrWords;
// A merge unit: one output token row, for every q head.
// {out_row, stripe_base, n_stripes, 0}
constexpr int kUnitWords = 4;

// Query blocks of a token (prefill) plan for the MFMA prefill kernel:
// {run, first token, token count, last token's position + 1}, at most
// kPrefillTokens consecutive tokens of one run, longest key range first.
constexpr int kQBlockWords = 4;
constexpr int kPrefillTokens = 64;
// Page-table entries the MFMA prefill kernels hold in LDS: the full-attention
// kernels move a window of this many entries along the run; the sliding
// kernel holds the run's whole ring, so rings of more pages take the token
// kernels.
constexpr int kPrefillLdsPages = 4096;

constexpr int kTile = 16;  // reference TILE = f32 SIMD width on AVX-512
constexpr float kNegBig = -1e30f;

// ---------------------------------------------------------------------------
// Scalar numerics shared by every kernel.
// ---------------------------------------------------------------------------
__device__ __forceinline__ float bf16_lo(uint32_t packed) {
  return __uint_as_float(packed << 16);
}
__device__ __forceinline__ float bf16_hi(uint32_t packed) {
  return __uint_as_float(packed & 0xFFFF0000u);
}
__device__ __forceinline__ float bf16_to_f32(uint16_t b) {
  return __uint_as_float(static_cast<uint32_t>(b) << 16);
}
// Round-to-nearest-even f32 -> bf16 bits (butterquant/convert.mojo:14-17).
__device__ __forceinline__ uint32_t f32_to_bf16_bits(float f) {
  uint32_t u = __float_as_uint(f);
  return (u + ((u >> 16) & 1u) + 0x7FFFu) >> 16;
}

// fast_exp_softmax_biased (simd_math/exponential.mojo:177-194), evaluated
// with the same float operations in the same order (no contraction: the
// library is compiled with -ffp-contract=off).
__device__ __forceinline__ float fexp(float x) {
  const float a_magic = 12102203.16156148f;
  const float bias_f = 1059208216.0f;
  const float qc_a = 1.6501418352127075f;
  const float qc_b = -0.37554836273193359f;
  const float qc_c = 0.38696467876434326f;
  float t = a_magic * x;
  t = t + bias_f;
  int32_t i = static_cast<int32_t>(t);
  uint32_t u = static_cast<uint32_t>(i);
  float k = __uint_as_float(u);
  // f = (float)(u & 0x7FFFFF) / 2^23, formed as F - 1 with F = 1.f (the
  // mantissa bits under a biased exponent of 0): both are m / 2^23 exactly
  // (F - 1 is exact by Sterbenz' lemma, and m / 2^23 needs no rounding), so
  // the bits are the reference's, in one and-or and one subtract instead of
  // an and, an int-to-float conversion and a multiply.
  float f = __uint_as_float((u & 0x7FFFFFu) | 0x3F800000u) - 1.0f;
  float p = f * qc_c;
  p = qc_b + p;
  p = f * p;
  p = qc_a + p;
  return k * p;
}

__device__ __forceinline__ float max_ref(float a, float b) {
  return a > b ? a : b;
}

// ---------------------------------------------------------------------------
// Cross-lane helpers (wave64).
// ---------------------------------------------------------------------------
template <int kCtrl>
__device__ __forceinline__ float dpp_f32(float v) {
  return __int_as_float(__builtin_amdgcn_update_dpp(
      0, __float_as_int(v), kCtrl, 0xF, 0xF, true));
}
template <int kCtrl>
__device__ __forceinline__ int dpp_i32(int v) {
  return __builtin_amdgcn_update_dpp(0, v, kCtrl, 0xF, 0xF, true);
}
constexpr int kDppXor1 = 0xB1;         // quad_perm [1,0,3,2]
constexpr int kDppXor2 = 0x4E;         // quad_perm [2,3,0,1]
constexpr int kDppHalfMirror = 0x141;  // lane i <-> 7-i within 8 lanes
constexpr int kDppQuadReverse = 0x1B;  // quad_perm [3,2,1,0]: lane i <- i ^ 3
constexpr int kDppRowRor8 = 0x128;     // lane i <- (i-8)%16 = lane i ^ 8 within 16 lanes

__device__ __forceinline__ float shfl_xor_f32(float v, int mask) {
  int lane = __lane_id();
  return __int_as_float(
      __builtin_amdgcn_ds_bpermute((lane ^ mask) << 2, __float_as_int(v)));
}
__device__ __forceinline__ int shfl_xor_i32(int v, int mask) {
  int lane = __lane_id();
  return __builtin_amdgcn_ds_bpermute((lane ^ mask) << 2, v);
}
__device__ __forceinline__ float readlane_f32(float v, int lane) {
  return __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), lane));
}

// gfx950 lane swaps.  v_permlane32_swap exchanges the upper 32 lanes of its
// first operand with the lower 32 lanes of its second; v_permlane16_swap the
// odd 16-lane rows of the first with the even rows of the second.  With x as
// both operands the two results hold the two members of each (lane,
// lane ^ 32) or (lane, lane ^ 16) pair, lower lane first, in both lanes of
// the pair.  A commutative op on them therefore gives, bit for bit, what
// x op shfl_xor(x, 32 | 16) gives, as one VALU operation instead of an LDS
// permute round trip.
constexpr int kDppRowRor4 = 0x124;  // lane i <- (i-4)%16 within 16 lanes
__device__ __forceinline__ float pair_sum32(float x) {
  const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x),
                                                  false, false);
  return __uint_as_float(r[0]) + __uint_as_float(r[1]);
}
__device__ __forceinline__ float pair_sum16(float x) {
  const auto r = __builtin_amdgcn_permlane16_swap(__float_as_uint(x), __float_as_uint(x),
                                                  false, false);
  return __uint_as_float(r[0]) + __uint_as_float(r[1]);
}
__device__ __forceinline__ float pair_max32(float x) {
  const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x),
                                                  false, false);
  return max_ref(__uint_as_float(r[0]), __uint_as_float(r[1]));
}
__device__ __forceinline__ float pair_max16(float x) {
  const auto r = __builtin_amdgcn_permlane16_swap(__float_as_uint(x), __float_as_uint(x),
                                                  false, false);
  return max_ref(__uint_as_float(r[0]), __uint_as_float(r[1]));
}
// Max over the 64 lanes (exact in any pairing order): quad swaps, the
// 8-lane mirror, the 16-lane rotate by 8, then the two lane swaps.
__device__ __forceinline__ float wave_max_ref(float x) {
  x = max_ref(x, dpp_f32<kDppXor1>(x));
  x = max_ref(x, dpp_f32<kDppXor2>(x));
  x = max_ref(x, dpp_f32<kDppHalfMirror>(x));
  x = max_ref(x, dpp_f32<kDppRowRor8>(x));
  return pair_max32(pair_max16(x));
}
// x + x[lane ^ 8], then ^ 4, ^ 2, ^ 1 inside each 16-lane row (the halving
// tree of a 16-wide SIMD reduce_add), on DPP.  After the ^ 8 step lanes i and
// i ^ 8 hold the same bits, so the rotate by 4 reads a lane equal to i ^ 4;
// the quad swaps are exact.  Same operands, same order as the shuffles.
__device__ __forceinline__ float tree16_sum(float x) {
  x = x + dpp_f32<kDppRowRor8>(x);
  x = x + dpp_f32<kDppRowRor4>(x);
  x = x + dpp_f32<kDppXor2>(x);
  return x + dpp_f32<kDppXor1>(x);
}
__device__ __forceinline__ int uniform_i32(int v) {
  return __builtin_amdgcn_readfirstlane(v);
}

// A wave-uniform read of read-only data through the scalar cache.  A vector
// load would be counted with the K/V loads in flight (vmcnt is in order), and
// waiting for it would wait for all of them.
__device__ __forceinline__ int32_t sload(const int32_t* p) {
  return *reinterpret_cast<const __attribute__((address_space(4))) int32_t*>(
      reinterpret_cast<uintptr_t>(p));
}

}  // namespace ifr
