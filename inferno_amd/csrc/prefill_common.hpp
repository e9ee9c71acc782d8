// Shared pieces of the MFMA chunked-prefill kernels (prefill.hip: full
// attention; prefill_wide.hip: full attention at head_dim 512 / GQA 8;
// prefill_sliding.hip: sliding window): block geometry, LDS tile sizes,
// lane-pair reductions, the biased exp with fused multiply-adds and the
// per-tile online-softmax step.
#pragma once

#include "common.hpp"

namespace ifr {
namespace prefill {

typedef __bf16 bf16x8_t __attribute__((ext_vector_type(8)));
typedef short s16x4_t __attribute__((ext_vector_type(4)));
typedef float f32x16_t __attribute__((ext_vector_type(16)));
typedef __attribute__((address_space(3))) s16x4_t lds_s16x4_t;
typedef __attribute__((address_space(3))) void lds_void_t;
typedef __bf16 bf16x2_t __attribute__((ext_vector_type(2)));
typedef float f32x2_t __attribute__((ext_vector_type(2)));

constexpr int kPD = 256;             // head_dim
constexpr int kPWaves = 4;           // waves per block (one per SIMD, one block per CU)
constexpr int kPThreads = 64 * kPWaves;
constexpr int kPTokensPerWave = 16;  // x 2 q heads = 32 rows
constexpr int kPTokens = kPWaves * kPTokensPerWave;  // tokens per block
static_assert(kPTokens == kPrefillTokens, "plan query blocks must match the kernel");
constexpr int kKeys = 64;                // keys per iteration
constexpr int kBlocks = kKeys / 32;      // 32-key S blocks (tile pairs) per iteration
constexpr int kDimBlocks = kPD / 32;     // 32-dim blocks of O^T
constexpr int kRowBytes = kPD * 2;       // one key row of K or V in LDS
constexpr int kTileBytes = kKeys * kRowBytes;  // 32 KiB: one iteration of K (or V)
constexpr int kStageRows = kKeys / kPWaves;  // key rows each wave stages per iteration
static_assert(kStageRows % 2 == 0, "two rows per 64-lane load");
static_assert(4 * kTileBytes + 4 * kPrefillLdsPages <= 160 * 1024, "LDS budget");

// x + x[lane ^ 32] and max(x, x[lane ^ 32]) through the gfx950 lane swap:
// with both operands x, the two results hold the low and high member of
// each pair, so their sum (low + high) is the same in both lanes.
__device__ __forceinline__ float sum_xor32(float x) {
  const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x),
                                                  false, false);
  return __uint_as_float(r[0]) + __uint_as_float(r[1]);
}
__device__ __forceinline__ float max_xor32(float x) {
  const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x),
                                                  false, false);
  return fmaxf(__uint_as_float(r[0]), __uint_as_float(r[1]));
}

// The reference's biased exp (the steps of fexp) with fused multiply-adds
// (fexp_fused_u below).
constexpr float kExpA = 12102203.16156148f;
constexpr float kExpBias = 1059208216.0f;
// The quadratic a + f*(b + c*f) in the mantissa fraction f = F - 1 is
// evaluated in F = 1 + f itself, F taken straight from the bits:
// (a - b + c) + F*((b - 2c) + c*F).
constexpr double kExpQa = 1.6501418352127075, kExpQb = -0.37554836273193359,
                 kExpQc = 0.38696467876434326;
// P.V takes P as bf16 hi parts; a tile whose weight sum exceeds this share
// of the row's running l (l after the tile) also takes the lo parts
// p - bf16(p).  The row's final share of a tile can only be smaller (later
// tiles rescale the tile and l alike and add to l), so leaving the lo parts
// out of a tile below the share moves the output by at most
// 2^-9 * kLoShare * max|v|.
constexpr float kLoShare = 0x1p-7f;

// F = 1.0 with the mantissa bits of i: (i & 0x7FFFFF) | 0x3F800000 as one
// v_and_or_b32 (the mask from a scalar register, 1.0 as an inline constant)
// instead of an AND and an OR that each carry a literal.  The mask's s_mov
// has no side effects, so the compiler hoists it out of the loops.
__device__ __forceinline__ float mantissa_one(int32_t i) {
  uint32_t m, r;
  asm("s_mov_b32 %0, 0x7fffff" : "=s"(m));
  asm("v_and_or_b32 %0, %1, %2, 1.0" : "=v"(r) : "v"(i), "s"(m));
  return __uint_as_float(r);
}
// The maximum of 8 values as three v_max3_f32 and one v_max_f32 (the
// maximum of finite values is the same in any order).  Written as
// instructions: fmaxf on values the compiler cannot prove canonical (MFMA
// results copied out of AGPRs) gets a v_max_f32 x, x canonicalisation per
// input, 8 extra VALU instructions per tile.
__device__ __forceinline__ float max3_raw(float a, float b, float c) {
  float r;
  asm("v_max3_f32 %0, %1, %2, %3" : "=v"(r) : "v"(a), "v"(b), "v"(c));
  return r;
}
__device__ __forceinline__ float max8(const float (&v)[8]) {
  float r;
  asm("v_max_f32 %0, %1, %2"
      : "=v"(r)
      : "v"(max3_raw(v[0], v[1], v[2])), "v"(max3_raw(max3_raw(v[3], v[4], v[5]), v[6], v[7])));
  return r;
}

// The biased exp of a pre-scaled argument t = a_magic * x + bias_f, without
// the reference's clamp at x = -87: the conversion to unsigned
// (v_cvt_u32_f32) takes t < 0, i.e. x below about -87.5, to 0 and so to a
// weight of 0 instead of fexp(-87) = 1.4e-38, and t between 0 and the
// clamp's t gives weights below 1.4e-38.  A row's running l holds its
// largest weight (fexp(0) = 0.99963 when it entered, then rescaled by
// fexp(0) per tile without a new maximum: above 0.2 over 4,096 tiles), so
// weights this small change neither l nor any weighted sum in f32: the
// results are those of the clamped form, one VALU instruction less per
// score.
__device__ __forceinline__ float fexp_fused_u(float t) {
  uint32_t i;
  asm("v_cvt_u32_f32 %0, %1" : "=v"(i) : "v"(t));
  const float F = mantissa_one(static_cast<int32_t>(i));
  float p = __builtin_fmaf(F, static_cast<float>(kExpQc), static_cast<float>(kExpQb - 2 * kExpQc));
  p = __builtin_fmaf(F, p, static_cast<float>(kExpQa - kExpQb + kExpQc));
  return __uint_as_float(i) * p;
}

// One tile's online-softmax step for this lane's row (process_kv_tile's
// m / corr / w / l updates, attention_ops.mojo:165-180).  sv[0..7] are the
// lane's 8 keys of the tile, key 8*(i/4) + 4*half + i%4 for value i.
// Masked: the tile reaches past some row's last key (or the row is empty);
// a row with no key in the tile is left untouched (corr 1, weights 0), pads
// score -1e30 (the reference's fexp(-87) of a pad enters l; here its weight
// is 0, which leaves l as it is, see fexp_fused_u).  The in-lane sum of the 8 weights comes
// first, then lane ^32's (the same 16 weights as the reference's halving
// tree, added in another order).  Maxima use v_max_f32 (the scores are
// finite for finite inputs).  big: the tile's weight sum exceeds kLoShare of
// the updated l.
template <bool kMasked>
__device__ __forceinline__ void softmax_tile(const float (&sv)[8], int valid, int half,
                                             float& m, float& l, float& corr, float (&w)[8],
                                             bool& big) {
  float sc[8];
#pragma unroll
  for (int i = 0; i < 8; ++i) {
    const int key = 8 * (i >> 2) + 4 * half + (i & 3);
    sc[i] = (!kMasked || key < valid) ? sv[i] : kNegBig;
  }
  float mx = max8(sc);
  mx = max_xor32(mx);
  const float m_new = fmaxf(mx, m);
  // corr without the clamp as well: below -87.5 it is 0 instead of
  // fexp(-87) = 1.4e-38, which scales an l of at least 0.2 (or 0) and acc
  // alike to nothing next to the tile's own weights.
  const float c = fexp_fused_u(__builtin_fmaf(kExpA, m - m_new, kExpBias));
  // a*(s - m_new) + bias as one fma per key (weights below fexp(-87) go to
  // 0 or below it, as fexp_fused_u states).
  const float t0 = __builtin_fmaf(-kExpA, m_new, kExpBias);
  float e[8];
#pragma unroll
  for (int i = 0; i < 8; ++i) e[i] = fexp_fused_u(__builtin_fmaf(kExpA, sc[i], t0));
  float ts = ((e[0] + e[1]) + (e[2] + e[3])) + ((e[4] + e[5]) + (e[6] + e[7]));
  ts = sum_xor32(ts);
  if (kMasked) {
    const bool any = valid > 0;
    l = any ? l * c + ts : l;
    m = any ? m_new : m;
    corr = any ? c : 1.0f;
    big = any && ts > kLoShare * l;
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      const int key = 8 * (i >> 2) + 4 * half + (i & 3);
      w[i] = key < valid ? e[i] : 0.0f;
    }
  } else {
    l = l * c + ts;
    m = m_new;
    corr = c;
    big = ts > kLoShare * l;
#pragma unroll
    for (int i = 0; i < 8; ++i) w[i] = e[i];
  }
}

}  // namespace prefill
}  // namespace ifr
