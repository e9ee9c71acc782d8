// Chunked prefill with MFMA for sliding-window layers (gfx950).  Semantics:
// FlashPrefillSlidingKernel (kernels/flash_attention_prefill.mojo:18-114) at
// degree 1 -- every query token at absolute position p walks keys
// [lo, p], lo = max(0, p - window + 1), in tiles of 16 from lo with the
// online softmax of process_kv_tile (kernels/attention_ops.mojo:165-253), and
// is finalised as acc * (1/l).
//
// The block shape, LDS staging, score MFMAs (S^T = K . Q^T on
// v_mfma_f32_32x32x16_bf16) and P.V MFMAs are those of the full-attention
// kernel (prefill.hip).  What differs is where a row's tiles start: lo moves
// by one key per query token, so the reference's tiles of the rows of a
// block are not aligned with each other.  They are aligned with the key
// space up to a per-row offset r = lo % 16: each aligned 16-key tile t (keys
// 16t .. 16t + 15) splits at r into a low part (keys < 16t + r) and a high
// part, and the row's reference tile J is the high part of aligned tile
// t - 1 followed by the low part of aligned tile t (r = 0: tile t - 1 whole).
// A row's tile J is therefore complete once aligned tile t is scored: at
// that step the row takes the tile's max over its 16 keys (its lane and lane
// ^ 32), m_new, corr = fexp(m - m_new), the 16 weights and l = l*corr + sum,
// exactly the reference's per-tile steps.  The weights of aligned tile t - 1
// are then complete (its low part belonged to tile J - 1, its high part to J)
// and its P.V MFMA runs; tile t's low-part weights wait one step.  Rows whose
// window lies before the tile, or that ended earlier, add nothing.  A row's
// last tile J_K (K = (p - lo) / 16) completes at aligned step
// lo / 16 + K + 1, which a final step past the last staged tile covers.
// Pads (keys past p in a row's last tile: with lo = 0, or when the window is
// not a multiple of 16, in its high or its low part) score -1e30 and get
// weight 0 (the reference's fexp(-87) = 1.4e-38 of a pad enters l, which
// cannot change l in f32; see fexp_fused_u).
//
// As in the full kernel the accumulator is kept as acc_stored with acc =
// acc_stored * S; a weight enters the MFMA divided by S right after its own
// tile, so later rescales need not touch the 128 accumulators (the pending
// low-part weights follow the rare S -> 1 renormalisation).  P enters as
// bf16 hi parts plus, for tiles that hold a large share of some row's l, the
// lo parts (the full kernel's gate), and the biased exp is the fused-FMA form
// (about 2e-5 relative from the reference's separately rounded steps).
//
// kBq: the butterquant variant (BqFlashPrefillSlidingKernel, butterquant_
// kernels/attention.mojo:170-264; bq_process_kv_tile :27-102).  K codes are
// staged straight into LDS (256-byte rows, the same XOR swizzle) and the
// scores come from v_mfma_i32_32x32x32_i8: sum k*q is exact, plus 128 *
// sum q it is the reference's VNNI raw dot, and each score is then formed in
// the reference's order, ((raw - qi_bias) * f_q) * k_scale / 127^2, so the
// scores equal the oracle's bit for bit.  V codes pass through registers on
// their way to LDS, converted to bf16 (exact for int8), so P.V is the bf16
// path above; a weight enters it as (w * v_scale) / 127.
#include <type_traits>

#include "common.hpp"
#include "launch.hpp"
#include "prefill_common.hpp"

namespace ifr {
namespace {

using namespace prefill;

typedef int i32x4_t __attribute__((ext_vector_type(4)));
typedef int i32x16_t __attribute__((ext_vector_type(16)));

// Bytes of one head's row of int8 codes.
constexpr int kBqRowBytes = kPD;

template <bool kBq>
__global__ __launch_bounds__(kPThreads) __attribute__((amdgpu_waves_per_eu(1, 1)))
void prefill_sliding_mfma_kernel(
    const int32_t* __restrict__ image, const void* __restrict__ qp,
    const float* __restrict__ qi_bias, const float* __restrict__ f_q,
    const void* __restrict__ kcp, const float* __restrict__ k_scale,
    const void* __restrict__ vcp, const float* __restrict__ v_scale,
    uint16_t* __restrict__ out, int num_q, int num_kv, int64_t kv_stride, int shift,
    int row_mask, int page_mask, int window) {
  __shared__ __align__(16) uint8_t kbuf0[kBq ? kKeys * kBqRowBytes : kTileBytes];
  __shared__ __align__(16) uint8_t kbuf1[kBq ? kKeys * kBqRowBytes : kTileBytes];
  __shared__ __align__(16) uint8_t vbuf0[kTileBytes];
  __shared__ __align__(16) uint8_t vbuf1[kTileBytes];
  __shared__ int32_t page_rows[kPrefillLdsPages];
  // bq: K and V scales of the staged keys, per buffer.
  __shared__ __align__(16) float kscl[2][kBq ? kKeys : 1];
  __shared__ __align__(16) float vscl[2][kBq ? kKeys : 1];
  const int tid = threadIdx.x;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int lane = tid & 63;
  const int half = lane >> 5;
  const int row = lane & 31;
  const int g = blockIdx.x % num_kv;
  const int qb = blockIdx.x / num_kv;

  const int32_t* blk = image + image[kHdrOffQBlocks] + qb * kQBlockWords;
  const int run = blk[0];
  const int t0 = blk[1];
  const int ntok = blk[2];
  const int32_t* rp = image + image[kHdrOffRuns] + run * 4;
  const int buf_start = rp[0];
  const int base_pos = rp[1];
  const int32_t* rows = image + image[kHdrOffRows] + rp[2];

  // Keys of the block: [k_lo, p_last]; iterations of 64 keys from k_lo
  // rounded down to 64.
  const int p_first = base_pos + (t0 - buf_start);
  const int p_last = p_first + ntok - 1;
  const int k_lo = max(0, p_first - window + 1);
  const int kb0 = k_lo & ~(kKeys - 1);
  const int n_iters = (p_last + 1 - kb0 + kKeys - 1) / kKeys;
  const int tile0 = kb0 >> 4;

  // This lane's row: token wave*16 + (l%32)/2, q head 2g + (l%32)%2.
  const int tok_local = wave * kPTokensPerWave + (row >> 1);
  const int head = g * 2 + (row & 1);
  const bool row_live = tok_local < ntok;
  const int tok = t0 + tok_local;
  const int p = p_first + tok_local;
  const int lo = max(0, p - window + 1);
  const int r = lo & 15;
  // Aligned tiles at which the row completes a reference tile: (t_first,
  // t_end], t_end the step of its last tile J_K, K = (p - lo) / 16.
  const int t_first = row_live ? (lo >> 4) : (1 << 30);
  const int t_end = row_live ? (lo >> 4) + ((p - lo) >> 4) + 1 : -1;

  // Q^T fragments.  bf16: lane holds Q[row][16*d + 8*half .. +7]; bq: the
  // codes Q[row][32*d + 16*half .. +15], with the row's 128 * sum q, bias
  // and f_q.
  constexpr int kQFrags = kBq ? kPD / 32 : kPD / 16;
  using QFrag = typename std::conditional<kBq, i32x4_t, bf16x8_t>::type;
  QFrag qf[kQFrags];
  int qs128 = 0;
  float qb_row = 0.0f, fq_row = 0.0f;
  const int64_t q_off = (static_cast<int64_t>(row_live ? tok : t0) * num_q + head) * kPD;
  if constexpr (kBq) {
    const int8_t* qr = static_cast<const int8_t*>(qp) + q_off + 16 * half;
    int qs = 0;
#pragma unroll
    for (int d = 0; d < kQFrags; ++d) {
      const uint4 v = *reinterpret_cast<const uint4*>(qr + 32 * d);
      qf[d] = __builtin_bit_cast(i32x4_t, v);
      qs = __builtin_amdgcn_sdot4(static_cast<int>(v.x), 0x01010101, qs, false);
      qs = __builtin_amdgcn_sdot4(static_cast<int>(v.y), 0x01010101, qs, false);
      qs = __builtin_amdgcn_sdot4(static_cast<int>(v.z), 0x01010101, qs, false);
      qs = __builtin_amdgcn_sdot4(static_cast<int>(v.w), 0x01010101, qs, false);
    }
    // The row's other 128 codes are in lane ^ 32.
    const auto sw = __builtin_amdgcn_permlane32_swap(static_cast<uint32_t>(qs),
                                                    static_cast<uint32_t>(qs), false, false);
    qs128 = 128 * (static_cast<int>(sw[0]) + static_cast<int>(sw[1]));
    const int64_t qh = static_cast<int64_t>(row_live ? tok : t0) * num_q + head;
    qb_row = qi_bias[qh];
    fq_row = f_q[qh];
  } else {
    const uint16_t* qr = static_cast<const uint16_t*>(qp) + q_off + 8 * half;
#pragma unroll
    for (int d = 0; d < kQFrags; ++d) {
      const uint4 v = *reinterpret_cast<const uint4*>(qr + 16 * d);
      qf[d] = __builtin_bit_cast(bf16x8_t, v);
    }
  }
#pragma unroll
  for (int d = 0; d < kQFrags; ++d) asm volatile("" : "+a"(qf[d]));

  f32x16_t acc[kDimBlocks];
#pragma unroll
  for (int b = 0; b < kDimBlocks; ++b)
#pragma unroll
    for (int v = 0; v < 16; ++v) acc[b][v] = 0.0f;
  float m = kNegBig, l = 0.0f, S = 1.0f;

  // The run's ring of pages (the planner validated every ordinal the keys
  // [k_lo, p_last] reach; a run may list fewer pages than the ring holds).
  const int n_pages = min(page_mask + 1, rp[3]);
  for (int i = tid; i < n_pages; i += kPThreads) page_rows[i] = rows[i];
  __syncthreads();

  // Staging of one iteration (as the full kernel's): keys clamped into
  // [k_lo, p_last]; V rows of keys outside it are zeroed after landing.
  const uint16_t* kbase = static_cast<const uint16_t*>(kcp) + static_cast<int64_t>(g) * kPD;
  const uint16_t* vbase = static_cast<const uint16_t*>(vcp) + static_cast<int64_t>(g) * kPD;
  const int8_t* kbase8 = static_cast<const int8_t*>(kcp) + static_cast<int64_t>(g) * kPD;
  const int8_t* vbase8 = static_cast<const int8_t*>(vcp) + static_cast<int64_t>(g) * kPD;
  const int stage_row0 = wave * kStageRows + half;
  auto slot_of = [&](int key) -> int64_t {
    return static_cast<int64_t>(page_rows[(key >> shift) & page_mask]) + (key & row_mask);
  };
  // bq: V codes of the wave's kStageRows rows, 4 rows per 64 lanes (lane p:
  // row p / 16, 16 codes from 16 * (p % 16)), held until converted.
  uint4 vcodes[kBq ? kStageRows / 4 : 1];
  auto stage = [&](int it, uint8_t* kdst, uint8_t* vdst, int buf) {
    if constexpr (kBq) {
#pragma unroll
      for (int i = 0; i < kStageRows / 4; ++i) {
        const int rr = wave * kStageRows + 4 * i + (lane >> 4);
        const int key = min(max(kb0 + it * kKeys + rr, k_lo), p_last);
        const int64_t off = slot_of(key) * kv_stride;
        const int c = lane & 15;
        __builtin_amdgcn_global_load_lds(
            kbase8 + off + 16 * (c ^ (rr & 15)),
            (lds_void_t*)(kdst + (wave * kStageRows + 4 * i) * kBqRowBytes), 16, 0, 0);
        vcodes[i] = *reinterpret_cast<const uint4*>(vbase8 + off + 16 * c);
      }
      if (wave == 0) {
        // The staged keys' scales, lane p: key p of the iteration.
        const int key = min(max(kb0 + it * kKeys + lane, k_lo), p_last);
        const int64_t si = slot_of(key) * num_kv + g;
        __builtin_amdgcn_global_load_lds(k_scale + si, (lds_void_t*)(&kscl[buf][0]), 4, 0, 0);
        __builtin_amdgcn_global_load_lds(v_scale + si, (lds_void_t*)(&vscl[buf][0]), 4, 0, 0);
      }
    } else {
#pragma unroll
      for (int i = 0; i < kStageRows / 2; ++i) {
        const int rr = stage_row0 + 2 * i;
        const int key = min(max(kb0 + it * kKeys + rr, k_lo), p_last);
        const int64_t off = slot_of(key) * kv_stride;
        const int lds_row = wave * kStageRows + 2 * i;
        __builtin_amdgcn_global_load_lds(kbase + off + 8 * (row ^ (rr & 15)),
                                         (lds_void_t*)(kdst + lds_row * kRowBytes), 16, 0, 0);
        __builtin_amdgcn_global_load_lds(vbase + off + 8 * (row ^ (2 * (rr & 3))),
                                         (lds_void_t*)(vdst + lds_row * kRowBytes), 16, 0, 0);
      }
    }
  };
  // The same for an iteration whose keys all lie in [k_lo, p_last] (pages
  // of >= 16 rows): iterations start at multiples of 64 keys, so a wave's
  // kStageRows rows sit in one page, reached by one lookup; the per-lane
  // byte offsets are fixed for the kernel.  bf16: row rr = 2i + half at
  // i * 4 * kv_stride + hk bytes, K chunk (row ^ half) ^ 2i, V chunk one of
  // two lane constants.  bq: row rr = 4i + lr (lr = lane / 16) at
  // i * 4 * kv_stride + lr * kv_stride bytes, K chunk (c ^ lr) ^ 4i.
  const int lr = lane >> 4;
  const int cq = lane & 15;
  const uint32_t hk = kBq ? static_cast<uint32_t>(lr * static_cast<int>(kv_stride))
                          : static_cast<uint32_t>(half * static_cast<int>(kv_stride) * 2);
  const uint32_t kx = kBq ? 16u * static_cast<uint32_t>(cq ^ lr)
                          : 16u * static_cast<uint32_t>(row ^ half);
  const uint32_t hv0 = kBq ? hk + 16u * static_cast<uint32_t>(cq)
                           : hk + 16u * static_cast<uint32_t>(row ^ (2 * half));
  const uint32_t hv1 = hk + 16u * static_cast<uint32_t>(row ^ (4 + 2 * half));
  auto stage_page = [&](int it, uint8_t* kdst, uint8_t* vdst, int buf) {
    const int key0 = kb0 + it * kKeys + wave * kStageRows;  // wave-uniform
    const int prow = __builtin_amdgcn_readfirstlane(page_rows[(key0 >> shift) & page_mask]);
    const int64_t slot0 = static_cast<int64_t>(prow) + (key0 & row_mask);
    if constexpr (kBq) {
      const char* kb = reinterpret_cast<const char*>(kbase8 + slot0 * kv_stride);
      const char* vb = reinterpret_cast<const char*>(vbase8 + slot0 * kv_stride);
      const int64_t step = 4 * kv_stride;
#pragma unroll
      for (int i = 0; i < kStageRows / 4; ++i) {
        __builtin_amdgcn_global_load_lds(
            kb + i * step + (hk + (kx ^ (64u * i))),
            (lds_void_t*)(kdst + (wave * kStageRows + 4 * i) * kBqRowBytes), 16, 0, 0);
        vcodes[i] = *reinterpret_cast<const uint4*>(vb + i * step + hv0);
      }
      if (wave == 0) {
        const int key = kb0 + it * kKeys + lane;
        const int64_t si = slot_of(key) * num_kv + g;
        __builtin_amdgcn_global_load_lds(k_scale + si, (lds_void_t*)(&kscl[buf][0]), 4, 0, 0);
        __builtin_amdgcn_global_load_lds(v_scale + si, (lds_void_t*)(&vscl[buf][0]), 4, 0, 0);
      }
    } else {
      const char* kb = reinterpret_cast<const char*>(kbase + slot0 * kv_stride);
      const char* vb = reinterpret_cast<const char*>(vbase + slot0 * kv_stride);
      const int64_t step = 4 * kv_stride;
#pragma unroll
      for (int i = 0; i < kStageRows / 2; ++i) {
        const int lds_row = wave * kStageRows + 2 * i;  // wave-uniform
        __builtin_amdgcn_global_load_lds(kb + i * step + (hk + (kx ^ (32u * i))),
                                         (lds_void_t*)(kdst + lds_row * kRowBytes), 16, 0, 0);
        __builtin_amdgcn_global_load_lds(vb + i * step + ((i & 1) ? hv1 : hv0),
                                         (lds_void_t*)(vdst + lds_row * kRowBytes), 16, 0, 0);
      }
    }
  };
  // Iteration it's keys all in [k_lo, p_last] with pages of >= 16 rows.
  auto interior = [&](int it) {
    const int first = kb0 + it * kKeys;
    return shift >= 4 && first >= k_lo && first + kKeys <= p_last + 1;  // block-uniform
  };
  // After the wave's loads have landed: bf16 keeps the staged V rows and
  // zeroes those outside [k_lo, p_last]; bq writes its V codes as bf16 (the
  // bf16 swizzle: 16-byte chunk c of row rr at c ^ 2*(rr & 3)), zeros for
  // keys outside the range.
  auto land_v = [&](int it, uint8_t* vdst) {
    const int first = kb0 + it * kKeys;
    if constexpr (kBq) {
#pragma unroll
      for (int i = 0; i < kStageRows / 4; ++i) {
        const int rr = wave * kStageRows + 4 * i + (lane >> 4);
        const int key = first + rr;
        const bool in = key >= k_lo && key <= p_last;
        const uint32_t w[4] = {vcodes[i].x, vcodes[i].y, vcodes[i].z, vcodes[i].w};
        uint32_t bf[8];
#pragma unroll
        for (int j = 0; j < 4; ++j) {
#pragma unroll
          for (int b = 0; b < 4; b += 2) {
            const float f0 = static_cast<float>(static_cast<int8_t>(w[j] >> (8 * b)));
            const float f1 = static_cast<float>(static_cast<int8_t>(w[j] >> (8 * b + 8)));
            bf[2 * j + b / 2] = in ? ((__float_as_uint(f0) >> 16) | (__float_as_uint(f1) & 0xFFFF0000u))
                                   : 0u;
          }
        }
        const int c0 = 2 * (lane & 15);
        uint8_t* vr = vdst + rr * kRowBytes;
        *reinterpret_cast<uint4*>(vr + 16 * (c0 ^ (2 * (rr & 3)))) =
            make_uint4(bf[0], bf[1], bf[2], bf[3]);
        *reinterpret_cast<uint4*>(vr + 16 * ((c0 + 1) ^ (2 * (rr & 3)))) =
            make_uint4(bf[4], bf[5], bf[6], bf[7]);
      }
    } else {
      if (first >= k_lo && first + kKeys <= p_last + 1) return;  // block-uniform
#pragma unroll
      for (int i = 0; i < kStageRows / 2; ++i) {
        const int rr = stage_row0 + 2 * i;
        const int key = first + rr;
        if (key < k_lo || key > p_last)
          *reinterpret_cast<uint4*>(vdst + rr * kRowBytes + 16 * row) =
              make_uint4(0u, 0u, 0u, 0u);
      }
    }
  };

  if (n_iters > 0) stage(0, kbuf0, vbuf0, 0);
  __builtin_amdgcn_s_waitcnt(0);
  if (n_iters > 0) land_v(0, vbuf0);
  __syncthreads();

  const int k_lane = row * kRowBytes + 16 * ((row & 15) ^ half);
  const int vj = lane & 15;
  const int v_row = (4 * half + (vj >> 2)) * kRowBytes +
                    32 * (((lane >> 4) & 1) ^ ((vj >> 2) & 1)) + 8 * (vj & 3);
  int v_even = v_row + 64 * (vj >> 3);
  int v_odd1 = v_row - 64 * (vj >> 3) + 64;  // odd block b at v_odd1 + 64 * (b - 1)
  // Opaque to the compiler: from the known low bits of these offsets it
  // would combine them with the buffer address by OR, one VALU instruction
  // per read, instead of a base register and immediate offsets.
  asm("" : "+v"(v_even), "+v"(v_odd1));

  // bq K operand reads: chunk 2d + half of key row (row & 31) of 256 bytes,
  // stored at (2d + half) ^ (row & 15): byte address kq_lane ^ 32d.
  const int kq_lane = row * kBqRowBytes + 16 * ((row & 15) ^ half);
  constexpr float kInv127 = 1.0f / 127.0f;
  constexpr float kInv127Sq = kInv127 * kInv127;

  constexpr int kKAhead = 6;
  // Scores of 32-key block h of the staged iteration (buffer buf).
  auto qk = [&](const uint8_t* kl, int h, int buf) {
    if constexpr (kBq) {
      i32x16_t si;
#pragma unroll
      for (int v = 0; v < 16; ++v) si[v] = qs128;  // the raw dot's 128 * sum q, exact in int32
      const uint8_t* kh = kl + 32 * h * kBqRowBytes;
      uint4 kf[kQFrags];
#pragma unroll
      for (int d = 0; d < kQFrags; ++d)
        kf[d] = *reinterpret_cast<const uint4*>(kh + (kq_lane ^ (32 * d)));
#pragma unroll
      for (int d = 0; d < kQFrags; ++d)
        si = __builtin_amdgcn_mfma_i32_32x32x32_i8(__builtin_bit_cast(i32x4_t, kf[d]), qf[d],
                                                   si, 0, 0, 0);
      // ((raw - qi_bias) * f_q) * k_scale / 127^2 per (row, key); value
      // 4j + i holds key 8j + 4*half + i of the block.
      f32x16_t sblk;
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        const float4 ks4 =
            *reinterpret_cast<const float4*>(&kscl[buf][32 * h + 8 * j + 4 * half]);
        const float ks[4] = {ks4.x, ks4.y, ks4.z, ks4.w};
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          float sc = static_cast<float>(si[4 * j + i]) - qb_row;
          sc = sc * fq_row;
          sc = sc * ks[i];
          sblk[4 * j + i] = sc * kInv127Sq;
        }
      }
      return sblk;
    } else {
    f32x16_t sblk;
#pragma unroll
    for (int v = 0; v < 16; ++v) sblk[v] = 0.0f;
    const uint8_t* kh = kl + 32 * h * kRowBytes;
    uint4 kf[kPD / 16];
#pragma unroll
    for (int d = 0; d < kKAhead; ++d)
      kf[d] = *reinterpret_cast<const uint4*>(kh + (k_lane ^ (32 * d)));
#pragma unroll
    for (int d = 0; d < kPD / 16; ++d) {
      if (d + kKAhead < kPD / 16)
        kf[d + kKAhead] = *reinterpret_cast<const uint4*>(kh + (k_lane ^ (32 * (d + kKAhead))));
      sblk = __builtin_amdgcn_mfma_f32_32x32x16_bf16(__builtin_bit_cast(bf16x8_t, kf[d]), qf[d],
                                                     sblk, 0, 0, 0);
    }
    __builtin_amdgcn_sched_group_barrier(0x100, kKAhead, 0);
#pragma unroll
    for (int d = 0; d < kPD / 16 - kKAhead; ++d) {
      __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
      __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);
    }
    __builtin_amdgcn_sched_group_barrier(0x008, kKAhead, 0);
    return sblk;
    }
  };

  // acc_stored += V^T P^T for the 16-key tile at rows tile_row .. +15 of vl:
  // P as bf16 hi parts, and the lo parts p - bf16(p) in a second pass when
  // some row of the wave draws more than kLoShare of its running l from a
  // reference tile with weights in this tile (the full kernel's gate: the
  // lo parts of a smaller share move that row's output by at most
  // 2^-9 * kLoShare * max|v|).
  auto pv = [&](const uint8_t* vl, int tile_row, const float (&pw0)[8], bool need_lo,
                int buf) {
    float pw[8];
#pragma unroll
    for (int i = 0; i < 8; ++i) pw[i] = pw0[i];
    if constexpr (kBq) {
      // Lane value i is key tile_row + 8*(i/4) + 4*half + i%4.
#pragma unroll
      for (int j = 0; j < 2; ++j) {
        const float4 vs4 =
            *reinterpret_cast<const float4*>(&vscl[buf][tile_row + 8 * j + 4 * half]);
        pw[4 * j] = (pw[4 * j] * vs4.x) * kInv127;
        pw[4 * j + 1] = (pw[4 * j + 1] * vs4.y) * kInv127;
        pw[4 * j + 2] = (pw[4 * j + 2] * vs4.z) * kInv127;
        pw[4 * j + 3] = (pw[4 * j + 3] * vs4.w) * kInv127;
      }
    }
    bf16x8_t phi;
#pragma unroll
    for (int i = 0; i < 8; i += 2) {
      const bf16x2_t hb = __builtin_convertvector(f32x2_t{pw[i], pw[i + 1]}, bf16x2_t);
      phi[i] = hb[0];
      phi[i + 1] = hb[1];
    }
    const uint8_t* vt = vl + tile_row * kRowBytes;
    bf16x8_t av[kDimBlocks];
#pragma unroll
    for (int b = 0; b < kDimBlocks; ++b) {
      const uint8_t* vb = (b & 1) ? vt + v_odd1 + 64 * (b - 1) : vt + v_even + 64 * b;
      const s16x4_t v0 = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_s16x4_t*)vb);
      const s16x4_t v1 =
          __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_s16x4_t*)(vb + 8 * kRowBytes));
      av[b] = __builtin_bit_cast(bf16x8_t, __builtin_shufflevector(v0, v1, 0, 1, 2, 3, 4, 5, 6, 7));
      acc[b] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(av[b], phi, acc[b], 0, 0, 0);
    }
    if (__builtin_amdgcn_ballot_w64(need_lo) != 0) {  // wave-uniform
      bf16x8_t plo;
#pragma unroll
      for (int i = 0; i < 8; ++i) plo[i] = static_cast<__bf16>(pw[i] - static_cast<float>(phi[i]));
#pragma unroll
      for (int b = 0; b < kDimBlocks; ++b)
        acc[b] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(av[b], plo, acc[b], 0, 0, 0);
    }
  };

  // Per-step state: the previous aligned tile's scores and the pending
  // (low-part) weights of the current one.
  float s_prev[8], pend[8];
  bool pend_big = false;  // the pending weights' reference tile exceeded kLoShare
#pragma unroll
  for (int i = 0; i < 8; ++i) {
    s_prev[i] = kNegBig;
    pend[i] = 0.0f;
  }
  // Key offset inside an aligned tile of the lane's value i (32x32 C layout).
  auto key_of = [&](int i) { return 8 * (i >> 2) + 4 * half + (i & 3); };

  // Step of aligned tile t with scores st: completes the row's reference
  // tile (high part of t - 1, low part of t) when t_first < t <= t_end, then
  // P.V of tile t - 1 (vprev, rows prev_row ..) unless do_pv is false.
  // kInner: every row of the wave completes a reference tile at t and none
  // of its keys lies past the row's position (no fin or pad tests).
  auto step_impl = [&](auto inner_c, int t, const float (&st)[8], const uint8_t* vprev,
                       int prev_row, bool do_pv, int prev_buf) {
    constexpr bool kInner = decltype(inner_c)::value;
    const bool fin = kInner || (t > t_first && t <= t_end);
    float sel[8];
    bool low[8];
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      const int kk = key_of(i);
      low[i] = kk < r;
      const bool pad = !kInner && (low[i] ? 16 * t : 16 * (t - 1)) + kk > p;
      sel[i] = (fin && !pad) ? (low[i] ? st[i] : s_prev[i]) : kNegBig;
    }
    float mx = max8(sel);
    mx = max_xor32(mx);
    const float m_new = fmaxf(mx, m);
    const float c = fexp_fused_u(__builtin_fmaf(kExpA, m - m_new, kExpBias));
    const float te = __builtin_fmaf(-kExpA, m_new, kExpBias);
    float e[8];
#pragma unroll
    for (int i = 0; i < 8; ++i) e[i] = fexp_fused_u(__builtin_fmaf(kExpA, sel[i], te));
    float ts = ((e[0] + e[1]) + (e[2] + e[3])) + ((e[4] + e[5]) + (e[6] + e[7]));
    ts = sum_xor32(ts);
    const float corr = fin ? c : 1.0f;
    if (fin) {
      l = l * c + ts;
      m = m_new;
    }
    const bool big = fin && ts > kLoShare * l;
    float S_new = S * corr;
    if (__builtin_amdgcn_ballot_w64(S_new < 0x1p-64f) != 0) {  // wave-uniform
#pragma unroll
      for (int b = 0; b < kDimBlocks; ++b) {
        f32x16_t tv = acc[b];
        asm volatile("" : "+v"(tv));
        acc[b] = tv * S_new;
        asm volatile("" : "+a"(acc[b]));
        __builtin_amdgcn_sched_barrier(0);
      }
#pragma unroll
      for (int i = 0; i < 8; ++i) pend[i] = pend[i] * S_new;
      S_new = 1.0f;
    }
    S = S_new;
    const float inv_s = __builtin_amdgcn_rcpf(S_new);
    float pw[8];
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      const int kk = key_of(i);
      const bool pad = !kInner && (low[i] ? 16 * t : 16 * (t - 1)) + kk > p;
      const float w = (fin && !pad) ? e[i] * inv_s : 0.0f;
      pw[i] = low[i] ? pend[i] : w;
      pend[i] = low[i] ? w : 0.0f;
      s_prev[i] = st[i];
    }
    const bool need_lo = pend_big || big;
    pend_big = big && r != 0;
    if (do_pv) pv(vprev, prev_row, pw, need_lo, prev_buf);
  };
  // The steps at which every row of the wave is inside: t_first < t <=
  // t_end, and the row's last key at step t (16t + r - 1 for its low part,
  // 16t - 1 for its high part) at most p.  Wave-uniform bounds [in_lo,
  // in_hi] (a wave with rows past the block's last token has none).
  int in_lo = t_first + 1;
  int in_hi = min(t_end, r > 0 ? (p - r + 1) >> 4 : (p + 1) >> 4);
  if (!row_live) in_hi = -1;
#pragma unroll
  for (int o = 1; o < 64; o <<= 1) {
    in_lo = max(in_lo, __shfl_xor(in_lo, o));
    in_hi = min(in_hi, __shfl_xor(in_hi, o));
  }
  in_lo = __builtin_amdgcn_readfirstlane(in_lo);
  in_hi = __builtin_amdgcn_readfirstlane(in_hi);
  const std::true_type inner_yes{};
  const std::false_type inner_no{};
  // One iteration: the scores of its two 32-key blocks and its four steps,
  // all of them kInner or none.
  auto iteration = [&](auto inner_c, int it) {
    uint8_t* kl = (it & 1) ? kbuf1 : kbuf0;
    uint8_t* vl = (it & 1) ? vbuf1 : vbuf0;
    uint8_t* kn = (it & 1) ? kbuf0 : kbuf1;
    uint8_t* vn = (it & 1) ? vbuf0 : vbuf1;
    const int cb = it & 1, nb = cb ^ 1;
    const int tb = tile0 + 4 * it;
    float st[8];
    const f32x16_t s0 = qk(kl, 0, cb);
#pragma unroll
    for (int i = 0; i < 8; ++i) st[i] = s0[i];
    // Tile tb - 1 lies in the other buffer (the previous iteration's last
    // tile); it is read before that buffer is restaged.
    step_impl(inner_c, tb, st, vn, 48, it > 0, nb);
    __syncthreads();
    if (it + 1 < n_iters) {
      if (interior(it + 1))
        stage_page(it + 1, kn, vn, nb);
      else
        stage(it + 1, kn, vn, nb);
    }
#pragma unroll
    for (int i = 0; i < 8; ++i) st[i] = s0[8 + i];
    step_impl(inner_c, tb + 1, st, vl, 0, true, cb);
    const f32x16_t s1 = qk(kl, 1, cb);
#pragma unroll
    for (int i = 0; i < 8; ++i) st[i] = s1[i];
    step_impl(inner_c, tb + 2, st, vl, 16, true, cb);
#pragma unroll
    for (int i = 0; i < 8; ++i) st[i] = s1[8 + i];
    step_impl(inner_c, tb + 3, st, vl, 32, true, cb);
#pragma unroll
    for (int b = 0; b < kDimBlocks; ++b) asm volatile("" : "+a"(acc[b]));
#pragma unroll
    for (int d = 0; d < kQFrags; ++d) asm volatile("" : "+a"(qf[d]));
    __builtin_amdgcn_s_waitcnt(0);
    if (it + 1 < n_iters) land_v(it + 1, vn);
    __syncthreads();
  };
  // Iterations whose four steps tile0 + 4it .. +3 all lie in [in_lo, in_hi]
  // run the kInner form, in a loop of their own (one form per loop keeps
  // the register allocation of each loop to one iteration body).
  const int it_in0 = min(n_iters, max(0, (in_lo - tile0 + 3) >> 2));
  const int it_in1 = max(it_in0, min(n_iters, (in_hi - 3 - tile0 >= 0) ? ((in_hi - 3 - tile0) >> 2) + 1 : 0));
  int it = 0;
  for (; it < it_in0; ++it) iteration(inner_no, it);
  for (; it < it_in1; ++it) iteration(inner_yes, it);
  for (; it < n_iters; ++it) iteration(inner_no, it);
  // The step past the last staged tile: completes the last reference tile of
  // rows with r = 0 and runs the last tile's P.V.
  if (n_iters > 0) {
    float st[8];
#pragma unroll
    for (int i = 0; i < 8; ++i) st[i] = kNegBig;
    const int lb = (n_iters - 1) & 1;
    step_impl(inner_no, tile0 + 4 * n_iters, st, lb ? vbuf1 : vbuf0, 48, true, lb);
  }

  // Finalisation of the sliding prefill: acc * (1/l).
  if (row_live) {
    const bool live = l > 0.0f;
    const float inv_l = live ? 1.0f / l : 0.0f;
    uint16_t* dst = out + (static_cast<int64_t>(tok) * num_q + head) * kPD + 4 * half;
#pragma unroll
    for (int b = 0; b < kDimBlocks; ++b) {
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        uint32_t e[4];
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          const float av = acc[b][4 * j + i] * S;
          e[i] = live ? f32_to_bf16_bits(av * inv_l) : 0u;
        }
        *reinterpret_cast<uint2*>(dst + 32 * b + 8 * j) =
            make_uint2(e[0] | (e[1] << 16), e[2] | (e[3] << 16));
      }
    }
  }
}

}  // namespace

hipError_t launch_prefill_sliding_mfma(const int32_t* image, int num_qblocks, const void* q,
                                       const void* k, const void* v, void* output, int num_q,
                                       int num_kv, int64_t kv_stride, PagedGeom geom,
                                       int window, hipStream_t stream) {
  if (num_qblocks <= 0) return hipSuccess;
  hipLaunchKernelGGL(prefill_sliding_mfma_kernel<false>, dim3(num_qblocks * num_kv),
                     dim3(kPThreads), 0, stream, image, q, nullptr, nullptr, k, nullptr, v,
                     nullptr, static_cast<uint16_t*>(output), num_q, num_kv, kv_stride,
                     geom.shift, geom.row_mask, geom.page_mask, window);
  return hipGetLastError();
}

hipError_t launch_prefill_sliding_mfma_bq(const int32_t* image, int num_qblocks,
                                          const void* q_i8, const float* qi_bias,
                                          const float* f_q, const void* k,
                                          const float* k_scale, const void* v,
                                          const float* v_scale, void* output, int num_q,
                                          int num_kv, int64_t kv_stride, PagedGeom geom,
                                          int window, hipStream_t stream) {
  if (num_qblocks <= 0) return hipSuccess;
  hipLaunchKernelGGL(prefill_sliding_mfma_kernel<true>, dim3(num_qblocks * num_kv),
                     dim3(kPThreads), 0, stream, image, q_i8, qi_bias, f_q, k, k_scale, v,
                     v_scale, static_cast<uint16_t*>(output), num_q, num_kv, kv_stride,
                     geom.shift, geom.row_mask, geom.page_mask, window);
  return hipGetLastError();
}

}  // namespace ifr
