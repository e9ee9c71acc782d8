// Chunked causal prefill with MFMA for Gemma-4's full-attention layers:
// head_dim 512 with 8 q heads per kv head (16 q / 2 kv heads,
// modeling/gemma4_common.mojo:14-20, prefilled through dispatch_full_attention
// at modeling/gemma_4_moe.mojo:415-479).  Semantics: FlashPrefillFullKernel +
// PrefillMergeKernel (kernels/flash_attention_prefill.mojo:117-248) at
// degree 1, as in prefill_full_mfma_kernel -- every query token at position
// p walks keys [0, p] in tiles of 16 from key 0 with the online softmax of
// process_kv_tile (kernels/attention_ops.mojo:165-253), then its one-segment
// merge (kernels/logsum_merge.mojo:28-122).
//
// A row is one (query token, q head).  A wave owns 32 rows = 4 tokens x the
// 8 q heads of one kv head, with all 512 dims: the O^T accumulator of all
// 512 output dims fills the 256 AGPRs, and the Q^T fragments of the rows
// (128 VGPRs; 64 for bq codes) leave the other 128 VGPRs to the scores, the
// softmax and the operand reads (one group of V^T reads and two K reads in
// flight; the staging addresses are a scalar base plus a 32-bit lane
// offset).  Each wave therefore computes its rows' whole scores itself,
// S^T = K . Q^T (32 x v_mfma_f32_32x32x16_bf16 per 32 keys), runs their
// softmax once, and accumulates O^T += V^T . P'^T over its 16 dim blocks.  A block of 4 waves (one per SIMD, one block per CU)
// owns 16 tokens = 128 rows sharing each staged K/V tile; a plan query block
// of 64 tokens is 4 such blocks.  Every K and V fragment read from LDS feeds
// 32 rows.
//
// The C layout, the per-tile softmax (softmax_tile), the folded rescales
// with the per-row scale S, the hi + lo bf16 parts of P under the kLoShare
// gate, the fused-FMA biased exp, the swizzled K/V rows staged straight
// into LDS (32 keys of 1 KiB rows, double-buffered) and the transposing
// V^T reads are those of prefill_full_mfma_kernel (prefill.hip).
//
// The run's page table is held in LDS as a window of kWLdsPages entries,
// moved forward at an iteration boundary when the next staged keys pass its
// end, so a run of any length stays on this kernel.
//
// kBq: the butterquant variant (BqFlashPrefillFullKernel, butterquant_
// kernels/attention.mojo:267-351, at Gemma-4's bq full layer, modeling/
// gemma_4_moe_bq.mojo:527-553).  K codes (512-byte rows) are staged straight
// into LDS; the score's integer part is sum k*q over the 512 dims from
// v_mfma_i32_32x32x32_i8 plus 128 * sum q, the reference's VNNI raw dot
// (it reads k ^ 0x80 as unsigned), and the score is formed in the
// reference's order, ((raw - qi_bias) * f_q) * k_scale / 127^2.  V codes
// pass through registers to LDS as bf16 (exact for int8) and the V scale
// enters the weight as (w * v_scale) / 127.
//
// Blocks run in an XCD-aware order.  Workgroups go to the 8 XCDs round
// robin (block b to XCD b % 8, in order of b on each), and the plan lists
// its query blocks run-major, longest first.  When num_kv divides 8, XCD x
// serves kv head x % num_kv and the query blocks x / num_kv, x / num_kv +
// 8 / num_kv, ...: every XCD gets an even share of every run (a run-per-XCD
// split left the XCD holding the longest run working long after the
// others), each key tile is fetched by 8 / num_kv XCDs rather than all 8,
// and the blocks running together on one XCD belong to one run and kv head
// and walk its keys in step through that XCD's L2.  Otherwise XCD x takes
// query blocks x, x + 8, ... with all their kv heads.
#include <type_traits>

#include "common.hpp"
#include "launch.hpp"
#include "prefill_common.hpp"

namespace ifr {
namespace {

using namespace prefill;

constexpr int kWD = 512;                   // head_dim
constexpr int kWG = 8;                     // q heads per kv head
constexpr int kWTokensPerWave = 32 / kWG;  // 4 tokens x 8 heads = 32 rows
constexpr int kWTokens = kPWaves * kWTokensPerWave;  // 16 tokens per block
constexpr int kWSub = kPrefillTokens / kWTokens;     // blocks per plan query block
constexpr int kWKeys = 32;                 // keys per iteration (one S block, two tiles)
constexpr int kWRowBytes = kWD * 2;        // one key row of K or V in LDS
constexpr int kWTileBytes = kWKeys * kWRowBytes;  // 32 KiB
constexpr int kWDimBlocks = kWD / 32;      // 32-dim blocks of O^T
constexpr int kWStageRows = kWKeys / kPWaves;  // key rows each wave stages
constexpr int kWLdsPages = 2048;           // page-table window held in LDS
constexpr int kXcds = 8;
static_assert(kPrefillTokens % kWTokens == 0, "plan query blocks split into kernel blocks");
static_assert(4 * kWTileBytes + 4 * kWLdsPages <= 160 * 1024, "LDS budget");

typedef int wi32x4_t __attribute__((ext_vector_type(4)));
typedef int wi32x16_t __attribute__((ext_vector_type(16)));
constexpr int kWBqRowBytes = kWD;  // one kv head's row of int8 codes

template <bool kBq>
__global__ __launch_bounds__(kPThreads) __attribute__((amdgpu_waves_per_eu(1, 1)))
void prefill_wide_mfma_kernel(
    const int32_t* __restrict__ image, const void* __restrict__ qp,
    const float* __restrict__ qi_bias, const float* __restrict__ f_q,
    const void* __restrict__ kcp, const float* __restrict__ k_scale,
    const void* __restrict__ vcp, const float* __restrict__ v_scale,
    uint16_t* __restrict__ out, int num_q, int num_kv, int64_t kv_stride, int shift,
    int row_mask, int num_qblocks) {
  __shared__ __align__(16) uint8_t kbuf0[kBq ? kWKeys * kWBqRowBytes : kWTileBytes];
  __shared__ __align__(16) uint8_t kbuf1[kBq ? kWKeys * kWBqRowBytes : kWTileBytes];
  __shared__ __align__(16) uint8_t vbuf0[kWTileBytes];
  __shared__ __align__(16) uint8_t vbuf1[kWTileBytes];
  __shared__ int32_t page_rows[kWLdsPages];
  // bq: the staged keys' K scales (0 .. 31) and V scales (32 .. 63), per buffer.
  __shared__ __align__(16) float scl[2][kBq ? 2 * kWKeys : 1];
  const int x = blockIdx.x % kXcds;
  const int slot = blockIdx.x / kXcds;
  int qb, g, sub;
  if (kXcds % num_kv == 0) {
    // XCD x serves kv head x % num_kv and every (8 / num_kv)-th query block.
    const int lanes = kXcds / num_kv;
    qb = (slot / kWSub) * lanes + x / num_kv;
    g = x % num_kv;
    sub = slot % kWSub;
  } else {
    const int items_per_qb = num_kv * kWSub;
    qb = (slot / items_per_qb) * kXcds + x;
    g = (slot % items_per_qb) % num_kv;
    sub = (slot % items_per_qb) / num_kv;
  }
  if (qb >= num_qblocks) return;  // block-uniform, before any barrier
  const int tid = threadIdx.x;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int lane = tid & 63;
  const int half = lane >> 5;
  const int row = lane & 31;

  const int32_t* blk = image + image[kHdrOffQBlocks] + qb * kQBlockWords;
  const int run = blk[0];
  const int t0 = blk[1] + sub * kWTokens;
  const int ntok = min(kWTokens, blk[2] - sub * kWTokens);
  if (ntok <= 0) return;  // block-uniform
  const int32_t* rp = image + image[kHdrOffRuns] + run * 4;
  const int buf_start = rp[0];
  const int base_pos = rp[1];
  const int32_t* rows = image + image[kHdrOffRows] + rp[2];

  // Keys the block needs: [0, count_max).
  const int count_max = base_pos + (t0 + ntok - 1 - buf_start) + 1;
  const int n_iters = (count_max + kWKeys - 1) / kWKeys;
  const int n_pages = count_max > 0 ? ((count_max - 1) >> shift) + 1 : 0;

  // This lane's row: token 4*wave + (l%32)/8, q head 8g + (l%32)%8.
  const int tok_local = wave * kWTokensPerWave + (row >> 3);
  const int head = g * kWG + (row & 7);
  const bool row_live = tok_local < ntok;
  const int tok = t0 + tok_local;
  const int count = row_live ? base_pos + (tok - buf_start) + 1 : 0;
  const int wave_first = wave * kWTokensPerWave;
  const int wave_last = min(ntok, wave_first + kWTokensPerWave) - 1;
  const int wave_count = wave_first < ntok ? base_pos + (t0 + wave_last - buf_start) + 1 : 0;
  // Keys below wave_min are valid for every row of the wave.
  const int wave_min = wave_first + kWTokensPerWave <= ntok
                           ? base_pos + (t0 + wave_first - buf_start) + 1
                           : 0;

  // Q^T fragments: lane holds Q[row][16*d + 8*half .. +7] for the 32 16-dim
  // steps d.  bq: the codes Q[row][32*d + 16*half .. +15] for the 16 32-dim
  // steps, 128 * the sum of the row's 512 codes, and its bias and f_q.
  constexpr int kQFrags = kBq ? kWD / 32 : kWD / 16;
  using QFrag = typename std::conditional<kBq, wi32x4_t, bf16x8_t>::type;
  QFrag qf[kQFrags];
  int qs128 = 0;
  float qb_row = 0.0f, fq_row = 0.0f;
  const int64_t q_row = static_cast<int64_t>(row_live ? tok : t0) * num_q + head;
  if constexpr (kBq) {
    const int8_t* qr = static_cast<const int8_t*>(qp) + q_row * kWD + 16 * half;
    int qs = 0;
#pragma unroll
    for (int d = 0; d < kQFrags; ++d) {
      const uint4 v = *reinterpret_cast<const uint4*>(qr + 32 * d);
      qf[d] = __builtin_bit_cast(wi32x4_t, v);
      qs = __builtin_amdgcn_sdot4(static_cast<int>(v.x), 0x01010101, qs, false);
      qs = __builtin_amdgcn_sdot4(static_cast<int>(v.y), 0x01010101, qs, false);
      qs = __builtin_amdgcn_sdot4(static_cast<int>(v.z), 0x01010101, qs, false);
      qs = __builtin_amdgcn_sdot4(static_cast<int>(v.w), 0x01010101, qs, false);
    }
    const auto sw = __builtin_amdgcn_permlane32_swap(static_cast<uint32_t>(qs),
                                                    static_cast<uint32_t>(qs), false, false);
    qs128 = 128 * (static_cast<int>(sw[0]) + static_cast<int>(sw[1]));
    qb_row = qi_bias[q_row];
    fq_row = f_q[q_row];
  } else {
    const uint16_t* qr = static_cast<const uint16_t*>(qp) + q_row * kWD + 8 * half;
#pragma unroll
    for (int d = 0; d < kQFrags; ++d) {
      const uint4 v = *reinterpret_cast<const uint4*>(qr + 16 * d);
      qf[d] = __builtin_bit_cast(bf16x8_t, v);
    }
  }
  // The fragments stay in VGPRs: the accumulators fill the 256 AGPRs.

  // acc = acc_stored * S (prefill_full_mfma_kernel's scheme).
  f32x16_t acc[kWDimBlocks];
#pragma unroll
  for (int b = 0; b < kWDimBlocks; ++b)
#pragma unroll
    for (int v = 0; v < 16; ++v) acc[b][v] = 0.0f;
  float m = kNegBig, l = 0.0f, S = 1.0f;

  // Page-table window: LDS entry i holds the run's page wbase + i.
  int wbase = 0;
  auto load_window = [&](int first) {
    const int n = min(kWLdsPages, n_pages - first);
    for (int i = tid; i < n; i += kPThreads) page_rows[i] = rows[first + i];
  };
  load_window(0);
  __syncthreads();

  // Staging: wave w moves key rows kWStageRows*w .. +7 of K and of V.  bf16:
  // one 1 KiB row per load (lane p: 16 bytes); lane p writes LDS chunk p, for
  // K holding global chunk p ^ (key & 15), for V chunk p ^ 2*(key & 3).  Keys
  // past count_max read the last key (in bounds); their V rows are zeroed
  // once the loads have landed.  bq: K rows of 512 bytes, two per load (lane
  // p: row p / 32, LDS chunk p % 32 holding global chunk (p % 32) ^ (key &
  // 15)); V codes to registers (lane p: row 2i + p / 32, 16 codes from
  // 16 * (p % 32)), written to LDS as bf16 rows once landed; wave 0 moves the
  // 32 keys' K scales (lanes 0-31) and V scales (lanes 32-63).
  const uint16_t* kbase = static_cast<const uint16_t*>(kcp) + static_cast<int64_t>(g) * kWD;
  const uint16_t* vbase = static_cast<const uint16_t*>(vcp) + static_cast<int64_t>(g) * kWD;
  const int8_t* kbase8 = static_cast<const int8_t*>(kcp) + static_cast<int64_t>(g) * kWD;
  const int8_t* vbase8 = static_cast<const int8_t*>(vcp) + static_cast<int64_t>(g) * kWD;
  uint4 vcodes[kBq ? kWStageRows / 2 : 1];
  auto page_of = [&](int key) { return page_rows[(key >> shift) - wbase]; };
  auto stage = [&](int it, uint8_t* kdst, uint8_t* vdst, int buf) {
    if constexpr (kBq) {
#pragma unroll
      for (int i = 0; i < kWStageRows / 2; ++i) {
        const int r = wave * kWStageRows + 2 * i + (lane >> 5);
        const int key = min(it * kWKeys + r, count_max - 1);
        const int64_t off = (static_cast<int64_t>(page_of(key)) + (key & row_mask)) * kv_stride;
        const int c = lane & 31;
        __builtin_amdgcn_global_load_lds(
            kbase8 + off + 16 * (c ^ (r & 15)),
            (lds_void_t*)(kdst + (wave * kWStageRows + 2 * i) * kWBqRowBytes), 16, 0, 0);
        vcodes[i] = *reinterpret_cast<const uint4*>(vbase8 + off + 16 * c);
      }
      if (wave == 0) {
        const int key = min(it * kWKeys + (lane & 31), count_max - 1);
        const int64_t si = (static_cast<int64_t>(page_of(key)) + (key & row_mask)) * num_kv + g;
        __builtin_amdgcn_global_load_lds((lane < 32 ? k_scale : v_scale) + si,
                                         (lds_void_t*)(&scl[buf][0]), 4, 0, 0);
      }
    } else {
#pragma unroll
      for (int i = 0; i < kWStageRows; ++i) {
        const int r = wave * kWStageRows + i;  // wave-uniform key row of the iteration
        const int key = min(it * kWKeys + r, count_max - 1);
        const int prow = __builtin_amdgcn_readfirstlane(page_of(key));
        const int64_t off = (static_cast<int64_t>(prow) + (key & row_mask)) * kv_stride;
        const uint8_t* krow = reinterpret_cast<const uint8_t*>(kbase + off);  // uniform
        const uint8_t* vrow = reinterpret_cast<const uint8_t*>(vbase + off);
        uint32_t lk = static_cast<uint32_t>(16 * lane) ^ static_cast<uint32_t>(16 * (r & 15));
        uint32_t lv = static_cast<uint32_t>(16 * lane) ^ static_cast<uint32_t>(32 * (r & 3));
        // Opaque lane offsets: the address stays a uniform base plus a 32-bit
        // lane offset (the load's scalar-base form) rather than 64-bit lane
        // addresses hoisted out of the loop.
        asm volatile("" : "+v"(lk), "+v"(lv));
        __builtin_amdgcn_global_load_lds(krow + lk, (lds_void_t*)(kdst + r * kWRowBytes), 16,
                                         0, 0);
        __builtin_amdgcn_global_load_lds(vrow + lv, (lds_void_t*)(vdst + r * kWRowBytes), 16,
                                         0, 0);
      }
    }
  };
  // After the wave's loads have landed: bf16 zeroes the V rows of keys past
  // count_max; bq writes its V codes as bf16 rows (zeros past count_max).
  auto land_v = [&](int it, uint8_t* vdst) {
    if constexpr (kBq) {
#pragma unroll
      for (int i = 0; i < kWStageRows / 2; ++i) {
        const int r = wave * kWStageRows + 2 * i + (lane >> 5);
        const bool in = it * kWKeys + r < count_max;
        const uint32_t w[4] = {vcodes[i].x, vcodes[i].y, vcodes[i].z, vcodes[i].w};
        uint32_t bf[8];
#pragma unroll
        for (int j = 0; j < 4; ++j) {
#pragma unroll
          for (int b = 0; b < 4; b += 2) {
            const float f0 = static_cast<float>(static_cast<int8_t>(w[j] >> (8 * b)));
            const float f1 = static_cast<float>(static_cast<int8_t>(w[j] >> (8 * b + 8)));
            bf[2 * j + b / 2] =
                in ? ((__float_as_uint(f0) >> 16) | (__float_as_uint(f1) & 0xFFFF0000u)) : 0u;
          }
        }
        const int c0 = 2 * (lane & 31);
        uint8_t* vr = vdst + r * kWRowBytes;
        *reinterpret_cast<uint4*>(vr + 16 * (c0 ^ (2 * (r & 3)))) =
            make_uint4(bf[0], bf[1], bf[2], bf[3]);
        *reinterpret_cast<uint4*>(vr + 16 * ((c0 + 1) ^ (2 * (r & 3)))) =
            make_uint4(bf[4], bf[5], bf[6], bf[7]);
      }
    } else {
      if ((it + 1) * kWKeys <= count_max) return;  // block-uniform
#pragma unroll
      for (int i = 0; i < kWStageRows; ++i) {
        const int r = wave * kWStageRows + i;
        if (it * kWKeys + r >= count_max)
          *reinterpret_cast<uint4*>(vdst + r * kWRowBytes + 16 * lane) =
              make_uint4(0u, 0u, 0u, 0u);
      }
    }
  };

  if (n_iters > 0) stage(0, kbuf0, vbuf0, 0);
  __builtin_amdgcn_s_waitcnt(0);
  if (n_iters > 0) land_v(0, vbuf0);
  __syncthreads();

  // QK operand reads: chunk 2d + half of key row (row & 31), stored at chunk
  // (2d + half) ^ (row & 15): byte address k_lane ^ 32d.
  const int k_lane = row * kWRowBytes + 16 * ((row & 15) ^ half);
  // Transposing V^T reads, as in prefill_full_mfma_kernel at 1 KiB rows.
  const int vj = lane & 15;
  const int v_row = (4 * half + (vj >> 2)) * kWRowBytes +
                    32 * (((lane >> 4) & 1) ^ ((vj >> 2) & 1)) + 8 * (vj & 3);
  int v_even = v_row + 64 * (vj >> 3);
  int v_odd1 = v_row - 64 * (vj >> 3) + 64;  // odd block b at v_odd1 + 64 * (b - 1)
  // Opaque to the compiler: from the known low bits of these offsets it
  // would combine them with the buffer address by OR, one VALU instruction
  // per read, instead of a base register and immediate offsets.
  asm("" : "+v"(v_even), "+v"(v_odd1));
  // bq K operand reads: chunk 2d + half of key row (row & 31) of 512 bytes,
  // stored at (2d + half) ^ (row & 15): kq_lane ^ 32d.
  const int kq_lane = row * kWBqRowBytes + 16 * ((row & 15) ^ half);
  constexpr float kInv127 = 1.0f / 127.0f;
  constexpr float kInv127Sq = kInv127 * kInv127;

  // K operand reads in flight ahead of their MFMAs (measured best: 6 for
  // bf16, 4 for the int8 codes).
  constexpr int kKAhead = kBq ? 4 : 6;
  // The rows' scores over the 32 staged keys (value 4j + i holds key
  // 8j + 4*half + i of the block).  bq: ((raw - qi_bias) * f_q) * k_scale /
  // 127^2 with raw the integer dot plus 128 * sum q.
  auto qk = [&](const uint8_t* kl, int buf) -> f32x16_t {
    if constexpr (kBq) {
      wi32x16_t si;
#pragma unroll
      for (int v = 0; v < 16; ++v) si[v] = 0;
      uint4 kf[kQFrags];
#pragma unroll
      for (int d = 0; d < kKAhead; ++d)
        kf[d] = *reinterpret_cast<const uint4*>(kl + (kq_lane ^ (32 * d)));
#pragma unroll
      for (int d = 0; d < kQFrags; ++d) {
        if (d + kKAhead < kQFrags)
          kf[d + kKAhead] =
              *reinterpret_cast<const uint4*>(kl + (kq_lane ^ (32 * (d + kKAhead))));
        si = __builtin_amdgcn_mfma_i32_32x32x32_i8(__builtin_bit_cast(wi32x4_t, kf[d]), qf[d],
                                                   si, 0, 0, 0);
      }
      __builtin_amdgcn_sched_group_barrier(0x100, kKAhead, 0);
#pragma unroll
      for (int d = 0; d < kQFrags - kKAhead; ++d) {
        __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
        __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);
      }
      __builtin_amdgcn_sched_group_barrier(0x008, kKAhead, 0);
      f32x16_t sfull;
#pragma unroll
      for (int c = 0; c < 4; ++c) {
        const float4 ks4 = *reinterpret_cast<const float4*>(&scl[buf][8 * c + 4 * half]);
        const float ks[4] = {ks4.x, ks4.y, ks4.z, ks4.w};
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          float sc = static_cast<float>(si[4 * c + i] + qs128) - qb_row;
          sc = sc * fq_row;
          sc = sc * ks[i];
          sfull[4 * c + i] = sc * kInv127Sq;
        }
      }
      return sfull;
    } else {
      f32x16_t sblk;
#pragma unroll
      for (int v = 0; v < 16; ++v) sblk[v] = 0.0f;
      uint4 kf[kQFrags];
#pragma unroll
      for (int d = 0; d < kKAhead; ++d)
        kf[d] = *reinterpret_cast<const uint4*>(kl + (k_lane ^ (32 * d)));
#pragma unroll
      for (int d = 0; d < kQFrags; ++d) {
        if (d + kKAhead < kQFrags)
          kf[d + kKAhead] =
              *reinterpret_cast<const uint4*>(kl + (k_lane ^ (32 * (d + kKAhead))));
        sblk = __builtin_amdgcn_mfma_f32_32x32x16_bf16(__builtin_bit_cast(bf16x8_t, kf[d]),
                                                       qf[d], sblk, 0, 0, 0);
      }
      __builtin_amdgcn_sched_group_barrier(0x100, kKAhead, 0);
#pragma unroll
      for (int d = 0; d < kQFrags - kKAhead; ++d) {
        __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
        __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);
      }
      __builtin_amdgcn_sched_group_barrier(0x008, kKAhead, 0);
      return sblk;
    }
  };
  // bf16 scores with the next iteration's page-staged rows loaded between
  // the MFMAs (K and V of row i after MFMAs 4i + 1 and 4i + 3): a load's
  // issue then overlaps the MFMA pipe instead of holding up the wave ahead
  // of the scores.  kb / vb: the wave's first staged row; kdst / vdst: the
  // next buffers.
  auto qk_staging = [&](const uint8_t* kl, const uint8_t* kb, const uint8_t* vb, uint8_t* kdst,
                        uint8_t* vdst) -> f32x16_t {
    const int64_t row_bytes = 2 * kv_stride;
    f32x16_t sblk;
#pragma unroll
    for (int v = 0; v < 16; ++v) sblk[v] = 0.0f;
    uint4 kf[kQFrags];
#pragma unroll
    for (int d = 0; d < kKAhead; ++d)
      kf[d] = *reinterpret_cast<const uint4*>(kl + (k_lane ^ (32 * d)));
#pragma unroll
    for (int d = 0; d < kQFrags; ++d) {
      if (d + kKAhead < kQFrags)
        kf[d + kKAhead] = *reinterpret_cast<const uint4*>(kl + (k_lane ^ (32 * (d + kKAhead))));
      sblk = __builtin_amdgcn_mfma_f32_32x32x16_bf16(__builtin_bit_cast(bf16x8_t, kf[d]), qf[d],
                                                     sblk, 0, 0, 0);
      if (d & 1) {
        const int i = d >> 2;
        const int r = wave * kWStageRows + i;  // wave-uniform key row of the iteration
        if ((d & 2) == 0) {
          uint32_t lk = static_cast<uint32_t>(16 * lane) ^ static_cast<uint32_t>(16 * (r & 15));
          asm volatile("" : "+v"(lk));
          __builtin_amdgcn_global_load_lds(kb + i * row_bytes + lk,
                                           (lds_void_t*)(kdst + r * kWRowBytes), 16, 0, 0);
        } else {
          uint32_t lv = static_cast<uint32_t>(16 * lane) ^ static_cast<uint32_t>(32 * (r & 3));
          asm volatile("" : "+v"(lv));
          __builtin_amdgcn_global_load_lds(vb + i * row_bytes + lv,
                                           (lds_void_t*)(vdst + r * kWRowBytes), 16, 0, 0);
        }
      }
    }
    __builtin_amdgcn_sched_group_barrier(0x100, kKAhead, 0);
#pragma unroll
    for (int d = 0; d < kQFrags; ++d) {
      __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
      if (d + kKAhead < kQFrags) __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);
      if (d & 1) __builtin_amdgcn_sched_group_barrier(0x010, 1, 0);
    }
    return sblk;
  };
  auto softmax_pair = [&](const f32x16_t& sblk, int tile_key0, bool masked, float (&w)[2][8],
                          float (&corr)[2], bool (&big)[2]) {
#pragma unroll
    for (int u = 0; u < 2; ++u) {
      float sv[8];
#pragma unroll
      for (int i = 0; i < 8; ++i) sv[i] = sblk[8 * u + i];
      if (!masked) {
        softmax_tile<false>(sv, 16, half, m, l, corr[u], w[u], big[u]);
      } else {
        corr[u] = 1.0f;
        big[u] = false;
#pragma unroll
        for (int i = 0; i < 8; ++i) w[u][i] = 0.0f;
        const int tk = tile_key0 + 16 * u;
        if (tk < wave_count) {  // wave-uniform
          if (tk + 16 <= wave_min) {
            softmax_tile<false>(sv, 16, half, m, l, corr[u], w[u], big[u]);
          } else {
            const int valid = min(16, max(0, count - tk));
            softmax_tile<true>(sv, valid, half, m, l, corr[u], w[u], big[u]);
          }
        }
      }
    }
  };
  // Fold of the two tiles and acc_stored += V^T P''^T (prefill.hip's fold_pv
  // on one 32-key block, over the 16 dim blocks).
  auto fold_pv = [&](const uint8_t* vl, const float (&w0)[2][8], const float (&corr)[2],
                     const bool (&big)[2], int buf) {
    // bq: the weights as (w * v_scale) / 127; lane value i of tile u is key
    // 16u + 8*(i/4) + 4*half + i%4.
    float w[2][8];
#pragma unroll
    for (int u = 0; u < 2; ++u) {
#pragma unroll
      for (int j = 0; j < 2; ++j) {
        float vs[4] = {1.0f, 1.0f, 1.0f, 1.0f};
        if constexpr (kBq) {
          const float4 v4 =
              *reinterpret_cast<const float4*>(&scl[buf][kWKeys + 16 * u + 8 * j + 4 * half]);
          vs[0] = v4.x;
          vs[1] = v4.y;
          vs[2] = v4.z;
          vs[3] = v4.w;
        }
#pragma unroll
        for (int i = 0; i < 4; ++i)
          w[u][4 * j + i] = kBq ? (w0[u][4 * j + i] * vs[i]) * kInv127 : w0[u][4 * j + i];
      }
    }
    float S_new = S * (corr[0] * corr[1]);
    if (__builtin_amdgcn_ballot_w64(S_new < 0x1p-64f) != 0) {  // wave-uniform
#pragma unroll
      for (int b = 0; b < kWDimBlocks; ++b) {
        f32x16_t t = acc[b];
        asm volatile("" : "+v"(t));
        acc[b] = t * S_new;
        asm volatile("" : "+a"(acc[b]));
        __builtin_amdgcn_sched_barrier(0);
      }
      S_new = 1.0f;
    }
    S = S_new;
    const float inv_s = __builtin_amdgcn_rcpf(S_new);
    const float fs[2] = {corr[1] * inv_s, inv_s};
    bf16x8_t phi[2];
#pragma unroll
    for (int u = 0; u < 2; ++u) {
#pragma unroll
      for (int i = 0; i < 8; i += 2) {
        const bf16x2_t hb =
            __builtin_convertvector(f32x2_t{w[u][i] * fs[u], w[u][i + 1] * fs[u]}, bf16x2_t);
        phi[u][i] = hb[0];
        phi[u][i + 1] = hb[1];
      }
    }
    // V^T operands of tile u, dim blocks b0 .. b0+3 (8 transposing reads).
    auto read_group = [&](int u, int b0, bf16x8_t (&av)[4]) {
      const uint8_t* vt = vl + 16 * u * kWRowBytes;
#pragma unroll
      for (int b = 0; b < 4; ++b) {
        const uint8_t* vb = ((b0 + b) & 1) ? vt + v_odd1 + 64 * (b0 + b - 1)
                                           : vt + v_even + 64 * (b0 + b);
        const s16x4_t v0 = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_s16x4_t*)vb);
        const s16x4_t v1 =
            __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_s16x4_t*)(vb + 8 * kWRowBytes));
        av[b] = __builtin_bit_cast(bf16x8_t,
                                   __builtin_shufflevector(v0, v1, 0, 1, 2, 3, 4, 5, 6, 7));
      }
    };
    auto mfma_group = [&](const bf16x8_t& p, int b0, const bf16x8_t (&av)[4]) {
#pragma unroll
      for (int b = 0; b < 4; ++b)
        acc[b0 + b] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(av[b], p, acc[b0 + b], 0, 0, 0);
    };
    // Eight groups of four MFMAs (tile u, dim blocks 4q .. 4q+3), one group
    // of V^T reads in flight (a second one does not fit the VGPRs left).
    // A tile's lo parts (p - bf16(p)) take the MFMAs right after its hi
    // parts on the same fragments when some row of the wave has its big
    // flag (per accumulator: hi 0, lo 0, hi 1, lo 1).
#pragma unroll
    for (int u = 0; u < 2; ++u) {
      const bool lo = __builtin_amdgcn_ballot_w64(big[u]) != 0;  // wave-uniform
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        bf16x8_t ga[4];
        read_group(u, 4 * q, ga);
        mfma_group(phi[u], 4 * q, ga);
        if (lo) {
          bf16x8_t plo;
#pragma unroll
          for (int i = 0; i < 8; ++i)
            plo[i] = static_cast<__bf16>(w[u][i] * fs[u] - static_cast<float>(phi[u][i]));
          mfma_group(plo, 4 * q, ga);
        }
      }
    }
  };

  // End of iteration it: the next iteration's rows have landed (each wave
  // waits for its own loads; the barrier publishes them to the block).  If
  // the keys staged during the next iteration (those of iteration it + 2)
  // reach past the page-table window, the window moves to their first page
  // (nothing reads it between the barrier and the refill's barrier).
  auto iteration_end = [&](int it, uint8_t* vnext) {
#pragma unroll
    for (int b = 0; b < kWDimBlocks; ++b) asm volatile("" : "+a"(acc[b]));
    __builtin_amdgcn_s_waitcnt(0);
    if (it + 1 < n_iters) land_v(it + 1, vnext);
    __syncthreads();
    const int j = it + 2;
    if (j < n_iters) {  // block-uniform
      const int p_hi = (min((j + 1) * kWKeys, count_max) - 1) >> shift;
      if (p_hi >= wbase + kWLdsPages) {
        wbase = (j * kWKeys) >> shift;
        load_window(wbase);
        __syncthreads();
      }
    }
  };
  // An iteration whose keys are valid for every row of the block.  The
  // next iteration's rows are staged unconditionally (past the last
  // iteration they are clamped, in-bounds rows of an unused buffer).
  auto full_iteration = [&](int it, const uint8_t* kl, const uint8_t* vl, uint8_t* knext,
                            uint8_t* vnext) {
    f32x16_t s;
    if (!kBq && shift >= 3 && (it + 2) * kWKeys <= count_max) {  // block-uniform
      // The wave's kWStageRows rows of the next iteration lie in one page.
      const int key0 = (it + 1) * kWKeys + wave * kWStageRows;  // wave-uniform
      const int prow = __builtin_amdgcn_readfirstlane(page_of(key0));
      const int64_t slot0 = static_cast<int64_t>(prow) + (key0 & row_mask);
      s = qk_staging(kl, reinterpret_cast<const uint8_t*>(kbase + slot0 * kv_stride),
                     reinterpret_cast<const uint8_t*>(vbase + slot0 * kv_stride), knext, vnext);
    } else {
      stage(it + 1, knext, vnext, (it + 1) & 1);
      s = qk(kl, it & 1);
    }
    float w[2][8], corr[2];
    bool big[2];
    softmax_pair(s, 0, false, w, corr, big);
    fold_pv(vl, w, corr, big, it & 1);
    iteration_end(it, vnext);
  };
  // An iteration on the causal diagonal: per-tile masks (a wave whose rows
  // all end before a tile gets corr 1 and zero weights for it).  One call
  // site with the buffers chosen at run time keeps the register allocation
  // of the whole kernel within the register file.
  auto masked_iteration = [&](int it, const uint8_t* kl, const uint8_t* vl, uint8_t* knext,
                              uint8_t* vnext) {
    const int key_base = it * kWKeys;
    if (it + 1 < n_iters) stage(it + 1, knext, vnext, (it + 1) & 1);
    float w[2][8], corr[2];
    bool big[2];
    const f32x16_t s = qk(kl, it & 1);
    softmax_pair(s, key_base, true, w, corr, big);
    fold_pv(vl, w, corr, big, it & 1);
    iteration_end(it, vnext);
  };
  // Iterations whose keys are valid for every row of the block run the
  // unmasked code, in pairs so that each buffer is a fixed LDS object; the
  // rest (the causal diagonal, and an odd one left over) the masked code.
  // All waves of the block run the same iterations and barriers.
  const int block_min = ntok == kWTokens ? base_pos + (t0 - buf_start) + 1 : 0;
  const int it_full = min(n_iters, block_min / kWKeys) & ~1;
  int it = 0;
  for (; it < it_full; it += 2) {
    full_iteration(it, kbuf0, vbuf0, kbuf1, vbuf1);
    full_iteration(it + 1, kbuf1, vbuf1, kbuf0, vbuf0);
  }
#pragma unroll 1
  for (; it < n_iters; ++it) {
    const bool odd = it & 1;
    masked_iteration(it, odd ? kbuf1 : kbuf0, odd ? vbuf1 : vbuf0, odd ? kbuf0 : kbuf1,
                     odd ? vbuf0 : vbuf1);
  }

  // ---- one-segment merge and bf16 store (PrefillMergeKernel) ----
  // Lane l holds dims 32*b + 8*j + 4*half + i (value 4*j + i of block b).
  if (row_live) {
    const float c0 = l > 0.0f ? fexp(max_ref(-87.0f, m - m)) : 0.0f;
    const float gl = l * c0;
    const bool live = gl > 0.0f;
    const float inv_l = live ? 1.0f / gl : 0.0f;
    uint16_t* dst = out + (static_cast<int64_t>(tok) * num_q + head) * kWD + 4 * half;
#pragma unroll
    for (int b = 0; b < kWDimBlocks; ++b) {
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        uint32_t e[4];
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          const float av = (acc[b][4 * j + i] * S) * c0;
          e[i] = live ? f32_to_bf16_bits(av * inv_l) : 0u;
        }
        *reinterpret_cast<uint2*>(dst + 32 * b + 8 * j) =
            make_uint2(e[0] | (e[1] << 16), e[2] | (e[3] << 16));
      }
    }
  }
}

// Grid of the XCD-aware order above (blocks past the last query block exit).
int wide_blocks(int num_qblocks, int num_kv) {
  const int lanes = kXcds % num_kv == 0 ? kXcds / num_kv : kXcds;
  const int per_lane = kXcds % num_kv == 0 ? kWSub : kWSub * num_kv;
  return (num_qblocks + lanes - 1) / lanes * per_lane * kXcds;
}

}  // namespace

hipError_t launch_prefill_wide_mfma(const int32_t* image, int num_qblocks, const void* q,
                                    const void* k, const void* v, void* output, int num_q,
                                    int num_kv, int64_t kv_stride, PagedGeom geom,
                                    hipStream_t stream) {
  if (num_qblocks <= 0) return hipSuccess;
  const int blocks = wide_blocks(num_qblocks, num_kv);
  hipLaunchKernelGGL(prefill_wide_mfma_kernel<false>, dim3(blocks), dim3(kPThreads), 0,
                     stream, image, q, nullptr, nullptr, k, nullptr, v, nullptr,
                     static_cast<uint16_t*>(output), num_q, num_kv, kv_stride, geom.shift,
                     geom.row_mask, num_qblocks);
  return hipGetLastError();
}

hipError_t launch_prefill_wide_mfma_bq(const int32_t* image, int num_qblocks, const void* q_i8,
                                       const float* qi_bias, const float* f_q, const void* k,
                                       const float* k_scale, const void* v,
                                       const float* v_scale, void* output, int num_q,
                                       int num_kv, int64_t kv_stride, PagedGeom geom,
                                       hipStream_t stream) {
  if (num_qblocks <= 0) return hipSuccess;
  const int blocks = wide_blocks(num_qblocks, num_kv);
  hipLaunchKernelGGL(prefill_wide_mfma_kernel<true>, dim3(blocks), dim3(kPThreads), 0,
                     stream, image, q_i8, qi_bias, f_q, k, k_scale, v, v_scale,
                     static_cast<uint16_t*>(output), num_q, num_kv, kv_stride, geom.shift,
                     geom.row_mask, num_qblocks);
  return hipGetLastError();
}

}  // namespace ifr
