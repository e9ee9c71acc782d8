// Chunked causal prefill over the paged cache with MFMA (gfx950), full
// attention.  Semantics: FlashPrefillFullKernel + PrefillMergeKernel
// (kernels/flash_attention_prefill.mojo:117-248) at degree 1 -- every query
// token t at absolute position p walks keys [0, p] in tiles of 16 from key 0
// with the online softmax of process_kv_tile (kernels/attention_ops.mojo:
// 165-253), then its one-segment merge (kernels/logsum_merge.mojo:28-122).
// Because all queries start at key 0 the tiles line up across queries, so a
// block of query tokens shares every K/V tile of its kv head.
//
// A row is one (query token, q head); a wave owns 32 rows = 16 tokens x the
// 2 q heads of one kv head; a block of 4 waves (one per SIMD) owns 64
// tokens.  Each iteration stages 64 keys (4 tiles) in LDS and computes, per
// wave:
//
//   S^T (32 keys x 32 rows) = K . Q^T, per pair of tiles     v_mfma_f32_32x32x16_bf16
//   O^T (32 dims x 32 rows) += V^T . P'^T, 16 keys/MFMA       v_mfma_f32_32x32x16_bf16
//
// In the 32x32 C layout lane l holds row l%32 and keys 8j + 4*(l/32) + i
// (j, i < 4) of a 32-key block, so a 16-key tile is 8 keys in lane l and 8 in
// lane l^32: the per-row softmax state stays in the lane pair.  Each K / V
// fragment read from LDS feeds 32 rows (the transposing V reads are the
// costliest LDS operation on gfx950).
// The reference's per-tile steps are kept in tile order: a row skips tiles
// past its position (the reference never visits them), pads of its last
// tile score -1e30 (the reference adds their fexp(-87) = 1.4e-38 to l;
// here they weigh 0, the same l in f32), and m, corr, w use the biased
// exp; l is updated tile by tile.  The accumulator rescales of a pair of
// tiles are folded: acc*c0*c1 + (w0*c1) V0 + w1 V1 equals the
// reference's nested (acc*c0 + w0 V0)*c1 + w1 V1 up to f32 rounding, and
// the product of the rescales is carried as a per-row scale S (acc =
// acc_stored * S) that divides the weights instead of multiplying the 128
// accumulators.  P' enters the bf16 MFMA as hi + lo bf16 parts (~16
// significant bits per weight); QK^T products are exact in f32.  The biased
// exp is evaluated with fused multiply-adds (fexp_fused_u): its value differs
// from the reference's separately rounded steps by about 2e-5 relative,
// far inside the bf16 output tolerance, and it saves a third of the
// softmax's VALU work, which bounds this kernel together with the MFMAs.
//
// K and V reach LDS straight from global memory (global_load_lds_dwordx4,
// no registers) one iteration ahead.  K rows are stored XOR-swizzled (16-byte
// chunk c of key k at position c ^ (k & 15)) so the 16 keys a QK operand read
// touches fall in distinct banks; V rows are stored plainly and read with
// ds_read_b64_tr_b16 (a 16-lane transposing read).  A window of the run's
// page table is held in LDS.
// Blocks are numbered kv-head-fastest so every block of a kv head lands on
// one XCD (block id mod 8) and shares that XCD's L2.
//
// kBq: the butterquant variant (BqFlashPrefillFullKernel, butterquant_
// kernels/attention.mojo:267-351) at 16 q / 8 kv x 256, with the sliding
// kernel's int8 pieces: K codes (256-byte rows) staged straight into LDS,
// scores from v_mfma_i32_32x32x32_i8 plus 128 * sum q (the reference's VNNI
// raw dot, which reads k ^ 0x80 as unsigned) formed in the reference's order
// ((raw - qi_bias) * f_q) * k_scale / 127^2, V codes through registers into
// the bf16 V tile (exact for int8), and the V scale entering each weight as
// (w * v_scale) / 127.
#include <type_traits>

#include "common.hpp"
#include "launch.hpp"
#include "prefill_common.hpp"

namespace ifr {
namespace {

using namespace prefill;

typedef int i32x4_t __attribute__((ext_vector_type(4)));
typedef int i32x16_t __attribute__((ext_vector_type(16)));
constexpr int kBqRowBytes = kPD;  // one kv head's row of int8 codes

// One wave per SIMD (up to 512 VGPR + AGPR per lane); one block per CU.
template <bool kBq>
__global__ __launch_bounds__(kPThreads) __attribute__((amdgpu_waves_per_eu(1, 1)))
void prefill_full_mfma_kernel(
    const int32_t* __restrict__ image, const void* __restrict__ qp,
    const float* __restrict__ qi_bias, const float* __restrict__ f_q,
    const void* __restrict__ kcp, const float* __restrict__ k_scale,
    const void* __restrict__ vcp, const float* __restrict__ v_scale,
    uint16_t* __restrict__ out, int num_q, int num_kv, int64_t kv_stride,
    int shift, int row_mask) {
  // Two K and two V buffers as separate LDS objects: the LDS reads of one
  // buffer then provably do not alias the loads landing in the other, and
  // no wait for those loads is inserted before the reads.
  __shared__ __align__(16) uint8_t kbuf0[kBq ? kKeys * kBqRowBytes : kTileBytes];
  __shared__ __align__(16) uint8_t kbuf1[kBq ? kKeys * kBqRowBytes : kTileBytes];
  __shared__ __align__(16) uint8_t vbuf0[kTileBytes];
  __shared__ __align__(16) uint8_t vbuf1[kTileBytes];
  __shared__ int32_t page_rows[kPrefillLdsPages];
  // bq: the staged keys' K and V scales, per buffer.
  __shared__ __align__(16) float kscl[2][kBq ? kKeys : 1];
  __shared__ __align__(16) float vscl[2][kBq ? kKeys : 1];
  const int tid = threadIdx.x;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int lane = tid & 63;
  const int half = lane >> 5;  // key half of the C layout / k half of the operands
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

  // Keys the block needs: [0, count_max), count_max = last token's position + 1.
  const int count_max = base_pos + (t0 + ntok - 1 - buf_start) + 1;
  const int n_iters = (count_max + kKeys - 1) / kKeys;

  // This lane's row: token wave*16 + (l%32)/2, q head 2g + (l%32)%2.
  const int tok_local = wave * kPTokensPerWave + (row >> 1);
  const int head = g * 2 + (row & 1);
  const bool row_live = tok_local < ntok;
  const int tok = t0 + tok_local;
  const int count = row_live ? base_pos + (tok - buf_start) + 1 : 0;
  const int wave_first = wave * kPTokensPerWave;
  const int wave_last = min(ntok, wave_first + kPTokensPerWave) - 1;
  const int wave_count = wave_first < ntok ? base_pos + (t0 + wave_last - buf_start) + 1 : 0;
  // Keys below wave_min are valid for every row of the wave (0 if the wave
  // has rows past the block's last token).
  const int wave_min = wave_first + kPTokensPerWave <= ntok
                           ? base_pos + (t0 + wave_first - buf_start) + 1
                           : 0;

  // Q^T fragments.  bf16: lane holds Q[row][16*d + 8*half .. +7] for 16-dim
  // steps d; bq: the codes Q[row][32*d + 16*half .. +15], with the row's
  // 128 * sum q, bias and f_q.
  constexpr int kQFrags = kBq ? kPD / 32 : kPD / 16;
  using QFrag = typename std::conditional<kBq, i32x4_t, bf16x8_t>::type;
  QFrag qf[kQFrags];
  int qs128 = 0;
  float qb_row = 0.0f, fq_row = 0.0f;
  const int64_t q_row = static_cast<int64_t>(row_live ? tok : t0) * num_q + head;
  if constexpr (kBq) {
    const int8_t* qr = static_cast<const int8_t*>(qp) + q_row * kPD + 16 * half;
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
    qb_row = qi_bias[q_row];
    fq_row = f_q[q_row];
  } else {
    const uint16_t* qr = static_cast<const uint16_t*>(qp) + q_row * kPD + 8 * half;
#pragma unroll
    for (int d = 0; d < kQFrags; ++d) {
      const uint4 v = *reinterpret_cast<const uint4*>(qr + 16 * d);
      qf[d] = __builtin_bit_cast(bf16x8_t, v);
    }
  }
  // The Q^T fragments live in AGPRs (MFMA operands may come from there),
  // which leaves the VGPRs to the softmax and the operand reads.
#pragma unroll
  for (int d = 0; d < kQFrags; ++d) asm volatile("" : "+a"(qf[d]));

  // The O^T accumulator is kept as acc_stored with acc = acc_stored * S: a
  // tile's rescale multiplies S, and the weights entering the MFMA are
  // divided by the new S, so the 128 accumulators are not rescaled per
  // iteration.  When S would fall below 2^-64 the accumulators take it over
  // (acc_stored *= S, S = 1) for the whole wave.
  f32x16_t acc[kDimBlocks];
#pragma unroll
  for (int b = 0; b < kDimBlocks; ++b)
#pragma unroll
    for (int v = 0; v < 16; ++v) acc[b][v] = 0.0f;
  float m = kNegBig, l = 0.0f, S = 1.0f;

  // The run's page table in LDS, so that the staging addresses of an
  // iteration wait on an LDS read rather than on a global load: a window of
  // kPrefillLdsPages entries (entry i holds page wbase + i), moved forward at
  // an iteration boundary when the next staged keys pass its end.
  const int n_pages = count_max > 0 ? ((count_max - 1) >> shift) + 1 : 0;
  int wbase = 0;
  auto load_window = [&](int first) {
    const int n = min(kPrefillLdsPages, n_pages - first);
    for (int i = tid; i < n; i += kPThreads) page_rows[i] = rows[first + i];
  };
  load_window(0);
  __syncthreads();

  // Staging of one iteration: wave w moves key rows kStageRows*w .. +15 of
  // K and of V, two rows per load (lanes 0-31 the first, 32-63 the second,
  // 16 bytes each).  Lane p of a row writes LDS chunk p; for K that chunk
  // holds global chunk p ^ (key & 15), for V chunk p ^ 2*(key & 3).  Keys past count_max read the last
  // key (in bounds); their V rows are zeroed once the last iteration's
  // loads have landed.
  // bq: K code rows of 256 bytes, four per load (lane p: row p / 16, LDS
  // chunk p % 16 holding global chunk (p % 16) ^ (key & 15)); V codes to
  // registers (the same rows, 16 codes from 16 * (p % 16)), written to LDS as
  // bf16 rows once landed; wave 0 moves the 64 keys' K and V scales.
  const uint16_t* kbase = static_cast<const uint16_t*>(kcp) + static_cast<int64_t>(g) * kPD;
  const uint16_t* vbase = static_cast<const uint16_t*>(vcp) + static_cast<int64_t>(g) * kPD;
  const int8_t* kbase8 = static_cast<const int8_t*>(kcp) + static_cast<int64_t>(g) * kPD;
  const int8_t* vbase8 = static_cast<const int8_t*>(vcp) + static_cast<int64_t>(g) * kPD;
  const int stage_row0 = wave * kStageRows + half;
  auto slot_of = [&](int key) -> int64_t {
    return static_cast<int64_t>(page_rows[(key >> shift) - wbase]) + (key & row_mask);
  };
  uint4 vcodes[kBq ? kStageRows / 4 : 1];
  auto stage_scales = [&](int it, int buf) {
    if (wave == 0) {
      const int key = min(it * kKeys + lane, count_max - 1);
      const int64_t si = slot_of(key) * num_kv + g;
      __builtin_amdgcn_global_load_lds(k_scale + si, (lds_void_t*)(&kscl[buf][0]), 4, 0, 0);
      __builtin_amdgcn_global_load_lds(v_scale + si, (lds_void_t*)(&vscl[buf][0]), 4, 0, 0);
    }
  };
  auto stage = [&](int it, uint8_t* kdst, uint8_t* vdst, int buf) {
    if constexpr (kBq) {
#pragma unroll
      for (int i = 0; i < kStageRows / 4; ++i) {
        const int rr = wave * kStageRows + 4 * i + (lane >> 4);
        const int key = min(it * kKeys + rr, count_max - 1);
        const int64_t off = slot_of(key) * kv_stride;
        const int c = lane & 15;
        __builtin_amdgcn_global_load_lds(
            kbase8 + off + 16 * (c ^ (rr & 15)),
            (lds_void_t*)(kdst + (wave * kStageRows + 4 * i) * kBqRowBytes), 16, 0, 0);
        vcodes[i] = *reinterpret_cast<const uint4*>(vbase8 + off + 16 * c);
      }
      stage_scales(it, buf);
      return;
    }
#pragma unroll
    for (int i = 0; i < kStageRows / 2; ++i) {
      const int r = stage_row0 + 2 * i;  // key row within the iteration
      const int key = min(it * kKeys + r, count_max - 1);
      const int64_t slot =
          static_cast<int64_t>(page_rows[(key >> shift) - wbase]) + (key & row_mask);
      const int64_t off = slot * kv_stride;
      const int kchunk = row ^ (r & 15);
      const int lds_row = wave * kStageRows + 2 * i;  // wave-uniform
      __builtin_amdgcn_global_load_lds(
          kbase + off + 8 * kchunk,
          (lds_void_t*)(kdst + lds_row * kRowBytes), 16, 0, 0);
      __builtin_amdgcn_global_load_lds(
          vbase + off + 8 * (row ^ (2 * (r & 3))),
          (lds_void_t*)(vdst + lds_row * kRowBytes), 16, 0, 0);
    }
  };
  // The same for an iteration whose kStageRows rows per wave all lie below
  // count_max and inside one page (pages of >= 16 rows): one page lookup, a
  // wave-uniform row base and per-lane byte offsets fixed for the kernel.
  // Row rr = 2i + half of the wave's rows sits rr * kv_stride * 2 bytes past
  // the base, i.e. i * 4 * kv_stride (uniform) + hk (lane); its K chunk
  // row ^ rr = (row ^ half) ^ 2i gives the byte offset x16 ^ 32i, its V
  // chunk row ^ 2*(rr & 3) one of two lane constants (i even or odd).
  // bq: row rr = 4i + lr (lr = lane / 16) at i * 4 * kv_stride + lr *
  // kv_stride bytes, K chunk (c ^ lr) ^ 4i.
  const int lr = lane >> 4;
  const int cq = lane & 15;
  const int hk = kBq ? lr * static_cast<int>(kv_stride) : half * static_cast<int>(kv_stride) * 2;
  const uint32_t x16 = kBq ? 16u * static_cast<uint32_t>(cq ^ lr)
                           : 16u * static_cast<uint32_t>(row ^ half);
  const uint32_t hv0 = kBq ? static_cast<uint32_t>(hk) + 16u * static_cast<uint32_t>(cq)
                           : static_cast<uint32_t>(hk) + 16u * static_cast<uint32_t>(row ^ (2 * half));
  const uint32_t hv1 =
      static_cast<uint32_t>(hk) + 16u * static_cast<uint32_t>(row ^ (4 + 2 * half));
  auto stage_page = [&](int it, uint8_t* kdst, uint8_t* vdst, int buf) {
    const int key0 = it * kKeys + wave * kStageRows;  // wave-uniform
    const int prow = __builtin_amdgcn_readfirstlane(page_rows[(key0 >> shift) - wbase]);
    const int64_t slot0 = static_cast<int64_t>(prow) + (key0 & row_mask);
    if constexpr (kBq) {
      const char* kb = reinterpret_cast<const char*>(kbase8 + slot0 * kv_stride);
      const char* vb = reinterpret_cast<const char*>(vbase8 + slot0 * kv_stride);
      const int64_t step = 4 * kv_stride;
#pragma unroll
      for (int i = 0; i < kStageRows / 4; ++i) {
        __builtin_amdgcn_global_load_lds(
            kb + i * step + (static_cast<uint32_t>(hk) + (x16 ^ (64u * i))),
            (lds_void_t*)(kdst + (wave * kStageRows + 4 * i) * kBqRowBytes), 16, 0, 0);
        vcodes[i] = *reinterpret_cast<const uint4*>(vb + i * step + hv0);
      }
      stage_scales(it, buf);
      return;
    }
    const char* kb = reinterpret_cast<const char*>(kbase + slot0 * kv_stride);
    const char* vb = reinterpret_cast<const char*>(vbase + slot0 * kv_stride);
    const int64_t step = 4 * kv_stride;  // bytes from row pair i to i + 1
#pragma unroll
    for (int i = 0; i < kStageRows / 2; ++i) {
      const int lds_row = wave * kStageRows + 2 * i;  // wave-uniform
      const uint32_t ko = static_cast<uint32_t>(hk) + (x16 ^ (32u * i));
      __builtin_amdgcn_global_load_lds(kb + i * step + ko,
                                       (lds_void_t*)(kdst + lds_row * kRowBytes), 16, 0, 0);
      __builtin_amdgcn_global_load_lds(vb + i * step + ((i & 1) ? hv1 : hv0),
                                       (lds_void_t*)(vdst + lds_row * kRowBytes), 16, 0, 0);
    }
  };
  // After the wave's loads have landed: bf16 zeroes the V rows of keys past
  // count_max; bq writes its V codes as bf16 rows (the bf16 swizzle: chunk c
  // of row rr at c ^ 2*(rr & 3)), zeros past count_max.
  auto zero_tail = [&](int it, uint8_t* vdst) {
    if constexpr (kBq) {
#pragma unroll
      for (int i = 0; i < kStageRows / 4; ++i) {
        const int rr = wave * kStageRows + 4 * i + (lane >> 4);
        const bool in = it * kKeys + rr < count_max;
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
        const int c0 = 2 * (lane & 15);
        uint8_t* vr = vdst + rr * kRowBytes;
        *reinterpret_cast<uint4*>(vr + 16 * (c0 ^ (2 * (rr & 3)))) =
            make_uint4(bf[0], bf[1], bf[2], bf[3]);
        *reinterpret_cast<uint4*>(vr + 16 * ((c0 + 1) ^ (2 * (rr & 3)))) =
            make_uint4(bf[4], bf[5], bf[6], bf[7]);
      }
      return;
    }
    if ((it + 1) * kKeys <= count_max) return;  // block-uniform
#pragma unroll
    for (int i = 0; i < kStageRows / 2; ++i) {
      const int r = stage_row0 + 2 * i;
      if (it * kKeys + r >= count_max)
        *reinterpret_cast<uint4*>(vdst + r * kRowBytes + 16 * row) =
            make_uint4(0u, 0u, 0u, 0u);
    }
  };

  if (n_iters > 0) stage(0, kbuf0, vbuf0, 0);
  __builtin_amdgcn_s_waitcnt(0);  // the Q fragments and iteration 0's rows
  if (n_iters > 0) zero_tail(0, vbuf0);
  __syncthreads();

  // QK operand reads: lane reads chunk 2d + half of key 32*sb + row, found
  // at position (2d + half) ^ (row & 15) = 2d ^ kx with kx = (row & 15) ^ half;
  // the byte address is therefore k_lane ^ 32d.
  const int k_lane = row * kRowBytes + 16 * ((row & 15) ^ half);
  // Transposing-read address of this lane inside a 16-key tile of V: lane
  // j of 16-lane group q addresses key 4*(q/2) + j/4 (+8 for the second
  // read), dims 16*(q%2) + 4*(j%4) .. +3 of 32-dim block b; the read
  // returns, in lane j, 4 keys of dim 16*(q%2) + j.  Lane l thus gets the
  // keys 4*half + 0..3 and 8 + 4*half + 0..3 of dim l%32, the k order of its
  // P values.  Unswizzled, that is chunk c = 4b + 2*(q%2) + (j%4)/2 of the
  // row, stored at c ^ 2*(j/4) (key & 3 = j/4): position
  // 4*(b ^ (j/8)) + 2*((q%2) ^ ((j/4)%2)) + (j%4)/2.  b ^ (j/8) is b + j/8
  // for even b and b - j/8 for odd b, so the per-block addresses are
  // immediate offsets from two lane bases.  The 4 rows a 16-lane group reads
  // then cover 8 distinct 16-byte chunks (32 banks).
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

  // S^T of tile pair h (32 keys) of the staged iteration (buffer buf).
  // The K operand reads run kKAhead steps ahead of their MFMAs.  bq:
  // ((raw - qi_bias) * f_q) * k_scale / 127^2 per (row, key), raw the
  // integer dot plus 128 * sum q; value 4j + i holds key 8j + 4*half + i.
  constexpr int kKAhead = 6;
  // bf16 page staging split into 16 single loads (K then V of row pair i
  // for load j = 2i, 2i + 1), so they can be issued between MFMAs.
  auto page_load = [&](int j, const char* kb, const char* vb, uint8_t* kdst, uint8_t* vdst) {
    const int i = j >> 1;
    const int64_t step = 4 * kv_stride;  // bytes from row pair i to i + 1
    const int lds_row = wave * kStageRows + 2 * i;  // wave-uniform
    if ((j & 1) == 0)
      __builtin_amdgcn_global_load_lds(kb + i * step + (static_cast<uint32_t>(hk) + (x16 ^ (32u * i))),
                                       (lds_void_t*)(kdst + lds_row * kRowBytes), 16, 0, 0);
    else
      __builtin_amdgcn_global_load_lds(vb + i * step + ((i & 1) ? hv1 : hv0),
                                       (lds_void_t*)(vdst + lds_row * kRowBytes), 16, 0, 0);
  };
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
    }
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
    // Keep that order: kKAhead reads, then each MFMA followed by the read
    // kKAhead steps ahead of it.
    __builtin_amdgcn_sched_group_barrier(0x100, kKAhead, 0);
#pragma unroll
    for (int d = 0; d < kPD / 16 - kKAhead; ++d) {
      __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
      __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);
    }
    __builtin_amdgcn_sched_group_barrier(0x008, kKAhead, 0);
    return sblk;
  };
  // bf16 S^T of tile pair h with the next iteration's page-staged loads
  // 8h .. 8h + 7 issued after the odd MFMAs: a load's issue then overlaps
  // the MFMA pipe instead of holding up the wave ahead of the scores (the
  // 64 staging loads of a block take about a thousand cycles to pass the
  // texture unit).
  auto qk_staging = [&](const uint8_t* kl, int h, const char* kb, const char* vb,
                        uint8_t* kdst, uint8_t* vdst) {
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
      if (d & 1) page_load(8 * h + (d >> 1), kb, vb, kdst, vdst);
    }
    __builtin_amdgcn_sched_group_barrier(0x100, kKAhead, 0);
#pragma unroll
    for (int d = 0; d < kPD / 16; ++d) {
      __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
      if (d + kKAhead < kPD / 16) __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);
      if (d & 1) __builtin_amdgcn_sched_group_barrier(0x010, 1, 0);
    }
    return sblk;
  };
  // Online softmax of the pair's two tiles; tile_key0 is the first key of
  // tile a.  Tiles past the wave's last row are skipped (corr 1, weights 0).
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
  // Fold of the pair and acc_stored += V^T P''^T:
  // acc*c_a*c_b + w_a*c_b V_a + w_b V_b = S' (acc_stored + (w_a*c_b V_a +
  // w_b V_b) / S'),  S' = S*c_a*c_b.
  auto fold_pv = [&](const uint8_t* vl, int h, const float (&w0)[2][8], const float (&corr)[2],
                     const bool (&big)[2], int buf) {
    // bq: the weights as (w * v_scale) / 127; lane value i of tile u is key
    // 32h + 16u + 8*(i/4) + 4*half + i%4.
    float w[2][8];
#pragma unroll
    for (int u = 0; u < 2; ++u) {
#pragma unroll
      for (int j = 0; j < 2; ++j) {
        float vs[4] = {1.0f, 1.0f, 1.0f, 1.0f};
        if constexpr (kBq) {
          const float4 v4 = *reinterpret_cast<const float4*>(
              &vscl[buf][32 * h + 16 * u + 8 * j + 4 * half]);
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
      // The accumulators are copied to VGPRs here, inside the rare branch
      // (the asm keeps the copy from being hoisted to the loop).
#pragma unroll
      for (int b = 0; b < kDimBlocks; ++b) {
        asm volatile("" : "+a"(acc[b]));  // no copy out of AGPRs ahead of the branch
        f32x16_t t = acc[b];
        asm volatile("" : "+v"(t));
        acc[b] = t * S_new;
        asm volatile("" : "+a"(acc[b]));
        __builtin_amdgcn_sched_barrier(0);  // one block of 16 at a time in VGPRs
      }
      S_new = 1.0f;
    }
    S = S_new;
    const float inv_s = __builtin_amdgcn_rcpf(S_new);
    const float fs[2] = {corr[1] * inv_s, inv_s};
    // P''^T of both tiles in bf16 (hi): k index 8*half + i holds the lane's
    // value i.  A tile's lo parts (p - bf16(p), about 8 more bits) join the
    // pass when some row of the wave has the tile's big flag (more than
    // kLoShare of its running l).
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
    // V^T operands in groups of four 32-dim blocks (8 transposing reads);
    // two groups are in flight, so each group's reads are issued a group of
    // MFMAs ahead of their use.
    auto read_group = [&](int u, int b0, bf16x8_t (&av)[4]) {
      const uint8_t* vt = vl + (32 * h + 16 * u) * kRowBytes;
#pragma unroll
      for (int b = 0; b < 4; ++b) {
        const uint8_t* vb = ((b0 + b) & 1) ? vt + v_odd1 + 64 * (b0 + b - 1)
                                           : vt + v_even + 64 * (b0 + b);
        const s16x4_t v0 = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_s16x4_t*)vb);
        const s16x4_t v1 =
            __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_s16x4_t*)(vb + 8 * kRowBytes));
        av[b] = __builtin_bit_cast(bf16x8_t,
                                   __builtin_shufflevector(v0, v1, 0, 1, 2, 3, 4, 5, 6, 7));
      }
    };
    // One pass over the pair's V^T fragments.  A tile's lo parts (kLo0 /
    // kLo1) take the MFMAs right after its hi parts on the same fragments,
    // so they cost MFMA issue only, no LDS reads of their own; per
    // accumulator the order is hi 0, lo 0, hi 1, lo 1.
    auto mfma_group = [&](const bf16x8_t& p, int b0, const bf16x8_t (&av)[4]) {
#pragma unroll
      for (int b = 0; b < 4; ++b)
        acc[b0 + b] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(av[b], p, acc[b0 + b], 0, 0, 0);
    };
    auto lo_part = [&](int u) {
      bf16x8_t plo;
#pragma unroll
      for (int i = 0; i < 8; ++i)
        plo[i] = static_cast<__bf16>(w[u][i] * fs[u] - static_cast<float>(phi[u][i]));
      return plo;
    };
    const bool lo0 = __builtin_amdgcn_ballot_w64(big[0]) != 0;  // wave-uniform
    const bool lo1 = __builtin_amdgcn_ballot_w64(big[1]) != 0;
    bf16x8_t ga[4], gb[4];
    read_group(0, 0, ga);
    read_group(0, 4, gb);
    mfma_group(phi[0], 0, ga);
    if (lo0) mfma_group(lo_part(0), 0, ga);
    read_group(1, 0, ga);
    mfma_group(phi[0], 4, gb);
    if (lo0) mfma_group(lo_part(0), 4, gb);
    read_group(1, 4, gb);
    mfma_group(phi[1], 0, ga);
    if (lo1) mfma_group(lo_part(1), 0, ga);
    mfma_group(phi[1], 4, gb);
    if (lo1) mfma_group(lo_part(1), 4, gb);
  };

  // End of one iteration: the accumulators and the Q^T fragments stay in
  // AGPRs across iterations (the MFMAs read and write them there; only the
  // rare rescale moves the accumulators through VGPRs); the next iteration's
  // rows have landed (each wave waits for its own loads; the barrier
  // publishes them to the block).  If the keys staged during the next
  // iteration (those of iteration it + 2) reach past the page-table window,
  // the window moves to their first page (nothing reads it between the
  // barrier and the refill's barrier).
  auto iteration_end = [&](int it, uint8_t* vnext) {
#pragma unroll
    for (int b = 0; b < kDimBlocks; ++b) asm volatile("" : "+a"(acc[b]));
#pragma unroll
    for (int d = 0; d < kQFrags; ++d) asm volatile("" : "+a"(qf[d]));
    __builtin_amdgcn_s_waitcnt(0);
    if (it + 1 < n_iters) zero_tail(it + 1, vnext);
    __syncthreads();
    const int j = it + 2;
    if (j < n_iters) {  // block-uniform
      const int p_hi = (min((j + 1) * kKeys, count_max) - 1) >> shift;
      if (p_hi >= wbase + kPrefillLdsPages) {
        wbase = (j * kKeys) >> shift;
        load_window(wbase);
        __syncthreads();
      }
    }
  };
  // An iteration whose keys are valid for every row: straight-line code.
  // The next iteration's rows are staged unconditionally (past the last
  // iteration they are clamped, in-bounds rows of an unused buffer), so the
  // staging shares a block with the score MFMAs.
  auto full_iteration = [&](bool page_stage, int it, const uint8_t* kl, const uint8_t* vl,
                            uint8_t* knext, uint8_t* vnext) {
    const int buf = it & 1;
    f32x16_t s0, s1;
    if (!kBq && page_stage) {  // block-uniform
      // One page lookup for the wave's rows of the next iteration; the
      // loads go out between the score MFMAs.
      const int key0 = (it + 1) * kKeys + wave * kStageRows;  // wave-uniform
      const int prow = __builtin_amdgcn_readfirstlane(page_rows[(key0 >> shift) - wbase]);
      const int64_t slot0 = static_cast<int64_t>(prow) + (key0 & row_mask);
      const char* kb = reinterpret_cast<const char*>(kbase + slot0 * kv_stride);
      const char* vb = reinterpret_cast<const char*>(vbase + slot0 * kv_stride);
      s0 = qk_staging(kl, 0, kb, vb, knext, vnext);
      s1 = qk_staging(kl, 1, kb, vb, knext, vnext);
    } else {
      if (page_stage)  // block-uniform
        stage_page(it + 1, knext, vnext, buf ^ 1);
      else
        stage(it + 1, knext, vnext, buf ^ 1);
      s0 = qk(kl, 0, buf);
      s1 = qk(kl, 1, buf);
    }
    // Straight-line order that lets the pair-1 scores (MFMA) run under the
    // pair-0 softmax (VALU), and the pair-0 PV (MFMA) under the pair-1
    // softmax.
    float w0[2][8], c0[2], w1[2][8], c1[2];
    bool g0[2], g1[2];
    softmax_pair(s0, 0, false, w0, c0, g0);
    fold_pv(vl, 0, w0, c0, g0, buf);
    softmax_pair(s1, 0, false, w1, c1, g1);
    fold_pv(vl, 1, w1, c1, g1, buf);
    iteration_end(it, vnext);
  };
  // An iteration on the causal diagonal: per-tile masks.
  auto masked_iteration = [&](int it, const uint8_t* kl, const uint8_t* vl, uint8_t* knext,
                              uint8_t* vnext) {
    const int key_base = it * kKeys;
    const int buf = it & 1;
    if (it + 1 < n_iters) stage(it + 1, knext, vnext, buf ^ 1);
#pragma unroll 1
    for (int h = 0; h < kBlocks; ++h) {
      if (key_base + 32 * h >= wave_count) break;  // wave-uniform
      float w[2][8], corr[2];
      bool big[2];
      const f32x16_t sb = qk(kl, h, buf);
      softmax_pair(sb, key_base + 32 * h, true, w, corr, big);
      fold_pv(vl, h, w, corr, big, buf);
    }
    iteration_end(it, vnext);
  };

  // Iterations whose keys are valid for every row of the block (the first
  // row's count bounds them; a partial block has none) run unmasked
  // straight-line code, in pairs so that each buffer is a fixed LDS object;
  // the remaining ones (the causal diagonal, and an odd one left over) the
  // masked per-tile code.  All waves of the block run the same iterations
  // and barriers.  Iteration it reads buffer it % 2.
  const int block_min = ntok == kPTokens ? base_pos + (t0 - buf_start) + 1 : 0;
  const int it_full = min(n_iters, block_min / kKeys) & ~1;
  int it = 0;
  // A staged iteration below it_full has every row below count_max, so with
  // pages of >= 16 rows it stages through stage_page.
  const bool pages16 = shift >= 4;
  for (; it < it_full; it += 2) {
    full_iteration(pages16, it, kbuf0, vbuf0, kbuf1, vbuf1);
    full_iteration(pages16 && it + 2 < it_full, it + 1, kbuf1, vbuf1, kbuf0, vbuf0);
  }
  for (; it < n_iters; ++it) {
    if (it & 1)
      masked_iteration(it, kbuf1, vbuf1, kbuf0, vbuf0);
    else
      masked_iteration(it, kbuf0, vbuf0, kbuf1, vbuf1);
  }

  // ---- one-segment merge and bf16 store (PrefillMergeKernel) ----
  // Lane l holds dims 32*b + 8*j + 4*half + i (value 4*j + i of block b).
  if (row_live) {
    const float c0 = l > 0.0f ? fexp(max_ref(-87.0f, m - m)) : 0.0f;
    const float gl = l * c0;
    const bool live = gl > 0.0f;
    const float inv_l = live ? 1.0f / gl : 0.0f;
    uint16_t* dst = out + (static_cast<int64_t>(tok) * num_q + head) * kPD + 4 * half;
#pragma unroll
    for (int b = 0; b < kDimBlocks; ++b) {
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

}  // namespace

hipError_t launch_prefill_full_mfma(const int32_t* image, int num_qblocks, const void* q,
                                    const void* k, const void* v, void* output, int num_q,
                                    int num_kv, int64_t kv_stride, PagedGeom geom,
                                    hipStream_t stream) {
  if (num_qblocks <= 0) return hipSuccess;
  hipLaunchKernelGGL(prefill_full_mfma_kernel<false>, dim3(num_qblocks * num_kv),
                     dim3(kPThreads), 0, stream, image, q, nullptr, nullptr, k, nullptr, v,
                     nullptr, static_cast<uint16_t*>(output), num_q, num_kv, kv_stride,
                     geom.shift, geom.row_mask);
  return hipGetLastError();
}

hipError_t launch_prefill_full_mfma_bq(const int32_t* image, int num_qblocks, const void* q_i8,
                                       const float* qi_bias, const float* f_q, const void* k,
                                       const float* k_scale, const void* v,
                                       const float* v_scale, void* output, int num_q,
                                       int num_kv, int64_t kv_stride, PagedGeom geom,
                                       hipStream_t stream) {
  if (num_qblocks <= 0) return hipSuccess;
  hipLaunchKernelGGL(prefill_full_mfma_kernel<true>, dim3(num_qblocks * num_kv),
                     dim3(kPThreads), 0, stream, image, q_i8, qi_bias, f_q, k, k_scale, v,
                     v_scale, static_cast<uint16_t*>(output), num_q, num_kv, kv_stride,
                     geom.shift, geom.row_mask);
  return hipGetLastError();
}

}  // namespace ifr
