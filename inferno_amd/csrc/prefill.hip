// Chunked causal prefill over the paged cache with MFMA (gfx950), full
// attention.  Semantics: FlashPrefillFullKernel + PrefillMergeKernel
// (kernels/flash_attention_prefill.mojo:117-248) at degree 1 -- every query
// token t at absolute position p walks keys [0, p] in tiles of 16 from key 0
// with the online softmax of process_kv_tile (kernels/attention_ops.mojo:
// 165-253), then its one-segment merge (kernels/logsum_merge.mojo:28-122).
// Because all queries start at key 0 the tiles line up across queries, so a
// block of queries can share each K/V tile:
//
//   S^T (16 keys x 16 rows) = K_tile (16 x 256) . Q^T      v_mfma_f32_16x16x32_bf16
//   O^T (16 dims x 16 rows) += V^T (16 x 16 keys) . P^T    v_mfma_f32_16x16x16_bf16
//
// A row is one (query token, q head); a wave owns 16 rows = 8 tokens x the
// 2 q heads of one kv head.  In the MFMA C layout lane l holds keys
// 4*(l/16)..+3 of row l%16, which is also the B layout P^T needs, and the
// O^T accumulator keeps row l%16 in lane l, so the per-row softmax state and
// the per-tile rescale stay lane-local.  Per row and tile the reference's
// steps are kept: a row skips tiles past its position (the reference never
// visits them), pads of its last tile score -1e30 (their fexp(-87) enters l,
// not PV), m/corr/w use the biased exp, and the 16 weights are summed by the
// halving tree (key ^8 = lane ^32, ^4 = lane ^16, ^2 and ^1 inside the lane).
// P is fed to the bf16 MFMA as hi + lo bf16 parts, so the products carry ~16
// significant bits of each weight; QK^T products are exact in f32.
//
// K/V tiles are gathered through the page table into LDS (K row-major, V
// transposed) with one barrier per tile; the next tile's global loads are in
// flight while the current tile is computed.  Blocks are numbered
// kv-head-fastest so every block of a kv head lands on one XCD (block id mod
// 8) and shares that XCD's L2.
#include "common.hpp"
#include "launch.hpp"

namespace ifr {
namespace {

typedef __bf16 bf16x8_t __attribute__((ext_vector_type(8)));
typedef short s16x4_t __attribute__((ext_vector_type(4)));
typedef float f32x4_t __attribute__((ext_vector_type(4)));

constexpr int kPD = 256;             // head_dim
constexpr int kPWaves = 8;           // waves per block
constexpr int kPTokensPerWave = 8;   // x 2 q heads = 16 rows
constexpr int kPTokens = kPWaves * kPTokensPerWave;  // tokens per block
static_assert(kPTokens == kPrefillTokens, "plan query blocks must match the kernel");
constexpr int kKPitch = kPD * 2 + 16;   // bytes per K row in LDS (padded)
constexpr int kVPitch = 16 * 2 + 8;     // bytes per V^T dim row in LDS (padded)
constexpr int kKBytes = 16 * kKPitch;
constexpr int kVBytes = kPD * kVPitch;
constexpr int kBufBytes = kKBytes + kVBytes;

__device__ __forceinline__ uint32_t bf16_rne_bits(float f) { return f32_to_bf16_bits(f); }

// Two waves per SIMD (<= 256 VGPR + AGPR per lane).
__global__ __launch_bounds__(64 * kPWaves) __attribute__((amdgpu_waves_per_eu(2)))
void prefill_full_mfma_kernel(
    const int32_t* __restrict__ image, const uint16_t* __restrict__ q,
    const uint16_t* __restrict__ kc, const uint16_t* __restrict__ vc,
    uint16_t* __restrict__ out, int num_q, int num_kv, int64_t kv_stride,
    int shift, int row_mask) {
  extern __shared__ __align__(16) uint8_t lds[];
  const int tid = threadIdx.x;
  const int wave = tid >> 6;
  const int lane = tid & 63;
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
  const int n_tiles = (count_max + 15) >> 4;

  // This lane's row: token wave*8 + (l%16)/2, q head 2g + (l%16)%2.
  const int row = lane & 15;
  const int tok_local = wave * kPTokensPerWave + (row >> 1);
  const int head = g * 2 + (row & 1);
  const bool row_live = tok_local < ntok;
  const int tok = t0 + tok_local;
  const int count = row_live ? base_pos + (tok - buf_start) + 1 : 0;
  const int wave_last = min(ntok, (wave + 1) * kPTokensPerWave) - 1;
  const int wave_count =
      wave * kPTokensPerWave < ntok ? base_pos + (t0 + wave_last - buf_start) + 1 : 0;

  // Q^T fragments: lane holds Q[row][32c + 8*(l/16) .. +7] for chunks c.
  bf16x8_t qf[8];
  {
    const uint16_t* qr =
        q + (static_cast<int64_t>(row_live ? tok : t0) * num_q + head) * kPD + 8 * (lane >> 4);
#pragma unroll
    for (int c = 0; c < 8; ++c) {
      const uint4 v = *reinterpret_cast<const uint4*>(qr + 32 * c);
      qf[c] = __builtin_bit_cast(bf16x8_t, v);
    }
  }

  f32x4_t acc[16];
#pragma unroll
  for (int b = 0; b < 16; ++b) acc[b] = f32x4_t{0.0f, 0.0f, 0.0f, 0.0f};
  float m = kNegBig, l = 0.0f;

  // Global -> register staging of one tile: 16 keys x 512 B of K and of V =
  // 512 chunks of 16 B each; thread tid takes chunk tid of K and of V.  Chunk
  // c -> key c/32, dims 8*(c%32) .. +7.  Two register sets keep the loads of
  // tiles j+1 and j+2 in flight while tile j is computed from LDS.
  static_assert(kPWaves * 64 == 512, "one 16-byte chunk of K and V per thread");
  const uint16_t* kbase = kc + static_cast<int64_t>(g) * kPD;
  const uint16_t* vbase = vc + static_cast<int64_t>(g) * kPD;
  const int ckey = tid >> 5, cd0 = 8 * (tid & 31);
  uint4 kreg[2], vreg[2];
  auto gload = [&](int tile, int set) {
    const int key = tile * 16 + ckey;
    if (key < count_max) {
      const int64_t slot = static_cast<int64_t>(rows[key >> shift]) + (key & row_mask);
      const int64_t off = slot * kv_stride + cd0;
      kreg[set] = *reinterpret_cast<const uint4*>(kbase + off);
      vreg[set] = *reinterpret_cast<const uint4*>(vbase + off);
    } else {
      kreg[set] = make_uint4(0, 0, 0, 0);
      vreg[set] = make_uint4(0, 0, 0, 0);
    }
  };
  auto lstore = [&](int buf, int set) {
    uint8_t* kl = lds + buf * kBufBytes;
    uint8_t* vl = kl + kKBytes;
    *reinterpret_cast<uint4*>(kl + ckey * kKPitch + 2 * cd0) = kreg[set];
    const uint32_t w[4] = {vreg[set].x, vreg[set].y, vreg[set].z, vreg[set].w};
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      *reinterpret_cast<uint16_t*>(vl + (cd0 + 2 * e) * kVPitch + 2 * ckey) =
          static_cast<uint16_t>(w[e] & 0xFFFFu);
      *reinterpret_cast<uint16_t*>(vl + (cd0 + 2 * e + 1) * kVPitch + 2 * ckey) =
          static_cast<uint16_t>(w[e] >> 16);
    }
  };

  if (n_tiles > 0) {
    gload(0, 0);
    lstore(0, 0);
  }
  if (n_tiles > 1) gload(1, 1);
  __syncthreads();

  for (int tile = 0; tile < n_tiles; ++tile) {
    const int buf = tile & 1;
    // set (tile+1)&1 holds tile+1 (issued last iteration); reuse set tile&1
    // for tile+2.
    if (tile + 2 < n_tiles) gload(tile + 2, tile & 1);
    const uint8_t* kl = lds + buf * kBufBytes;
    const uint8_t* vl = kl + kKBytes;

    if (tile * 16 < wave_count) {
      // ---- S^T = K . Q^T ----
      f32x4_t s = f32x4_t{0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
      for (int c = 0; c < 8; ++c) {
        const uint4 kv = *reinterpret_cast<const uint4*>(kl + row * kKPitch + 64 * c +
                                                         16 * (lane >> 4));
        s = __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8_t, kv), qf[c],
                                                    s, 0, 0, 0);
      }
      // ---- online softmax of this tile for row (lane & 15) ----
      const int valid = min(16, max(0, count - tile * 16));
      const int key0 = 4 * (lane >> 4);
      float sc[4];
#pragma unroll
      for (int j = 0; j < 4; ++j) sc[j] = key0 + j < valid ? s[j] : kNegBig;
      float mx = max_ref(max_ref(sc[0], sc[1]), max_ref(sc[2], sc[3]));
      mx = max_ref(mx, shfl_xor_f32(mx, 16));
      mx = max_ref(mx, shfl_xor_f32(mx, 32));
      float corr = 1.0f;
      float w[4] = {0.0f, 0.0f, 0.0f, 0.0f};
      if (valid > 0) {
        const float m_new = mx > m ? mx : m;
        corr = fexp(max_ref(-87.0f, m - m_new));
#pragma unroll
        for (int j = 0; j < 4; ++j) w[j] = fexp(max_ref(-87.0f, sc[j] - m_new));
        float a[4];
#pragma unroll
        for (int j = 0; j < 4; ++j) a[j] = w[j] + shfl_xor_f32(w[j], 32);  // key ^ 8
#pragma unroll
        for (int j = 0; j < 4; ++j) a[j] = a[j] + shfl_xor_f32(a[j], 16);  // key ^ 4
        const float t0s = a[0] + a[2];                                      // key ^ 2
        const float t1s = a[1] + a[3];
        const float ts = t0s + t1s;                                         // key ^ 1
        const float lc = l * corr;
        l = lc + ts;
        m = m_new;
#pragma unroll
        for (int j = 0; j < 4; ++j)
          if (key0 + j >= valid) w[j] = 0.0f;  // pads enter l only
      }
      // ---- P^T as bf16 hi + lo ----
      uint32_t hi[4], lo[4];
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        hi[j] = bf16_rne_bits(w[j]);
        lo[j] = bf16_rne_bits(w[j] - __uint_as_float(hi[j] << 16));
      }
      const s16x4_t phi = s16x4_t{static_cast<short>(hi[0]), static_cast<short>(hi[1]),
                                  static_cast<short>(hi[2]), static_cast<short>(hi[3])};
      const s16x4_t plo = s16x4_t{static_cast<short>(lo[0]), static_cast<short>(lo[1]),
                                  static_cast<short>(lo[2]), static_cast<short>(lo[3])};
      // ---- O^T = O^T * corr + V^T . P^T ----
#pragma unroll
      for (int b = 0; b < 16; ++b) {
        acc[b] = acc[b] * corr;
        const uint2 vv = *reinterpret_cast<const uint2*>(vl + (16 * b + row) * kVPitch +
                                                         8 * (lane >> 4));
        const s16x4_t va = __builtin_bit_cast(s16x4_t, vv);
        acc[b] = __builtin_amdgcn_mfma_f32_16x16x16bf16_1k(va, phi, acc[b], 0, 0, 0);
        acc[b] = __builtin_amdgcn_mfma_f32_16x16x16bf16_1k(va, plo, acc[b], 0, 0, 0);
      }
    }
    if (tile + 1 < n_tiles) lstore(buf ^ 1, (tile + 1) & 1);
    __syncthreads();
  }

  // ---- one-segment merge and bf16 store (PrefillMergeKernel) ----
  if (row_live) {
    const float c0 = l > 0.0f ? fexp(max_ref(-87.0f, m - m)) : 0.0f;
    const float gl = l * c0;
    const bool live = gl > 0.0f;
    const float inv_l = live ? 1.0f / gl : 0.0f;
    uint16_t* dst = out + (static_cast<int64_t>(tok) * num_q + head) * kPD + 4 * (lane >> 4);
#pragma unroll
    for (int b = 0; b < 16; ++b) {
      uint32_t e[4];
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        const float a = acc[b][j] * c0;
        e[j] = live ? f32_to_bf16_bits(a * inv_l) : 0u;
      }
      *reinterpret_cast<uint2*>(dst + 16 * b) = make_uint2(e[0] | (e[1] << 16), e[2] | (e[3] << 16));
    }
  }
}

}  // namespace

hipError_t launch_prefill_full_mfma(const int32_t* image, int num_qblocks, const void* q,
                                    const void* k, const void* v, void* output, int num_q,
                                    int num_kv, int64_t kv_stride, PagedGeom geom,
                                    hipStream_t stream) {
  if (num_qblocks <= 0) return hipSuccess;
  hipLaunchKernelGGL(prefill_full_mfma_kernel, dim3(num_qblocks * num_kv), dim3(64 * kPWaves),
                     2 * kBufBytes, stream, image, static_cast<const uint16_t*>(q),
                     static_cast<const uint16_t*>(k), static_cast<const uint16_t*>(v),
                     static_cast<uint16_t*>(output), num_q, num_kv, kv_stride, geom.shift,
                     geom.row_mask);
  return hipGetLastError();
}

}  // namespace ifr
