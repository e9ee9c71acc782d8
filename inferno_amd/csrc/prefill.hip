// Chunked causal prefill over the paged cache with MFMA (gfx950), full
// attention.  Semantics: FlashPrefillFullKernel + PrefillMergeKernel
// (kernels/flash_attention_prefill.mojo:117-248) at degree 1 -- every query
// token t at absolute position p walks keys [0, p] in tiles of 16 from key 0
// with the online softmax of process_kv_tile (kernels/attention_ops.mojo:
// 165-253), then its one-segment merge (kernels/logsum_merge.mojo:28-122).
// Because all queries start at key 0 the tiles line up across queries, so a
// block of query tokens shares every K/V tile of its kv head.
//
// A row is one (query token, q head); a wave owns 16 rows = 8 tokens x the
// 2 q heads of one kv head; a block of 8 waves owns 64 tokens.  Each
// iteration stages 64 keys (4 tiles) in LDS and computes, per wave:
//
//   S^T (16 keys x 16 rows) = K_tile . Q^T, per tile     v_mfma_f32_16x16x32_bf16
//   O^T (16 dims x 16 rows) += V^T . P'^T, 32 keys/MFMA  v_mfma_f32_16x16x32_bf16
//
// In the MFMA C layout lane l holds keys 4*(l/16)..+3 of row l%16, and O^T
// keeps row l%16 in lane l, so the per-row softmax state stays lane-local.
// The reference's per-tile steps are kept in tile order: a row skips tiles
// past its position (the reference never visits them), pads of its last
// tile score -1e30 (their fexp(-87) enters l, not PV), and m, corr, w use
// the biased exp; l is updated tile by tile.  The accumulator rescales of
// a pair of tiles are folded: acc*c0*c1 + (w0*c1) V0 + w1 V1 equals the
// reference's nested (acc*c0 + w0 V0)*c1 + w1 V1 up to f32 rounding, and
// the product of the rescales is carried as a per-row scale S (acc =
// acc_stored * S) that divides the weights instead of multiplying the 64
// accumulators.  P' enters the bf16 MFMA as hi + lo bf16 parts (~16
// significant bits per weight); QK^T products are exact in f32.
//
// K and V tiles are staged row-major in LDS; V^T operands come from
// ds_read_b64_tr_b16 (a 16-lane transposing read).  The next iteration's
// keys are loaded into registers while the current one is computed; the
// run's page table is staged in LDS first.
// Blocks are numbered kv-head-fastest so every block of a kv head lands on
// one XCD (block id mod 8) and shares that XCD's L2.
#include "common.hpp"
#include "launch.hpp"

namespace ifr {
namespace {

typedef __bf16 bf16x8_t __attribute__((ext_vector_type(8)));
typedef short s16x4_t __attribute__((ext_vector_type(4)));
typedef short s16x8_t __attribute__((ext_vector_type(8)));
typedef float f32x4_t __attribute__((ext_vector_type(4)));
typedef __attribute__((address_space(3))) s16x4_t lds_s16x4_t;
typedef __bf16 bf16x2_t __attribute__((ext_vector_type(2)));
typedef float f32x2_t __attribute__((ext_vector_type(2)));

constexpr int kPD = 256;             // head_dim
constexpr int kPWaves = 8;           // waves per block (one block per CU)
constexpr int kPTokensPerWave = 8;   // x 2 q heads = 16 rows
constexpr int kPTokens = kPWaves * kPTokensPerWave;  // tokens per block
static_assert(kPTokens == kPrefillTokens, "plan query blocks must match the kernel");
constexpr int kKeys = 64;                // keys per iteration
constexpr int kTiles = kKeys / 16;       // 16-key tiles per iteration
constexpr int kHalves = kTiles / 2;      // 32-key MFMA operands per iteration
static_assert(kTiles % 2 == 0, "tiles pair up into 32-key MFMA operands");
constexpr int kKPitch = kPD * 2 + 16;    // bytes per K row in LDS: 132 dwords
constexpr int kVPitch = kPD * 2 + 32;    // bytes per V row in LDS: 136 dwords
constexpr int kKBytes = kKeys * kKPitch;
constexpr int kVBytes = kKeys * kVPitch;
constexpr int kBufBytes = kKBytes + kVBytes;
constexpr int kChunksPerThread = kKeys * kPD * 2 / 16 / (64 * kPWaves);  // of K and of V
static_assert(kChunksPerThread == 4, "staging layout");
constexpr int kKeyStep = kKeys / kChunksPerThread;  // keys between a thread's chunks

static_assert(kKeyStep * 32 == 64 * kPWaves, "32 lanes per key row");

// x + x[lane ^ 16] and x + x[lane ^ 32] through the gfx950 lane swaps: with
// both operands x, the two results hold the low and high member of each
// pair, so their sum (low + high) is the same in both lanes.
__device__ __forceinline__ float sum_xor16(float x) {
  const auto r = __builtin_amdgcn_permlane16_swap(__float_as_uint(x), __float_as_uint(x),
                                                  false, false);
  return __uint_as_float(r[0]) + __uint_as_float(r[1]);
}
__device__ __forceinline__ float sum_xor32(float x) {
  const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x),
                                                  false, false);
  return __uint_as_float(r[0]) + __uint_as_float(r[1]);
}
__device__ __forceinline__ float max_xor16(float x) {
  const auto r = __builtin_amdgcn_permlane16_swap(__float_as_uint(x), __float_as_uint(x),
                                                  false, false);
  return max_ref(__uint_as_float(r[0]), __uint_as_float(r[1]));
}
__device__ __forceinline__ float max_xor32(float x) {
  const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x),
                                                  false, false);
  return max_ref(__uint_as_float(r[0]), __uint_as_float(r[1]));
}

// One tile's online-softmax step for this lane's row (process_kv_tile's
// m / corr / w / l updates, attention_ops.mojo:165-180).  Masked: the tile
// reaches past some row's last key (or the row is empty); a row with no key
// in the tile is left untouched (corr 1, weights 0), pads score -1e30 and
// enter l only.  The in-lane sum of the 4 weights comes first, then the
// lanes ^16 and ^32 (the same 16 weights as the reference's halving tree,
// added in another order).
template <bool kMasked>
__device__ __forceinline__ void softmax_tile(const f32x4_t s, int valid, int key0, float& m,
                                             float& l, float& corr, float (&w)[4]) {
  float sc[4];
#pragma unroll
  for (int j = 0; j < 4; ++j) sc[j] = (!kMasked || key0 + j < valid) ? s[j] : kNegBig;
  float mx = max_ref(max_ref(sc[0], sc[1]), max_ref(sc[2], sc[3]));
  mx = max_xor16(mx);
  mx = max_xor32(mx);
  const float m_new = mx > m ? mx : m;
  const float c = fexp(max_ref(-87.0f, m - m_new));
  float e[4];
#pragma unroll
  for (int j = 0; j < 4; ++j) e[j] = fexp(max_ref(-87.0f, sc[j] - m_new));
  float ts = (e[0] + e[1]) + (e[2] + e[3]);
  ts = sum_xor16(ts);
  ts = sum_xor32(ts);
  if (kMasked) {
    const bool any = valid > 0;
    l = any ? l * c + ts : l;
    m = any ? m_new : m;
    corr = any ? c : 1.0f;
#pragma unroll
    for (int j = 0; j < 4; ++j) w[j] = key0 + j < valid ? e[j] : 0.0f;
  } else {
    l = l * c + ts;
    m = m_new;
    corr = c;
#pragma unroll
    for (int j = 0; j < 4; ++j) w[j] = e[j];
  }
}

// Two waves per SIMD (<= 256 VGPR + AGPR per lane); one block per CU.
__global__ __launch_bounds__(64 * kPWaves) __attribute__((amdgpu_waves_per_eu(2)))
void prefill_full_mfma_kernel(
    const int32_t* __restrict__ image, const uint16_t* __restrict__ q,
    const uint16_t* __restrict__ kc, const uint16_t* __restrict__ vc,
    uint16_t* __restrict__ out, int num_q, int num_kv, int64_t kv_stride,
    int shift, int row_mask) {
  __shared__ __align__(16) uint8_t lds[2 * kBufBytes];
  __shared__ int32_t page_rows[kPrefillLdsPages];
  const int tid = threadIdx.x;
  const int wave = tid >> 6;
  const int lane = tid & 63;
  const int grp = lane >> 4;   // key group within a tile / k group of the MFMA
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

  // This lane's row: token wave*8 + (l%16)/2, q head 2g + (l%16)%2.
  const int row = lane & 15;
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

  // Q^T fragments: lane holds Q[row][32c + 8*(l/16) .. +7] for chunks c.
  bf16x8_t qf[8];
  {
    const uint16_t* qr =
        q + (static_cast<int64_t>(row_live ? tok : t0) * num_q + head) * kPD + 8 * grp;
#pragma unroll
    for (int c = 0; c < 8; ++c) {
      const uint4 v = *reinterpret_cast<const uint4*>(qr + 32 * c);
      qf[c] = __builtin_bit_cast(bf16x8_t, v);
    }
  }

  // The O^T accumulator is kept as acc_stored with acc = acc_stored * S: a
  // tile's rescale multiplies S, and the weights entering the MFMA are
  // divided by the new S, so the 64 accumulators are not rescaled per
  // iteration.  When S would fall below 2^-64 the accumulators take it over
  // (acc_stored *= S, S = 1) for the whole wave.
  f32x4_t acc[16];
#pragma unroll
  for (int b = 0; b < 16; ++b) acc[b] = f32x4_t{0.0f, 0.0f, 0.0f, 0.0f};
  float m = kNegBig, l = 0.0f, S = 1.0f;

  // The run's page table, staged once (the host routes runs with more than
  // kPrefillLdsPages pages elsewhere): the K/V loads of an iteration then
  // wait on an LDS read rather than on a global load.
  const int n_pages = count_max > 0 ? ((count_max - 1) >> shift) + 1 : 0;
  for (int i = tid; i < n_pages; i += 64 * kPWaves) page_rows[i] = rows[i];
  __syncthreads();

  // Staging of one iteration: kKeys keys x 512 B of K and of V, 16-byte
  // chunks; thread tid takes dims 8*(tid%32) of keys tid/32 + kKeyStep*r
  // (32 consecutive lanes read one key's 512 contiguous bytes).  Keys past
  // count_max read the last key (in bounds) and are stored as zeros.
  const uint16_t* kbase = kc + static_cast<int64_t>(g) * kPD;
  const uint16_t* vbase = vc + static_cast<int64_t>(g) * kPD;
  const int ckey = tid >> 5, cd0 = 8 * (tid & 31);
  uint4 kreg[kChunksPerThread], vreg[kChunksPerThread];
  uint32_t in_range = 0;  // bit r: chunk r holds a key below count_max
  // All page-table reads first, then all K/V loads: no load waits on
  // another, and the zero fill of keys past count_max happens at the LDS
  // store, when the loaded data is needed anyway.
  auto gload = [&](int it) {
    int32_t page_row[kChunksPerThread];
    in_range = 0;
#pragma unroll
    for (int r = 0; r < kChunksPerThread; ++r) {
      const int key = it * kKeys + ckey + kKeyStep * r;
      in_range |= (key < count_max ? 1u : 0u) << r;
      const int kk = min(key, count_max - 1);
      page_row[r] = kk;
    }
#pragma unroll
    for (int r = 0; r < kChunksPerThread; ++r) page_row[r] = page_rows[page_row[r] >> shift];
#pragma unroll
    for (int r = 0; r < kChunksPerThread; ++r) {
      const int kk = min(it * kKeys + ckey + kKeyStep * r, count_max - 1);
      const int64_t slot = static_cast<int64_t>(page_row[r]) + (kk & row_mask);
      const int64_t off = slot * kv_stride + cd0;
      kreg[r] = *reinterpret_cast<const uint4*>(kbase + off);
      vreg[r] = *reinterpret_cast<const uint4*>(vbase + off);
    }
  };
  auto lstore = [&](int buf) {
    uint8_t* kl = lds + buf * kBufBytes;
    uint8_t* vl = kl + kKBytes;
#pragma unroll
    for (int r = 0; r < kChunksPerThread; ++r) {
      const uint32_t keep = ((in_range >> r) & 1u) ? 0xFFFFFFFFu : 0u;
      const uint4 kv = make_uint4(kreg[r].x & keep, kreg[r].y & keep, kreg[r].z & keep,
                                  kreg[r].w & keep);
      const uint4 vv = make_uint4(vreg[r].x & keep, vreg[r].y & keep, vreg[r].z & keep,
                                  vreg[r].w & keep);
      *reinterpret_cast<uint4*>(kl + (ckey + kKeyStep * r) * kKPitch + 2 * cd0) = kv;
      *reinterpret_cast<uint4*>(vl + (ckey + kKeyStep * r) * kVPitch + 2 * cd0) = vv;
    }
  };

  if (n_iters > 0) {
    gload(0);
    lstore(0);
  }
  if (n_iters > 1) gload(1);
  __syncthreads();

  // Transposing-read address of this lane inside a 16-key tile of V: lane
  // R = l%16 of group grp addresses key 4*grp + R/4, dims 4*(R%4) .. +3;
  // the read returns, in lane R, keys 4*grp .. +3 of dim R (per 16 dims).
  const int tr_off = (4 * grp + (row >> 2)) * kVPitch + 8 * (row & 3);
  const int key0 = 4 * grp;
  // Settle every load issued so far (the Q fragments among them) before the
  // loop, so that the loop's own waits track only the K/V prefetch and the
  // prefetch stays in flight across a whole iteration.
  __builtin_amdgcn_s_waitcnt(0);

  for (int it = 0; it < n_iters; ++it) {
    const int buf = it & 1;
    const uint8_t* kl = lds + buf * kBufBytes;
    const uint8_t* vl = kl + kKBytes;
    const int key_base = it * kKeys;

    if (key_base < wave_count) {
      // ---- S^T for the 4 tiles ----
      f32x4_t s[kTiles];
#pragma unroll
      for (int t = 0; t < kTiles; ++t) {
        s[t] = f32x4_t{0.0f, 0.0f, 0.0f, 0.0f};
        if (key_base + 16 * t < wave_count) {
#pragma unroll
          for (int c = 0; c < 8; ++c) {
            const uint4 kv = *reinterpret_cast<const uint4*>(
                kl + (16 * t + row) * kKPitch + 64 * c + 16 * grp);
            s[t] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8_t, kv),
                                                           qf[c], s[t], 0, 0, 0);
          }
        }
      }
      // ---- per pair of tiles: online softmax, fold, acc_stored += V^T P''^T ----
      // The pair's MFMAs depend only on its own tiles, so they run while
      // the next pair's softmax is computed.
#pragma unroll
      for (int h = 0; h < kHalves; ++h) {
        if (key_base + 32 * h >= wave_count) continue;  // wave-uniform
        float w[2][4];
        float corr[2];
#pragma unroll
        for (int u = 0; u < 2; ++u) {
          const int t = 2 * h + u;
          const int tile_key0 = key_base + 16 * t;
          corr[u] = 1.0f;
#pragma unroll
          for (int j = 0; j < 4; ++j) w[u][j] = 0.0f;
          if (tile_key0 < wave_count) {  // wave-uniform
            if (tile_key0 + 16 <= wave_min) {
              softmax_tile<false>(s[t], 16, key0, m, l, corr[u], w[u]);
            } else {
              const int valid = min(16, max(0, count - tile_key0));
              softmax_tile<true>(s[t], valid, key0, m, l, corr[u], w[u]);
            }
          }
        }
        // acc*c_a*c_b + w_a*c_b V_a + w_b V_b = S' (acc_stored + (w_a*c_b V_a +
        // w_b V_b) / S'),  S' = S*c_a*c_b.
        float S_new = S * (corr[0] * corr[1]);
        if (__builtin_amdgcn_ballot_w64(S_new < 0x1p-64f) != 0) {  // wave-uniform
#pragma unroll
          for (int b = 0; b < 16; ++b) acc[b] = acc[b] * S_new;
          S_new = 1.0f;
        }
        S = S_new;
        const float inv_s = 1.0f / S_new;
        const float fs[2] = {corr[1] * inv_s, inv_s};
        // P''^T as bf16 hi + lo: k index 8*grp + i holds tile a key 4*grp + i
        // (i < 4), tile b key 4*grp + i - 4 (i >= 4), the order the V^T
        // reads below produce.
        bf16x8_t phi, plo;
#pragma unroll
        for (int i = 0; i < 8; i += 2) {
          const int u = i >> 2;
          const float p0 = w[u][i & 3] * fs[u];
          const float p1 = w[u][(i & 3) + 1] * fs[u];
          const bf16x2_t hb = __builtin_convertvector(f32x2_t{p0, p1}, bf16x2_t);
          const float r0 = p0 - static_cast<float>(hb[0]);
          const float r1 = p1 - static_cast<float>(hb[1]);
          const bf16x2_t lb = __builtin_convertvector(f32x2_t{r0, r1}, bf16x2_t);
          phi[i] = hb[0];
          phi[i + 1] = hb[1];
          plo[i] = lb[0];
          plo[i + 1] = lb[1];
        }
#pragma unroll
        for (int b = 0; b < 16; ++b) {
          const uint8_t* va = vl + (32 * h) * kVPitch + tr_off + 32 * b;
          const s16x4_t v0 = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_s16x4_t*)(va));
          const s16x4_t v1 =
              __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_s16x4_t*)(va + 16 * kVPitch));
          const s16x8_t a8 = __builtin_shufflevector(v0, v1, 0, 1, 2, 3, 4, 5, 6, 7);
          const bf16x8_t av = __builtin_bit_cast(bf16x8_t, a8);
          acc[b] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(av, phi, acc[b], 0, 0, 0);
          acc[b] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(av, plo, acc[b], 0, 0, 0);
        }
      }
    }
    if (it + 1 < n_iters) {
      lstore(buf ^ 1);
      if (it + 2 < n_iters) gload(it + 2);
    }
    __syncthreads();
  }

  // ---- one-segment merge and bf16 store (PrefillMergeKernel) ----
  if (row_live) {
    const float c0 = l > 0.0f ? fexp(max_ref(-87.0f, m - m)) : 0.0f;
    const float gl = l * c0;
    const bool live = gl > 0.0f;
    const float inv_l = live ? 1.0f / gl : 0.0f;
    uint16_t* dst = out + (static_cast<int64_t>(tok) * num_q + head) * kPD + 4 * grp;
#pragma unroll
    for (int b = 0; b < 16; ++b) {
      uint32_t e[4];
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        const float av = (acc[b][j] * S) * c0;
        e[j] = live ? f32_to_bf16_bits(av * inv_l) : 0u;
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
                     0, stream, image, static_cast<const uint16_t*>(q),
                     static_cast<const uint16_t*>(k), static_cast<const uint16_t*>(v),
                     static_cast<uint16_t*>(output), num_q, num_kv, kv_stride, geom.shift,
                     geom.row_mask);
  return hipGetLastError();
}

}  // namespace ifr
