// MiniMax-M3 block-sparse paged attention at degree 1 (prototypes/
// lightning_indexer.mojo, prototypes/sparse_attention.mojo): the lightning
// indexer scores every 128-position block of each token's causal context,
// keeps the top 16 blocks per index head, and the attention walks only those
// blocks.  The run table, page table and token->run map come from a
// full-attention plan image (ifr_plan_attention).
//
// index_scores_kernel   one wave per (token, block): each lane takes one index
//                       head and whole positions, and forms the dots in the
//                       reference's VDPBF16PS order, so block scores, and with
//                       them the selected blocks, are bit-identical.
// select_blocks_kernel  one wave per (token, index head): the reference's
//                       32-slot streaming bank, each reduction done as a rank
//                       count under reduce_argmax's order (value, then slot
//                       lane, then slot register).
// sparse_attention_kernel  one wave per (token, kv head): S = K.Q^T for the 16
//                       q heads of the kv head on MFMA, the reference's
//                       per-tile online softmax, P.V in f32 in position order,
//                       and the one-stripe finalisation.
#include "common.hpp"
#include "launch.hpp"

namespace ifr {
namespace {

typedef __bf16 bf16x8_t __attribute__((ext_vector_type(8)));
typedef float f32x4_t __attribute__((ext_vector_type(4)));

struct TokenPos {
  int abs_pos;
  const int32_t* rows;
};

__device__ __forceinline__ TokenPos token_position(const int32_t* image, int t) {
  const int run = image[image[kHdrOffTokRun] + t];
  const int32_t* rp = image + image[kHdrOffRuns] + run * 4;
  return TokenPos{rp[1] + (t - rp[0]), image + image[kHdrOffRows] + rp[2]};
}

// ---------------------------------------------------------------------------
// IndexBlockScoreKernel (lightning_indexer.mojo:134-202).  Dots of the index
// key with each head's query follow bf16_panel_dot_to_scalars with
// port_unroll = D/32 (one strip of D): accumulator (p, j) takes the pair
// (32p + 2j + 1, 32p + 2j) as odd*odd + even*even, lane j sums its
// accumulators p = 0.. in order, then the 16-lane halving tree.
// ---------------------------------------------------------------------------
template <int D, int H>
__global__ __launch_bounds__(256) void index_scores_kernel(
    const int32_t* __restrict__ image, const uint16_t* __restrict__ index_q,
    const uint16_t* __restrict__ index_k, float* __restrict__ scores, int block_stride,
    int block_size, float scale, int shift, int row_mask) {
  static_assert(64 % H == 0, "heads must divide the wave");
  constexpr int kP = D / 32;        // port-unroll accumulators, one strip
  constexpr int kLanes = 64 / H;    // positions a pass
  const int wave = threadIdx.x >> 6;
  const int lane = threadIdx.x & 63;
  const int head = lane / kLanes;   // lane = (head, position)
  const int sub = lane % kLanes;
  const int t = blockIdx.y;
  const int b = blockIdx.x * 4 + wave;
  const TokenPos tp = token_position(image, t);
  const int nb = min(tp.abs_pos / block_size + 1, block_stride);
  if (b >= nb) return;
  const int lo = b * block_size;
  const int hi = min(lo + block_size, tp.abs_pos + 1);

  uint32_t qp[D / 2];  // this lane's head query, bf16 pairs
  {
    const uint4* qr = reinterpret_cast<const uint4*>(
        index_q + (static_cast<int64_t>(t) * H + head) * D);
#pragma unroll
    for (int c = 0; c < D / 8; ++c) {
      const uint4 v = qr[c];
      qp[4 * c] = v.x;
      qp[4 * c + 1] = v.y;
      qp[4 * c + 2] = v.z;
      qp[4 * c + 3] = v.w;
    }
  }
  float best = kNegBig;
  for (int pos = lo + sub; pos < hi; pos += kLanes) {
    const int64_t slot = static_cast<int64_t>(tp.rows[pos >> shift]) + (pos & row_mask);
    const uint4* kr = reinterpret_cast<const uint4*>(index_k + slot * D);
    float s[16];
#pragma unroll
    for (int p = 0; p < kP; ++p) {
      uint32_t kp[16];
#pragma unroll
      for (int c = 0; c < 4; ++c) {
        const uint4 v = kr[4 * p + c];
        kp[4 * c] = v.x;
        kp[4 * c + 1] = v.y;
        kp[4 * c + 2] = v.z;
        kp[4 * c + 3] = v.w;
      }
#pragma unroll
      for (int j = 0; j < 16; ++j) {
        const uint32_t q2 = qp[16 * p + j];
        // bf16 products are exact in f32, so the fma rounds (odd + even) once.
        const float odd = bf16_hi(kp[j]) * bf16_hi(q2);
        const float a = fmaf(bf16_lo(kp[j]), bf16_lo(q2), odd);
        s[j] = p == 0 ? a : s[j] + a;
      }
    }
#pragma unroll
    for (int w = 8; w >= 1; w >>= 1) {
#pragma unroll
      for (int j = 0; j < w; ++j) s[j] = s[j] + s[j + w];
    }
    const float sh = s[0] * scale;
    best = sh > best ? sh : best;
  }
#pragma unroll
  for (int msk = 1; msk < kLanes; msk <<= 1) best = fmaxf(best, shfl_xor_f32(best, msk));
  if (sub == 0) scores[(static_cast<int64_t>(t) * H + head) * block_stride + b] = best;
}

// ---------------------------------------------------------------------------
// stream_select_blocks (lightning_indexer.mojo:48-126) per (token, head) row.
// Lane s < cap holds bank slot s.  reduce_top_k's successive argmax passes
// (matrixops.mojo:125-218) pick slots in one total order -- larger value,
// then smaller lane s % 16, then smaller register s / 16 -- so a slot's
// selection index is the number of slots ahead of it in that order.
// ---------------------------------------------------------------------------
__device__ __forceinline__ int bank_rank(float v, int slot, int cap) {
  const int key = (slot & 15) * 64 + (slot >> 4);
  int rank = 0;
  for (int s2 = 0; s2 < cap; ++s2) {
    const float v2 = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), s2));
    const int key2 = (s2 & 15) * 64 + (s2 >> 4);
    rank += (v2 > v || (v2 == v && key2 < key)) ? 1 : 0;
  }
  return rank;
}

__global__ __launch_bounds__(256) void select_blocks_kernel(
    const int32_t* __restrict__ image, const float* __restrict__ scores,
    int32_t* __restrict__ block_idx, int block_stride, int num_heads, int block_size,
    int topk, int local_blocks, int init_blocks, int cap, int num_rows) {
  __shared__ float bank_v[4][64];
  __shared__ int bank_b[4][64];
  const int wave = threadIdx.x >> 6;
  const int lane = threadIdx.x & 63;
  const int row = blockIdx.x * 4 + wave;
  if (row >= num_rows) return;
  const int t = row / num_heads;
  const TokenPos tp = token_position(image, t);
  const int nb = min(tp.abs_pos / block_size + 1, block_stride);
  const float* sr = scores + static_cast<int64_t>(row) * block_stride;
  const int local_start = max(nb - local_blocks, 0);

  float v = kNegBig;
  int id = -1;
  int fill = 0;
  for (int b = 0; b < nb;) {
    const int n_new = min(cap - fill, nb - b);
    if (lane >= fill && lane < fill + n_new) {
      const int blk = b + lane - fill;
      v = (blk >= local_start || blk < init_blocks) ? 1.0e30f : sr[blk];
      id = blk;
    }
    fill += n_new;
    b += n_new;
    if (fill == cap) {
      // Keep the top `topk` slots, in selection order, in slots 0..topk-1.
      const int rank = bank_rank(v, lane, cap);
      bank_v[wave][lane] = kNegBig;
      bank_b[wave][lane] = -1;
      __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
      __builtin_amdgcn_wave_barrier();
      __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
      if (lane < cap && rank < topk) {
        bank_v[wave][rank] = v;
        bank_b[wave][rank] = id;
      }
      __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
      __builtin_amdgcn_wave_barrier();
      __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
      v = bank_v[wave][lane];
      id = bank_b[wave][lane];
      __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
      __builtin_amdgcn_wave_barrier();
      __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
      fill = topk;
    }
  }
  const int rank = bank_rank(v, lane, cap);
  const bool sel = lane < cap && rank < topk && v > kNegBig;
  const uint64_t mask = __ballot(sel);
  const int count = __popcll(mask);
  int32_t* out = block_idx + static_cast<int64_t>(row) * topk;
  if (sel) {
    // Ids are distinct: the output slot is the number of selected ids below.
    int below = 0;
    for (int s2 = 0; s2 < cap; ++s2) {
      const int id2 = __builtin_amdgcn_readlane(id, s2);
      const bool sel2 = (mask >> s2) & 1ull;
      below += (sel2 && id2 < id) ? 1 : 0;
    }
    out[below] = id;
  }
  if (lane >= count && lane < topk) out[lane] = -1;
}

// ---------------------------------------------------------------------------
// BlockSparseFlashKernel (sparse_attention.mojo:58-125) + the one-stripe
// write_finalized_head of PrefillMergeKernel (flash_attention_prefill.mojo:
// 221-240), for head_dim 128 and 16 q heads per kv head.
//
// Scores: v_mfma_f32_16x16x32_bf16 with A = the tile's 16 keys x 32 dims and
// B = the 16 queries' dims, so lane l holds S[pos 4*(l/16)+j][head l%16].
// Softmax per tile follows online_softmax_tile with the biased exp; the tile
// weight sum uses the 16-position halving tree (xor 32, xor 16, then in-lane).
// P.V: lane l owns dims 2l, 2l+1 of all 16 heads and adds w*v in position
// order, as process_kv_tile's fma chain does per element.
// ---------------------------------------------------------------------------
constexpr int kSD = 128;  // head_dim
constexpr int kSG = 16;   // q heads per kv head

__global__ __launch_bounds__(256) void sparse_attention_kernel(
    const int32_t* __restrict__ image, const uint16_t* __restrict__ q,
    const uint16_t* __restrict__ k_base, const uint16_t* __restrict__ v_base,
    const int32_t* __restrict__ block_idx, uint16_t* __restrict__ out, int64_t kv_stride,
    int num_q, int num_kv, int block_size, int topk, int shift, int row_mask, int num_rows) {
  const int wave = threadIdx.x >> 6;
  const int lane = threadIdx.x & 63;
  const int row = blockIdx.x * 4 + wave;
  if (row >= num_rows) return;
  const int t = row / num_kv;
  const int h = row - t * num_kv;
  const TokenPos tp = token_position(image, t);
  const int64_t cap = static_cast<int64_t>(tp.abs_pos) + 1;
  const int r16 = lane & 15;
  const int g = lane >> 4;

  // B operand: Q[head r16][32c + 8g .. +8] for c = 0..3.
  bf16x8_t qf[4];
  {
    const uint16_t* qrow =
        q + (static_cast<int64_t>(t) * num_q + h * kSG + r16) * kSD + 8 * g;
#pragma unroll
    for (int c = 0; c < 4; ++c)
      qf[c] = __builtin_bit_cast(bf16x8_t, *reinterpret_cast<const uint4*>(qrow + 32 * c));
  }
  const uint16_t* kh = k_base + static_cast<int64_t>(h) * kSD;
  const uint16_t* vh = v_base + static_cast<int64_t>(h) * kSD + 2 * lane;

  float m = kNegBig;     // state of head r16 (same in the 4 lanes of the head)
  float lsum = 0.0f;
  float acc[kSG][2];     // dims 2*lane, 2*lane+1 of every head
#pragma unroll
  for (int hh = 0; hh < kSG; ++hh) acc[hh][0] = acc[hh][1] = 0.0f;

  const int32_t* brow = block_idx + static_cast<int64_t>(row) * topk;
  for (int s = 0; s < topk; ++s) {
    const int b = brow[s];
    if (b < 0) break;
    const int64_t plo = static_cast<int64_t>(b) * block_size;
    const int64_t phi = min(plo + block_size, cap);
    for (int64_t pos = plo; pos < phi; pos += kTile) {
      const int tl = static_cast<int>(min<int64_t>(kTile, phi - pos));
      // K: row pos + r16 (a pad row repeats pos and is masked below).
      const int pk = static_cast<int>(pos) + (r16 < tl ? r16 : 0);
      const int64_t kslot = static_cast<int64_t>(tp.rows[pk >> shift]) + (pk & row_mask);
      const uint16_t* kp = kh + kslot * kv_stride + 8 * g;
      f32x4_t sc = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
      for (int c = 0; c < 4; ++c) {
        const bf16x8_t kf = __builtin_bit_cast(bf16x8_t, *reinterpret_cast<const uint4*>(kp + 32 * c));
        sc = __builtin_amdgcn_mfma_f32_16x16x32_bf16(kf, qf[c], sc, 0, 0, 0);
      }
      // V rows of the tile: 4 bytes (2 dims) each.
      uint32_t vv[kTile];
#pragma unroll
      for (int j = 0; j < kTile; ++j) {
        const int pj = static_cast<int>(pos) + (j < tl ? j : 0);
        const int64_t vslot = static_cast<int64_t>(tp.rows[pj >> shift]) + (pj & row_mask);
        vv[j] = *reinterpret_cast<const uint32_t*>(vh + vslot * kv_stride);
      }
      // Scores of pad positions are -1e30 (they enter l through fexp(-87)).
      float sj[4];
#pragma unroll
      for (int j = 0; j < 4; ++j) sj[j] = (4 * g + j < tl) ? sc[j] : kNegBig;
      float tmax = max_ref(max_ref(sj[0], sj[1]), max_ref(sj[2], sj[3]));
      tmax = max_ref(tmax, shfl_xor_f32(tmax, 16));
      tmax = max_ref(tmax, shfl_xor_f32(tmax, 32));
      const float m_new = tmax > m ? tmax : m;
      const float corr = fexp(max_ref(-87.0f, m - m_new));
      float w[4];
#pragma unroll
      for (int j = 0; j < 4; ++j) w[j] = fexp(max_ref(-87.0f, sj[j] - m_new));
      // 16-position halving tree: t with t+8 (xor 32), t+4 (xor 16), then j+2, j+1.
      float ws[4];
#pragma unroll
      for (int j = 0; j < 4; ++j) ws[j] = w[j] + shfl_xor_f32(w[j], 32);
#pragma unroll
      for (int j = 0; j < 4; ++j) ws[j] = ws[j] + shfl_xor_f32(ws[j], 16);
      const float wsum = (ws[0] + ws[2]) + (ws[1] + ws[3]);
      lsum = lsum * corr + wsum;
      m = m_new;
      // scale_unrolled, then the tile's P.V in position order.
#pragma unroll
      for (int hh = 0; hh < kSG; ++hh) {
        const float c = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(corr), hh));
        acc[hh][0] = acc[hh][0] * c;
        acc[hh][1] = acc[hh][1] * c;
      }
#pragma unroll
      for (int j = 0; j < kTile; ++j) {
        if (j >= tl) break;
        const float v0 = bf16_lo(vv[j]);
        const float v1 = bf16_hi(vv[j]);
#pragma unroll
        for (int hh = 0; hh < kSG; ++hh) {
          const float wj = __int_as_float(
              __builtin_amdgcn_readlane(__float_as_int(w[j & 3]), 16 * (j >> 2) + hh));
          acc[hh][0] = fmaf(v0, wj, acc[hh][0]);
          acc[hh][1] = fmaf(v1, wj, acc[hh][1]);
        }
      }
    }
  }

  // write_finalized_head over one stripe: cv = fexp(0) scales both acc and
  // l (l > 0), out = (acc * cv) * (1 / (l * cv)).
  uint16_t* orow = out + (static_cast<int64_t>(t) * num_q + h * kSG) * kSD + 2 * lane;
#pragma unroll
  for (int hh = 0; hh < kSG; ++hh) {
    const float lh = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(lsum), hh));
    const float mh = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(m), hh));
    const float gm = mh > kNegBig ? mh : kNegBig;
    float cv = fexp(max_ref(-87.0f, mh - gm));
    cv = lh > 0.0f ? cv : 0.0f;
    const float gl = 0.0f + lh * cv;
    uint32_t packed = 0;
    if (gl > 0.0f) {
      const float inv = 1.0f / gl;
      packed = f32_to_bf16_bits((acc[hh][0] * cv) * inv) |
               (f32_to_bf16_bits((acc[hh][1] * cv) * inv) << 16);
    }
    *reinterpret_cast<uint32_t*>(orow + static_cast<int64_t>(hh) * kSD) = packed;
  }
}

}  // namespace

int index_block_stride(int64_t max_pos, int64_t block_size) {
  return static_cast<int>(((max_pos / block_size + 1) + 15) / 16 * 16);
}

int select_bank_cap(int topk) {
  int cap = 1;
  while (cap < 2 * topk) cap <<= 1;
  return cap < 16 ? 16 : cap;
}

hipError_t launch_lightning_indexer(const int32_t* image, int seq_len, const void* index_q,
                                    const void* index_k, int32_t* block_idx, float* scores,
                                    int block_stride, int num_heads, int head_dim,
                                    int block_size, int topk, int local_blocks,
                                    int init_blocks, float scale, int shift, int row_mask,
                                    hipStream_t stream) {
  if (seq_len <= 0) return hipSuccess;
  if (head_dim != 128 || num_heads != 4) return hipErrorInvalidValue;
  dim3 grid((block_stride + 3) / 4, seq_len);
  hipLaunchKernelGGL((index_scores_kernel<128, 4>), grid, dim3(256), 0, stream, image,
                     static_cast<const uint16_t*>(index_q), static_cast<const uint16_t*>(index_k),
                     scores, block_stride, block_size, scale, shift, row_mask);
  hipError_t err = hipGetLastError();
  if (err != hipSuccess) return err;
  const int rows = seq_len * num_heads;
  hipLaunchKernelGGL(select_blocks_kernel, dim3((rows + 3) / 4), dim3(256), 0, stream, image,
                     scores, block_idx, block_stride, num_heads, block_size, topk,
                     local_blocks, init_blocks, select_bank_cap(topk), rows);
  return hipGetLastError();
}

hipError_t launch_block_sparse_attention(const int32_t* image, int seq_len, const void* q,
                                         const void* k_base, const void* v_base,
                                         const int32_t* block_idx, void* output,
                                         int64_t kv_stride, int num_q, int num_kv,
                                         int block_size, int topk, int shift, int row_mask,
                                         hipStream_t stream) {
  if (seq_len <= 0) return hipSuccess;
  const int rows = seq_len * num_kv;
  hipLaunchKernelGGL(sparse_attention_kernel, dim3((rows + 3) / 4), dim3(256), 0, stream,
                     image, static_cast<const uint16_t*>(q),
                     static_cast<const uint16_t*>(k_base), static_cast<const uint16_t*>(v_base),
                     block_idx, static_cast<uint16_t*>(output), kv_stride, num_q, num_kv,
                     block_size, topk, shift, row_mask, rows);
  return hipGetLastError();
}

}  // namespace ifr
