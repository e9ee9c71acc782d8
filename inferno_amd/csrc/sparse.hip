// MiniMax-M3 block-sparse paged attention at degree 1 (prototypes/
// lightning_indexer.mojo, prototypes/sparse_attention.mojo): the lightning
// indexer scores every 128-position block of each token's causal context,
// keeps the top 16 blocks per index head, and the attention walks only those
// blocks.  The run table, page table and token->run map come from a
// full-attention plan image (ifr_plan_attention).
//
// index_scores_kernel   one wave per (token, block): each lane takes whole
//                       positions and all index heads (queries from SGPRs),
//                       and forms the dots in the reference's VDPBF16PS order,
//                       so block scores, and with them the selected blocks,
//                       are bit-identical.
// select_blocks_kernel  one wave per (token, index head): the reference's
//                       32-slot streaming bank, each reduction done as a rank
//                       count under reduce_argmax's order (value, then slot
//                       lane, then slot register).
// sparse_attention_kernel  four waves per (token, kv head): S = K.Q^T and P.V
//                       for the 16 q heads of the kv head on MFMA around the
//                       reference's per-tile online softmax (each wave forms
//                       the same scores and owns 32 output dims), then the
//                       one-stripe finalisation.
#include "common.hpp"
#include "launch.hpp"

namespace ifr {
namespace {

typedef __bf16 bf16x8_t __attribute__((ext_vector_type(8)));
typedef float f32x4_t __attribute__((ext_vector_type(4)));

__device__ __forceinline__ void wave_sync() {
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
  __builtin_amdgcn_wave_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
}

struct TokenPos {
  int abs_pos;
  const int32_t* rows;
};

__device__ __forceinline__ TokenPos token_position(const int32_t* image, int t) {
  const int run = sload(image + sload(image + kHdrOffTokRun) + t);
  const int32_t* rp = image + sload(image + kHdrOffRuns) + run * 4;
  return TokenPos{sload(rp + 1) + (t - sload(rp)), image + sload(image + kHdrOffRows) + sload(rp + 2)};
}

// ---------------------------------------------------------------------------
// IndexBlockScoreKernel (lightning_indexer.mojo:146-204).  Dots of the index
// key with each head's query follow bf16_panel_dot_to_scalars with
// port_unroll = D/32 (one strip of D): accumulator (p, j) takes the pair
// (32p + 2j + 1, 32p + 2j) as odd*odd + even*even, lane j sums its
// accumulators p = 0.. in order, then the 16-lane halving tree.
// ---------------------------------------------------------------------------
template <int D, int H, bool kPageRows>
__global__ __launch_bounds__(256) void index_scores_kernel(
    const int32_t* __restrict__ image, const uint16_t* __restrict__ index_q,
    const uint16_t* __restrict__ index_k, float* __restrict__ scores, int block_stride,
    int block_size, float scale, int shift, int row_mask) {
  constexpr int kP = D / 32;  // port-unroll accumulators, one strip
  static_assert(H * D == 64 * 8, "one 16-byte query load per lane");
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);  // wave-uniform
  const int lane = threadIdx.x & 63;
  const int t = blockIdx.y;
  const int b = blockIdx.x * 4 + wave;
  const TokenPos tp = token_position(image, t);
  const int nb = min(tp.abs_pos / block_size + 1, block_stride);
  if (b >= nb) return;
  const int lo = b * block_size;
  const int hi = min(lo + block_size, tp.abs_pos + 1);

  // One round = 64 positions, one per lane.  A lane past the block rereads
  // the block's last position (in bounds) and is left out of the maxima.
  // kPageRows (pages of >= 64 rows): a round spans at most two pages, whose
  // rows come from scalar loads.
  auto load_round = [&](int p0, uint4 (&kv)[D / 8]) {
    const int pos = min(p0 + lane, hi - 1);
    int64_t slot;
    if constexpr (kPageRows) {
      const int pg0 = p0 >> shift;
      const int pg1 = min(p0 + 63, hi - 1) >> shift;
      const int64_t ra = sload(tp.rows + pg0);
      const int64_t rb = pg1 != pg0 ? sload(tp.rows + pg1) : ra;
      slot = ((pos >> shift) == pg0 ? ra : rb) + (pos & row_mask);
    } else {
      slot = static_cast<int64_t>(tp.rows[pos >> shift]) + (pos & row_mask);
    }
    const uint4* kr = reinterpret_cast<const uint4*>(index_k + slot * D);
#pragma unroll
    for (int c = 0; c < D / 8; ++c) kv[c] = kr[c];
  };
  uint4 kv[D / 8];
  load_round(lo, kv);
  // The token's queries are wave-uniform: bf16 pairs read as scalar dwords
  // and unpacked on the SALU, so each FMA takes its query value from an
  // SGPR (no LDS staging or reads).
  const int32_t* qg = reinterpret_cast<const int32_t*>(index_q + static_cast<int64_t>(t) * H * D);
  float best[H];
#pragma unroll
  for (int h = 0; h < H; ++h) best[h] = kNegBig;
  // A lane takes whole positions and all heads: the key's pairs are unpacked
  // once, the queries are read from LDS (every lane the same address).
  for (int p0 = lo; p0 < hi; p0 += 64) {
    const bool valid = p0 + lane < hi;
    // The query reads stay inside the loop (hoisted, 256 dwords would not
    // fit in SGPRs).
    int qoff = 0;
    asm volatile("" : "+s"(qoff));
    float s[H][16];
#pragma unroll
    for (int p = 0; p < kP; ++p) {
      float klo[16], khi[16];
#pragma unroll
      for (int c = 0; c < 4; ++c) {
        const uint4 v = kv[4 * p + c];
        const uint32_t w4[4] = {v.x, v.y, v.z, v.w};
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          klo[4 * c + e] = bf16_lo(w4[e]);
          khi[4 * c + e] = bf16_hi(w4[e]);
        }
      }
#pragma unroll
      for (int h = 0; h < H; ++h) {
        const int32_t* qh = qg + qoff + (h * D + 32 * p) / 2;  // 16 dwords: pairs j = 0..15
#pragma unroll
        for (int j = 0; j < 16; ++j) {
          const uint32_t qw = static_cast<uint32_t>(sload(qh + j));
          const float qe = __uint_as_float(qw << 16), qo = __uint_as_float(qw & 0xFFFF0000u);
          // bf16 products are exact in f32, so the fma rounds (odd + even) once.
          const float a = fmaf(klo[j], qe, khi[j] * qo);
          s[h][j] = p == 0 ? a : s[h][j] + a;
        }
      }
    }
#pragma unroll
    for (int h = 0; h < H; ++h) {
#pragma unroll
      for (int w = 8; w >= 1; w >>= 1) {
#pragma unroll
        for (int jj = 0; jj < w; ++jj) s[h][jj] = s[h][jj] + s[h][jj + w];
      }
      const float sh = s[h][0] * scale;
      best[h] = valid && sh > best[h] ? sh : best[h];
    }
    // The next round's loads are issued after this round's math (with its
    // registers, 3 waves fit per SIMD; a prefetch into a second set, at 2
    // waves per SIMD, measured slower).
    if (p0 + 64 < hi) load_round(p0 + 64, kv);  // wave-uniform
  }
#pragma unroll
  for (int h = 0; h < H; ++h) {
    float v = best[h];
#pragma unroll
    for (int msk = 1; msk < 64; msk <<= 1) v = fmaxf(v, shfl_xor_f32(v, msk));
    if (lane == 0) scores[(static_cast<int64_t>(t) * H + h) * block_stride + b] = v;
  }
}

// ---------------------------------------------------------------------------
// stream_select_blocks (lightning_indexer.mojo:48-126) per (token, head) row.
// Lane s < kCap holds bank slot s.  reduce_top_k's successive argmax passes
// (matrixops.mojo:125-218) pick slots in one total order -- larger value,
// then smaller lane s % 16, then smaller register s / 16 -- so a bitonic
// sort of the bank under that order leaves the kept slots, in selection
// order, in lanes 0..topk-1: exactly the refilled bank of the reference.
// ---------------------------------------------------------------------------
template <int kCap>
__device__ __forceinline__ void bank_sort(float& v, int& id, int lane) {
  int key = (lane & 15) * 64 + ((lane & (kCap - 1)) >> 4);  // slot order on ties
#pragma unroll
  for (int k = 2; k <= kCap; k <<= 1) {
#pragma unroll
    for (int j = k >> 1; j > 0; j >>= 1) {
      const float v2 = shfl_xor_f32(v, j);
      const int key2 = shfl_xor_i32(key, j);
      const int id2 = shfl_xor_i32(id, j);
      const bool other_first = v2 > v || (v2 == v && key2 < key);
      const bool keep_first = ((lane & j) == 0) == ((lane & k) == 0);
      if (keep_first ? other_first : !other_first) {
        v = v2;
        key = key2;
        id = id2;
      }
    }
  }
}

// Ascending sort of ids over kCap lanes (empty lanes carry INT_MAX).
template <int kCap>
__device__ __forceinline__ void id_sort(int& id, int lane) {
#pragma unroll
  for (int k = 2; k <= kCap; k <<= 1) {
#pragma unroll
    for (int j = k >> 1; j > 0; j >>= 1) {
      const int id2 = shfl_xor_i32(id, j);
      const bool keep_low = ((lane & j) == 0) == ((lane & k) == 0);
      id = keep_low ? min(id, id2) : max(id, id2);
    }
  }
}

constexpr int kFastChunks = 32;  // fast path: rows of up to 64 * 32 blocks

template <int kCap>
__global__ __launch_bounds__(256) void select_blocks_kernel(
    const int32_t* __restrict__ image, const float* __restrict__ scores,
    int32_t* __restrict__ block_idx, int block_stride, int num_heads, int block_size,
    int topk, int local_blocks, int init_blocks, int num_rows) {
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);  // wave-uniform
  const int lane = threadIdx.x & 63;
  const int row = blockIdx.x * 4 + wave;
  if (row >= num_rows) return;
  const int t = row / num_heads;
  const TokenPos tp = token_position(image, t);
  const int nb = min(tp.abs_pos / block_size + 1, block_stride);
  const float* sr = scores + static_cast<int64_t>(row) * block_stride;
  const int local_start = max(nb - local_blocks, 0);

  int32_t* out = block_idx + static_cast<int64_t>(row) * topk;
  // Short rows keep every block.
  if (nb <= topk) {
    if (lane < topk) out[lane] = lane < nb ? lane : -1;
    return;
  }
  // Fast path.  If exactly topk scores are >= the topk-th largest score T,
  // every bank reduction keeps them (at most topk - 1 entries can precede
  // one of them) and the final pass returns them: the result is the set
  // {score >= T} whatever the tie order.  T comes from a radix select over
  // the scores held in registers (nb <= 2048); ties straddling T, or longer
  // rows, take the bank below.
  if (nb <= 64 * kFastChunks) {
    float vals[kFastChunks];
    uint32_t keys[kFastChunks];
    const int n_chunks = (nb + 63) / 64;
#pragma unroll
    for (int i = 0; i < kFastChunks; ++i) {
      const int blk = 64 * i + lane;
      float x = -INFINITY;
      const bool in = i < n_chunks && blk < nb;
      if (in) x = (blk >= local_start || blk < init_blocks) ? 1.0e30f : sr[blk] + 0.0f;  // -0 -> +0
      vals[i] = x;
      const uint32_t u = __float_as_uint(x);
      // Order-preserving key; 0 for slots past the row, which no candidate
      // (at least one bit set) counts, so the counting loop needs no
      // per-chunk branch.
      keys[i] = in ? ((u & 0x80000000u) ? ~u : (u | 0x80000000u)) : 0u;
      asm volatile("" : "+v"(keys[i]));  // a plain register: one compare per chunk below
    }
    uint32_t prefix = 0;
    for (int bit = 31; bit >= 0; --bit) {
      const uint32_t cand = prefix | (1u << bit);
      int cnt = 0;
#pragma unroll
      for (int i = 0; i < kFastChunks; ++i)
        cnt += __popcll(__builtin_amdgcn_ballot_w64(keys[i] >= cand));
      if (cnt >= topk) prefix = cand;
    }
    const uint32_t tu = (prefix & 0x80000000u) ? (prefix & 0x7FFFFFFFu) : ~prefix;
    const float thr = __uint_as_float(tu);
    // Slots past the row hold -inf, below any threshold of finite scores.
    int cnt_ge = 0;
#pragma unroll
    for (int i = 0; i < kFastChunks; ++i)
      cnt_ge += __popcll(__builtin_amdgcn_ballot_w64(vals[i] >= thr));
    if (cnt_ge == topk) {
      const uint64_t below = (lane == 0) ? 0ull : (~0ull >> (64 - lane));
      int written = 0;
#pragma unroll
      for (int i = 0; i < kFastChunks; ++i) {
        const bool sel = vals[i] >= thr;
        const uint64_t mask = __ballot(sel);
        if (sel) out[written + __popcll(mask & below)] = 64 * i + lane;
        written += __popcll(mask);
      }
      return;
    }
  }

  float v = kNegBig;
  int id = -1;
  int fill = 0;
  // Scores stream through two 64-block register windows [base, base + 128),
  // the next one loading while the bank works on the current.
  int base = 0;
  float win0 = lane < nb ? sr[lane] : kNegBig;
  float win1 = 64 + lane < nb ? sr[64 + lane] : kNegBig;
  for (int b = 0; b < nb;) {
    const int n_new = min(kCap - fill, nb - b);
    {
      const int blk = b + lane - fill;  // block this lane would take
      const int rel = min(max(blk - base, 0), 127);
      const float x0 = __shfl(win0, rel & 63);
      const float x1 = __shfl(win1, rel & 63);
      if (lane >= fill && lane < fill + n_new) {
        v = (blk >= local_start || blk < init_blocks) ? 1.0e30f : (rel < 64 ? x0 : x1);
        id = blk;
      }
    }
    if (b + n_new - base >= 64) {
      base += 64;
      win0 = win1;
      win1 = base + 64 + lane < nb ? sr[base + 64 + lane] : kNegBig;
    }
    fill += n_new;
    b += n_new;
    if (fill == kCap) {
      bank_sort<kCap>(v, id, lane);
      if (lane >= topk) {
        v = kNegBig;
        id = -1;
      }
      fill = topk;
    }
  }
  bank_sort<kCap>(v, id, lane);
  const bool sel = lane < kCap && lane < topk && v > kNegBig;
  const int count = __popcll(__ballot(sel));
  int sid = sel ? id : INT32_MAX;
  id_sort<kCap>(sid, lane);
  if (lane < topk) out[lane] = lane < count ? sid : -1;
}

// ---------------------------------------------------------------------------
// BlockSparseFlashKernel (sparse_attention.mojo:59-131) + the one-stripe
// write_finalized_head of PrefillMergeKernel (flash_attention_prefill.mojo:
// 221-240), for head_dim 128 and 16 q heads per kv head.
//
// Scores: v_mfma_f32_16x16x32_bf16 with A = the tile's 16 keys x 32 dims and
// B = the 16 queries' dims, so lane l holds S[pos 4*(l/16)+j][head l%16].
// Softmax per tile follows online_softmax_tile with the biased exp; the tile
// weight sum uses the 16-position halving tree (xor 32, xor 16, then in-lane).
// P.V: v_mfma_f32_16x16x16_bf16 per 16-dim block with A = V^T (a transposing
// LDS read of the tile's rows) and B = P^T, which is the softmax layout
// itself, so the accumulator C[dim][head] rescales lane-locally.  P enters as
// bf16 hi + lo parts (about 16 significant bits per weight); pad positions
// carry their fexp(-87) into l but a zero weight into P.V, as in the
// reference.  The next two tiles' keys and values load while a tile
// computes.
// ---------------------------------------------------------------------------
constexpr int kSD = 128;                // head_dim
constexpr int kSG = 16;                 // q heads per kv head
constexpr int kSVPitch = kSD * 2 + 32;  // bytes per V row in LDS
constexpr int kSVBytes = kTile * kSVPitch;

typedef short s16x4_t __attribute__((ext_vector_type(4)));
typedef __attribute__((address_space(3))) s16x4_t lds_s16x4_t;
typedef __bf16 bf16x2_t __attribute__((ext_vector_type(2)));
typedef float f32x2_t __attribute__((ext_vector_type(2)));

// The tile walk: blocks in list order, stopping at the first -1, each from
// its first position to min(end, cap) in 16-position steps.
struct TileCursor {
  int s;
  int64_t pos, phi;
  bool valid;
};

__device__ __forceinline__ TileCursor next_tile(TileCursor c, const int32_t* brow, int topk,
                                                int block_size, int64_t cap) {
  c.pos += kTile;
  while (c.pos >= c.phi) {
    ++c.s;
    if (c.s >= topk) {
      c.valid = false;
      return c;
    }
    const int b = sload(brow + c.s);
    if (b < 0) {
      c.valid = false;
      return c;
    }
    c.pos = static_cast<int64_t>(b) * block_size;
    c.phi = min(c.pos + block_size, cap);
  }
  c.valid = true;
  return c;
}

struct TileRegs {
  uint4 k0, k1, k2, k3;  // keys: row r16, dims 32c + 8g .. +8
  uint4 v0;              // values: row lane/4, 16 bytes of the wave's 32 dims
};
// The four waves of a workgroup share one (token, kv head): each forms the
// same scores and softmax (identical arithmetic) and owns 32 of the 128
// output dims in P.V, so a decode step has four times as many waves on its
// block lists.  V rows of the wave's dims are staged at a 96-byte pitch
// (4 rows x 32 bytes of a transposing read fall on distinct banks).
constexpr int kSDW = kSD / 4;                 // output dims per wave
constexpr int kSVPitchW = kSDW * 2 + 32;      // bytes per V row in LDS
constexpr int kSVBytesW = kTile * kSVPitchW;

__global__ __launch_bounds__(256) void sparse_attention_kernel(
    const int32_t* __restrict__ image, const uint16_t* __restrict__ q,
    const uint16_t* __restrict__ k_base, const uint16_t* __restrict__ v_base,
    const int32_t* __restrict__ block_idx, uint16_t* __restrict__ out, int64_t kv_stride,
    int num_q, int num_kv, int block_size, int topk, int shift, int row_mask, int num_rows) {
  __shared__ __align__(16) uint8_t vlds[4][2][kSVBytesW];
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);  // wave-uniform
  const int lane = threadIdx.x & 63;
  const int row = blockIdx.x;
  if (row >= num_rows) return;
  const int dq = wave;  // the wave's quarter of the output dims
  const int t = row / num_kv;
  const int h = row - t * num_kv;
  const TokenPos tp = token_position(image, t);
  const int64_t cap = static_cast<int64_t>(tp.abs_pos) + 1;
  const int r16 = lane & 15;
  const int g = lane >> 4;

  // B operand of the scores: Q[head r16][32c + 8g .. +8] for c = 0..3.
  bf16x8_t qf[4];
  {
    const uint16_t* qrow =
        q + (static_cast<int64_t>(t) * num_q + h * kSG + r16) * kSD + 8 * g;
#pragma unroll
    for (int c = 0; c < 4; ++c)
      qf[c] = __builtin_bit_cast(bf16x8_t, *reinterpret_cast<const uint4*>(qrow + 32 * c));
  }
  const uint16_t* kh = k_base + static_cast<int64_t>(h) * kSD;
  const uint16_t* vh = v_base + static_cast<int64_t>(h) * kSD;
  const int32_t* brow = block_idx + static_cast<int64_t>(row) * topk;
  // V staging: lane takes 16 bytes (chunk lane%4) of row lane/4 of the
  // wave's 32 dims.
  const int vrow_l = lane >> 2;
  const int vcol = 16 * (lane & 3);
  // Transposing read: lane r16 of group g addresses row 4g + r16/4, dims
  // 4*(r16%4) .. +3 of a 16-dim block, and receives V[4g + k][16b + r16].
  const int tr_off = (4 * g + (r16 >> 2)) * kSVPitchW + 8 * (r16 & 3);

  // A tile never straddles a page (page_len >= 16, tiles 16-aligned), so its
  // page row is one uniform (scalar) load, not a vector load the K/V loads
  // would have to wait behind.
  auto page_row = [&](const TileCursor& c) -> int64_t {
    return sload(tp.rows + static_cast<int>(c.pos >> shift));
  };
  auto load_tile = [&](const TileCursor& c, int64_t prow) {
    TileRegs d;
    const int tl = static_cast<int>(min<int64_t>(kTile, c.phi - c.pos));
    const int off0 = static_cast<int>(c.pos) & row_mask;
    const int64_t kslot = prow + off0 + (r16 < tl ? r16 : 0);
    const uint16_t* kp = kh + kslot * kv_stride + 8 * g;
    d.k0 = *reinterpret_cast<const uint4*>(kp);
    d.k1 = *reinterpret_cast<const uint4*>(kp + 32);
    d.k2 = *reinterpret_cast<const uint4*>(kp + 64);
    d.k3 = *reinterpret_cast<const uint4*>(kp + 96);
    const int64_t vslot = prow + off0 + (vrow_l < tl ? vrow_l : 0);
    d.v0 = *reinterpret_cast<const uint4*>(
        reinterpret_cast<const uint8_t*>(vh + vslot * kv_stride + kSDW * dq) + vcol);
    return d;
  };

  float m = kNegBig;  // state of head r16 (the same in its four lanes)
  float lsum = 0.0f;
  f32x4_t acc[kSDW / 16];  // acc[b][j] = O[dim 32dq + 16b + 4g + j][head r16]
#pragma unroll
  for (int b = 0; b < kSDW / 16; ++b) acc[b] = f32x4_t{0.0f, 0.0f, 0.0f, 0.0f};

  // A tile's scores and softmax, then P.V; between the two the caller
  // reuses the tile's registers for the loads of a later tile.
  auto scores = [&](const TileRegs& rg, const TileCursor& c, int buf) {
    uint8_t* vb = vlds[wave][buf];
    wave_sync();
    *reinterpret_cast<uint4*>(vb + vrow_l * kSVPitchW + vcol) = rg.v0;
    f32x4_t sc = {0.0f, 0.0f, 0.0f, 0.0f};
    sc = __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8_t, rg.k0), qf[0], sc, 0, 0, 0);
    sc = __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8_t, rg.k1), qf[1], sc, 0, 0, 0);
    sc = __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8_t, rg.k2), qf[2], sc, 0, 0, 0);
    sc = __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8_t, rg.k3), qf[3], sc, 0, 0, 0);
    return sc;
  };
  auto softmax_pv = [&](const f32x4_t& sc, const TileCursor& c, int buf) {
    const int tl = static_cast<int>(min<int64_t>(kTile, c.phi - c.pos));
    uint8_t* vb = vlds[wave][buf];
    // Scores of pad positions are -1e30 (their fexp(-87) enters l only).
    float sj[4];
#pragma unroll
    for (int j = 0; j < 4; ++j) sj[j] = (4 * g + j < tl) ? sc[j] : kNegBig;
    float tmax = max_ref(max_ref(sj[0], sj[1]), max_ref(sj[2], sj[3]));
    tmax = pair_max32(pair_max16(tmax));  // lane swaps, not LDS permutes
    const float m_new = tmax > m ? tmax : m;
    const float corr = fexp(max_ref(-87.0f, m - m_new));
    float w[4];
#pragma unroll
    for (int j = 0; j < 4; ++j) w[j] = fexp(max_ref(-87.0f, sj[j] - m_new));
    // 16-position halving tree: t with t+8 (xor 32), t+4 (xor 16), then j+2, j+1.
    float ws[4];
#pragma unroll
    for (int j = 0; j < 4; ++j) ws[j] = pair_sum16(pair_sum32(w[j]));
    const float wsum = (ws[0] + ws[2]) + (ws[1] + ws[3]);
    lsum = lsum * corr + wsum;
    m = m_new;
    // P^T as bf16 hi + lo, zero at pads.
    s16x4_t phi, plo;
#pragma unroll
    for (int j = 0; j < 4; j += 2) {
      const float p0 = (4 * g + j < tl) ? w[j] : 0.0f;
      const float p1 = (4 * g + j + 1 < tl) ? w[j + 1] : 0.0f;
      const bf16x2_t hb = __builtin_convertvector(f32x2_t{p0, p1}, bf16x2_t);
      const float r0 = p0 - static_cast<float>(hb[0]);
      const float r1 = p1 - static_cast<float>(hb[1]);
      const bf16x2_t lb = __builtin_convertvector(f32x2_t{r0, r1}, bf16x2_t);
      const s16x4_t hs = __builtin_bit_cast(s16x4_t, __builtin_shufflevector(hb, hb, 0, 1, 0, 1));
      const s16x4_t ls = __builtin_bit_cast(s16x4_t, __builtin_shufflevector(lb, lb, 0, 1, 0, 1));
      phi[j] = hs[0];
      phi[j + 1] = hs[1];
      plo[j] = ls[0];
      plo[j + 1] = ls[1];
    }
    wave_sync();
#pragma unroll
    for (int b = 0; b < kSDW / 16; ++b) {
      acc[b] = acc[b] * corr;  // scale_unrolled for head r16
      const s16x4_t va =
          __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_s16x4_t*)(vb + tr_off + 32 * b));
      acc[b] = __builtin_amdgcn_mfma_f32_16x16x16bf16_1k(va, phi, acc[b], 0, 0, 0);
      acc[b] = __builtin_amdgcn_mfma_f32_16x16x16bf16_1k(va, plo, acc[b], 0, 0, 0);
    }
  };

  // kAhead tiles in flight in rotating register sets (no copies between
  // them): set s holds tile i + s; once tile i's scores have read its keys
  // and its values are in LDS, the set takes the loads of tile i + kAhead.
  // The loads are unconditional -- past the block list they all read the
  // sequence's first row (in bounds, unused) -- so every step leaves the same
  // loads in flight and each wait covers only older loads.  The next
  // cursor's page row is read (scalar) one step before its loads use it.
  // An even depth keeps each step's LDS buffer a compile-time choice
  // (measured: depths 2 and 4 93 us, 3 and 5 100 us, 6 and 8 98.5 us).
  constexpr int kAhead = 4;
  auto advance = [&](const TileCursor& c) {
    return c.valid ? next_tile(c, brow, topk, block_size, cap) : c;
  };
  auto dummy_or = [&](const TileCursor& c) {
    TileCursor d = c;  // selects, not a branch: one code path for the loads
    d.pos = c.valid ? c.pos : 0;
    d.phi = c.valid ? c.phi : kTile;
    return d;
  };
  TileCursor cs[kAhead];
  TileRegs rs[kAhead];
  cs[0] = next_tile(TileCursor{-1, 0, 0, false}, brow, topk, block_size, cap);
#pragma unroll
  for (int i = 1; i < kAhead; ++i) cs[i] = advance(cs[i - 1]);
  // Issued in set order, as the loop issues them (the waits count on it).
#pragma unroll
  for (int i = 0; i < kAhead; ++i) {
    const TileCursor d = dummy_or(cs[i]);
    rs[i] = load_tile(d, page_row(d));
    __builtin_amdgcn_sched_barrier(0);
  }
  TileCursor pend = dummy_or(advance(cs[kAhead - 1]));  // the next tile to issue
  bool pend_valid = advance(cs[kAhead - 1]).valid;
  TileCursor last = advance(cs[kAhead - 1]);
  int64_t pend_row = page_row(pend);
  int buf = 0;
  for (;;) {
#pragma unroll
    for (int s = 0; s < kAhead; ++s) {
      // Leaving the loop is the only branch: every path that goes on has
      // issued the same loads.
      if (!cs[s].valid) goto tiles_done;  // uniform
      const TileCursor c = cs[s];
      const f32x4_t sc = scores(rs[s], c, buf);
      __builtin_amdgcn_sched_barrier(0);
      rs[s] = load_tile(pend, pend_row);
      __builtin_amdgcn_sched_barrier(0);
      cs[s] = pend;
      cs[s].valid = pend_valid;
      last = advance(last);
      pend_valid = last.valid;
      pend = dummy_or(last);
      pend_row = page_row(pend);
      softmax_pv(sc, c, buf);
      buf ^= 1;
    }
  }
tiles_done:

  // write_finalized_head over one stripe: cv = fexp(0) scales both acc and
  // l (l > 0), out = (acc * cv) * (1 / (0 + l * cv)).
  const float gm = m > kNegBig ? m : kNegBig;
  float cv = fexp(max_ref(-87.0f, m - gm));
  cv = lsum > 0.0f ? cv : 0.0f;
  const float gl = 0.0f + lsum * cv;
  const float inv = gl > 0.0f ? 1.0f / gl : 0.0f;
  uint16_t* orow =
      out + (static_cast<int64_t>(t) * num_q + h * kSG + r16) * kSD + kSDW * dq + 4 * g;
#pragma unroll
  for (int b = 0; b < kSDW / 16; ++b) {
    uint32_t lo = 0, hi = 0;
    if (gl > 0.0f) {
      lo = f32_to_bf16_bits((acc[b][0] * cv) * inv) | (f32_to_bf16_bits((acc[b][1] * cv) * inv) << 16);
      hi = f32_to_bf16_bits((acc[b][2] * cv) * inv) | (f32_to_bf16_bits((acc[b][3] * cv) * inv) << 16);
    }
    *reinterpret_cast<uint2*>(orow + 16 * b) = make_uint2(lo, hi);
  }
}

// ---------------------------------------------------------------------------
// bq_process_kv_tile_head (prototypes/bq_sparse_attention.mojo:29-91) inside
// BqBlockSparseFlashKernel (:94-200, one (token, kv head) per wave, blocks in
// order, -1 ends the list, one-stripe finalisation) and
// BqBlockSparseFlashDecodeKernel (:254-364, one (worker, kv head) per wave over
// the worker's band of block slots, -1 skipped, a partial stripe per worker).
//
// Scores: raw = sum (k ^ 0x80) * q over u8 x i8 equals sum k*q + 128 * sum q,
// both exact integers; sum k*q comes from v_mfma_i32_16x16x64_i8, so
// ((raw - qi_bias) * f_q * k_scale) / 127^2 is the reference's value.
// P.V: the tile's int8 values enter LDS as bf16 (exact), weights are
// (w * v_scale) / 127 as in the reference, on the bf16 MFMA as hi + lo.
// ---------------------------------------------------------------------------
typedef int i32x4_t __attribute__((ext_vector_type(4)));

struct BqTileRegs {
  uint4 k0, k1;          // keys: row r16, bytes 16g and 64 + 16g
  uint2 v0, v1, v2, v3;  // values: 32 bytes of row l/4 at 32*(l%4)
  float ks[4], vs[4];    // scales of positions 4g + j
};

template <bool kDecode>
__global__ __launch_bounds__(256) void bq_sparse_kernel(
    const int32_t* __restrict__ image, const int8_t* __restrict__ q_i8,
    const float* __restrict__ qi_bias, const float* __restrict__ f_q,
    const int8_t* __restrict__ k_base, const float* __restrict__ k_scale,
    const int8_t* __restrict__ v_base, const float* __restrict__ v_scale,
    const int32_t* __restrict__ block_idx, uint16_t* __restrict__ out,
    float* __restrict__ partials, int64_t partial_stride, int64_t kv_stride, int num_q,
    int num_kv, int block_size, int topk, int decode_slots, int decode_workers, int shift,
    int row_mask, int num_rows) {
  __shared__ __align__(16) uint8_t vlds[4][2][kSVBytes];
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);  // wave-uniform
  const int lane = threadIdx.x & 63;
  const int row = blockIdx.x * 4 + wave;
  if (row >= num_rows) return;
  const int r16 = lane & 15;
  const int g = lane >> 4;
  // Unit: (token t | worker w, kv head h) and its slot range.
  const int unit = row / num_kv;
  const int h = row - unit * num_kv;
  const int t = kDecode ? 0 : unit;
  int s_lo = 0, s_hi = topk;
  if (kDecode) {
    const int total = num_kv * decode_slots;  // worker_range over (head, slot) units
    const int per = (total + decode_workers - 1) / decode_workers;
    const int lo = min(unit * per, total), hi = min(lo + per, total);
    s_lo = max(lo, h * decode_slots) - h * decode_slots;
    s_hi = min(hi, (h + 1) * decode_slots) - h * decode_slots;
  }
  const TokenPos tp = token_position(image, t);
  const int64_t cap = static_cast<int64_t>(tp.abs_pos) + 1;
  const int gh = h * kSG + r16;  // q head of this lane's column
  const int64_t qrow = static_cast<int64_t>(t) * num_q + gh;

  // B operand of the scores: q codes of head r16, bytes 16g and 64 + 16g;
  // qsum = sum of the head's 128 codes (exact).
  const int8_t* qp = q_i8 + qrow * kSD + 16 * g;
  const uint4 qa = *reinterpret_cast<const uint4*>(qp);
  const uint4 qb4 = *reinterpret_cast<const uint4*>(qp + 64);
  int qsum = 0;
  {
    const uint32_t w8[8] = {qa.x, qa.y, qa.z, qa.w, qb4.x, qb4.y, qb4.z, qb4.w};
#pragma unroll
    for (int i = 0; i < 8; ++i)
      qsum += static_cast<int8_t>(w8[i]) + static_cast<int8_t>(w8[i] >> 8) +
              static_cast<int8_t>(w8[i] >> 16) + static_cast<int8_t>(w8[i] >> 24);
    qsum += __shfl_xor(qsum, 16);
    qsum += __shfl_xor(qsum, 32);
  }
  const float qbias = qi_bias[qrow];
  const float fq = f_q[qrow];
  const float inv127 = 1.0f / 127.0f;
  const float inv127sq = inv127 * inv127;

  const int8_t* kh = k_base + static_cast<int64_t>(h) * kSD;
  const int8_t* vh = v_base + static_cast<int64_t>(h) * kSD;
  const int32_t* brow =
      block_idx + (kDecode ? static_cast<int64_t>(h) : static_cast<int64_t>(row)) * topk;
  const int tr_off = (4 * g + (r16 >> 2)) * kSVPitch + 8 * (r16 & 3);

  // V staging: lane takes 32 bytes (dims 32*(l%4) ..) of row l/4.
  const int vr_row = lane >> 2;
  const int vr_col = 32 * (lane & 3);
  auto load_tile = [&](const TileCursor& c) {
    BqTileRegs d;
    const int tl = static_cast<int>(min<int64_t>(kTile, c.phi - c.pos));
    const int64_t prow = sload(tp.rows + static_cast<int>(c.pos >> shift));  // uniform
    const int off0 = static_cast<int>(c.pos) & row_mask;
    const int64_t base = prow + off0;
    const int8_t* kp = kh + (base + (r16 < tl ? r16 : 0)) * kv_stride + 16 * g;
    d.k0 = *reinterpret_cast<const uint4*>(kp);
    d.k1 = *reinterpret_cast<const uint4*>(kp + 64);
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const int64_t sl = (base + (4 * g + j < tl ? 4 * g + j : 0)) * num_kv + h;
      d.ks[j] = k_scale[sl];
      d.vs[j] = v_scale[sl];
    }
    const int8_t* vp = vh + (base + (vr_row < tl ? vr_row : 0)) * kv_stride + vr_col;
    d.v0 = *reinterpret_cast<const uint2*>(vp);
    d.v1 = *reinterpret_cast<const uint2*>(vp + 8);
    d.v2 = *reinterpret_cast<const uint2*>(vp + 16);
    d.v3 = *reinterpret_cast<const uint2*>(vp + 24);
    return d;
  };
  auto next = [&](TileCursor c) {
    c.pos += kTile;
    while (c.pos >= c.phi) {
      ++c.s;
      if (c.s >= s_hi) {
        c.valid = false;
        return c;
      }
      const int b = sload(brow + c.s);
      if (b < 0) {
        if (!kDecode) {
          c.valid = false;
          return c;
        }
        c.pos = 0;
        c.phi = 0;
        continue;
      }
      c.pos = static_cast<int64_t>(b) * block_size;
      c.phi = min(c.pos + block_size, cap);
    }
    c.valid = true;
    return c;
  };

  float m = kNegBig;
  float lsum = 0.0f;
  f32x4_t acc[kSD / 16];
#pragma unroll
  for (int b = 0; b < kSD / 16; ++b) acc[b] = f32x4_t{0.0f, 0.0f, 0.0f, 0.0f};

  auto advance = [&](const TileCursor& c) { return c.valid ? next(c) : c; };
  TileCursor cur = next(TileCursor{s_lo - 1, 0, 0, false});
  TileCursor c1 = advance(cur);
  BqTileRegs rg{}, r1{};
  if (cur.valid) rg = load_tile(cur);
  if (c1.valid) r1 = load_tile(c1);
  int buf = 0;
  while (cur.valid) {
    const TileCursor c2 = advance(c1);
    const int tl = static_cast<int>(min<int64_t>(kTile, cur.phi - cur.pos));
    uint8_t* vb = vlds[wave][buf];
    wave_sync();
    {
      // 32 int8 values -> 32 bf16 (exact) at row vr_row, dims vr_col ..
      const uint32_t w8[8] = {rg.v0.x, rg.v0.y, rg.v1.x, rg.v1.y,
                              rg.v2.x, rg.v2.y, rg.v3.x, rg.v3.y};
      uint32_t o16[16];
#pragma unroll
      for (int i = 0; i < 8; ++i) {
#pragma unroll
        for (int b = 0; b < 4; b += 2) {
          const float f0 = static_cast<float>(static_cast<int8_t>(w8[i] >> (8 * b)));
          const float f1 = static_cast<float>(static_cast<int8_t>(w8[i] >> (8 * b + 8)));
          o16[2 * i + b / 2] = (__float_as_uint(f0) >> 16) | (__float_as_uint(f1) & 0xFFFF0000u);
        }
      }
      uint8_t* dst = vb + vr_row * kSVPitch + 2 * vr_col;
#pragma unroll
      for (int i = 0; i < 4; ++i)
        *reinterpret_cast<uint4*>(dst + 16 * i) =
            make_uint4(o16[4 * i], o16[4 * i + 1], o16[4 * i + 2], o16[4 * i + 3]);
    }
    BqTileRegs r2{};
    if (c2.valid) r2 = load_tile(c2);

    i32x4_t si = {0, 0, 0, 0};
    si = __builtin_amdgcn_mfma_i32_16x16x64_i8(
        __builtin_bit_cast(i32x4_t, rg.k0), __builtin_bit_cast(i32x4_t, qa), si, 0, 0, 0);
    si = __builtin_amdgcn_mfma_i32_16x16x64_i8(
        __builtin_bit_cast(i32x4_t, rg.k1), __builtin_bit_cast(i32x4_t, qb4), si, 0, 0, 0);
    // Lane holds positions 4g + j of head r16.
    float sj[4], vsj[4];
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      vsj[j] = rg.vs[j];
      const float raw = static_cast<float>(si[j] + 128 * qsum);
      float sc = raw - qbias;
      sc = sc * fq;
      sc = sc * rg.ks[j];
      sc = sc * inv127sq;
      sj[j] = (4 * g + j < tl) ? sc : kNegBig;
    }
    float tmax = max_ref(max_ref(sj[0], sj[1]), max_ref(sj[2], sj[3]));
    tmax = pair_max32(pair_max16(tmax));  // lane swaps, not LDS permutes
    const float m_new = tmax > m ? tmax : m;
    const float corr = fexp(max_ref(-87.0f, m - m_new));
    float w[4];
#pragma unroll
    for (int j = 0; j < 4; ++j) w[j] = fexp(max_ref(-87.0f, sj[j] - m_new));
    float ws[4];
#pragma unroll
    for (int j = 0; j < 4; ++j) ws[j] = pair_sum16(pair_sum32(w[j]));
    const float wsum = (ws[0] + ws[2]) + (ws[1] + ws[3]);
    lsum = lsum * corr + wsum;
    m = m_new;
    s16x4_t phi, plo;
#pragma unroll
    for (int j = 0; j < 4; j += 2) {
      float p0 = w[j] * vsj[j];
      p0 = p0 * inv127;
      float p1 = w[j + 1] * vsj[j + 1];
      p1 = p1 * inv127;
      p0 = (4 * g + j < tl) ? p0 : 0.0f;
      p1 = (4 * g + j + 1 < tl) ? p1 : 0.0f;
      const bf16x2_t hb = __builtin_convertvector(f32x2_t{p0, p1}, bf16x2_t);
      const float r0 = p0 - static_cast<float>(hb[0]);
      const float r1 = p1 - static_cast<float>(hb[1]);
      const bf16x2_t lb = __builtin_convertvector(f32x2_t{r0, r1}, bf16x2_t);
      const s16x4_t hs = __builtin_bit_cast(s16x4_t, __builtin_shufflevector(hb, hb, 0, 1, 0, 1));
      const s16x4_t ls = __builtin_bit_cast(s16x4_t, __builtin_shufflevector(lb, lb, 0, 1, 0, 1));
      phi[j] = hs[0];
      phi[j + 1] = hs[1];
      plo[j] = ls[0];
      plo[j + 1] = ls[1];
    }
    wave_sync();
#pragma unroll
    for (int b = 0; b < kSD / 16; ++b) {
      acc[b] = acc[b] * corr;
      const s16x4_t va =
          __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_s16x4_t*)(vb + tr_off + 32 * b));
      acc[b] = __builtin_amdgcn_mfma_f32_16x16x16bf16_1k(va, phi, acc[b], 0, 0, 0);
      acc[b] = __builtin_amdgcn_mfma_f32_16x16x16bf16_1k(va, plo, acc[b], 0, 0, 0);
    }
    rg = r1;
    r1 = r2;
    cur = c1;
    c1 = c2;
    buf ^= 1;
  }

  if constexpr (kDecode) {
    // The worker's stripe: acc, m, l of the kv head's 16 q heads (the
    // identity m = -1e30, l = 0 when its band does not reach the head).
    float* pw = partials + static_cast<int64_t>(unit) * partial_stride;
    float* prow = pw + static_cast<int64_t>(gh) * kSD + 4 * g;
#pragma unroll
    for (int b = 0; b < kSD / 16; ++b)
      *reinterpret_cast<float4*>(prow + 16 * b) =
          make_float4(acc[b][0], acc[b][1], acc[b][2], acc[b][3]);
    if (g == 0) {
      pw[num_q * kSD + gh] = m;
      pw[num_q * kSD + num_q + gh] = lsum;
    }
  } else {
    const float gm = m > kNegBig ? m : kNegBig;
    float cv = fexp(max_ref(-87.0f, m - gm));
    cv = lsum > 0.0f ? cv : 0.0f;
    const float gl = 0.0f + lsum * cv;
    const float inv = gl > 0.0f ? 1.0f / gl : 0.0f;
    uint16_t* orow = out + qrow * kSD + 4 * g;
#pragma unroll
    for (int b = 0; b < kSD / 16; ++b) {
      uint32_t lo = 0, hi = 0;
      if (gl > 0.0f) {
        lo = f32_to_bf16_bits((acc[b][0] * cv) * inv) |
             (f32_to_bf16_bits((acc[b][1] * cv) * inv) << 16);
        hi = f32_to_bf16_bits((acc[b][2] * cv) * inv) |
             (f32_to_bf16_bits((acc[b][3] * cv) * inv) << 16);
      }
      *reinterpret_cast<uint2*>(orow + 16 * b) = make_uint2(lo, hi);
    }
  }
}

// The batched route of bq_sparse_kernel (one sequential pass per (token, kv
// head)) with the bf16 kernel's split: four waves per (token, kv head), each
// forming the same int8 scores (exact integers, so identical) and owning 32
// of the 128 output dims, with kSAhead tiles in flight in rotating register
// sets.  One wave per (token, kv head) left three quarters of the SIMDs idle
// at B = 64 with 4 kv heads.
struct BqSplitRegs {
  uint4 k0, k1;       // keys: row r16, bytes 16g and 64 + 16g
  uint2 v;            // values: 8 bytes of the wave's 32 dims of row lane/4
  float ks[4], vs[4];  // scales of positions 4g + j
};
constexpr int kSAhead = 4;

__global__ __launch_bounds__(256) void bq_sparse_split_kernel(
    const int32_t* __restrict__ image, const int8_t* __restrict__ q_i8,
    const float* __restrict__ qi_bias, const float* __restrict__ f_q,
    const int8_t* __restrict__ k_base, const float* __restrict__ k_scale,
    const int8_t* __restrict__ v_base, const float* __restrict__ v_scale,
    const int32_t* __restrict__ block_idx, uint16_t* __restrict__ out, int64_t kv_stride,
    int num_q, int num_kv, int block_size, int topk, int shift, int row_mask, int num_rows) {
  __shared__ __align__(16) uint8_t vlds[4][2][kSVBytesW];
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);  // wave-uniform
  const int lane = threadIdx.x & 63;
  const int row = blockIdx.x;
  if (row >= num_rows) return;
  const int dq = wave;  // the wave's quarter of the output dims
  const int t = row / num_kv;
  const int h = row - t * num_kv;
  const TokenPos tp = token_position(image, t);
  const int64_t cap = static_cast<int64_t>(tp.abs_pos) + 1;
  const int r16 = lane & 15;
  const int g = lane >> 4;
  const int gh = h * kSG + r16;  // q head of this lane's column
  const int64_t qrow = static_cast<int64_t>(t) * num_q + gh;

  // B operand of the scores: q codes of head r16, bytes 16g and 64 + 16g;
  // qsum = sum of the head's 128 codes (exact).
  const int8_t* qp = q_i8 + qrow * kSD + 16 * g;
  const uint4 qa = *reinterpret_cast<const uint4*>(qp);
  const uint4 qb4 = *reinterpret_cast<const uint4*>(qp + 64);
  int qsum = 0;
  {
    const uint32_t w8[8] = {qa.x, qa.y, qa.z, qa.w, qb4.x, qb4.y, qb4.z, qb4.w};
#pragma unroll
    for (int i = 0; i < 8; ++i)
      qsum += static_cast<int8_t>(w8[i]) + static_cast<int8_t>(w8[i] >> 8) +
              static_cast<int8_t>(w8[i] >> 16) + static_cast<int8_t>(w8[i] >> 24);
    qsum += __shfl_xor(qsum, 16);
    qsum += __shfl_xor(qsum, 32);
  }
  const float qbias = qi_bias[qrow];
  const float fq = f_q[qrow];
  const float inv127 = 1.0f / 127.0f;
  const float inv127sq = inv127 * inv127;

  const int8_t* kh = k_base + static_cast<int64_t>(h) * kSD;
  const int8_t* vh = v_base + static_cast<int64_t>(h) * kSD + kSDW * dq;
  const int32_t* brow = block_idx + static_cast<int64_t>(row) * topk;
  // V staging: lane takes 8 bytes (dims 8*(l%4) ..) of the wave's 32 dims of
  // row l/4 and writes them as 8 bf16 (exact); the transposing read as in
  // sparse_attention_kernel.
  const int vrow_l = lane >> 2;
  const int vcol = 8 * (lane & 3);
  const int tr_off = (4 * g + (r16 >> 2)) * kSVPitchW + 8 * (r16 & 3);

  auto page_row = [&](const TileCursor& c) -> int64_t {
    return sload(tp.rows + static_cast<int>(c.pos >> shift));
  };
  auto load_tile = [&](const TileCursor& c, int64_t prow) {
    BqSplitRegs d;
    const int tl = static_cast<int>(min<int64_t>(kTile, c.phi - c.pos));
    const int64_t base = prow + (static_cast<int>(c.pos) & row_mask);
    const int8_t* kp = kh + (base + (r16 < tl ? r16 : 0)) * kv_stride + 16 * g;
    d.k0 = *reinterpret_cast<const uint4*>(kp);
    d.k1 = *reinterpret_cast<const uint4*>(kp + 64);
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const int64_t sl = (base + (4 * g + j < tl ? 4 * g + j : 0)) * num_kv + h;
      d.ks[j] = k_scale[sl];
      d.vs[j] = v_scale[sl];
    }
    d.v = *reinterpret_cast<const uint2*>(vh + (base + (vrow_l < tl ? vrow_l : 0)) * kv_stride +
                                          vcol);
    return d;
  };

  float m = kNegBig;
  float lsum = 0.0f;
  f32x4_t acc[kSDW / 16];  // acc[b][j] = O[dim 32dq + 16b + 4g + j][head r16]
#pragma unroll
  for (int b = 0; b < kSDW / 16; ++b) acc[b] = f32x4_t{0.0f, 0.0f, 0.0f, 0.0f};

  // Values to LDS and the tile's scores; the caller then reuses the tile's
  // registers for the loads of a later tile.
  auto scores = [&](const BqSplitRegs& rg, const TileCursor& c, int buf, float (&sj)[4]) {
    const int tl = static_cast<int>(min<int64_t>(kTile, c.phi - c.pos));
    uint8_t* vb = vlds[wave][buf];
    wave_sync();
    {
      const uint32_t w8[2] = {rg.v.x, rg.v.y};
      uint32_t o16[4];
#pragma unroll
      for (int i = 0; i < 2; ++i) {
#pragma unroll
        for (int b = 0; b < 4; b += 2) {
          const float f0 = static_cast<float>(static_cast<int8_t>(w8[i] >> (8 * b)));
          const float f1 = static_cast<float>(static_cast<int8_t>(w8[i] >> (8 * b + 8)));
          o16[2 * i + b / 2] = (__float_as_uint(f0) >> 16) | (__float_as_uint(f1) & 0xFFFF0000u);
        }
      }
      *reinterpret_cast<uint4*>(vb + vrow_l * kSVPitchW + 2 * vcol) =
          make_uint4(o16[0], o16[1], o16[2], o16[3]);
    }
    i32x4_t si = {0, 0, 0, 0};
    si = __builtin_amdgcn_mfma_i32_16x16x64_i8(
        __builtin_bit_cast(i32x4_t, rg.k0), __builtin_bit_cast(i32x4_t, qa), si, 0, 0, 0);
    si = __builtin_amdgcn_mfma_i32_16x16x64_i8(
        __builtin_bit_cast(i32x4_t, rg.k1), __builtin_bit_cast(i32x4_t, qb4), si, 0, 0, 0);
    // Lane holds positions 4g + j of head r16.
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const float raw = static_cast<float>(si[j] + 128 * qsum);
      float sc = raw - qbias;
      sc = sc * fq;
      sc = sc * rg.ks[j];
      sc = sc * inv127sq;
      sj[j] = (4 * g + j < tl) ? sc : kNegBig;
    }
  };
  auto softmax_pv = [&](const float (&sj)[4], const float (&vsj)[4], const TileCursor& c,
                        int buf) {
    const int tl = static_cast<int>(min<int64_t>(kTile, c.phi - c.pos));
    uint8_t* vb = vlds[wave][buf];
    float tmax = max_ref(max_ref(sj[0], sj[1]), max_ref(sj[2], sj[3]));
    tmax = pair_max32(pair_max16(tmax));
    const float m_new = tmax > m ? tmax : m;
    const float corr = fexp(max_ref(-87.0f, m - m_new));
    float w[4];
#pragma unroll
    for (int j = 0; j < 4; ++j) w[j] = fexp(max_ref(-87.0f, sj[j] - m_new));
    float ws[4];
#pragma unroll
    for (int j = 0; j < 4; ++j) ws[j] = pair_sum16(pair_sum32(w[j]));
    const float wsum = (ws[0] + ws[2]) + (ws[1] + ws[3]);
    lsum = lsum * corr + wsum;
    m = m_new;
    s16x4_t phi, plo;
#pragma unroll
    for (int j = 0; j < 4; j += 2) {
      float p0 = w[j] * vsj[j];
      p0 = p0 * inv127;
      float p1 = w[j + 1] * vsj[j + 1];
      p1 = p1 * inv127;
      p0 = (4 * g + j < tl) ? p0 : 0.0f;
      p1 = (4 * g + j + 1 < tl) ? p1 : 0.0f;
      const bf16x2_t hb = __builtin_convertvector(f32x2_t{p0, p1}, bf16x2_t);
      const float r0 = p0 - static_cast<float>(hb[0]);
      const float r1 = p1 - static_cast<float>(hb[1]);
      const bf16x2_t lb = __builtin_convertvector(f32x2_t{r0, r1}, bf16x2_t);
      const s16x4_t hs = __builtin_bit_cast(s16x4_t, __builtin_shufflevector(hb, hb, 0, 1, 0, 1));
      const s16x4_t ls = __builtin_bit_cast(s16x4_t, __builtin_shufflevector(lb, lb, 0, 1, 0, 1));
      phi[j] = hs[0];
      phi[j + 1] = hs[1];
      plo[j] = ls[0];
      plo[j + 1] = ls[1];
    }
    wave_sync();
#pragma unroll
    for (int b = 0; b < kSDW / 16; ++b) {
      acc[b] = acc[b] * corr;
      const s16x4_t va =
          __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_s16x4_t*)(vb + tr_off + 32 * b));
      acc[b] = __builtin_amdgcn_mfma_f32_16x16x16bf16_1k(va, phi, acc[b], 0, 0, 0);
      acc[b] = __builtin_amdgcn_mfma_f32_16x16x16bf16_1k(va, plo, acc[b], 0, 0, 0);
    }
  };

  // Rotating register sets as in sparse_attention_kernel: unconditional
  // loads (past the block list they read the sequence's first row), leaving
  // the loop the only branch, page rows read one step ahead.
  auto advance = [&](const TileCursor& c) {
    return c.valid ? next_tile(c, brow, topk, block_size, cap) : c;
  };
  auto dummy_or = [&](const TileCursor& c) {
    TileCursor d = c;
    d.pos = c.valid ? c.pos : 0;
    d.phi = c.valid ? c.phi : kTile;
    return d;
  };
  TileCursor cs[kSAhead];
  BqSplitRegs rs[kSAhead];
  cs[0] = next_tile(TileCursor{-1, 0, 0, false}, brow, topk, block_size, cap);
#pragma unroll
  for (int i = 1; i < kSAhead; ++i) cs[i] = advance(cs[i - 1]);
#pragma unroll
  for (int i = 0; i < kSAhead; ++i) {
    const TileCursor d = dummy_or(cs[i]);
    rs[i] = load_tile(d, page_row(d));
    __builtin_amdgcn_sched_barrier(0);
  }
  TileCursor last = advance(cs[kSAhead - 1]);
  TileCursor pend = dummy_or(last);
  bool pend_valid = last.valid;
  int64_t pend_row = page_row(pend);
  int buf = 0;
  for (;;) {
#pragma unroll
    for (int s = 0; s < kSAhead; ++s) {
      if (!cs[s].valid) goto tiles_done;  // uniform
      const TileCursor c = cs[s];
      float sj[4], vsj[4];
      scores(rs[s], c, buf, sj);
#pragma unroll
      for (int j = 0; j < 4; ++j) vsj[j] = rs[s].vs[j];
      __builtin_amdgcn_sched_barrier(0);
      rs[s] = load_tile(pend, pend_row);
      __builtin_amdgcn_sched_barrier(0);
      cs[s] = pend;
      cs[s].valid = pend_valid;
      last = advance(last);
      pend_valid = last.valid;
      pend = dummy_or(last);
      pend_row = page_row(pend);
      softmax_pv(sj, vsj, c, buf);
      buf ^= 1;
    }
  }
tiles_done:
  {
    // write_finalized_head over one stripe.
    const float gm = m > kNegBig ? m : kNegBig;
    float cv = fexp(max_ref(-87.0f, m - gm));
    cv = lsum > 0.0f ? cv : 0.0f;
    const float gl = 0.0f + lsum * cv;
    const float inv = gl > 0.0f ? 1.0f / gl : 0.0f;
    uint16_t* orow = out + qrow * kSD + kSDW * dq + 4 * g;
#pragma unroll
    for (int b = 0; b < kSDW / 16; ++b) {
      uint32_t lo = 0, hi = 0;
      if (gl > 0.0f) {
        lo = f32_to_bf16_bits((acc[b][0] * cv) * inv) |
             (f32_to_bf16_bits((acc[b][1] * cv) * inv) << 16);
        hi = f32_to_bf16_bits((acc[b][2] * cv) * inv) |
             (f32_to_bf16_bits((acc[b][3] * cv) * inv) << 16);
      }
      *reinterpret_cast<uint2*>(orow + 16 * b) = make_uint2(lo, hi);
    }
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
  const auto* iq = static_cast<const uint16_t*>(index_q);
  const auto* ik = static_cast<const uint16_t*>(index_k);
  if (row_mask + 1 >= 64)
    hipLaunchKernelGGL((index_scores_kernel<128, 4, true>), grid, dim3(256), 0,
                       stream, image, iq, ik, scores, block_stride, block_size, scale, shift,
                       row_mask);
  else
    hipLaunchKernelGGL((index_scores_kernel<128, 4, false>), grid, dim3(256), 0,
                       stream, image, iq, ik, scores, block_stride, block_size, scale, shift,
                       row_mask);
  hipError_t err = hipGetLastError();
  if (err != hipSuccess) return err;
  const int rows = seq_len * num_heads;
  const int cap = select_bank_cap(topk);
  dim3 sgrid((rows + 3) / 4);
  if (cap == 16) {
    hipLaunchKernelGGL(select_blocks_kernel<16>, sgrid, dim3(256), 0, stream, image, scores,
                       block_idx, block_stride, num_heads, block_size, topk, local_blocks,
                       init_blocks, rows);
  } else if (cap == 32) {
    hipLaunchKernelGGL(select_blocks_kernel<32>, sgrid, dim3(256), 0, stream, image, scores,
                       block_idx, block_stride, num_heads, block_size, topk, local_blocks,
                       init_blocks, rows);
  } else if (cap == 64) {
    hipLaunchKernelGGL(select_blocks_kernel<64>, sgrid, dim3(256), 0, stream, image, scores,
                       block_idx, block_stride, num_heads, block_size, topk, local_blocks,
                       init_blocks, rows);
  } else {
    return hipErrorInvalidValue;
  }
  return hipGetLastError();
}

hipError_t launch_bq_block_sparse_attention(
    const int32_t* image, int seq_len, const void* q_i8, const float* qi_bias,
    const float* f_q, const void* k_base, const float* k_scale, const void* v_base,
    const float* v_scale, const int32_t* block_idx, void* output, float* partials,
    int64_t partial_stride, int64_t kv_stride, int num_q, int num_kv, int block_size,
    int topk, int decode_slots, int decode_workers, int shift, int row_mask,
    hipStream_t stream) {
  if (seq_len <= 0) return hipSuccess;
  const auto* q = static_cast<const int8_t*>(q_i8);
  const auto* k = static_cast<const int8_t*>(k_base);
  const auto* v = static_cast<const int8_t*>(v_base);
  auto* o = static_cast<uint16_t*>(output);
  if (seq_len == 1) {
    const int rows = decode_workers * num_kv;
    hipLaunchKernelGGL(bq_sparse_kernel<true>, dim3((rows + 3) / 4), dim3(256), 0, stream,
                       image, q, qi_bias, f_q, k, k_scale, v, v_scale, block_idx, o, partials,
                       partial_stride, kv_stride, num_q, num_kv, block_size, topk,
                       decode_slots, decode_workers, shift, row_mask, rows);
    hipError_t err = hipGetLastError();
    if (err != hipSuccess) return err;
    return launch_merge_stripes(partials, output, partial_stride, decode_workers, num_q,
                                stream);
  }
  const int rows = seq_len * num_kv;
  hipLaunchKernelGGL(bq_sparse_split_kernel, dim3(rows), dim3(256), 0, stream, image, q,
                     qi_bias, f_q, k, k_scale, v, v_scale, block_idx, o, kv_stride, num_q,
                     num_kv, block_size, topk, shift, row_mask, rows);
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
  hipLaunchKernelGGL(sparse_attention_kernel, dim3(rows), dim3(256), 0, stream,
                     image, static_cast<const uint16_t*>(q),
                     static_cast<const uint16_t*>(k_base), static_cast<const uint16_t*>(v_base),
                     block_idx, static_cast<uint16_t*>(output), kv_stride, num_q, num_kv,
                     block_size, topk, shift, row_mask, rows);
  return hipGetLastError();
}

}  // namespace ifr
