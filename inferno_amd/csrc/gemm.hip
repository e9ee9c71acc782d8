// o_proj after the attention: out[m][n] = bf16(sum_k x[m][k] * w[n][k]) for
// bf16 x [seq_len][cols] and w [rows][cols], f32 accumulation
// (dispatch_gemm_cols, kernels/gemm.mojo:198-225, called at
// modeling/gemma_4_moe.mojo:387-392 and :485-490 with rows = HIDDEN).
//
// v_mfma_f32_16x16x32_bf16 with x as the A operand (16 token rows x 32 k)
// and w as B (32 k x 16 output columns): both fragments are 16-byte runs
// along k of one row, so w streams straight from HBM into registers and x is
// staged once per workgroup in LDS.  A workgroup covers 64 tokens x 64
// columns (4 waves x 16 columns, each wave up to 4 MFMA tiles down the
// tokens) over a k range.  Decode batches (<= 64 tokens) have too few tiles
// to fill 256 CUs: gemm_cols_split_kernel gives each workgroup a 512-wide k
// slice loaded in one round trip and writes f32 partials that
// gemm_cols_reduce_kernel adds in slice order.  Larger batches run
// gemm_cols_kernel, which walks k in double-buffered 128-wide chunks (and
// splits k the same way only while the grid is under 512 workgroups).
#include "common.hpp"
#include "launch.hpp"

namespace ifr {
namespace {

typedef __bf16 bf16x8_t __attribute__((ext_vector_type(8)));
typedef float f32x4_t __attribute__((ext_vector_type(4)));
typedef uint32_t u32x4_t __attribute__((ext_vector_type(4)));

constexpr int kBM = 64;               // token rows per workgroup
constexpr int kBN = 64;               // output columns per workgroup
constexpr int kKC = 128;              // k per LDS chunk
constexpr int kPitch = kKC + 8;       // LDS row pitch in bf16 (272 B: rows 4 banks apart)
constexpr int kSegs = kBM * kKC / 8;  // 16-byte x segments per chunk
constexpr int kSegsPerThread = kSegs / 256;
constexpr int kMaxSplits = 16;        // k slices the reduce adds

template <bool kStream>
__device__ __forceinline__ uint4 load_w(const uint16_t* p) {
  if constexpr (kStream) {
    const u32x4_t v = __builtin_nontemporal_load(reinterpret_cast<const u32x4_t*>(p));
    return make_uint4(v.x, v.y, v.z, v.w);
  } else {
    return *reinterpret_cast<const uint4*>(p);
  }
}

// kStream: w is read by one token tile only (decode), so its loads bypass
// the caches' retention.  kSplit: write f32 partials [split][m][n] instead of
// bf16 outputs.
template <bool kStream, bool kSplit>
__global__ __launch_bounds__(256) void gemm_cols_kernel(
    const uint16_t* __restrict__ x, const uint16_t* __restrict__ w,
    uint16_t* __restrict__ out, float* __restrict__ part, int M, int N, int K,
    int k_span) {
  __shared__ __align__(16) uint16_t xs[2][kBM * kPitch];
  const int wave = threadIdx.x >> 6;
  const int lane = threadIdx.x & 63;
  const int r = lane & 15;
  const int g = lane >> 4;
  const int n0 = blockIdx.x * kBN + wave * 16;
  const int m0 = blockIdx.y * kBM;
  const int k0 = blockIdx.z * k_span;
  const bool live = n0 < N;  // a wave past the last column still stages x
  const uint16_t* wp = w + static_cast<int64_t>(live ? n0 + r : 0) * K + k0 + 8 * g;

  // x staging: thread t moves segments t, t+256, ... (row s/16, 8 bf16 at
  // 8*(s%16)); rows past M repeat row M-1 and are never stored.
  const uint16_t* xsrc[kSegsPerThread];
  int xdst[kSegsPerThread];
#pragma unroll
  for (int i = 0; i < kSegsPerThread; ++i) {
    const int s = threadIdx.x + 256 * i;
    const int row = s >> 4;
    const int col = (s & 15) * 8;
    xsrc[i] = x + static_cast<int64_t>(min(m0 + row, M - 1)) * K + k0 + col;
    xdst[i] = row * kPitch + col;
  }

  const int chunks = k_span / kKC;
  uint4 xr[kSegsPerThread];
  uint4 wr[kKC / 32];
#pragma unroll
  for (int i = 0; i < kSegsPerThread; ++i) xr[i] = *reinterpret_cast<const uint4*>(xsrc[i]);
  if (live) {
#pragma unroll
    for (int j = 0; j < kKC / 32; ++j) wr[j] = load_w<kStream>(wp + 32 * j);
  }
#pragma unroll
  for (int i = 0; i < kSegsPerThread; ++i)
    *reinterpret_cast<uint4*>(&xs[0][xdst[i]]) = xr[i];
  __syncthreads();

  f32x4_t acc[kBM / 16];
#pragma unroll
  for (int t = 0; t < kBM / 16; ++t) acc[t] = f32x4_t{0.0f, 0.0f, 0.0f, 0.0f};

  for (int c = 0; c < chunks; ++c) {
    const int buf = c & 1;
    const bool more = c + 1 < chunks;
    uint4 wn[kKC / 32];
    if (more) {
      const int koff = (c + 1) * kKC;
#pragma unroll
      for (int i = 0; i < kSegsPerThread; ++i)
        xr[i] = *reinterpret_cast<const uint4*>(xsrc[i] + koff);
      if (live) {
#pragma unroll
        for (int j = 0; j < kKC / 32; ++j) wn[j] = load_w<kStream>(wp + koff + 32 * j);
      }
    }
    if (live) {
      const uint16_t* xb = &xs[buf][r * kPitch + 8 * g];
#pragma unroll
      for (int j = 0; j < kKC / 32; ++j) {
        const bf16x8_t b = __builtin_bit_cast(bf16x8_t, wr[j]);
#pragma unroll
        for (int t = 0; t < kBM / 16; ++t) {
          const uint4 av = *reinterpret_cast<const uint4*>(xb + 16 * t * kPitch + 32 * j);
          acc[t] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8_t, av), b,
                                                           acc[t], 0, 0, 0);
        }
      }
    }
    if (more) {
#pragma unroll
      for (int i = 0; i < kSegsPerThread; ++i)
        *reinterpret_cast<uint4*>(&xs[buf ^ 1][xdst[i]]) = xr[i];
#pragma unroll
      for (int j = 0; j < kKC / 32; ++j) wr[j] = wn[j];
    }
    __syncthreads();
  }

  if (!live) return;
  // C layout: acc[t][j] is token m0 + 16t + 4g + j, column n0 + r.
#pragma unroll
  for (int t = 0; t < kBM / 16; ++t) {
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const int m = m0 + 16 * t + 4 * g + j;
      if (m >= M) continue;
      const int64_t o = static_cast<int64_t>(m) * N + n0 + r;
      if constexpr (kSplit) {
        part[static_cast<int64_t>(blockIdx.z) * M * N + o] = acc[t][j];
      } else {
        out[o] = static_cast<uint16_t>(f32_to_bf16_bits(acc[t][j]));
      }
    }
  }
}

// Decode batches (M <= 64 tokens): one workgroup takes 64 columns and one
// 512-wide slice of k, and issues every load of the slice at once (16
// weight loads a lane straight into registers, the x slice of TM 16-row
// tiles into LDS), so the slice costs one memory round trip.  Partials f32
// [split][m][n].
template <int TM, int kSpan>
__global__ __launch_bounds__(256) void gemm_cols_split_kernel(
    const uint16_t* __restrict__ x, const uint16_t* __restrict__ w, float* __restrict__ part,
    int M, int N, int K) {
  constexpr int kSpanPitch = kSpan + 8;  // rows 4 banks apart
  __shared__ __align__(16) uint16_t xs[TM * 16 * kSpanPitch];
  constexpr int kXSegs = TM * 16 * (kSpan / 8) / 256;  // 16-byte x segments a thread
  const int wave = threadIdx.x >> 6;
  const int lane = threadIdx.x & 63;
  const int r = lane & 15;
  const int g = lane >> 4;
  const int n0 = blockIdx.x * kBN + wave * 16;
  const int k0 = blockIdx.y * kSpan;
  const bool live = n0 < N;

  uint4 wr[kSpan / 32];
  if (live) {
    const uint16_t* wp = w + static_cast<int64_t>(n0 + r) * K + k0 + 8 * g;
#pragma unroll
    for (int j = 0; j < kSpan / 32; ++j) wr[j] = load_w<true>(wp + 32 * j);
  }
  uint4 xr[kXSegs];
#pragma unroll
  for (int i = 0; i < kXSegs; ++i) {
    const int seg = threadIdx.x + 256 * i;
    const int row = seg / (kSpan / 8);
    const int col = (seg % (kSpan / 8)) * 8;
    xr[i] = *reinterpret_cast<const uint4*>(x + static_cast<int64_t>(min(row, M - 1)) * K +
                                            k0 + col);
  }
#pragma unroll
  for (int i = 0; i < kXSegs; ++i) {
    const int seg = threadIdx.x + 256 * i;
    const int row = seg / (kSpan / 8);
    const int col = (seg % (kSpan / 8)) * 8;
    *reinterpret_cast<uint4*>(&xs[row * kSpanPitch + col]) = xr[i];
  }
  __syncthreads();
  if (!live) return;

  f32x4_t acc[TM];
#pragma unroll
  for (int t = 0; t < TM; ++t) acc[t] = f32x4_t{0.0f, 0.0f, 0.0f, 0.0f};
  const uint16_t* xb = &xs[r * kSpanPitch + 8 * g];
#pragma unroll
  for (int j = 0; j < kSpan / 32; ++j) {
    const bf16x8_t b = __builtin_bit_cast(bf16x8_t, wr[j]);
#pragma unroll
    for (int t = 0; t < TM; ++t) {
      const uint4 av = *reinterpret_cast<const uint4*>(xb + 16 * t * kSpanPitch + 32 * j);
      acc[t] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8_t, av), b,
                                                       acc[t], 0, 0, 0);
    }
  }
  float* pz = part + static_cast<int64_t>(blockIdx.y) * M * N;
#pragma unroll
  for (int t = 0; t < TM; ++t) {
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const int m = 16 * t + 4 * g + j;
      if (m < M) pz[static_cast<int64_t>(m) * N + n0 + r] = acc[t][j];
    }
  }
}

// out = bf16(part[0] + part[1] + ... + part[NS-1]), four columns a thread:
// every load issues before the first add, the adds run in split order.
template <int NS>
__global__ __launch_bounds__(256) void gemm_cols_reduce_kernel(
    const float* __restrict__ part, uint16_t* __restrict__ out, int64_t quads, int64_t mn) {
  const int64_t i = static_cast<int64_t>(blockIdx.x) * 256 + threadIdx.x;
  if (i >= quads) return;
  float4 v[NS];
#pragma unroll
  for (int z = 0; z < NS; ++z) v[z] = reinterpret_cast<const float4*>(part + z * mn)[i];
  float4 s = v[0];
#pragma unroll
  for (int z = 1; z < NS; ++z) {
    s.x = s.x + v[z].x;
    s.y = s.y + v[z].y;
    s.z = s.z + v[z].z;
    s.w = s.w + v[z].w;
  }
  const uint32_t lo = f32_to_bf16_bits(s.x) | (f32_to_bf16_bits(s.y) << 16);
  const uint32_t hi = f32_to_bf16_bits(s.z) | (f32_to_bf16_bits(s.w) << 16);
  reinterpret_cast<uint2*>(out)[i] = make_uint2(lo, hi);
}

template <int NS>
hipError_t launch_reduce_n(const float* part, uint16_t* out, int64_t quads, int64_t mn,
                           int splits, hipStream_t stream) {
  if constexpr (NS > kMaxSplits) {
    return hipErrorInvalidValue;
  } else {
    if (splits != NS) return launch_reduce_n<NS + 1>(part, out, quads, mn, splits, stream);
    hipLaunchKernelGGL((gemm_cols_reduce_kernel<NS>),
                       dim3(static_cast<unsigned>((quads + 255) / 256)), dim3(256), 0, stream,
                       part, out, quads, mn);
    return hipGetLastError();
  }
}

// k slice of gemm_cols_split_kernel, or 0 when the batch takes gemm_cols_kernel.
int decode_span(int64_t M, int64_t K) {
  if (M <= 16 && K % 256 == 0 && K / 256 <= kMaxSplits) return 256;
  if (M <= kBM && K % 512 == 0 && K / 512 <= kMaxSplits) return 512;
  return 0;
}

}  // namespace

int gemm_cols_splits(int64_t M, int64_t N, int64_t K) {
  const int span = decode_span(M, K);
  if (span) return static_cast<int>(K / span);
  const int64_t tiles = ((N + kBN - 1) / kBN) * ((M + kBM - 1) / kBM);
  const int64_t chunks = K / kKC;
  int splits = 1;
  while (tiles * splits * 2 <= 512 && chunks % (splits * 2) == 0 && splits * 2 <= kMaxSplits)
    splits *= 2;
  return splits;
}

int64_t gemm_cols_workspace_bytes(int64_t M, int64_t N, int64_t K) {
  const int splits = gemm_cols_splits(M, N, K);
  const bool sliced = decode_span(M, K) != 0;  // always writes partials
  return splits > 1 || sliced ? static_cast<int64_t>(splits) * M * N * 4 : 0;
}

hipError_t launch_gemm_cols(const void* x, const void* w, void* out, float* workspace,
                            int64_t M, int64_t N, int64_t K, hipStream_t stream) {
  if (M <= 0) return hipSuccess;
  const int splits = gemm_cols_splits(M, N, K);
  const int k_span = static_cast<int>(K / splits);
  dim3 grid(static_cast<unsigned>((N + kBN - 1) / kBN),
            static_cast<unsigned>((M + kBM - 1) / kBM), static_cast<unsigned>(splits));
  const auto* xp = static_cast<const uint16_t*>(x);
  const auto* wp = static_cast<const uint16_t*>(w);
  auto* op = static_cast<uint16_t*>(out);
  const bool stream_w = grid.y == 1;
  if (const int span = decode_span(M, K)) {
    dim3 sgrid(grid.x, static_cast<unsigned>(splits));
    const int tm = static_cast<int>((M + 15) / 16);
    const int m = static_cast<int>(M), n = static_cast<int>(N), k = static_cast<int>(K);
    if (span == 256) {  // M <= 16
      hipLaunchKernelGGL((gemm_cols_split_kernel<1, 256>), sgrid, dim3(256), 0, stream, xp,
                         wp, workspace, m, n, k);
    } else if (tm == 1) {
      hipLaunchKernelGGL((gemm_cols_split_kernel<1, 512>), sgrid, dim3(256), 0, stream, xp,
                         wp, workspace, m, n, k);
    } else if (tm == 2) {
      hipLaunchKernelGGL((gemm_cols_split_kernel<2, 512>), sgrid, dim3(256), 0, stream, xp,
                         wp, workspace, m, n, k);
    } else if (tm == 3) {
      hipLaunchKernelGGL((gemm_cols_split_kernel<3, 512>), sgrid, dim3(256), 0, stream, xp,
                         wp, workspace, m, n, k);
    } else {
      hipLaunchKernelGGL((gemm_cols_split_kernel<4, 512>), sgrid, dim3(256), 0, stream, xp,
                         wp, workspace, m, n, k);
    }
    hipError_t err = hipGetLastError();
    if (err != hipSuccess) return err;
    return launch_reduce_n<1>(workspace, op, M * N / 4, M * N, splits, stream);
  }
  if (splits > 1) {
    if (stream_w) {
      hipLaunchKernelGGL((gemm_cols_kernel<true, true>), grid, dim3(256), 0, stream, xp, wp,
                         op, workspace, static_cast<int>(M), static_cast<int>(N),
                         static_cast<int>(K), k_span);
    } else {
      hipLaunchKernelGGL((gemm_cols_kernel<false, true>), grid, dim3(256), 0, stream, xp, wp,
                         op, workspace, static_cast<int>(M), static_cast<int>(N),
                         static_cast<int>(K), k_span);
    }
    hipError_t err = hipGetLastError();
    if (err != hipSuccess) return err;
    return launch_reduce_n<1>(workspace, op, M * N / 4, M * N, splits, stream);
  } else if (stream_w) {
    hipLaunchKernelGGL((gemm_cols_kernel<true, false>), grid, dim3(256), 0, stream, xp, wp, op,
                       nullptr, static_cast<int>(M), static_cast<int>(N), static_cast<int>(K),
                       k_span);
  } else {
    hipLaunchKernelGGL((gemm_cols_kernel<false, false>), grid, dim3(256), 0, stream, xp, wp,
                       op, nullptr, static_cast<int>(M), static_cast<int>(N),
                       static_cast<int>(K), k_span);
  }
  return hipGetLastError();
}

}  // namespace ifr
