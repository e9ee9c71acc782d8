// Page copy (copy-on-write of prefix pages), row gather and the seeded
// synthetic-input generator for gfx950.  All three are HBM streams: 16-byte
// vector loads and stores, one workgroup per chunk or row.
#include "common.hpp"
#include "launch.hpp"

namespace ifr {
namespace {

// Page copies stream through once: non-temporal loads and stores keep them
// from displacing the caches' working set (config 9: 4.60 -> 4.70 TB/s; the
// runtime's own 1 GiB device copy measures 5.0 TB/s).  The row gather keeps
// ordinary loads and stores (non-temporal measured 8 % slower there).
typedef unsigned int cu32x4_t __attribute__((ext_vector_type(4)));
__device__ __forceinline__ uint4 load_stream(const uint4* p) {
  const cu32x4_t v = __builtin_nontemporal_load(reinterpret_cast<const cu32x4_t*>(p));
  return make_uint4(v.x, v.y, v.z, v.w);
}
__device__ __forceinline__ void store_stream(uint4* p, uint4 v) {
  __builtin_nontemporal_store(cu32x4_t{v.x, v.y, v.z, v.w}, reinterpret_cast<cu32x4_t*>(p));
}

// PageCopyKernel (kernels/page_copy.mojo:25-60): the host splits every
// CopyJob into chunks of at most kCopyChunk bytes; one workgroup copies one
// chunk.  A chunk whose source and destination addresses agree modulo 16
// is copied as a byte head up to 16-byte alignment, 16-byte vectors (four
// loads in flight per thread before their stores) and a byte tail; any other
// chunk byte by byte.  The choice is per chunk, so one odd job does not slow
// the others of its call.
__global__ __launch_bounds__(256) void copy_chunks_kernel(
    uint8_t* __restrict__ arena, const int64_t* __restrict__ chunks) {
  const int64_t* ch = chunks + static_cast<int64_t>(blockIdx.x) * 4;
  const int64_t src = ch[0], dst = ch[1], bytes = ch[2];
  const int tid = threadIdx.x;
  const uintptr_t sa = reinterpret_cast<uintptr_t>(arena + src);
  const uintptr_t da = reinterpret_cast<uintptr_t>(arena + dst);
  if (((sa ^ da) & 15) != 0) {
    for (int64_t i = tid; i < bytes; i += blockDim.x) arena[dst + i] = arena[src + i];
    return;
  }
  const int64_t head = min<int64_t>(static_cast<int64_t>((16 - (da & 15)) & 15), bytes);
  if (tid < head) arena[dst + tid] = arena[src + tid];
  const int64_t n16 = (bytes - head) >> 4;
  const uint4* s = reinterpret_cast<const uint4*>(arena + src + head);
  uint4* d = reinterpret_cast<uint4*>(arena + dst + head);
  constexpr int kIn = 4;  // loads in flight per thread
  int64_t i = tid;
  for (; i + (kIn - 1) * 256 < n16; i += kIn * 256) {
    uint4 v[kIn];
#pragma unroll
    for (int u = 0; u < kIn; ++u) v[u] = load_stream(s + i + u * 256);
#pragma unroll
    for (int u = 0; u < kIn; ++u) store_stream(d + i + u * 256, v[u]);
  }
  for (; i < n16; i += 256) store_stream(d + i, load_stream(s + i));
  const int64_t tail0 = head + (n16 << 4);
  if (tail0 + tid < bytes) arena[dst + tail0 + tid] = arena[src + tail0 + tid];
}

// GatherRowsKernel (kernels/gather.mojo:8-27): one workgroup per output row.
__global__ __launch_bounds__(256) void gather_rows_kernel(
    const uint16_t* __restrict__ src, uint16_t* __restrict__ dst,
    const int32_t* __restrict__ rows, int cols) {
  const int j = blockIdx.x;
  const int64_t r = rows[j];
  const uint16_t* s = src + r * cols;
  uint16_t* d = dst + static_cast<int64_t>(j) * cols;
  if ((cols & 7) == 0) {
    const uint4* s4 = reinterpret_cast<const uint4*>(s);
    uint4* d4 = reinterpret_cast<uint4*>(d);
    for (int i = threadIdx.x; i < cols / 8; i += blockDim.x) d4[i] = s4[i];
  } else {
    for (int i = threadIdx.x; i < cols; i += blockDim.x) d[i] = s[i];
  }
}

__device__ __forceinline__ uint64_t splitmix64(uint64_t x) {
  uint64_t z = x + 0x9E3779B97F4A7C15ull;
  z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ull;
  z = (z ^ (z >> 27)) * 0x94D049BB133111EBull;
  return z ^ (z >> 31);
}

// rng_uniform (simd_math/sampling_rng.mojo:30-35).
__device__ __forceinline__ float rng_uniform(uint64_t seed, uint64_t counter) {
  const uint64_t h = splitmix64(seed ^ splitmix64(counter));
  return (static_cast<float>(static_cast<int64_t>(h >> 40)) + 1.0f) /
         (16777216.0f + 1.0f);
}

__global__ __launch_bounds__(256) void fill_normal_bf16_kernel(
    uint16_t* __restrict__ dst, int64_t n, uint64_t seed,
    int64_t outlier_every, float outlier_scale) {
  const int64_t stride = static_cast<int64_t>(gridDim.x) * blockDim.x;
  for (int64_t i = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
       i < n; i += stride) {
    const uint64_t c = 2ull * static_cast<uint64_t>(i);
    const float u1 = rng_uniform(seed, c);
    const float u2 = rng_uniform(seed, c + 1);
    float z = sqrtf(-2.0f * logf(u1)) * cosf(6.28318530717958648f * u2);
    if (outlier_every > 0 &&
        splitmix64(seed ^ 0x5DEECE66Dull ^ static_cast<uint64_t>(i)) %
                static_cast<uint64_t>(outlier_every) == 0)
      z = z * outlier_scale;
    dst[i] = static_cast<uint16_t>(f32_to_bf16_bits(z));
  }
}

}  // namespace

hipError_t launch_copy_chunks(void* arena, const int64_t* chunks, int num_chunks,
                              hipStream_t stream) {
  if (num_chunks <= 0) return hipSuccess;
  hipLaunchKernelGGL(copy_chunks_kernel, dim3(num_chunks), dim3(256), 0,
                     stream, static_cast<uint8_t*>(arena), chunks);
  return hipGetLastError();
}

hipError_t launch_gather_rows(const void* src, void* dst, const int32_t* rows,
                              int num_rows, int cols, hipStream_t stream) {
  if (num_rows <= 0) return hipSuccess;
  hipLaunchKernelGGL(gather_rows_kernel, dim3(num_rows), dim3(256), 0, stream,
                     static_cast<const uint16_t*>(src),
                     static_cast<uint16_t*>(dst), rows, cols);
  return hipGetLastError();
}

hipError_t launch_fill_normal_bf16(void* dst, int64_t n, uint64_t seed,
                                   int64_t outlier_every, float outlier_scale,
                                   hipStream_t stream) {
  if (n <= 0) return hipSuccess;
  int64_t blocks = (n + 255) / 256;
  if (blocks > 65536) blocks = 65536;
  hipLaunchKernelGGL(fill_normal_bf16_kernel, dim3(static_cast<unsigned>(blocks)),
                     dim3(256), 0, stream, static_cast<uint16_t*>(dst), n, seed,
                     outlier_every, outlier_scale);
  return hipGetLastError();
}

}  // namespace ifr
