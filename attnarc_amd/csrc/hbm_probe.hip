// HBM probes used by bench.py to measure the attainable bandwidth of the box
// and to calibrate rocprofv3 byte counters against a kernel of known traffic.
// Not part of the loom_hip ABI.

#include <hip/hip_runtime.h>
#include <stdint.h>
#include <stdint.h>

typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));

// Reads n16 16-byte vectors once (grid-stride) and writes one word per thread
// so that the loads are not dead.
__global__ __launch_bounds__(256) void stream_read_kernel(const u32x4* __restrict__ src, uint64_t n16,
                                                          uint32_t* __restrict__ sink) {
  const uint64_t tid = static_cast<uint64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
  const uint64_t stride = static_cast<uint64_t>(gridDim.x) * blockDim.x;
  u32x4 acc = {0U, 0U, 0U, 0U};
  uint64_t i = tid;
  for (; i + 7 * stride < n16; i += 8 * stride) {
    u32x4 v[8];
#pragma unroll
    for (int k = 0; k < 8; ++k) v[k] = __builtin_nontemporal_load(&src[i + k * stride]);
#pragma unroll
    for (int k = 0; k < 8; ++k) acc ^= v[k];
  }
  for (; i < n16; i += stride) acc ^= src[i];
  sink[tid] = acc[0] ^ acc[1] ^ acc[2] ^ acc[3];
}

__global__ __launch_bounds__(256) void copy_kernel(const u32x4* __restrict__ src, u32x4* __restrict__ dst,
                                                   uint64_t n16) {
  const uint64_t tid = static_cast<uint64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
  const uint64_t stride = static_cast<uint64_t>(gridDim.x) * blockDim.x;
  for (uint64_t i = tid; i < n16; i += stride) dst[i] = src[i];
}

extern "C" int loom_hip_probe_stream_read(const void* src, uint64_t bytes, uint32_t* sink, uint32_t blocks,
                                          void* stream) {
  if (src == nullptr || sink == nullptr || bytes % 16 != 0 || blocks == 0) return 1;
  hipLaunchKernelGGL(stream_read_kernel, dim3(blocks), dim3(256), 0, static_cast<hipStream_t>(stream),
                     static_cast<const u32x4*>(src), bytes / 16, sink);
  return hipGetLastError() == hipSuccess ? 0 : 3;
}

extern "C" int loom_hip_probe_copy(const void* src, void* dst, uint64_t bytes, uint32_t blocks, void* stream) {
  if (src == nullptr || dst == nullptr || bytes % 16 != 0 || blocks == 0) return 1;
  hipLaunchKernelGGL(copy_kernel, dim3(blocks), dim3(256), 0, static_cast<hipStream_t>(stream),
                     static_cast<const u32x4*>(src), static_cast<u32x4*>(dst), bytes / 16);
  return hipGetLastError() == hipSuccess ? 0 : 3;
}

// Random-chunk gather: reads `chunks` chunks of `chunk_bytes` (a multiple of
// 256) at offsets perm[i] * chunk_bytes, 256 contiguous bytes per 16 lanes.
// Measures the bandwidth a paged access pattern of that granularity attains.
template <int kUnroll>
__global__ __launch_bounds__(256) void gather_read_kernel(const uint8_t* __restrict__ base,
                                                          const uint32_t* __restrict__ perm, uint32_t chunks,
                                                          uint32_t chunk_bytes, uint32_t* __restrict__ sink) {
  const uint32_t pieces_per_chunk = chunk_bytes / 256;
  const uint64_t pieces = static_cast<uint64_t>(chunks) * pieces_per_chunk;
  const uint64_t group = (static_cast<uint64_t>(blockIdx.x) * blockDim.x + threadIdx.x) / 16;
  const uint64_t groups = static_cast<uint64_t>(gridDim.x) * blockDim.x / 16;
  const uint32_t sub = threadIdx.x & 15U;
  u32x4 acc = {0U, 0U, 0U, 0U};
  uint64_t p = group;
  for (; p + (kUnroll - 1) * groups < pieces; p += kUnroll * groups) {
    u32x4 v[kUnroll];
#pragma unroll
    for (int k = 0; k < kUnroll; ++k) {
      const uint64_t q = p + k * groups;
      const uint64_t chunk = perm[q / pieces_per_chunk];
      v[k] = *reinterpret_cast<const u32x4*>(base + chunk * chunk_bytes + (q % pieces_per_chunk) * 256 + sub * 16);
    }
#pragma unroll
    for (int k = 0; k < kUnroll; ++k) acc ^= v[k];
  }
  for (; p < pieces; p += groups) {
    const uint64_t chunk = perm[p / pieces_per_chunk];
    acc ^= *reinterpret_cast<const u32x4*>(base + chunk * chunk_bytes + (p % pieces_per_chunk) * 256 + sub * 16);
  }
  sink[static_cast<uint64_t>(blockIdx.x) * blockDim.x + threadIdx.x] = acc[0] ^ acc[1] ^ acc[2] ^ acc[3];
}

extern "C" int loom_hip_probe_gather_read(const void* base, const uint32_t* perm, uint32_t chunks,
                                          uint32_t chunk_bytes, uint32_t* sink, uint32_t blocks, uint32_t unroll,
                                          void* stream) {
  if (base == nullptr || perm == nullptr || sink == nullptr || chunk_bytes % 256 != 0 || blocks == 0) return 1;
  auto kernel = unroll >= 32 ? gather_read_kernel<32> : unroll >= 16 ? gather_read_kernel<16> : gather_read_kernel<8>;
  hipLaunchKernelGGL(kernel, dim3(blocks), dim3(256), 0, static_cast<hipStream_t>(stream),
                     static_cast<const uint8_t*>(base), perm, chunks, chunk_bytes, sink);
  return hipGetLastError() == hipSuccess ? 0 : 3;
}
