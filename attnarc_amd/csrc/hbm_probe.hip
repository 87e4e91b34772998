// HBM probes used by bench.py to measure the attainable bandwidth of the box
// and to calibrate rocprofv3 byte counters against a kernel of known traffic.
// Not part of the loom_hip ABI.

#include <hip/hip_runtime.h>
#include <stdint.h>

typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));

// Reads n16 16-byte vectors once with non-temporal loads: workgroup b reads
// the contiguous range [b * n16 / grid, (b + 1) * n16 / grid), eight loads
// per thread in flight, and writes one word per thread so that the loads are
// not dead. (A grid-stride order, each load instruction of the grid 1 KiB
// apart per wave, measured 6.4 TB/s; contiguous ranges per workgroup 7.0-7.1;
// the same ranges without the non-temporal hint 6.1-6.2.)
__global__ __launch_bounds__(256) void stream_read_kernel(const u32x4* __restrict__ src, uint64_t n16,
                                                          uint32_t* __restrict__ sink) {
  const uint64_t lo = n16 * blockIdx.x / gridDim.x;
  const uint64_t hi = n16 * (blockIdx.x + 1ULL) / gridDim.x;
  u32x4 acc = {0U, 0U, 0U, 0U};
  for (uint64_t i = lo + threadIdx.x; i < hi; i += 8ULL * blockDim.x) {
    u32x4 v[8];
#pragma unroll
    for (int k = 0; k < 8; ++k) {
      const uint64_t j = i + static_cast<uint64_t>(k) * blockDim.x;
      v[k] = j < hi ? __builtin_nontemporal_load(&src[j]) : u32x4{0U, 0U, 0U, 0U};
    }
#pragma unroll
    for (int k = 0; k < 8; ++k) acc ^= v[k];
  }
  sink[static_cast<uint64_t>(blockIdx.x) * blockDim.x + threadIdx.x] = acc[0] ^ acc[1] ^ acc[2] ^ acc[3];
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

// Contiguous-slice read: workgroup b of `blocks` reads bytes [b * bytes / blocks,
// (b + 1) * bytes / blocks), eight 16-byte loads per thread in flight. With
// one workgroup on each of n CUs it measures what n CUs can pull (a
// single-partition decode over n work items uses n CUs).
__global__ __launch_bounds__(512) void slice_read_kernel(const u32x4* __restrict__ src, uint64_t n16_per_block,
                                                         uint32_t* __restrict__ sink) {
  const u32x4* p = src + static_cast<uint64_t>(blockIdx.x) * n16_per_block;
  u32x4 acc = {0U, 0U, 0U, 0U};
  for (uint64_t i = threadIdx.x; i < n16_per_block; i += 8ULL * blockDim.x) {
    u32x4 v[8];
#pragma unroll
    for (int k = 0; k < 8; ++k) {
      const uint64_t j = i + static_cast<uint64_t>(k) * blockDim.x;
      v[k] = j < n16_per_block ? __builtin_nontemporal_load(&p[j]) : u32x4{0U, 0U, 0U, 0U};
    }
#pragma unroll
    for (int k = 0; k < 8; ++k) acc ^= v[k];
  }
  sink[static_cast<uint64_t>(blockIdx.x) * blockDim.x + threadIdx.x] = acc[0] ^ acc[1] ^ acc[2] ^ acc[3];
}

extern "C" int loom_hip_probe_slice_read(const void* src, uint64_t bytes, uint32_t* sink, uint32_t blocks,
                                         void* stream) {
  if (src == nullptr || sink == nullptr || blocks == 0 || bytes % (16ULL * blocks) != 0) return 1;
  hipLaunchKernelGGL(slice_read_kernel, dim3(blocks), dim3(512), 0, static_cast<hipStream_t>(stream),
                     static_cast<const u32x4*>(src), bytes / 16 / blocks, sink);
  return hipGetLastError() == hipSuccess ? 0 : 3;
}

// Random-chunk gather: the buffer is `chunks` chunks of `chunk_bytes` (a
// multiple of 16) and workgroup w reads chunks perm[w], perm[w + grid], ...
// whole, 16 bytes per lane and eight non-temporal loads per thread in
// flight (as the decode kernels load K/V). It is the attainable rate of a
// paged access pattern (K/V blocks scattered by a block table) with no
// computation. (Spreading each chunk over several workgroups
// measured 0.1-0.2 TB/s slower.)
__global__ __launch_bounds__(256) void gather_read_kernel(const uint8_t* __restrict__ base,
                                                          const uint32_t* __restrict__ perm, uint32_t chunks,
                                                          uint32_t chunk_bytes, uint32_t* __restrict__ sink) {
  const uint32_t per_round = 8U * blockDim.x * 16U;
  u32x4 acc = {0U, 0U, 0U, 0U};
  for (uint32_t c = blockIdx.x; c < chunks; c += gridDim.x) {
    const uint8_t* p = base + static_cast<uint64_t>(perm[c]) * chunk_bytes;
    for (uint32_t r = 0; r < chunk_bytes; r += per_round) {
      u32x4 v[8];
#pragma unroll
      for (int k = 0; k < 8; ++k) {
        const uint32_t off = r + (k * blockDim.x + threadIdx.x) * 16U;
        v[k] = off < chunk_bytes ? __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(p + off))
                                 : u32x4{0U, 0U, 0U, 0U};
      }
#pragma unroll
      for (int k = 0; k < 8; ++k) acc ^= v[k];
    }
  }
  sink[static_cast<uint64_t>(blockIdx.x) * blockDim.x + threadIdx.x] = acc[0] ^ acc[1] ^ acc[2] ^ acc[3];
}

extern "C" int loom_hip_probe_gather_read(const void* base, const uint32_t* perm, uint32_t chunks,
                                          uint32_t chunk_bytes, uint32_t* sink, uint32_t blocks, void* stream) {
  if (base == nullptr || perm == nullptr || sink == nullptr || chunk_bytes % 16 != 0 || blocks == 0) return 1;
  hipLaunchKernelGGL(gather_read_kernel, dim3(blocks), dim3(256), 0, static_cast<hipStream_t>(stream),
                     static_cast<const uint8_t*>(base), perm, chunks, chunk_bytes, sink);
  return hipGetLastError() == hipSuccess ? 0 : 3;
}

// Load-policy probe: the same contiguous ranges as stream_read_kernel, read
// with plain 16-byte loads (kPolicy 0), non-temporal 16-byte loads (1), LDS
// DMA (global_load_lds_dwordx4, 2) or LDS DMA with the non-temporal hint (3).
// The DMA forms keep eight 1 KiB loads per wave in flight into a ring of
// 8 KiB per wave, as the decode kernels' K/V stages do.
template <int kPolicy>
__global__ __launch_bounds__(256) void policy_read_kernel(const u32x4* __restrict__ src, uint64_t n16,
                                                          uint32_t* __restrict__ sink) {
  const uint64_t lo = n16 * blockIdx.x / gridDim.x;
  const uint64_t hi = n16 * (blockIdx.x + 1ULL) / gridDim.x;
  if constexpr (kPolicy < 2) {
    u32x4 acc = {0U, 0U, 0U, 0U};
    for (uint64_t i = lo + threadIdx.x; i < hi; i += 8ULL * blockDim.x) {
      u32x4 v[8];
#pragma unroll
      for (int k = 0; k < 8; ++k) {
        const uint64_t j = i + static_cast<uint64_t>(k) * blockDim.x;
        v[k] = j < hi ? (kPolicy == 1 ? __builtin_nontemporal_load(&src[j]) : src[j]) : u32x4{0U, 0U, 0U, 0U};
      }
#pragma unroll
      for (int k = 0; k < 8; ++k) acc ^= v[k];
    }
    sink[static_cast<uint64_t>(blockIdx.x) * blockDim.x + threadIdx.x] = acc[0] ^ acc[1] ^ acc[2] ^ acc[3];
  } else {
    __shared__ __attribute__((aligned(16))) uint8_t ring[4][8 * 1024];
    const uint32_t wave = threadIdx.x >> 6, lane = threadIdx.x & 63U;
    // Whole 1 KiB pieces of this workgroup's range, split over its 4 waves.
    const uint64_t first = (lo * 16 + 1023) / 1024, last = hi * 16 / 1024;
    const uint32_t base = __builtin_amdgcn_readfirstlane(
        static_cast<uint32_t>(reinterpret_cast<uintptr_t>((__attribute__((address_space(3))) uint8_t*)ring[wave])));
    const uint8_t* bytes = reinterpret_cast<const uint8_t*>(src);
    uint32_t k = 0;
    for (uint64_t piece = first + wave; piece < last; piece += 4, ++k) {
      const void* addr = bytes + piece * 1024 + lane * 16;
      const uint32_t m0 = base + (k & 7U) * 1024;
      if constexpr (kPolicy == 3) {
        asm volatile("s_mov_b32 m0, %1\n\tglobal_load_lds_dwordx4 %0, off nt" : : "v"(addr), "s"(m0) : "memory", "m0");
      } else {
        asm volatile("s_mov_b32 m0, %1\n\tglobal_load_lds_dwordx4 %0, off" : : "v"(addr), "s"(m0) : "memory", "m0");
      }
      if (k >= 7) asm volatile("s_waitcnt vmcnt(7)" : : : "memory");
    }
    asm volatile("s_waitcnt vmcnt(0)" : : : "memory");
    __syncthreads();
    sink[static_cast<uint64_t>(blockIdx.x) * blockDim.x + threadIdx.x] = ring[wave][lane * 4];
  }
}

extern "C" int loom_hip_probe_policy_read(const void* src, uint64_t bytes, uint32_t* sink, uint32_t blocks,
                                          uint32_t policy, void* stream) {
  if (src == nullptr || sink == nullptr || bytes % 16 != 0 || blocks == 0 || policy > 3) return 1;
  const hipStream_t s = static_cast<hipStream_t>(stream);
  const u32x4* p = static_cast<const u32x4*>(src);
  switch (policy) {
    case 0: hipLaunchKernelGGL(policy_read_kernel<0>, dim3(blocks), dim3(256), 0, s, p, bytes / 16, sink); break;
    case 1: hipLaunchKernelGGL(policy_read_kernel<1>, dim3(blocks), dim3(256), 0, s, p, bytes / 16, sink); break;
    case 2: hipLaunchKernelGGL(policy_read_kernel<2>, dim3(blocks), dim3(256), 0, s, p, bytes / 16, sink); break;
    default: hipLaunchKernelGGL(policy_read_kernel<3>, dim3(blocks), dim3(256), 0, s, p, bytes / 16, sink); break;
  }
  return hipGetLastError() == hipSuccess ? 0 : 3;
}
