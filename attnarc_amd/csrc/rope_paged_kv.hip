// Fused rotary embedding + paged K/V cache write for MI355X (gfx950).
//
// Replaces loom_cuda_rope_paged_kv_write_{f32,f16,bf16}
// (crates/loom-cuda-sys/cuda/include/loom_cuda.h:252-318). Semantics follow
// the Loom Kernels contract (crates/loom-kernels/src/rope_kv.rs:513-631):
//   - Q and K rows are rotated in place over the first rotary_dim dims, NeoX
//     (pair p with p + rotary_dim / 2) or interleaved (2p with 2p + 1), in F32
//     products and sums without fused multiply-add, rounded once to the
//     storage type (rope_kv.rs:759-777);
//   - for tokens below cache_tokens whose slot is non-negative and inside the
//     cache, the rotated K row (rotary part, then the unrotated tail) and the
//     V row are written to slot (block = slot / block_size, page = slot %
//     block_size) through explicit block/page/head element strides (NHD, HND
//     or the vLLM interleaved K/V views);
//   - an FP8 E4M3FN cache stores fp8(x / scale[head * scale_stride]) of the
//     stored (rotated, rounded) value, rounding to nearest even with finite
//     saturation at +-448 and NaN kept (quantization.rs:32-56);
//   - a token whose position is outside [0, max_position) is left untouched
//     (trusted metadata; the guard only keeps device reads in bounds).
//
// Work decomposition: one wave per (token, row), rows being the query heads
// followed by the KV heads; four waves per workgroup. A query row is rotated;
// a KV row is rotated and, when the token has a slot, written to the K and V
// caches, so each row is read once and written once.

#include <hip/hip_runtime.h>

#include <cmath>
#include <cstdint>
#include <limits>
#include <type_traits>

#include "../../include/loom_hip.h"
#include "loom_hip_internal.h"

namespace {

constexpr uint32_t kRopeThreads = 256;
constexpr uint32_t kRopeRowsPerGroup = kRopeThreads / 64;

struct RopeF32 {
  using T = float;
  static __device__ __forceinline__ float to_f(float x) { return x; }
  static __device__ __forceinline__ float from_f(float x) { return x; }
};

struct RopeF16 {
  using T = uint16_t;
  static __device__ __forceinline__ float to_f(uint16_t x) { return static_cast<float>(__builtin_bit_cast(_Float16, x)); }
  static __device__ __forceinline__ uint16_t from_f(float x) { return __builtin_bit_cast(uint16_t, static_cast<_Float16>(x)); }
};

struct RopeBf16 {
  using T = uint16_t;
  static __device__ __forceinline__ float to_f(uint16_t x) { return __builtin_bit_cast(float, static_cast<uint32_t>(x) << 16); }
  static __device__ __forceinline__ uint16_t from_f(float x) { return __builtin_bit_cast(uint16_t, static_cast<__bf16>(x)); }
};

// OCP FP8 E4M3FN encoding, round to nearest even, saturating to the largest
// finite value (448) and keeping NaN (sign | 0x7f). Subnormals are m * 2^-9.
__device__ __forceinline__ uint8_t encode_e4m3fn(float x) {
  const uint32_t bits = __builtin_bit_cast(uint32_t, x);
  const uint8_t sign = static_cast<uint8_t>((bits >> 24) & 0x80U);
  const uint32_t mag = bits & 0x7fffffffU;
  if (mag > 0x7f800000U) return sign | 0x7fU;          // NaN
  if (mag >= 0x43e00000U) return sign | 0x7eU;         // |x| >= 448 (and inf)
  if (mag < 0x3c800000U) {                             // |x| < 2^-6: subnormal range
    const float q = __builtin_bit_cast(float, mag) * 512.0f;  // exact: power-of-two scaling
    return sign | static_cast<uint8_t>(__builtin_rintf(q));    // 8 rounds up to the smallest normal
  }
  const uint32_t exp = (mag >> 23) - 127U + 7U;        // biased E4M3 exponent, 1..15
  uint32_t mant = mag & 0x7fffffU;
  uint32_t q = mant >> 20;
  const uint32_t rest = mant & 0xfffffU;
  if (rest > 0x80000U || (rest == 0x80000U && (q & 1U))) ++q;
  const uint32_t code = (exp << 3) + q;                // a mantissa carry moves into the exponent
  return sign | static_cast<uint8_t>(code > 0x7eU ? 0x7eU : code);
}

struct RopeArgs {
  void* query;
  void* key;
  const void* value;
  const int64_t* positions;
  const void* cos_sin;
  void* key_cache;
  void* value_cache;
  const float* key_scales;
  const float* value_scales;
  const int64_t* slot_mapping;
  uint32_t tokens, cache_tokens, query_heads, kv_heads, head_size, value_head_size, rotary_dim;
  uint32_t max_position, num_blocks, block_size, scale_stride, is_neox;
  uint64_t q_token, q_head, k_token, k_head, v_token, v_head;
  uint64_t kc_block, kc_page, kc_head, vc_block, vc_page, vc_head;
};

template <typename E, bool kFp8>
__global__ __launch_bounds__(kRopeThreads) void rope_paged_kv_kernel(RopeArgs a) {
#pragma clang fp contract(off)
  using T = typename E::T;
  using C = typename std::conditional<kFp8, uint8_t, T>::type;
  const uint32_t lane = threadIdx.x & 63U;
  const uint32_t rows = a.query_heads + a.kv_heads;
  const uint64_t unit = static_cast<uint64_t>(blockIdx.x) * kRopeRowsPerGroup +
                        __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  if (unit >= static_cast<uint64_t>(a.tokens) * rows) return;
  const uint32_t token = static_cast<uint32_t>(unit / rows);
  const uint32_t row = static_cast<uint32_t>(unit % rows);
  const int64_t position = a.positions[token];
  if (position < 0 || static_cast<uint64_t>(position) >= a.max_position) return;

  const bool is_key = row >= a.query_heads;
  const uint32_t head = is_key ? row - a.query_heads : row;
  T* x = static_cast<T*>(is_key ? a.key : a.query) +
         (is_key ? token * a.k_token + head * a.k_head : token * a.q_token + head * a.q_head);
  const T* cs = static_cast<const T*>(a.cos_sin) + static_cast<uint64_t>(position) * a.rotary_dim;
  const uint32_t half = a.rotary_dim / 2U;

  int64_t slot = -1;
  if (is_key && token < a.cache_tokens) slot = a.slot_mapping[token];
  const bool write = slot >= 0 && static_cast<uint64_t>(slot) < static_cast<uint64_t>(a.num_blocks) * a.block_size;
  C* kdst = nullptr;
  C* vdst = nullptr;
  float kscale = 1.0f, vscale = 1.0f;
  if (write) {
    const uint64_t blk = static_cast<uint64_t>(slot) / a.block_size, page = static_cast<uint64_t>(slot) % a.block_size;
    kdst = static_cast<C*>(a.key_cache) + blk * a.kc_block + page * a.kc_page + head * a.kc_head;
    vdst = static_cast<C*>(a.value_cache) + blk * a.vc_block + page * a.vc_page + head * a.vc_head;
    if (kFp8) {
      kscale = a.key_scales[static_cast<uint64_t>(head) * a.scale_stride];
      vscale = a.value_scales[static_cast<uint64_t>(head) * a.scale_stride];
    }
  }
  auto put = [&](C* dst, uint32_t d, T stored, float scale) {
    if constexpr (kFp8) {
      dst[d] = encode_e4m3fn(E::to_f(stored) / scale);
    } else {
      dst[d] = stored;
    }
  };

  for (uint32_t p = lane; p < half; p += 64) {
    const uint32_t i1 = a.is_neox ? p : 2 * p;
    const uint32_t i2 = a.is_neox ? p + half : 2 * p + 1;
    const float first = E::to_f(x[i1]);
    const float second = E::to_f(x[i2]);
    const float cosine = E::to_f(cs[p]);
    const float sine = E::to_f(cs[half + p]);
    const T r1 = E::from_f(first * cosine - second * sine);
    const T r2 = E::from_f(second * cosine + first * sine);
    x[i1] = r1;
    x[i2] = r2;
    if (write) {
      put(kdst, i1, r1, kscale);
      put(kdst, i2, r2, kscale);
    }
  }
  if (!write) return;
  for (uint32_t d = a.rotary_dim + lane; d < a.head_size; d += 64) put(kdst, d, x[d], kscale);
  const T* v = static_cast<const T*>(a.value) + token * a.v_token + head * a.v_head;
  for (uint32_t d = lane; d < a.value_head_size; d += 64) put(vdst, d, v[d], vscale);
}

template <typename E>
int rope_write(void* query, void* key, const void* value, const int64_t* positions, const void* cos_sin_cache,
               void* key_cache, void* value_cache, const float* key_scales, const float* value_scales,
               const int64_t* slot_mapping, uint32_t tokens, uint32_t cache_tokens, uint32_t query_heads,
               uint32_t kv_heads, uint32_t head_size, uint32_t value_head_size, uint32_t rotary_dim,
               uint32_t max_position, uint32_t num_blocks, uint32_t block_size, uint32_t cache_encoding,
               uint32_t scale_stride, uint64_t query_token_stride, uint64_t query_head_stride,
               uint64_t key_token_stride, uint64_t key_head_stride, uint64_t value_token_stride,
               uint64_t value_head_stride, uint64_t key_cache_block_stride, uint64_t key_cache_page_stride,
               uint64_t key_cache_head_stride, uint64_t value_cache_block_stride, uint64_t value_cache_page_stride,
               uint64_t value_cache_head_stride, uint32_t is_neox, void* stream) {
  using loom_hip_detail::fail;
  const bool fp8 = cache_encoding == LOOM_HIP_KV_CACHE_FP8_E4M3;
  if (cache_encoding != LOOM_HIP_KV_CACHE_NATIVE && !fp8)
    return fail(LOOM_HIP_INVALID_ARGUMENT, "unknown K/V cache encoding");
  // Host validation of the reference launcher (rope_paged_kv.cu:233-252).
  if (query == nullptr || key == nullptr || value == nullptr || positions == nullptr || cos_sin_cache == nullptr ||
      key_cache == nullptr || value_cache == nullptr)
    return fail(LOOM_HIP_INVALID_ARGUMENT, "null RoPE+paged-KV buffer");
  if (fp8 && (key_scales == nullptr || value_scales == nullptr))
    return fail(LOOM_HIP_INVALID_ARGUMENT, "FP8 K/V caches need key and value scales");
  if (tokens == 0 || (cache_tokens > 0 && slot_mapping == nullptr) || cache_tokens > tokens)
    return fail(LOOM_HIP_INVALID_ARGUMENT, "token counts or slot mapping are invalid");
  if (query_heads == 0 || kv_heads == 0 || head_size == 0 || value_head_size == 0 || max_position == 0 ||
      num_blocks == 0 || block_size == 0)
    return fail(LOOM_HIP_INVALID_ARGUMENT, "RoPE+paged-KV dimensions must be non-zero");
  if (rotary_dim == 0 || (rotary_dim & 1U) != 0 || rotary_dim > head_size)
    return fail(LOOM_HIP_INVALID_ARGUMENT, "rotary dimension must be non-zero, even and at most the head size");
  if (query_token_stride == 0 || query_head_stride == 0 || key_token_stride == 0 || key_head_stride == 0 ||
      value_token_stride == 0 || value_head_stride == 0 || key_cache_block_stride == 0 ||
      key_cache_page_stride == 0 || key_cache_head_stride == 0 || value_cache_block_stride == 0 ||
      value_cache_page_stride == 0 || value_cache_head_stride == 0)
    return fail(LOOM_HIP_INVALID_ARGUMENT, "RoPE+paged-KV strides must be non-zero");
  if (is_neox > 1U || scale_stride > 1U)
    return fail(LOOM_HIP_INVALID_ARGUMENT, "is_neox and scale_stride must be 0 or 1");
  if (tokens > static_cast<uint32_t>(std::numeric_limits<int>::max()))
    return fail(LOOM_HIP_INVALID_ARGUMENT, "token count exceeds the launch limit");
  const uint64_t units = static_cast<uint64_t>(tokens) * (static_cast<uint64_t>(query_heads) + kv_heads);
  const uint64_t groups = (units + kRopeRowsPerGroup - 1) / kRopeRowsPerGroup;
  if (groups > static_cast<uint64_t>(std::numeric_limits<int>::max()))
    return fail(LOOM_HIP_UNSUPPORTED, "RoPE+paged-KV grid exceeds the launch limit");
  const int avail = loom_hip_detail::device_available();
  if (avail != LOOM_HIP_SUCCESS) return avail;

  RopeArgs args{query, key, value, positions, cos_sin_cache, key_cache, value_cache, key_scales, value_scales,
                slot_mapping, tokens, cache_tokens, query_heads, kv_heads, head_size, value_head_size, rotary_dim,
                max_position, num_blocks, block_size, scale_stride, is_neox, query_token_stride, query_head_stride,
                key_token_stride, key_head_stride, value_token_stride, value_head_stride, key_cache_block_stride,
                key_cache_page_stride, key_cache_head_stride, value_cache_block_stride, value_cache_page_stride,
                value_cache_head_stride};
  hipStream_t s = static_cast<hipStream_t>(stream);
  if (fp8) {
    hipLaunchKernelGGL((rope_paged_kv_kernel<E, true>), dim3(static_cast<uint32_t>(groups)), dim3(kRopeThreads), 0,
                       s, args);
  } else {
    hipLaunchKernelGGL((rope_paged_kv_kernel<E, false>), dim3(static_cast<uint32_t>(groups)), dim3(kRopeThreads), 0,
                       s, args);
  }
  if (hipGetLastError() != hipSuccess) return fail(LOOM_HIP_LAUNCH_ERROR, "RoPE+paged-KV kernel launch failed");
  loom_hip_detail::count_launch(LOOM_HIP_ROPE_PAGED_KV_WRITE);
  return LOOM_HIP_SUCCESS;
}

}  // namespace

#define LOOM_HIP_ROPE_ARGS                                                                                      \
  query, key, value, positions, cos_sin_cache, key_cache, value_cache, key_scales, value_scales, slot_mapping, \
      tokens, cache_tokens, query_heads, kv_heads, head_size, value_head_size, rotary_dim, max_position,       \
      num_blocks, block_size, cache_encoding, scale_stride, query_token_stride, query_head_stride,             \
      key_token_stride, key_head_stride, value_token_stride, value_head_stride, key_cache_block_stride,        \
      key_cache_page_stride, key_cache_head_stride, value_cache_block_stride, value_cache_page_stride,         \
      value_cache_head_stride, is_neox, stream

extern "C" {

int loom_hip_rope_paged_kv_write_f32(
    float* query, float* key, const float* value, const int64_t* positions, const float* cos_sin_cache,
    void* key_cache, void* value_cache, const float* key_scales, const float* value_scales,
    const int64_t* slot_mapping, uint32_t tokens, uint32_t cache_tokens, uint32_t query_heads, uint32_t kv_heads,
    uint32_t head_size, uint32_t value_head_size, uint32_t rotary_dim, uint32_t max_position, uint32_t num_blocks,
    uint32_t block_size, uint32_t cache_encoding, uint32_t scale_stride, uint64_t query_token_stride,
    uint64_t query_head_stride, uint64_t key_token_stride, uint64_t key_head_stride, uint64_t value_token_stride,
    uint64_t value_head_stride, uint64_t key_cache_block_stride, uint64_t key_cache_page_stride,
    uint64_t key_cache_head_stride, uint64_t value_cache_block_stride, uint64_t value_cache_page_stride,
    uint64_t value_cache_head_stride, uint32_t is_neox, void* stream) {
  return rope_write<RopeF32>(LOOM_HIP_ROPE_ARGS);
}

int loom_hip_rope_paged_kv_write_f16(
    uint16_t* query, uint16_t* key, const uint16_t* value, const int64_t* positions, const uint16_t* cos_sin_cache,
    void* key_cache, void* value_cache, const float* key_scales, const float* value_scales,
    const int64_t* slot_mapping, uint32_t tokens, uint32_t cache_tokens, uint32_t query_heads, uint32_t kv_heads,
    uint32_t head_size, uint32_t value_head_size, uint32_t rotary_dim, uint32_t max_position, uint32_t num_blocks,
    uint32_t block_size, uint32_t cache_encoding, uint32_t scale_stride, uint64_t query_token_stride,
    uint64_t query_head_stride, uint64_t key_token_stride, uint64_t key_head_stride, uint64_t value_token_stride,
    uint64_t value_head_stride, uint64_t key_cache_block_stride, uint64_t key_cache_page_stride,
    uint64_t key_cache_head_stride, uint64_t value_cache_block_stride, uint64_t value_cache_page_stride,
    uint64_t value_cache_head_stride, uint32_t is_neox, void* stream) {
  return rope_write<RopeF16>(LOOM_HIP_ROPE_ARGS);
}

int loom_hip_rope_paged_kv_write_bf16(
    uint16_t* query, uint16_t* key, const uint16_t* value, const int64_t* positions, const uint16_t* cos_sin_cache,
    void* key_cache, void* value_cache, const float* key_scales, const float* value_scales,
    const int64_t* slot_mapping, uint32_t tokens, uint32_t cache_tokens, uint32_t query_heads, uint32_t kv_heads,
    uint32_t head_size, uint32_t value_head_size, uint32_t rotary_dim, uint32_t max_position, uint32_t num_blocks,
    uint32_t block_size, uint32_t cache_encoding, uint32_t scale_stride, uint64_t query_token_stride,
    uint64_t query_head_stride, uint64_t key_token_stride, uint64_t key_head_stride, uint64_t value_token_stride,
    uint64_t value_head_stride, uint64_t key_cache_block_stride, uint64_t key_cache_page_stride,
    uint64_t key_cache_head_stride, uint64_t value_cache_block_stride, uint64_t value_cache_page_stride,
    uint64_t value_cache_head_stride, uint32_t is_neox, void* stream) {
  return rope_write<RopeBf16>(LOOM_HIP_ROPE_ARGS);
}

}  // extern "C"
