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

// Vector-path FP8 helpers. The packed hardware conversion rounds to nearest
// even into OCP E4M3FN; saturation to +-448 is applied first (it returns NaN
// on overflow otherwise) and NaN inputs are re-encoded in software, since the
// hardware sets the sign bit of every NaN where the reference keeps it.
__device__ __forceinline__ float sat448(float x) {
  return __builtin_fabsf(x) > 448.0f ? __builtin_copysignf(448.0f, x) : x;
}

// Correctly rounded a / b given y = RN(1 / b): q = RN(a * y) is within one
// ulp, r = a - q * b is exact by FMA, and RN(q + r * y) = RN(a / b)
// (Markstein's theorem). Outside the range where no intermediate can
// underflow or overflow the quotient falls back to IEEE division; that range
// only holds quotients that encode to +-0 or saturate.
__device__ __forceinline__ float div_rn(float a, float b, float y) {
  const float q = a * y;
  if (!(__builtin_fabsf(a) >= 0x1p-100f && __builtin_fabsf(q) <= 0x1p20f)) return a / b;
  const float r = __builtin_fmaf(-q, b, a);
  return __builtin_fmaf(r, y, q);
}

// Four values -> four E4M3FN bytes (little-endian in one dword).
__device__ __forceinline__ uint32_t encode4_e4m3fn(float a, float b, float c, float d) {
  const int lo = __builtin_amdgcn_cvt_pk_fp8_f32(sat448(a), sat448(b), 0, false);
  uint32_t w = static_cast<uint32_t>(__builtin_amdgcn_cvt_pk_fp8_f32(sat448(c), sat448(d), lo, true));
  if (__builtin_expect(__builtin_isnan(a) | __builtin_isnan(b) | __builtin_isnan(c) | __builtin_isnan(d), 0)) {
    w = static_cast<uint32_t>(encode_e4m3fn(a)) | (static_cast<uint32_t>(encode_e4m3fn(b)) << 8) |
        (static_cast<uint32_t>(encode_e4m3fn(c)) << 16) | (static_cast<uint32_t>(encode_e4m3fn(d)) << 24);
  }
  return w;
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

// Vector path: one workgroup per (token, split); every thread moves whole
// 16-byte chunks. Items of a token, in order:
//   Q rotary items  query_heads * rot_items
//   K rotary items  kv_heads * rot_items          (also stored to the K cache)
//   K tail chunks   kv_heads * tail_chunks         (only when the token has a slot)
//   V chunks        kv_heads * value_chunks        (only when the token has a slot)
// A NeoX rotary item is chunk c of the first half plus chunk c of the second
// half (pairs (p, p + rotary_dim/2) stay in-lane); an interleaved item is one
// chunk holding VEC/2 adjacent pairs. Each thread takes kUnroll items and
// issues all of their loads before any arithmetic, so a workgroup keeps
// ~kUnroll * 256 * 48 bytes in flight.
constexpr uint32_t kVecUnroll = 2;

template <typename E>
struct Vec {
  using T = typename E::T;
  static constexpr uint32_t N = 16 / sizeof(T);  // elements per 16-byte chunk
  union Chunk {
    uint4 raw;
    T v[N];
  };
  union Half {
    uint2 raw;
    T v[N / 2];
  };
};

template <typename E, bool kFp8>
__device__ __forceinline__ void store_chunk(void* cache, uint64_t elem_off, const typename Vec<E>::Chunk& c,
                                            float scale, float inv_scale) {
  constexpr uint32_t N = Vec<E>::N;
  if constexpr (kFp8) {
    float x[N];
#pragma unroll
    for (uint32_t i = 0; i < N; ++i) x[i] = div_rn(E::to_f(c.v[i]), scale, inv_scale);
    uint32_t w[N / 4];
#pragma unroll
    for (uint32_t i = 0; i < N / 4; ++i) w[i] = encode4_e4m3fn(x[4 * i], x[4 * i + 1], x[4 * i + 2], x[4 * i + 3]);
    if constexpr (N == 8) {
      *reinterpret_cast<uint2*>(static_cast<uint8_t*>(cache) + elem_off) = uint2{w[0], w[1]};
    } else {
      *reinterpret_cast<uint32_t*>(static_cast<uint8_t*>(cache) + elem_off) = w[0];
    }
  } else {
    *reinterpret_cast<uint4*>(static_cast<typename E::T*>(cache) + elem_off) = c.raw;
  }
}

template <typename E, bool kFp8, bool kNeox>
__global__ __launch_bounds__(kRopeThreads) void rope_paged_kv_vec_kernel(RopeArgs a, uint32_t splits) {
#pragma clang fp contract(off)
  using T = typename E::T;
  using V = Vec<E>;
  constexpr uint32_t N = V::N;
  const uint32_t token = blockIdx.x / splits;
  const uint32_t split = blockIdx.x - token * splits;
  const int64_t position = a.positions[token];
  if (position < 0 || static_cast<uint64_t>(position) >= a.max_position) return;
  const int64_t slot = token < a.cache_tokens ? a.slot_mapping[token] : -1;
  const bool write = slot >= 0 && static_cast<uint64_t>(slot) < static_cast<uint64_t>(a.num_blocks) * a.block_size;
  uint64_t kc_base = 0, vc_base = 0;
  if (write) {
    const uint64_t blk = static_cast<uint64_t>(slot) / a.block_size, page = static_cast<uint64_t>(slot) % a.block_size;
    kc_base = blk * a.kc_block + page * a.kc_page;
    vc_base = blk * a.vc_block + page * a.vc_page;
  }
  const uint32_t half = a.rotary_dim / 2U;
  const uint32_t rot_items = kNeox ? half / N : a.rotary_dim / N;
  const uint32_t tail_chunks = (a.head_size - a.rotary_dim) / N;
  const uint32_t value_chunks = a.value_head_size / N;
  const uint32_t q_items = a.query_heads * rot_items;
  const uint32_t k_items = a.kv_heads * rot_items;
  const uint32_t t_items = write ? a.kv_heads * tail_chunks : 0U;
  const uint32_t v_items = write ? a.kv_heads * value_chunks : 0U;
  const uint32_t total = q_items + k_items + t_items + v_items;
  const T* cs = static_cast<const T*>(a.cos_sin) + static_cast<uint64_t>(position) * a.rotary_dim;
  T* qrow = static_cast<T*>(a.query) + token * a.q_token;
  T* krow = static_cast<T*>(a.key) + token * a.k_token;
  const T* vrow = static_cast<const T*>(a.value) + token * a.v_token;

  for (uint32_t base = split * kRopeThreads; base < total; base += splits * kRopeThreads * kVecUnroll) {
    // Phase 1: decode items and issue every load.
    uint32_t kind[kVecUnroll], head[kVecUnroll], c[kVecUnroll];
    typename V::Chunk x1[kVecUnroll], x2[kVecUnroll], co[kVecUnroll], si[kVecUnroll];
#pragma unroll
    for (uint32_t u = 0; u < kVecUnroll; ++u) {
      const uint32_t item = base + u * splits * kRopeThreads + threadIdx.x;
      kind[u] = 4;  // none
      head[u] = 0;
      c[u] = 0;
      if (item >= total) continue;
      uint32_t r = item;
      if (r < q_items) {
        kind[u] = 0;
      } else if ((r -= q_items) < k_items) {
        kind[u] = 1;
      } else if ((r -= k_items) < t_items) {
        kind[u] = 2;
      } else {
        r -= t_items;
        kind[u] = 3;
      }
      const uint32_t per = kind[u] <= 1 ? rot_items : (kind[u] == 2 ? tail_chunks : value_chunks);
      head[u] = r / per;
      c[u] = r - head[u] * per;
      if (kind[u] <= 1) {
        const T* row = kind[u] == 0 ? qrow + head[u] * a.q_head : krow + head[u] * a.k_head;
        if constexpr (kNeox) {
          x1[u].raw = *reinterpret_cast<const uint4*>(row + c[u] * N);
          x2[u].raw = *reinterpret_cast<const uint4*>(row + half + c[u] * N);
          co[u].raw = *reinterpret_cast<const uint4*>(cs + c[u] * N);
          si[u].raw = *reinterpret_cast<const uint4*>(cs + half + c[u] * N);
        } else {
          x1[u].raw = *reinterpret_cast<const uint4*>(row + c[u] * N);
          typename V::Half hc, hs;
          hc.raw = *reinterpret_cast<const uint2*>(cs + c[u] * (N / 2));
          hs.raw = *reinterpret_cast<const uint2*>(cs + half + c[u] * (N / 2));
#pragma unroll
          for (uint32_t i = 0; i < N / 2; ++i) {
            co[u].v[i] = hc.v[i];
            si[u].v[i] = hs.v[i];
          }
        }
      } else if (kind[u] == 2) {
        x1[u].raw = *reinterpret_cast<const uint4*>(krow + head[u] * a.k_head + a.rotary_dim + c[u] * N);
      } else {
        x1[u].raw = *reinterpret_cast<const uint4*>(vrow + head[u] * a.v_head + c[u] * N);
      }
    }
    // Phase 2: rotate, write back, store to the caches.
#pragma unroll
    for (uint32_t u = 0; u < kVecUnroll; ++u) {
      if (kind[u] == 4) continue;
      const float kscale = kFp8 && kind[u] != 0 ? a.key_scales[static_cast<uint64_t>(head[u]) * a.scale_stride] : 1.0f;
      const float kinv = 1.0f / kscale;
      if (kind[u] <= 1) {
        typename V::Chunk r1, r2;
        if constexpr (kNeox) {
#pragma unroll
          for (uint32_t i = 0; i < N; ++i) {
            const float f = E::to_f(x1[u].v[i]), s = E::to_f(x2[u].v[i]);
            const float cc = E::to_f(co[u].v[i]), ss = E::to_f(si[u].v[i]);
            r1.v[i] = E::from_f(f * cc - s * ss);
            r2.v[i] = E::from_f(s * cc + f * ss);
          }
        } else {
#pragma unroll
          for (uint32_t i = 0; i < N / 2; ++i) {
            const float f = E::to_f(x1[u].v[2 * i]), s = E::to_f(x1[u].v[2 * i + 1]);
            const float cc = E::to_f(co[u].v[i]), ss = E::to_f(si[u].v[i]);
            r1.v[2 * i] = E::from_f(f * cc - s * ss);
            r1.v[2 * i + 1] = E::from_f(s * cc + f * ss);
          }
        }
        T* row = kind[u] == 0 ? qrow + head[u] * a.q_head : krow + head[u] * a.k_head;
        const uint32_t o1 = c[u] * N, o2 = half + c[u] * N;
        *reinterpret_cast<uint4*>(row + o1) = r1.raw;
        if constexpr (kNeox) *reinterpret_cast<uint4*>(row + o2) = r2.raw;
        if (kind[u] == 1 && write) {
          const uint64_t dst = kc_base + head[u] * a.kc_head;
          store_chunk<E, kFp8>(a.key_cache, dst + o1, r1, kscale, kinv);
          if constexpr (kNeox) store_chunk<E, kFp8>(a.key_cache, dst + o2, r2, kscale, kinv);
        }
      } else if (kind[u] == 2) {
        store_chunk<E, kFp8>(a.key_cache, kc_base + head[u] * a.kc_head + a.rotary_dim + c[u] * N, x1[u], kscale,
                             kinv);
      } else {
        const float vscale = kFp8 ? a.value_scales[static_cast<uint64_t>(head[u]) * a.scale_stride] : 1.0f;
        store_chunk<E, kFp8>(a.value_cache, vc_base + head[u] * a.vc_head + c[u] * N, x1[u], vscale, 1.0f / vscale);
      }
    }
  }
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
  loom_hip_detail::KernelTimer timed(LOOM_HIP_KERNEL_ROPE, stream);

  // 16-byte vector path when every row, stride and base is chunk-aligned.
  constexpr uint64_t N = Vec<E>::N;
  const uint64_t cache_elem = fp8 ? 1 : sizeof(typename E::T);
  auto aligned = [](const void* p, uint64_t bytes) { return reinterpret_cast<uintptr_t>(p) % bytes == 0; };
  const bool vec_ok =
      (is_neox ? (rotary_dim / 2) % N == 0 : rotary_dim % N == 0) && head_size % N == 0 &&
      value_head_size % N == 0 && query_token_stride % N == 0 && query_head_stride % N == 0 &&
      key_token_stride % N == 0 && key_head_stride % N == 0 && value_token_stride % N == 0 &&
      value_head_stride % N == 0 && key_cache_block_stride % N == 0 && key_cache_page_stride % N == 0 &&
      key_cache_head_stride % N == 0 && value_cache_block_stride % N == 0 && value_cache_page_stride % N == 0 &&
      value_cache_head_stride % N == 0 && aligned(query, 16) && aligned(key, 16) && aligned(value, 16) &&
      aligned(cos_sin_cache, 16) && aligned(key_cache, N * cache_elem) && aligned(value_cache, N * cache_elem);
  const uint64_t rot_items = is_neox ? rotary_dim / 2 / N : rotary_dim / N;
  const uint64_t max_items = static_cast<uint64_t>(query_heads) * rot_items +
                             static_cast<uint64_t>(kv_heads) * (rot_items + (head_size - rotary_dim) / N +
                                                                value_head_size / N);
  if (vec_ok && max_items <= (1ULL << 31)) {
    // Enough workgroups to cover the chip even for a decode step of a few tokens.
    const uint64_t max_splits = (max_items + kRopeThreads - 1) / kRopeThreads;
    uint64_t splits = (2048 + tokens - 1) / tokens;
    if (splits > max_splits) splits = max_splits;
    if (splits < 1) splits = 1;
    const uint64_t vgroups = static_cast<uint64_t>(tokens) * splits;
    if (vgroups <= static_cast<uint64_t>(std::numeric_limits<int>::max())) {
      const dim3 grid(static_cast<uint32_t>(vgroups));
      const uint32_t sp = static_cast<uint32_t>(splits);
      if (fp8) {
        if (is_neox) hipLaunchKernelGGL((rope_paged_kv_vec_kernel<E, true, true>), grid, dim3(kRopeThreads), 0, s, args, sp);
        else hipLaunchKernelGGL((rope_paged_kv_vec_kernel<E, true, false>), grid, dim3(kRopeThreads), 0, s, args, sp);
      } else {
        if (is_neox) hipLaunchKernelGGL((rope_paged_kv_vec_kernel<E, false, true>), grid, dim3(kRopeThreads), 0, s, args, sp);
        else hipLaunchKernelGGL((rope_paged_kv_vec_kernel<E, false, false>), grid, dim3(kRopeThreads), 0, s, args, sp);
      }
      if (hipGetLastError() != hipSuccess) return fail(LOOM_HIP_LAUNCH_ERROR, "RoPE+paged-KV kernel launch failed");
      loom_hip_detail::count_launch(LOOM_HIP_ROPE_PAGED_KV_WRITE);
      return LOOM_HIP_SUCCESS;
    }
  }

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
