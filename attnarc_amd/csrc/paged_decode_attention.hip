// Paged MQA/GQA decode attention for MI355X (gfx950).
//
// Semantics: crates/loom-kernels/src/attention.rs:270-357 (one query token
// per sequence, softmax(scale * q.k) over the sequence's paged K, weighted sum
// of paged V). The launch ABI is include/loom_hip.h, a one-for-one
// replacement of the paged-decode part of
// crates/loom-cuda-sys/cuda/include/loom_cuda.h:175-250 plus extensions.
//
// Kernels
//   decode_stream_kernel / decode_stream_group_kernel
//                        the main path: 16-bit query, D = Dv = 64, 80, 96,
//                        112, 128 or 256 (native or FP8 E4M3FN cache), up to
//                        32 query heads per KV head (16 at 80-112 and 256),
//                        power-of-two blocks >= 16. One wave per (sequence,
//                        partition, KV head) item streams 16-token steps: K
//                        and V rows go to LDS by DMA (swizzled), QK^T and PV
//                        run on MFMA with
//                        the group's heads as the N dimension. Full grids
//                        put four adjacent-head items in one workgroup.
//   decode_stream_heads_kernel
//                        groups of 17-128 query heads at D = 64 or 128: one
//                        wave per 16 heads (17-32) or 32 heads (33-128), all
//                        reading one shared LDS ring.
//   decode_mfma_kernel   the same head layout with 32-token chunks and K in
//                        registers, for block sizes below 16 and partitions
//                        that are not a multiple of 16 tokens.
//   decode_vector_kernel any shape and dtype (including F32); fp32 VALU on
//                        64-token tiles. Covers the general contract.
//   merge_kernel / merge_rows_kernel / merge_wide_kernel
//                        stable log-sum-exp merge of per-partition states
//                        (the math of paged_decode_attention.cu:780-852).
//
// The decode kernels keep an online softmax in base-2 units (scores are
// multiplied by scale * log2(e)). A work item whose partition is the whole
// sequence writes the output (and optional LSE) directly; otherwise it
// writes (m, l) and its partial output to the caller's F32 workspace and a
// merge kernel finishes.

#include <hip/hip_runtime.h>

#include <atomic>
#include <cmath>
#include <cstdint>
#include <cstdlib>
#include <cstdio>
#include <cstring>
#include <limits>
#include <mutex>
#include <string>
#include <type_traits>
#include <vector>

#include "../../include/loom_hip.h"
#include "loom_hip_internal.h"

namespace {

constexpr float kLog2e = 1.44269504088896340736f;
constexpr float kLn2 = 0.69314718055994530942f;

typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));
typedef __bf16 bf16x2 __attribute__((ext_vector_type(2)));
typedef _Float16 f16x2 __attribute__((ext_vector_type(2)));

// ---------------------------------------------------------------------------
// Launch arguments shared by all kernels (passed by value as kernarg).
// ---------------------------------------------------------------------------
struct DecodeArgs {
  const void* query;
  const void* key_cache;
  const void* value_cache;
  const float* key_scales;
  const float* value_scales;
  const int32_t* block_tables;
  const int32_t* sequence_lengths;
  void* output;
  float* lse;
  float* ws_ml;  // [sequences][parts][query_heads][2] = (m in log2 units, l)
  float* ws_o;   // [sequences][parts][query_heads][Dv] partial outputs (F32 sums, put_partial)
  uint64_t k_block, k_page, k_head;  // element strides of the key cache
  uint64_t v_block, v_page, v_head;  // element strides of the value cache
  uint32_t query_heads;
  uint32_t kv_heads;
  uint32_t group;  // query heads per KV head
  uint32_t head_size;
  uint32_t value_head_size;
  uint32_t block_size;
  uint32_t block_shift;  // log2(block_size) when it is a power of two
  uint32_t max_blocks;
  uint32_t partition_tokens;
  uint32_t parts;  // partitions per (sequence, head); 1 = write output directly
  uint32_t scale_stride;
  uint32_t grid_y;  // decode kernels: work items per sequence besides partitions
  uint32_t sequences;
  float score_scale_log2;  // scale * log2(e)
};

// Index of the split-K state of output row (sequence, query head) = row and
// partition part. States are ordered [sequence][partition][query head], so
// the states one workgroup of adjacent KV heads writes for a partition are
// contiguous (whole cache lines for the (m, l) pairs).
__device__ __forceinline__ uint64_t state_of(const DecodeArgs& a, uint64_t row, uint32_t part) {
  const uint64_t seq = row / a.query_heads;
  return (seq * a.parts + part) * a.query_heads + (row - seq * a.query_heads);
}

// ---------------------------------------------------------------------------
// Element types.
// ---------------------------------------------------------------------------
struct F32Elem {
  using T = float;
  static __device__ __forceinline__ float to_f(float x) { return x; }
  static __device__ __forceinline__ float from_f(float x) { return x; }
};

struct F16Elem {
  using T = uint16_t;
  static __device__ __forceinline__ float to_f(uint16_t x) {
    return static_cast<float>(__builtin_bit_cast(_Float16, x));
  }
  static __device__ __forceinline__ uint16_t from_f(float x) {
    return __builtin_bit_cast(uint16_t, static_cast<_Float16>(x));
  }
};

struct Bf16Elem {
  using T = uint16_t;
  static __device__ __forceinline__ float to_f(uint16_t x) {
    return __uint_as_float(static_cast<uint32_t>(x) << 16);
  }
  static __device__ __forceinline__ uint16_t from_f(float x) {
    return __builtin_bit_cast(uint16_t, static_cast<__bf16>(x));  // RNE
  }
};

// OCP FP8 E4M3FN decode from its definition (quantization.rs:13-29):
// subnormal m * 2^-9, normal (1 + m/8) * 2^(e-7), 0x7f/0xff NaN.
struct Fp8Elem {
  using T = uint8_t;
  static __device__ __forceinline__ float to_f(uint8_t b) {
    const uint32_t mag = b & 0x7fU;
    const uint32_t e = mag >> 3;
    const uint32_t m = mag & 7U;
    float v = e == 0U ? static_cast<float>(m) * 0x1p-9f
                      : __uint_as_float(((e + 120U) << 23) | (m << 20));
    v = mag == 0x7fU ? __builtin_nanf("") : v;
    return (b & 0x80U) ? -v : v;
  }
};

__device__ __forceinline__ float wave_sum(float v) {
#pragma unroll
  for (int offset = 32; offset > 0; offset >>= 1) v += __shfl_xor(v, offset, 64);
  return v;
}

// Orders this wave's LDS accesses in the compiler only. The LDS unit
// executes one wave's DS instructions in issue order, so a write followed by
// a read of the same bytes (by any lanes of the wave) needs no hardware wait;
// a memory fence here would also wait for every outstanding global load.
__device__ __forceinline__ void wave_fence_lds() { asm volatile("" ::: "memory"); }

// s_waitcnt lgkmcnt(0) alone (vmcnt and expcnt left at their maxima).
__device__ __forceinline__ void wait_lds_reads() { __builtin_amdgcn_s_waitcnt(0xC07F); }

// Split-K partial outputs: the unnormalised F32 sum O_p = sum_t 2^(s_t -
// m_p) v_t (times the FP8 value scale) of each partition, as the reference
// keeps them (paged_decode_attention.cu:683-702): every output is rounded to
// its storage type once, by the merge. (16-bit o_p = O_p / l_p partials,
// half the bytes, were measured against the oracle: a partial rounded to
// BF16 carries up to half an ulp of |o_p|, which a merge of partials of
// opposite sign keeps in full, up to 7.8e-3 on 16-token partitions.)
__device__ __forceinline__ void put_partial(const DecodeArgs& a, uint64_t idx, float o) {
  static_cast<float*>(a.ws_o)[idx] = o;
}

// Four consecutive dims of one partial row (idx a multiple of 4), times
// scale. kNt: a non-temporal store.
template <bool kNt = false>
__device__ __forceinline__ void put_partial4(const DecodeArgs& a, uint64_t idx, f32x4 o, float scale) {
  f32x4* dst = reinterpret_cast<f32x4*>(static_cast<float*>(a.ws_o) + idx);
  if constexpr (kNt) {
    __builtin_nontemporal_store(o * scale, dst);
  } else {
    *dst = o * scale;
  }
}

// ---------------------------------------------------------------------------
// General kernel: any head size, dtype, stride and group size.
// grid.x = parts * grid_y * sequences, grid_y = kv_heads * head_chunks *
// value_tiles; 256 threads (4 waves). Each wave takes 64-token tiles of the
// partition in turn (wave w: tiles w, w + 4, ...). Within a tile
//   QK: lane i owns token i of the tile and forms its dot products with every
//       query head of the workgroup (query staged in LDS), so a tile costs
//       two wave reductions per head instead of one per token;
//   PV: the lanes split the value dims and walk the tile's tokens, taking
//       each token's probabilities and V row offset from its lane with
//       readlane; the V loads of a step are independent.
// The 64 block-table and K loads of a tile are all in flight together, so
// short sequences are not a chain of dependent loads.
// ---------------------------------------------------------------------------
constexpr uint32_t kVecThreads = 256;
constexpr uint32_t kVecWaves = kVecThreads / 64;
constexpr uint32_t kVecHeads = 8;      // query heads per workgroup
constexpr uint32_t kVecQLds = 512;     // largest head size staged in LDS

// Value dims per lane (1, 2 or 4; a workgroup covers 64 * kDvl of them) and
// the V rows each PV step loads before its FMAs.
__host__ __device__ constexpr uint32_t vec_pv_unroll(uint32_t dvl) { return 64 / dvl; }

__host__ __device__ constexpr uint32_t vec_dims_per_lane(uint32_t dv) { return dv <= 64 ? 1 : dv <= 128 ? 2 : 4; }

// Wave-wide reductions on DPP lane moves: quad swaps (xor 1, xor 2), the
// 8-lane and 16-lane mirrors, then the four 16-lane row results combined
// through scalar registers. Every lane gets the same value. (An xor-shuffle
// butterfly compiles to ds_bpermute, an LDS round trip per step.)
template <int kCtrl>
__device__ __forceinline__ float dpp_move(float v) {
  return __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v), kCtrl, 0xF, 0xF, false));
}
constexpr int kDppQuadXor1 = 0xB1;     // quad_perm [1, 0, 3, 2]
constexpr int kDppQuadXor2 = 0x4E;     // quad_perm [2, 3, 0, 1]
constexpr int kDppRowMirror = 0x140;   // lane 15 - i within each 16-lane row
constexpr int kDppHalfMirror = 0x141;  // lane 7 - i within each 8-lane half row

__device__ __forceinline__ float lane_value(float v, int lane) {
  return __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, v), lane));
}

__device__ __forceinline__ float wave_sum_dpp(float v) {
  v += dpp_move<kDppQuadXor1>(v);
  v += dpp_move<kDppQuadXor2>(v);
  v += dpp_move<kDppHalfMirror>(v);
  v += dpp_move<kDppRowMirror>(v);
  return (lane_value(v, 0) + lane_value(v, 16)) + (lane_value(v, 32) + lane_value(v, 48));
}

__device__ __forceinline__ float wave_max_dpp(float v) {
  v = fmaxf(v, dpp_move<kDppQuadXor1>(v));
  v = fmaxf(v, dpp_move<kDppQuadXor2>(v));
  v = fmaxf(v, dpp_move<kDppHalfMirror>(v));
  v = fmaxf(v, dpp_move<kDppRowMirror>(v));
  return fmaxf(fmaxf(lane_value(v, 0), lane_value(v, 16)), fmaxf(lane_value(v, 32), lane_value(v, 48)));
}

// 16 bytes of cache elements as floats.
template <typename CE>
__device__ __forceinline__ void load16_as_float(const typename CE::T* src,
                                                float (&out)[16 / sizeof(typename CE::T)]) {
  using CT = typename CE::T;
  constexpr uint32_t kW = 16 / sizeof(CT);
  union {
    uint4 u;
    CT e[kW];
  } w;
  w.u = *reinterpret_cast<const uint4*>(src);
#pragma unroll
  for (uint32_t i = 0; i < kW; ++i) out[i] = CE::to_f(w.e[i]);
}

// kVecK: K rows are read as 16-byte vectors (head size, K strides and the
// cache base all 16-byte aligned). kDvl: value dims per lane. kQLds: the
// query is staged in LDS (head size <= kVecQLds), zero-padded to whole
// 32-element chunks; otherwise it is read from global memory (uniform
// addresses) at every use. kH: query heads per workgroup as compiled (1, 2,
// 4 or 8; the group's own count may be smaller, the rest are zero rows).
template <typename QE, typename CE, bool kVecK, uint32_t kDvl, bool kQLds, uint32_t kH>
__global__ __launch_bounds__(kVecThreads) void decode_vector_kernel(DecodeArgs a) {
  using QT = typename QE::T;
  using CT = typename CE::T;
  const uint32_t bid = blockIdx.x;
  const uint32_t part = bid % a.parts;
  const uint32_t rest = bid / a.parts;
  uint32_t y = rest % a.grid_y;
  const uint32_t seq = rest / a.grid_y;
  constexpr uint32_t kDvTile = 64 * kDvl;
  constexpr uint32_t kUnroll = vec_pv_unroll(kDvl);
  constexpr uint32_t kCh = 32;  // K elements per QK chunk
  const uint32_t n_dvt = (a.value_head_size + kDvTile - 1) / kDvTile;
  const uint32_t dvt = y % n_dvt;
  y /= n_dvt;
  const uint32_t n_hc = (a.group + kVecHeads - 1) / kVecHeads;
  const uint32_t hc = y % n_hc;
  const uint32_t kvh = y / n_hc;

  const uint32_t len = static_cast<uint32_t>(a.sequence_lengths[seq]);
  const uint32_t p0 = part * a.partition_tokens;
  if (p0 >= len) return;  // uniform: no partition state is produced
  const uint32_t p1 = min(p0 + a.partition_tokens, len);

  const uint32_t heads = min(kVecHeads, a.group - hc * kVecHeads);  // <= kH
  const uint32_t qh0 = kvh * a.group + hc * kVecHeads;
  const uint32_t lane = threadIdx.x & 63U;
  const uint32_t wave = threadIdx.x >> 6;
  const uint32_t D = a.head_size;
  const uint32_t Dv = a.value_head_size;
  const uint32_t Dp = (D + kCh - 1) / kCh * kCh;  // LDS query row pitch

  float k_scale = 1.0f, v_scale = 1.0f;
  if (a.key_scales != nullptr) {
    k_scale = a.key_scales[kvh * a.scale_stride];
    v_scale = a.value_scales[kvh * a.scale_stride];
  }
  const float sl2 = a.score_scale_log2 * k_scale;

  const QT* q = static_cast<const QT*>(a.query) +
                (static_cast<uint64_t>(seq) * a.query_heads + qh0) * D;
  const CT* kc = static_cast<const CT*>(a.key_cache);
  const CT* vc = static_cast<const CT*>(a.value_cache);
  const int32_t* table = a.block_tables + static_cast<uint64_t>(seq) * a.max_blocks;

  // Block-table entry of this lane's token in the tile at t0; lanes past the
  // end of the partition repeat token t0.
  auto table_entry = [&](uint32_t t0) -> int32_t {
    const uint32_t t = t0 + lane;
    return table[(t < p1 ? t : t0) / a.block_size];
  };
  uint32_t t0 = p0 + wave * 64;
  int32_t next_blk = t0 < p1 ? table_entry(t0) : 0;  // in flight during the query staging

  __shared__ float sm_q[kQLds ? kVecHeads * kVecQLds : 1];
  if constexpr (kQLds) {
    for (uint32_t i = threadIdx.x; i < kH * Dp; i += kVecThreads) {
      const uint32_t h = i / Dp, d = i % Dp;
      sm_q[i] = h < heads && d < D ? QE::to_f(q[h * D + d]) : 0.0f;
    }
    __syncthreads();
  }
  auto qf = [&](uint32_t h, uint32_t d) -> float {
    if constexpr (kQLds) {
      return sm_q[h * Dp + d];
    } else {
      return h < heads && d < D ? QE::to_f(q[h * D + d]) : 0.0f;
    }
  };

  float m[kH], l[kH], o[kH][kDvl];
#pragma unroll
  for (uint32_t h = 0; h < kH; ++h) {
    m[h] = -INFINITY;
    l[h] = 0.0f;
#pragma unroll
    for (uint32_t j = 0; j < kDvl; ++j) o[h][j] = 0.0f;
  }

  for (; t0 < p1; t0 += kVecWaves * 64) {
    // ---- QK: this lane's token -----------------------------------------
    const uint32_t t = t0 + lane;
    const bool valid = t < p1;
    const uint32_t tc = valid ? t : t0;  // lanes past the end repeat token t0
    const uint64_t blk = static_cast<uint64_t>(next_blk);
    const uint32_t page = tc % a.block_size;
    if (t0 + kVecWaves * 64 < p1) next_blk = table_entry(t0 + kVecWaves * 64);
    const uint64_t krow = blk * a.k_block + page * a.k_page + kvh * a.k_head;
    const uint64_t vrow = blk * a.v_block + page * a.v_page + kvh * a.v_head;
    const uint32_t vrow_lo = static_cast<uint32_t>(vrow);
    const uint32_t vrow_hi = static_cast<uint32_t>(vrow >> 32);
    // V rows of tokens [i0, i0 + kUnroll) of the tile, lanes over value dims;
    // token u's row offset comes from lane u (rows past the end of the tile
    // repeat token t0). The first step is issued with the K loads below.
    float vv[kUnroll][kDvl];
    auto load_v = [&](uint32_t i0) {
#pragma unroll
      for (uint32_t u = 0; u < kUnroll; ++u) {
        const uint64_t row =
            (static_cast<uint64_t>(static_cast<uint32_t>(__builtin_amdgcn_readlane(vrow_hi, i0 + u))) << 32) |
            static_cast<uint32_t>(__builtin_amdgcn_readlane(vrow_lo, i0 + u));
        const CT* vr = vc + row + dvt * kDvTile + lane;
#pragma unroll
        for (uint32_t j = 0; j < kDvl; ++j) {
          const uint32_t d = dvt * kDvTile + j * 64 + lane;
          vv[u][j] = d < Dv ? CE::to_f(vr[j * 64]) : 0.0f;
        }
      }
    };
    load_v(0);
    float acc[kH];
#pragma unroll
    for (uint32_t h = 0; h < kH; ++h) acc[h] = 0.0f;
    if constexpr (kVecK) {
      // 32-element chunks of the K row as 16-byte loads, double-buffered:
      // chunk c + 1 is in flight while chunk c meets the query. Elements past
      // the head size load as zero and meet zero query padding.
      constexpr uint32_t kW = 16 / sizeof(CT);
      constexpr uint32_t kKU = kCh / kW;
      float ka[kKU][kW], kb[kKU][kW];
      auto load_chunk = [&](float (&buf)[kKU][kW], uint32_t d0) {
#pragma unroll
        for (uint32_t u = 0; u < kKU; ++u) {
          if (d0 + u * kW < D) {
            load16_as_float<CE>(kc + krow + d0 + u * kW, buf[u]);
          } else {
#pragma unroll
            for (uint32_t w = 0; w < kW; ++w) buf[u][w] = 0.0f;
          }
        }
      };
      auto fma_chunk = [&](const float (&buf)[kKU][kW], uint32_t d0) {
#pragma unroll
        for (uint32_t u = 0; u < kKU; ++u) {
#pragma unroll
          for (uint32_t h = 0; h < kH; ++h) {
#pragma unroll
            for (uint32_t w = 0; w < kW; ++w) acc[h] = fmaf(qf(h, d0 + u * kW + w), buf[u][w], acc[h]);
          }
        }
      };
      load_chunk(ka, 0);
      for (uint32_t d0 = 0; d0 < D; d0 += 2 * kCh) {
        const bool second = d0 + kCh < D;  // uniform
        if (second) load_chunk(kb, d0 + kCh);
        fma_chunk(ka, d0);
        if (!second) break;
        if (d0 + 2 * kCh < D) load_chunk(ka, d0 + 2 * kCh);
        fma_chunk(kb, d0 + kCh);
      }
    } else {
#pragma unroll 8
      for (uint32_t d = 0; d < D; ++d) {
        const float kv = CE::to_f(kc[krow + d]);
#pragma unroll
        for (uint32_t h = 0; h < kH; ++h) acc[h] = fmaf(qf(h, d), kv, acc[h]);
      }
    }

    // ---- online softmax over the tile -----------------------------------
    float alpha[kH], pv[kH];  // pv: v_scale * p of this lane's token
#pragma unroll
    for (uint32_t h = 0; h < kH; ++h) {
      alpha[h] = 1.0f;
      pv[h] = 0.0f;
      if (h < heads) {
        const float s = valid ? acc[h] * sl2 : -INFINITY;
        const float mn = fmaxf(m[h], wave_max_dpp(s));
        alpha[h] = exp2f(m[h] - mn);
        const float pr = valid ? exp2f(s - mn) : 0.0f;
        l[h] = fmaf(l[h], alpha[h], wave_sum_dpp(pr));
        m[h] = mn;
        pv[h] = pr * v_scale;
      }
    }

    // ---- PV: lanes over value dims, tokens of the tile in turn -------------
    // Token u's probabilities come from lane u by readlane (scalar operands,
    // no LDS round trip); past the end of the tile, and for absent heads,
    // they are zero.
#pragma unroll
    for (uint32_t h = 0; h < kH; ++h) {
#pragma unroll
      for (uint32_t j = 0; j < kDvl; ++j) o[h][j] *= alpha[h];
    }
    const uint32_t ntok = min(64U, p1 - t0);
    for (uint32_t i0 = 0; i0 < ntok; i0 += kUnroll) {
      if (i0 != 0) load_v(i0);
#pragma unroll
      for (uint32_t u = 0; u < kUnroll; ++u) {
#pragma unroll
        for (uint32_t h = 0; h < kH; ++h) {
          const float pr = __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, pv[h]), i0 + u));
#pragma unroll
          for (uint32_t j = 0; j < kDvl; ++j) o[h][j] = fmaf(pr, vv[u][j], o[h][j]);
        }
      }
    }
  }

  __shared__ float sm_m[kVecWaves][kH];
  __shared__ float sm_l[kVecWaves][kH];
  __shared__ float sm_o[kVecWaves][kH][kDvTile];
  if (lane == 0) {
#pragma unroll
    for (uint32_t h = 0; h < kH; ++h) {
      sm_m[wave][h] = m[h];
      sm_l[wave][h] = l[h];
    }
  }
#pragma unroll
  for (uint32_t h = 0; h < kH; ++h) {
#pragma unroll
    for (uint32_t j = 0; j < kDvl; ++j) sm_o[wave][h][j * 64 + lane] = o[h][j];
  }
  __syncthreads();

  for (uint32_t idx = threadIdx.x; idx < kH * kDvTile; idx += kVecThreads) {
    const uint32_t h = idx / kDvTile;
    const uint32_t dd = idx % kDvTile;
    const uint32_t d = dvt * kDvTile + dd;
    if (h >= heads || d >= Dv) continue;
    float M = -INFINITY;
#pragma unroll
    for (uint32_t w = 0; w < kVecWaves; ++w) M = fmaxf(M, sm_m[w][h]);
    float L = 0.0f, O = 0.0f;
#pragma unroll
    for (uint32_t w = 0; w < kVecWaves; ++w) {
      const float f = exp2f(sm_m[w][h] - M);  // 0 for a wave that saw no token
      L = fmaf(sm_l[w][h], f, L);
      O = fmaf(sm_o[w][h][dd], f, O);
    }
    const uint64_t row = static_cast<uint64_t>(seq) * a.query_heads + qh0 + h;
    if (a.parts == 1) {
      static_cast<QT*>(a.output)[row * Dv + d] = QE::from_f(O / L);
      if (a.lse != nullptr && d == 0) a.lse[row] = (M + log2f(L)) * kLn2;
    } else {
      const uint64_t state = state_of(a, row, part);
      put_partial(a, state * Dv + d, O);
      if (d == 0) {
        a.ws_ml[state * 2] = M;
        a.ws_ml[state * 2 + 1] = L;
      }
    }
  }
}


// ---------------------------------------------------------------------------
// Matrix-core kernel.
// ---------------------------------------------------------------------------
constexpr uint32_t kChunk = 32;        // tokens per wave iteration
constexpr uint32_t kDim = 128;         // head_size == value_head_size
constexpr uint32_t kTileRowBytes = kDim * 2;
constexpr uint32_t kTileBytes = kChunk * kTileRowBytes;  // 8 KiB V tile per wave

template <typename QE>
struct MfmaOps;

typedef short s16x4m __attribute__((ext_vector_type(4)));
typedef _Float16 f16x4 __attribute__((ext_vector_type(4)));

template <>
struct MfmaOps<Bf16Elem> {
  using vec8 = bf16x8;
  using vec4 = s16x4m;
  static __device__ __forceinline__ f32x4 mma(vec8 a, vec8 b, f32x4 c) {
    return __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, b, c, 0, 0, 0);
  }
  static __device__ __forceinline__ f32x4 mma16(vec4 a, vec4 b, f32x4 c) {
    return __builtin_amdgcn_mfma_f32_16x16x16bf16_1k(a, b, c, 0, 0, 0);
  }
  // Eight FP8 E4M3FN bytes (two dwords) to eight 16-bit values, exactly.
  static __device__ __forceinline__ vec8 from_fp8(uint32_t lo, uint32_t hi) {
    const bf16x2 a0 = __builtin_amdgcn_cvt_scalef32_pk_bf16_fp8(lo, 1.0f, false);
    const bf16x2 a1 = __builtin_amdgcn_cvt_scalef32_pk_bf16_fp8(lo, 1.0f, true);
    const bf16x2 a2 = __builtin_amdgcn_cvt_scalef32_pk_bf16_fp8(hi, 1.0f, false);
    const bf16x2 a3 = __builtin_amdgcn_cvt_scalef32_pk_bf16_fp8(hi, 1.0f, true);
    return vec8{a0[0], a0[1], a1[0], a1[1], a2[0], a2[1], a3[0], a3[1]};
  }
  static __device__ __forceinline__ uint32_t pack2(float x, float y) {
    const bf16x2 v{static_cast<__bf16>(x), static_cast<__bf16>(y)};
    return __builtin_bit_cast(uint32_t, v);
  }
  // PV takes the probabilities as a BF16 pair hi + lo: BF16's 8 significant
  // bits alone put up to 2^-9 of relative error on every weight, which a row
  // of large values of opposite sign keeps in full (measured 3.9e-3 against
  // the oracle on a 16-token head-256 row, past the 2e-3 parity bar). The
  // remainder x - hi rides in the same MFMA where the product has room for
  // it (StreamDecoder: one K = 32 instruction in place of K = 16), else in a
  // second one.
  static constexpr bool kSplitP = true;
  static __device__ __forceinline__ uint32_t rest2(float x, float y, uint32_t hi) {
    return pack2(x - __uint_as_float(hi << 16), y - __uint_as_float(hi & 0xFFFF0000U));
  }
};

template <>
struct MfmaOps<F16Elem> {
  using vec8 = f16x8;
  using vec4 = f16x4;
  static __device__ __forceinline__ f32x4 mma(vec8 a, vec8 b, f32x4 c) {
    return __builtin_amdgcn_mfma_f32_16x16x32_f16(a, b, c, 0, 0, 0);
  }
  static __device__ __forceinline__ f32x4 mma16(vec4 a, vec4 b, f32x4 c) {
    return __builtin_amdgcn_mfma_f32_16x16x16f16(a, b, c, 0, 0, 0);
  }
  static __device__ __forceinline__ vec8 from_fp8(uint32_t lo, uint32_t hi) {
    const f16x2 a0 = __builtin_amdgcn_cvt_scalef32_pk_f16_fp8(lo, 1.0f, false);
    const f16x2 a1 = __builtin_amdgcn_cvt_scalef32_pk_f16_fp8(lo, 1.0f, true);
    const f16x2 a2 = __builtin_amdgcn_cvt_scalef32_pk_f16_fp8(hi, 1.0f, false);
    const f16x2 a3 = __builtin_amdgcn_cvt_scalef32_pk_f16_fp8(hi, 1.0f, true);
    return vec8{a0[0], a0[1], a1[0], a1[1], a2[0], a2[1], a3[0], a3[1]};
  }
  static __device__ __forceinline__ uint32_t pack2(float x, float y) {
    const f16x2 v{static_cast<_Float16>(x), static_cast<_Float16>(y)};
    return __builtin_bit_cast(uint32_t, v);
  }
  // F16 probabilities keep 11 significant bits (P <= 1): one MFMA.
  static constexpr bool kSplitP = false;
  static __device__ __forceinline__ uint32_t rest2(float, float, uint32_t) { return 0U; }
};

__device__ __forceinline__ u32x4 load16(const void* p) {
  return *static_cast<const u32x4*>(p);
}

// ---------------------------------------------------------------------------
// Hand-scheduled memory pipeline. The decode loop's global loads are issued
// as inline assembly, which the compiler's wait-count insertion does not see,
// and every consumer is preceded by an explicit s_waitcnt vmcnt(N) that also
// names the destination registers as in/out operands (so no use of them can
// be scheduled above it). Vector-memory loads of a wave complete in issue
// order, so vmcnt(N) guarantees every load except the N most recent ones.
// (The compiler's own insertion waits for all outstanding loads at this
// loop's header and before DS instructions while LDS DMA is in flight, which
// would drain the prefetch pipeline on every chunk.)
// ---------------------------------------------------------------------------
__device__ __forceinline__ void vm_load16(u32x4& dst, const void* p) {
  asm volatile("global_load_dwordx4 %0, %1, off" : "=v"(dst) : "v"(p));
}

// K/V cache loads carry the non-temporal hint (nt): every cache byte is read
// once per call, and streaming reads with nt measured 7.0-7.1 TB/s against
// 6.1-6.2 TB/s without it (contiguous 4 GiB reads, plain or LDS DMA). On C3
// the decode kernel went from 217 to 199.5 us.
__device__ __forceinline__ void vm_load16_kv(u32x4& dst, const void* p) {
  asm volatile("global_load_dwordx4 %0, %1, off nt" : "=v"(dst) : "v"(p));
}

__device__ __forceinline__ void vm_load4(int32_t& dst, const void* p) {
  asm volatile("global_load_dword %0, %1, off" : "=v"(dst) : "v"(p));
}

// 16 bytes per lane from global memory straight into LDS at lds + 16 * lane
// (M0 holds the wave-uniform LDS base); K/V cache rows, non-temporal.
__device__ __forceinline__ void vm_load16_lds(const void* p, uint8_t* lds) {
  const uint32_t base = __builtin_amdgcn_readfirstlane(
      static_cast<uint32_t>(reinterpret_cast<uintptr_t>((__attribute__((address_space(3))) uint8_t*)lds)));
  asm volatile("s_mov_b32 m0, %1\n\tglobal_load_lds_dwordx4 %0, off nt" : : "v"(p), "s"(base) : "memory", "m0");
}

// Registers of one in-flight 32-token chunk plus the block IDs of the chunk
// two steps later.
//   16-bit caches: k[sb*4 + kc] = 8 dims kc*32 + (lane >> 4)*8 of token
//   sb*16 + (lane & 15), already in the QK^T MFMA operand layout; V goes
//   global -> LDS by DMA and has no registers.
//   FP8 caches: k[sb*2 + j] = 16 bytes at dims j*64 + (lane >> 4)*16 of the
//   same token; v[i] = 16 bytes (lane & 7)*16 of token 8*i + (lane >> 3).
template <bool kFp8>
struct ChunkBuf {
  static constexpr int kK = kFp8 ? 4 : 8;
  static constexpr int kLoads = kFp8 ? 8 : 16;  // vector-memory loads per chunk
  u32x4 k[kK];
  u32x4 v[4];
  int32_t ids;
};

// s_waitcnt vmcnt(N) bound to one chunk buffer's registers.
template <int N>
__device__ __forceinline__ void vm_wait(ChunkBuf<false>& b) {
  asm volatile("s_waitcnt vmcnt(%9)"
               : "+v"(b.k[0]), "+v"(b.k[1]), "+v"(b.k[2]), "+v"(b.k[3]), "+v"(b.k[4]), "+v"(b.k[5]),
                 "+v"(b.k[6]), "+v"(b.k[7]), "+v"(b.ids)
               : "n"(N)
               : "memory");
}

template <int N>
__device__ __forceinline__ void vm_wait(ChunkBuf<true>& b) {
  asm volatile("s_waitcnt vmcnt(%9)"
               : "+v"(b.k[0]), "+v"(b.k[1]), "+v"(b.k[2]), "+v"(b.k[3]), "+v"(b.v[0]), "+v"(b.v[1]),
                 "+v"(b.v[2]), "+v"(b.v[3]), "+v"(b.ids)
               : "n"(N)
               : "memory");
}

typedef short s16x4 __attribute__((ext_vector_type(4)));
typedef __attribute__((address_space(3))) uint8_t lds_u8;
typedef __attribute__((address_space(3))) s16x4 lds_s16x4;

// V tile in LDS: 32 token rows of 128 16-bit values (8 KiB). The 16-byte
// chunk ch of row t sits at chunk ch ^ 2*(t & 3): the transposed reads below
// (per 16-lane group: four rows t = 4g + k, 32 consecutive bytes each) then
// touch four disjoint 32-byte bank groups.
__device__ __forceinline__ uint32_t tile_off(uint32_t t, uint32_t ch) {
  return t * kTileRowBytes + ((ch ^ ((t & 3U) << 1)) << 4);
}

template <typename QE, bool kFp8, int kHeadTiles>
struct MfmaDecoder {
  using Ops = MfmaOps<QE>;
  using vec8 = typename Ops::vec8;
  using CT = typename std::conditional<kFp8, uint8_t, uint16_t>::type;
  using Buf = ChunkBuf<kFp8>;

  const DecodeArgs& a;
  uint32_t lane, g, c, p1;
  const int32_t* table;
  const CT* kbase;  // key cache + kv_head offset
  const CT* vbase;
  float sl2;

  vec8 qb[kHeadTiles][4];
  f32x4 acc[kHeadTiles][8];  // O^T tiles: dims dt*16 + 4g + r, head c
  float m[kHeadTiles];       // running max (log2 units) of head c
  float lsum[kHeadTiles];    // partial denominator over this lane's tokens

  __device__ __forceinline__ MfmaDecoder(const DecodeArgs& args) : a(args) {}

  // Lane i loads the table entry of logical block (c0 >> shift) + i (at most
  // 32 blocks per chunk); lanes past the chunk's last block reload the last
  // entry, so the load is branch-free.
  __device__ __forceinline__ void fetch_ids(int32_t& ids, uint32_t c0) const {
    const uint32_t lb0 = c0 >> a.block_shift;
    const uint32_t last = (min(c0 + kChunk, p1) - 1U) >> a.block_shift;
    vm_load4(ids, table + min(lb0 + lane, last));
  }

  // Element offset of the row of token t (clamped into the partition).
  __device__ __forceinline__ uint64_t row_of(uint32_t c0, int32_t ids, uint32_t t, uint64_t stride_b,
                                             uint64_t stride_p) const {
    t = min(t, p1 - 1U);
    const uint32_t src = (t >> a.block_shift) - (c0 >> a.block_shift);
    const uint32_t blk = static_cast<uint32_t>(__shfl(ids, static_cast<int>(src), 64));
    const uint32_t page = t & (a.block_size - 1U);
    return static_cast<uint64_t>(blk) * stride_b + static_cast<uint64_t>(page) * stride_p;
  }

  __device__ __forceinline__ void issue_k(Buf& b, int32_t ids, uint32_t c0) const {
    constexpr int kPerRow = kFp8 ? 2 : 4;
#pragma unroll
    for (int sb = 0; sb < 2; ++sb) {
      const CT* p = kbase + row_of(c0, ids, c0 + sb * 16 + c, a.k_block, a.k_page);
#pragma unroll
      for (int j = 0; j < kPerRow; ++j) {
        const uint32_t dim = kFp8 ? (j * 64 + g * 16) : (j * 32 + g * 8);
        vm_load16_kv(b.k[sb * kPerRow + j], p + dim);
      }
    }
  }

  // 16-bit V: eight global -> LDS DMA loads of 1 KiB. Load i fills tile rows
  // 4i..4i+3 in lane order (lane l -> byte 16*l), so lane l fetches the
  // logical chunk that the swizzle places at its slot.
  __device__ __forceinline__ void issue_v_dma(uint8_t* tile, int32_t ids, uint32_t c0) const {
    const uint32_t ch = (lane & 15U) ^ (((lane >> 4) & 3U) << 1);
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      const uint32_t t = c0 + 4 * i + (lane >> 4);
      vm_load16_lds(vbase + row_of(c0, ids, t, a.v_block, a.v_page) + ch * 8, tile + i * 1024);
    }
  }

  __device__ __forceinline__ void issue_v_fp8(Buf& b, int32_t ids, uint32_t c0) const {
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const uint32_t t = c0 + 8 * i + (lane >> 3);
      vm_load16_kv(b.v[i], vbase + row_of(c0, ids, t, a.v_block, a.v_page) + (lane & 7U) * 16);
    }
  }

  // One chunk's loads, in the order the steady state uses: V, K (FP8) or
  // K, V (16-bit); the IDs of chunk n + 2 follow separately.
  __device__ __forceinline__ void issue_chunk(Buf& b, uint8_t* tile, int32_t ids, uint32_t c0) const {
    if (kFp8) {
      issue_v_fp8(b, ids, c0);
      issue_k(b, ids, c0);
    } else {
      issue_k(b, ids, c0);
      issue_v_dma(tile, ids, c0);
    }
  }

  // FP8 V: exact conversion to 16-bit values, written in the tile layout.
  __device__ __forceinline__ void stage_v_fp8(const Buf& b, uint8_t* tile) const {
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const uint32_t t = 8 * i + (lane >> 3);
      const uint32_t ch = (lane & 7U) * 2;
      const vec8 lo = Ops::from_fp8(b.v[i][0], b.v[i][1]);
      const vec8 hi = Ops::from_fp8(b.v[i][2], b.v[i][3]);
      // 16-byte LDS writes are served 8 lanes at a time over 128 bytes of
      // banks: lanes 4..7 of each eight store their upper chunk first, so the
      // eight chunks of one store land in distinct 16-byte bank quarters.
      const uint32_t up = (lane >> 2) & 1U;
      *reinterpret_cast<vec8*>(tile + tile_off(t, ch + up)) = up ? hi : lo;
      *reinterpret_cast<vec8*>(tile + tile_off(t, ch + 1 - up)) = up ? lo : hi;
    }
  }

  __device__ __forceinline__ vec8 k_operand(const Buf& b, int sb, int kc) const {
    if (kFp8) {
      const u32x4 w = b.k[sb * 2 + (kc >> 1)];
      return (kc & 1) ? Ops::from_fp8(w[2], w[3]) : Ops::from_fp8(w[0], w[1]);
    } else {
      return __builtin_bit_cast(vec8, b.k[sb * 4 + kc]);
    }
  }

  // PV A operand: V^T[dims dt*16 + c][8 token slots of lane group g] by two
  // transposed reads. In a 16-lane group, ds_read_b64_tr_b16 hands lane i,
  // element k, the 16-bit element i % 4 of the 8 bytes addressed by lane
  // 4k + i / 4; lane (k = c >> 2, q = c & 3) therefore addresses dims
  // dt*16 + 4q of token 4g + k, and lane c receives dim dt*16 + c of tokens
  // 4g + k (first read) and 16 + 4g + k (second read): token slot j of group g
  // is token (j >> 2) * 16 + 4g + (j & 3), where the QK output placed P.
  __device__ __forceinline__ vec8 v_operand(const uint8_t* tile, uint32_t dt) const {
    const uint32_t k = c >> 2, q = c & 3U;
    const uint32_t off = tile_off(4 * g + k, 2 * dt + (q >> 1)) + (q & 1U) * 8;
    lds_u8* base = (lds_u8*)tile;  // generic -> LDS address space
    const s16x4 lo = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_s16x4*)(base + off));
    const s16x4 hi = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_s16x4*)(base + off + 16 * kTileRowBytes));
    typedef short s16x8 __attribute__((ext_vector_type(8)));
    const s16x8 w = {lo[0], lo[1], lo[2], lo[3], hi[0], hi[1], hi[2], hi[3]};
    return __builtin_bit_cast(vec8, w);
  }

  // QK^T of one chunk: S[token 4g + r][head c] for its two 16-token halves.
  __device__ __forceinline__ void qk(const Buf& b, f32x4 (&s)[kHeadTiles][2]) const {
#pragma unroll
    for (int ht = 0; ht < kHeadTiles; ++ht) {
#pragma unroll
      for (int sb = 0; sb < 2; ++sb) {
        f32x4 z = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
        for (int kc = 0; kc < 4; ++kc) z = Ops::mma(k_operand(b, sb, kc), qb[ht][kc], z);
        s[ht][sb] = z;
      }
    }
  }

  // Online softmax and PV of one chunk whose V is in `tile`.
  __device__ __forceinline__ void softmax_pv(f32x4 (&s)[kHeadTiles][2], uint32_t c0, const uint8_t* tile) {
    vec8 pb[kHeadTiles], pr[kHeadTiles];
#pragma unroll
    for (int ht = 0; ht < kHeadTiles; ++ht) {
      float cmax = -INFINITY;
#pragma unroll
      for (int sb = 0; sb < 2; ++sb) {
#pragma unroll
        for (int rr = 0; rr < 4; ++rr) {
          const uint32_t t = c0 + sb * 16 + 4 * g + rr;
          const float v = t < p1 ? s[ht][sb][rr] * sl2 : -INFINITY;
          s[ht][sb][rr] = v;
          cmax = fmaxf(cmax, v);
        }
      }
      cmax = fmaxf(cmax, __shfl_xor(cmax, 16, 64));
      cmax = fmaxf(cmax, __shfl_xor(cmax, 32, 64));
      const float mn = fmaxf(m[ht], cmax);  // finite: every chunk has a valid token
      const float alpha = __builtin_amdgcn_exp2f(m[ht] - mn);
      m[ht] = mn;
      float p[8];
      float psum = 0.0f;
#pragma unroll
      for (int j = 0; j < 8; ++j) {
        p[j] = __builtin_amdgcn_exp2f(s[ht][j >> 2][j & 3] - mn);
        psum += p[j];
      }
      lsum[ht] = fmaf(lsum[ht], alpha, psum);
#pragma unroll
      for (int dt = 0; dt < 8; ++dt) acc[ht][dt] *= alpha;
      u32x4 w;
      w[0] = Ops::pack2(p[0], p[1]);
      w[1] = Ops::pack2(p[2], p[3]);
      w[2] = Ops::pack2(p[4], p[5]);
      w[3] = Ops::pack2(p[6], p[7]);
      pb[ht] = __builtin_bit_cast(vec8, w);
      if constexpr (Ops::kSplitP) {
        const u32x4 r{Ops::rest2(p[0], p[1], w[0]), Ops::rest2(p[2], p[3], w[1]), Ops::rest2(p[4], p[5], w[2]),
                      Ops::rest2(p[6], p[7], w[3])};
        pr[ht] = __builtin_bit_cast(vec8, r);
      }
    }
#pragma unroll
    for (uint32_t dt = 0; dt < 8; ++dt) {
      const vec8 va = v_operand(tile, dt);
#pragma unroll
      for (int ht = 0; ht < kHeadTiles; ++ht) {
        acc[ht][dt] = Ops::mma(va, pb[ht], acc[ht][dt]);
        if constexpr (Ops::kSplitP) acc[ht][dt] = Ops::mma(va, pr[ht], acc[ht][dt]);
      }
    }
  }

  // Pipeline step for chunk n held in buffer b / tile. Every step issues the
  // same loads: chunk n + 2 into b and the tile (K once QK^T has consumed
  // b.k, V once PV has read the tile or, for FP8, once it is staged) and the
  // block IDs of chunk n + 4. Chunks past the wave's last one are not
  // skipped: their tokens clamp to the partition's last row, so those loads
  // hit in cache and are never consumed. With a uniform issue pattern the
  // loads in flight on entry are always, oldest first, chunk n's group and
  // chunk n + 1's group (L loads + 1 ID load each), so one wait of
  // vmcnt(L + 1) completes exactly chunk n's group.
  __device__ __forceinline__ void step(Buf& b, uint8_t* tile, uint32_t cn, uint32_t stride_tokens) {
    vm_wait<Buf::kLoads + 1>(b);
    const uint32_t c2 = cn + 2 * stride_tokens;
    if (kFp8) {
      stage_v_fp8(b, tile);
      wave_fence_lds();
      issue_v_fp8(b, b.ids, c2);
    }
    f32x4 s[kHeadTiles][2];
    qk(b, s);
    issue_k(b, b.ids, c2);
    softmax_pv(s, cn, tile);
    if (!kFp8) {
      wait_lds_reads();  // the tile's transposed reads have returned before the DMA refills it
      issue_v_dma(tile, b.ids, c2);
    }
    wave_fence_lds();
    fetch_ids(b.ids, cn + 4 * stride_tokens);
  }
};

template <typename QE, bool kFp8, int kHeadTiles, int kWaves>
__global__ __launch_bounds__(kWaves * 64) void decode_mfma_kernel(DecodeArgs a) {
  using Dec = MfmaDecoder<QE, kFp8, kHeadTiles>;
  using vec8 = typename Dec::vec8;
  using CT = typename Dec::CT;
  using Buf = typename Dec::Buf;
  __shared__ __attribute__((aligned(16))) uint8_t tile0[kWaves * kTileBytes];
  __shared__ __attribute__((aligned(16))) uint8_t tile1[kWaves * kTileBytes];

  // KV head fastest: the workgroups of one (sequence, partition) are
  // dispatched together (one per XCD for 8 KV heads), so the per-head slices
  // of each paged block are read at about the same time.
  const uint32_t bid = blockIdx.x;
  const uint32_t kvh = bid % a.kv_heads;
  const uint32_t rest = bid / a.kv_heads;
  const uint32_t part = rest % a.parts;
  const uint32_t seq = rest / a.parts;
  const uint32_t len = static_cast<uint32_t>(a.sequence_lengths[seq]);
  const uint32_t p0 = part * a.partition_tokens;
  if (p0 >= len) return;  // uniform across the workgroup

  Dec dec(a);
  dec.lane = threadIdx.x & 63U;
  dec.g = dec.lane >> 4;
  dec.c = dec.lane & 15U;
  dec.p1 = min(p0 + a.partition_tokens, len);
  dec.table = a.block_tables + static_cast<uint64_t>(seq) * a.max_blocks;
  dec.kbase = static_cast<const CT*>(a.key_cache) + static_cast<uint64_t>(kvh) * a.k_head;
  dec.vbase = static_cast<const CT*>(a.value_cache) + static_cast<uint64_t>(kvh) * a.v_head;
  const uint32_t wave = kWaves == 1 ? 0U : __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  uint8_t* tA = tile0 + wave * kTileBytes;
  uint8_t* tB = tile1 + wave * kTileBytes;

  float k_scale = 1.0f, v_scale = 1.0f;
  if (kFp8) {
    k_scale = a.key_scales[kvh * a.scale_stride];
    v_scale = a.value_scales[kvh * a.scale_stride];
  }
  dec.sl2 = a.score_scale_log2 * k_scale;

  // Chunks of this partition: chunk k covers [p0 + 32k, p0 + 32k + 32); wave
  // w takes chunks w, w + waves, ...
  const uint32_t nck = (dec.p1 - p0 + kChunk - 1) / kChunk;
  const uint32_t my_n = nck > wave ? (nck - wave + kWaves - 1) / kWaves : 0;
  const uint32_t st = kWaves * kChunk;
  const uint32_t c0 = p0 + wave * kChunk;

  // Query operand (head ht*16 + c, the dims paired with this lane's K dims)
  // and the first two chunks' block IDs; then everything is waited for.
  const uint16_t* qrow = static_cast<const uint16_t*>(a.query) +
                         (static_cast<uint64_t>(seq) * a.query_heads + kvh * a.group) * kDim;
  u32x4 qw[kHeadTiles][4];
#pragma unroll
  for (int ht = 0; ht < kHeadTiles; ++ht) {
    const uint32_t h = min(ht * 16 + dec.c, a.group - 1U);  // rows >= group are zeroed below
#pragma unroll
    for (int kc = 0; kc < 4; ++kc) {
      const uint32_t dim = kFp8 ? ((kc >> 1) * 64 + dec.g * 16 + (kc & 1) * 8) : (kc * 32 + dec.g * 8);
      vm_load16(qw[ht][kc], qrow + h * kDim + dim);
    }
  }
  Buf bA, bB;
  int32_t ids0, ids1;
  dec.fetch_ids(ids0, c0);
  dec.fetch_ids(ids1, c0 + st);
  asm volatile("s_waitcnt vmcnt(0)" : "+v"(ids0), "+v"(ids1) : : "memory");
#pragma unroll
  for (int ht = 0; ht < kHeadTiles; ++ht) {
#pragma unroll
    for (int kc = 0; kc < 4; ++kc) asm volatile("s_waitcnt vmcnt(0)" : "+v"(qw[ht][kc]));
  }
#pragma unroll
  for (int ht = 0; ht < kHeadTiles; ++ht) {
    const bool live = ht * 16 + dec.c < a.group;
#pragma unroll
    for (int kc = 0; kc < 4; ++kc) {
      const u32x4 w = live ? qw[ht][kc] : u32x4{0U, 0U, 0U, 0U};
      dec.qb[ht][kc] = __builtin_bit_cast(vec8, w);
    }
    dec.m[ht] = -INFINITY;
    dec.lsum[ht] = 0.0f;
#pragma unroll
    for (int dt = 0; dt < 8; ++dt) dec.acc[ht][dt] = f32x4{0.0f, 0.0f, 0.0f, 0.0f};
  }

  if (my_n > 0) {
    // Prologue in steady-state order: chunk 0, IDs of chunk 2, chunk 1, IDs
    // of chunk 3 (missing chunks clamp, as in step()).
    dec.issue_chunk(bA, tA, ids0, c0);
    dec.fetch_ids(bA.ids, c0 + 2 * st);
    dec.issue_chunk(bB, tB, ids1, c0 + st);
    dec.fetch_ids(bB.ids, c0 + 3 * st);
    for (uint32_t n = 0; n < my_n; n += 2) {
      const uint32_t cn = c0 + n * st;
      dec.step(bA, tA, cn, st);
      if (n + 1 >= my_n) break;
      dec.step(bB, tB, cn + st, st);
    }
    // Drain the trailing (clamped) loads: DMA into the tiles must land
    // before the tiles are reused below.
    asm volatile("s_waitcnt vmcnt(0)" : : : "memory");
  }

  // Per-lane partial denominators -> per head (sum over the 4 lane groups).
#pragma unroll
  for (int ht = 0; ht < kHeadTiles; ++ht) {
    float l = dec.lsum[ht];
    l += __shfl_xor(l, 16, 64);
    l += __shfl_xor(l, 32, 64);
    dec.lsum[ht] = l;
  }

  const uint32_t heads = min(a.group, static_cast<uint32_t>(kHeadTiles * 16));
  if (kWaves == 1) {
    // One wave: write straight from the accumulators. Lane (g, c) holds
    // dims dt*16 + 4g + r of head c.
#pragma unroll
    for (int ht = 0; ht < kHeadTiles; ++ht) {
      const uint32_t h = ht * 16 + dec.c;
      if (h >= heads) continue;
      const uint64_t row = static_cast<uint64_t>(seq) * a.query_heads + kvh * a.group + h;
      const float M = dec.m[ht], L = dec.lsum[ht];
      if (a.parts == 1) {
        const float inv = v_scale / L;
        uint16_t* o = static_cast<uint16_t*>(a.output) + row * kDim + 4 * dec.g;
#pragma unroll
        for (int dt = 0; dt < 8; ++dt) {
          uint32_t w0 = QE::from_f(dec.acc[ht][dt][0] * inv) | (static_cast<uint32_t>(QE::from_f(dec.acc[ht][dt][1] * inv)) << 16);
          uint32_t w1 = QE::from_f(dec.acc[ht][dt][2] * inv) | (static_cast<uint32_t>(QE::from_f(dec.acc[ht][dt][3] * inv)) << 16);
          *reinterpret_cast<uint2*>(o + dt * 16) = make_uint2(w0, w1);
        }
        if (a.lse != nullptr && dec.g == 0) a.lse[row] = (M + log2f(L)) * kLn2;
      } else {
        const uint64_t state = state_of(a, row, part);
#pragma unroll
        for (int dt = 0; dt < 8; ++dt) put_partial4(a, state * kDim + 4 * dec.g + dt * 16, dec.acc[ht][dt], v_scale);
        if (dec.g == 0) {
          a.ws_ml[state * 2] = M;
          a.ws_ml[state * 2 + 1] = L;
        }
      }
    }
    return;
  }

  // Several waves: reduce through LDS one head tile at a time. Wave w
  // publishes O[16 heads][128 dims] in its tile0 slot and (m, l) per head in
  // its tile1 slot.
  float* so = reinterpret_cast<float*>(tA);
  float* sml = reinterpret_cast<float*>(tB);
#pragma unroll
  for (int ht = 0; ht < kHeadTiles; ++ht) {
    __syncthreads();  // tiles are free (loop done / previous tile consumed)
    if (dec.g == 0) {
      sml[dec.c * 2] = dec.m[ht];
      sml[dec.c * 2 + 1] = dec.lsum[ht];
    }
#pragma unroll
    for (int dt = 0; dt < 8; ++dt) {
      *reinterpret_cast<f32x4*>(so + dec.c * kDim + dt * 16 + 4 * dec.g) = dec.acc[ht][dt];
    }
    __syncthreads();
    const uint32_t tile_heads = heads > ht * 16U ? min(16U, heads - ht * 16U) : 0U;
    for (uint32_t idx = threadIdx.x; idx < tile_heads * kDim; idx += kWaves * 64) {
      const uint32_t hl = idx / kDim;
      const uint32_t d = idx % kDim;
      float M = -INFINITY;
#pragma unroll
      for (int w = 0; w < kWaves; ++w) M = fmaxf(M, reinterpret_cast<const float*>(tile1 + w * kTileBytes)[hl * 2]);
      float L = 0.0f, O = 0.0f;
#pragma unroll
      for (int w = 0; w < kWaves; ++w) {
        const float* wml = reinterpret_cast<const float*>(tile1 + w * kTileBytes);
        const float* wo = reinterpret_cast<const float*>(tile0 + w * kTileBytes);
        const float f = exp2f(wml[hl * 2] - M);  // 0 for a wave that had no chunk
        L = fmaf(wml[hl * 2 + 1], f, L);
        O = fmaf(wo[hl * kDim + d], f, O);
      }
      O *= v_scale;
      const uint64_t row = static_cast<uint64_t>(seq) * a.query_heads + kvh * a.group + ht * 16 + hl;
      if (a.parts == 1) {
        static_cast<uint16_t*>(a.output)[row * kDim + d] = QE::from_f(O / L);
        if (a.lse != nullptr && d == 0) a.lse[row] = (M + log2f(L)) * kLn2;
      } else {
        const uint64_t state = state_of(a, row, part);
        put_partial(a, state * kDim + d, O);
        if (d == 0) {
          a.ws_ml[state * 2] = M;
          a.ws_ml[state * 2 + 1] = L;
        }
      }
    }
  }
}

// ---------------------------------------------------------------------------
// Streaming matrix-core kernel: 16-token steps, K and V through LDS.
//
// Each wave owns one (sequence, split-K partition, KV head) work item (or a
// quarter of one, when 4 waves split a partition) and walks it in 16-token
// steps with two steps in flight. It applies when the block size is a power
// of two >= 16 and partitions start on multiples of 16 tokens, so a step lies
// in one block: the block ID is one scalar load, the row base is scalar
// arithmetic, and each load is a global_load_lds_dwordx4 at a loop-invariant
// 32-bit lane offset from that base.
//
// The loads bring whole cache rows: each DMA instruction copies four full
// 256-byte rows (16-bit) or eight full 128-byte rows (FP8) of the wave's KV
// head into LDS. Measured on MI355X, this sustains ~11% more HBM bandwidth
// than loads shaped like the MFMA register operand (64 bytes of 16 rows per
// instruction). 16-byte chunks are XOR-swizzled by row so that operand reads
// are bank-conflict free.
//
// Per step: QK^T with v_mfma_f32_16x16x32 (S[token 4g + r][head c] lands in
// lane (g, c)); PV with v_mfma_f32_16x16x16, whose B operand is exactly that
// S layout (4 tokens of lane group g) and whose A operand (dims dt*16 + c of
// tokens 4g + k) is one ds_read_b64_tr_b16 from the 16-bit V tile. FP8 V is
// converted into that tile once per step; FP8 K is converted as it is read.
// ---------------------------------------------------------------------------
constexpr uint32_t kStep = 16;
constexpr uint32_t kStepTileBytes = kStep * kTileRowBytes;  // 4 KiB

// Chunk permutation of row t in a 16-bit V tile, so that a row's chunks stay
// inside the row: 2 (t & 7) for rows of 256 bytes or more (head size 128 and
// up); 2 (((t >> 1) & 3) ^ (t & 1)) for 128-byte rows (head size 64). The
// transposed 8-byte reads are served 32 lanes (rows 4g .. 4g + 3 of two lane
// groups g, eight rows) at a time over 256 bytes of banks, where rows t and
// t + 2 share bank offsets at the 128-byte pitch: the permutation differs
// across each such set of four rows. It also differs in bit 1 between rows
// 2k and 2k + 1, which keeps the FP8 conversion's 16-byte stores (8 lanes,
// two rows, 128 bytes of banks at a time) conflict-free.
template <uint32_t kPitch>
__host__ __device__ constexpr uint32_t vtile_swizzle(uint32_t t) {
  return kPitch >= 256 ? (t & 7U) << 1 : (((t >> 1) & 3U) ^ (t & 1U)) << 1;
}

// Byte offset of 16-byte chunk ch of row t in a 16-bit V tile (256-byte
// rows): chunk ch sits at ch ^ 2 (t & 7). The transposed reads fetch 8 bytes
// per lane from rows 4g .. 4g + 3 for two lane groups g at a time; XORing
// with three row bits spreads those eight rows over all 64 banks.
template <uint32_t kPitch = kTileRowBytes>
__device__ __forceinline__ uint32_t vtile_off(uint32_t t, uint32_t ch) {
  return t * kPitch + ((ch ^ vtile_swizzle<kPitch>(t)) << 4);
}

template <int N>
__device__ __forceinline__ void vm_wait_dma() {
  asm volatile("s_waitcnt vmcnt(%0)" : : "n"(N) : "memory");
}

// Waits for a step's DMA while the loads of min(later, kMax) later steps
// (kPer instructions each) stay in flight. `later` is wave-uniform: the
// steps issued after the awaited one, fewer than kMax near an item's end,
// where no load is issued past the item's last step.
template <int kPer, int kMax>
__device__ __forceinline__ void vm_wait_dma_later(uint32_t later) {
  if constexpr (kMax <= 0) {
    vm_wait_dma<0>();
  } else {
    if (later >= static_cast<uint32_t>(kMax)) {
      vm_wait_dma<kPer * kMax>();
    } else {
      vm_wait_dma_later<kPer, kMax - 1>(later);
    }
  }
}

// Waits for the query registers as well (loaded after the K/V DMA).
__device__ __forceinline__ void vm_wait_all(u32x4 (&q)[4]) {
  asm volatile("s_waitcnt vmcnt(0)" : "+v"(q[0]), "+v"(q[1]), "+v"(q[2]), "+v"(q[3]) : : "memory");
}

// kNt: with the non-temporal hint (rows of whole 128-byte lines; see
// StreamDecoder::kNtKV).
template <bool kNt>
__device__ __forceinline__ void vm_load16_lds_sv(uint32_t voff, uint64_t base, uint8_t* lds) {
  const uint32_t m0 = __builtin_amdgcn_readfirstlane(
      static_cast<uint32_t>(reinterpret_cast<uintptr_t>((__attribute__((address_space(3))) uint8_t*)lds)));
  if constexpr (kNt) {
    asm volatile("s_mov_b32 m0, %2\n\tglobal_load_lds_dwordx4 %0, %1 nt" : : "v"(voff), "s"(base), "s"(m0) : "memory", "m0");
  } else {
    asm volatile("s_mov_b32 m0, %2\n\tglobal_load_lds_dwordx4 %0, %1" : : "v"(voff), "s"(base), "s"(m0) : "memory", "m0");
  }
}

__device__ __forceinline__ void scalar_ready(uint32_t& v) { asm volatile("s_waitcnt lgkmcnt(0)" : "+s"(v)); }

// Pipeline stages per wave: a 16-bit stage is 8 KiB of K/V rows, an FP8
// stage 4 KiB. Deeper pipelines measured no faster (FP8 with 2, 3 and 4
// stages ran C4 at the same speed; two head tiles per wave ran C5 slower
// with 4 and 6 stages than with 2).
constexpr int kStreamStages = 2;
constexpr int kStreamStagesFp8 = 2;

// kHT: 16-query-head tiles per wave (1, or 2 for groups of 17-32 heads). The
// tiles share each step's K operand fetches and V transposed reads.
// kD: head size (= value head size): 128; 64, where 16-bit rows of 128 bytes
// take the FP8 path's DMA geometry (eight rows per instruction) without a
// conversion and FP8 rows of 64 bytes come sixteen per instruction; or 256
// with one head tile (16-bit rows of 512 bytes two per instruction, FP8 rows
// of 256 bytes four per instruction).
template <typename QE, bool kFp8, int kHT = 1, uint32_t kD = kDim,
          int kS = kFp8 ? kStreamStagesFp8 : kStreamStages, int kNt = -1>
struct StreamDecoder {
  static_assert(kD == kDim || kD == 64 || ((kD == 80 || kD == 96 || kD == 112 || kD == 256) && kHT == 1),
                "head size 64, 128, or 80 / 96 / 112 / 256 with one head tile");
  // K/V loads carry the non-temporal hint when a cache row is whole 128-byte
  // lines. Rows that share lines with their neighbours (head sizes 80, 96 and
  // 112, FP8 at 64-112) then fetch the shared lines twice; measured with the
  // hint (decode us, one partition of 512, B=64): 16-bit D64 187 -> 170, D128
  // 187 -> 172, D256 191 -> 176, FP8 D128 104.5 -> 95.5, FP8 D256 121.5 ->
  // 115, but 16-bit D80 183 -> 206, D96 181 -> 188, D112 167 -> 176, FP8
  // D64 108 -> 131, D80 118 -> 142, D96 119 -> 130, D112 98 -> 120.
  // kNt = 1 forces the hint: the launch passes it when each KV head's token
  // rows are contiguous (HND), so a step of 16 rows covers whole lines at
  // any head size (HND, 8-10% faster with it: 16-bit D80 178 -> 162 us, D96
  // 176 -> 161, D112 165 -> 152, FP8 D64 104 -> 95, D96 119 -> 115).
  static constexpr bool kNtKV = kNt >= 0 ? kNt != 0 : (kD * (kFp8 ? 1U : 2U)) % 128U == 0;
  static constexpr bool kNarrow = kD == 64 && !kFp8;         // 16-bit rows of 128 bytes
  static constexpr bool kF8Narrow = kD == 64 && kFp8;        // FP8 rows of 64 bytes
  static constexpr bool kWide = kD == 256 && !kFp8;          // 16-bit rows of 512 bytes
  static constexpr bool kF8Wide = kD == 256 && kFp8;         // FP8 rows of 256 bytes
  // Head size 96, 16-bit: rows of 12 chunks (192 bytes). Lanes map to chunks
  // by flat index (16 rows x 12 chunks = 3 DMA instructions per tensor), so a
  // stage holds rows at a 192-byte pitch; a row's chunks are rotated by
  // rot_shift(r) (mod 12).
  // Head sizes 80 and 112 take the same layout unrotated: rows of 10 or 14 chunks, a
  // tensor's step rounded up to whole DMA instructions (the spare lanes load
  // a valid chunk into the unused tail), QK over 3 or 4 operand chunks with
  // the chunks past the row read as zero.
  // FP8 rows at these head sizes (80, 96 or 112 bytes) are kept unrotated
  // and contiguous in LDS; the converted 16-bit V tile takes the rotated
  // layout.
  static constexpr bool kRot = kD == 80 || kD == 96 || kD == 112;
  static constexpr bool kF8Rot = kRot && kFp8;
  static constexpr uint32_t kRowChunks = kD / 8;               // 16-byte chunks of a 16-bit row
  static constexpr uint32_t kSrcChunks = kFp8 ? kD / 16 : kD / 8;  // 16-byte chunks of a cache row
  static constexpr int kRotDma = (kStep * kSrcChunks + 63) / 64;  // DMA instructions per tensor per step
  // Rotation of row r (in chunks); rot_slot places chunk `chunk` of row r.
  // Head size 96: 2 (r >> 2). Rows r and r + 4 share bank offsets at the
  // 192-byte pitch, and the shift interleaves their 32-byte pieces in the
  // transposed reads (8 rows per pass); measured free of bank conflicts, where
  // 3 (r >> 2) cost 24 cycles per step. Rows of 160 and 224 bytes (head sizes
  // 80, 112) measured conflict-free unrotated. The FP8 path's converted V
  // tile stays unrotated: its conversion stores (8 lanes over 128 bytes of
  // banks at a time) collide in the rotated layout.
  static __device__ __forceinline__ uint32_t rot_shift(uint32_t r) {
    return kD == 96 && !kFp8 ? 2U * (r >> 2) : 0U;
  }
  static __device__ __forceinline__ uint32_t rot_slot(uint32_t r, uint32_t chunk) {
    return (chunk + rot_shift(r)) % kRowChunks;
  }
  // Byte offset of 16-byte chunk ch of row t in the 16-bit V tile.
  static __device__ __forceinline__ uint32_t vt_off(uint32_t t, uint32_t ch) {
    if constexpr (kRot) {
      return t * kPitch + (rot_slot(t, ch) << 4);
    } else {
      return vtile_off<kD * 2>(t, ch);
    }
  }
  static constexpr uint32_t kPitch = kD * 2;  // bytes between consecutive tokens' rows in a 16-bit tile
  static constexpr int kDt = kD / 16;         // 16-dim PV tiles
  // 32-dim QK operand chunks (the last ones zero-padded); FP8 operands pair
  // them over 64 dims.
  static constexpr int kKc = kFp8 ? 2 * ((kD + 63) / 64) : (kD + 31) / 32;
  using Ops = MfmaOps<QE>;
  using vec8 = typename Ops::vec8;
  using vec4 = typename Ops::vec4;
  // PV's element type: the query's for 16-bit caches; F16 for FP8 caches,
  // whose E4M3 values convert to F16 exactly and whose probabilities then
  // keep 11 significant bits in one MFMA (BF16 ones need a hi + lo pair).
  using PvOps = std::conditional_t<kFp8, MfmaOps<F16Elem>, Ops>;
  using pv8 = typename PvOps::vec8;
  using pv4 = typename PvOps::vec4;
  // LDS per wave. 16-bit: kStages stages of [K 4 KiB | V 4 KiB]; PV reads V
  // in place. FP8: kStages stages of [K bytes 2 KiB | V bytes 2 KiB], then
  // one 4 KiB tile of the current step's V converted to 16 bits (kVTileOff).
  static constexpr int kStages = kS;
  static constexpr uint32_t kF8TileBytes = kRot ? kRotDma * 1024 : kStep * kD;  // FP8 bytes of one tensor's step
  static constexpr uint32_t kVOff = kRot ? kRotDma * 1024 : kStep * kPitch;  // 16-bit: V within a stage
  static constexpr uint32_t kStageBytes = kFp8 ? 2 * kF8TileBytes : 2 * kVOff;
  static constexpr uint32_t kVTileOff = kStages * kStageBytes;  // FP8: converted V tile
  static constexpr uint32_t kWaveBytes = kStages * kStageBytes + (kFp8 ? kStep * kPitch : 0);
  static constexpr int kDmaPerStep = kRot ? 2 * kRotDma : kWide ? 16 : kF8Wide ? 8 : kF8Narrow ? 2 : kFp8 || kNarrow ? 4 : 8;
  static constexpr uint32_t kElem = kFp8 ? 1 : 2;

  const DecodeArgs& a;
  uint32_t lane, g, c;
  uint32_t p1;   // end of this partition (exclusive)
  uint32_t len;  // sequence length
  uint32_t last_block;  // last active logical block of the sequence
  const int32_t* table;
  uint64_t kbase, vbase;  // byte address of (block 0, page 0, this kv head)
  uint64_t kstride_b, vstride_b, kstride_p, vstride_p;  // byte strides
  uint32_t k_voff[4];  // 16-bit: lane's K DMA offset for rows 4i..4i+3
  uint32_t v_voff[2];  // 16-bit: lane's V DMA offset for even / odd 4-row groups
  uint32_t f8_k_voff[2], f8_v_voff[2];  // FP8: lane's K / V DMA offsets, rows 8i .. 8i + 7
  uint32_t w_voff[kWide ? 16 : kF8Wide ? 8 : kRot ? 2 * kRotDma : 1];  // head size 256 / 96: K offsets, then V
  float sl2;

  vec8 qb[kHT][kKc];
  f32x4 acc[kHT][kDt];  // O^T of tile ht: dims dt*16 + 4g + r, head 16 ht + c
  float m[kHT];       // running max (log2 units) of head 16 ht + c
  float lsum[kHT];    // partial denominator over this lane's tokens

  __device__ __forceinline__ StreamDecoder(const DecodeArgs& args) : a(args) {}

  // Physical block of the step starting at token t0 (clamped to the last
  // active block, so steps past the sequence stay in valid memory).
  // A scalar load through the constant address space (the table is not
  // written during the launch): the compiler issues it where it stands and
  // waits for it before the value's first use (scalar_ready), so no register
  // copy or spill can read the destination while the load is in flight.
  __device__ __forceinline__ uint32_t block_of(uint32_t t0) const {
    const uint32_t lb = min(t0 >> a.block_shift, last_block);
    using ConstWord = const __attribute__((address_space(4))) int32_t;
    return static_cast<uint32_t>(((ConstWord*)table)[lb]);
  }

  __device__ __forceinline__ uint64_t row_base(uint64_t base, uint64_t stride_b, uint64_t stride_p, uint32_t blk,
                                               uint32_t t0) const {
    return base + blk * stride_b + (t0 & (a.block_size - 1U)) * stride_p;
  }

  // Lane DMA offsets. 16-bit K: instruction i brings rows 4i + lane / 16;
  // row r keeps its 16-byte chunk L at position L ^ (r & 15), so the 16 rows
  // of one MFMA operand fetch fall in different bank groups. 16-bit V: chunk
  // L of row r at L ^ 2 (r & 7) (vtile_off). FP8: eight 128-byte rows per
  // instruction, chunk L of row r at L ^ ((r >> 1) & 7), which keeps the K
  // operand reads and the V conversion reads bank-conflict free.
  __device__ __forceinline__ void init_offsets() {
    if constexpr (kRot) {
      // Lane l of instruction i fills LDS chunk 64 i + l = (row, slot); it
      // loads the row's logical chunk whose rotated slot that is.
#pragma unroll
      for (int i = 0; i < kRotDma; ++i) {
        const uint32_t idx = 64U * i + lane;
        const bool spare = idx >= kStep * kSrcChunks;  // past the step's rows: reload row 15, chunk 0
        const uint32_t r = spare ? kStep - 1 : idx / kSrcChunks, slot = spare ? 0U : idx % kSrcChunks;
        const uint32_t logical = spare || kFp8 ? slot : (slot + kRowChunks - rot_shift(r)) % kRowChunks;
        w_voff[i] = static_cast<uint32_t>(r * kstride_p) + (logical << 4);
        w_voff[kRotDma + i] = static_cast<uint32_t>(r * vstride_p) + (logical << 4);
      }
    } else if constexpr (kF8Narrow) {
      // FP8 rows of 64 bytes, all 16 rows of a step in one instruction: chunk
      // L of row r at L ^ ((r >> 2) & 3), so the rows sharing a 256-byte bank
      // window hold their chunks at distinct offsets.
      const uint32_t row = lane >> 2;
      const uint32_t chunk = ((lane & 3U) ^ ((row >> 2) & 3U)) << 4;
      f8_k_voff[0] = static_cast<uint32_t>(row * kstride_p) + chunk;
      f8_v_voff[0] = static_cast<uint32_t>(row * vstride_p) + chunk;
    } else if constexpr (kF8Wide) {
      // FP8 rows of 256 bytes, four per instruction: chunk L of row r at
      // L ^ (r & 15) in K and in V (the 8-byte K operand reads of 16 rows,
      // and the V conversion reads of 16 rows at one chunk, then cover all
      // banks).
      const uint32_t row = lane >> 4;
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const uint32_t r = 4 * i + row;
        const uint32_t chunk = ((lane & 15U) ^ (r & 15U)) << 4;
        w_voff[i] = static_cast<uint32_t>(row * kstride_p) + chunk;
        w_voff[4 + i] = static_cast<uint32_t>(row * vstride_p) + chunk;
      }
    } else if constexpr (kWide) {
      // 512-byte rows, two per instruction: K chunk L of row r at L ^ (r & 15),
      // V chunk L at L ^ vtile_swizzle(r) (the bank pattern of 256-byte rows).
      const uint32_t row = lane >> 5;
#pragma unroll
      for (int i = 0; i < 8; ++i) {
        const uint32_t r = 2 * i + row;
        w_voff[i] = static_cast<uint32_t>(row * kstride_p) + (((lane & 31U) ^ (r & 15U)) << 4);
        w_voff[8 + i] = static_cast<uint32_t>(row * vstride_p) + (((lane & 31U) ^ vtile_swizzle<kPitch>(r)) << 4);
      }
    } else if (kNarrow) {
      // 16-bit rows of 128 bytes: K chunk L of row r at L ^ ((r >> 1) & 7)
      // (as FP8 K), V chunk L at L ^ vtile_swizzle(r).
      const uint32_t row = lane >> 3;
#pragma unroll
      for (int i = 0; i < 2; ++i) {
        const uint32_t r = 8 * i + row;
        f8_k_voff[i] = static_cast<uint32_t>(row * kstride_p) + (((lane & 7U) ^ ((r >> 1) & 7U)) << 4);
        f8_v_voff[i] = static_cast<uint32_t>(row * vstride_p) + (((lane & 7U) ^ vtile_swizzle<kPitch>(r)) << 4);
      }
    } else if (kFp8) {
      const uint32_t row = lane >> 3;
#pragma unroll
      for (int i = 0; i < 2; ++i) {
        const uint32_t chunk = ((lane & 7U) ^ (((8 * i + row) >> 1) & 7U)) << 4;
        f8_k_voff[i] = static_cast<uint32_t>(row * kstride_p) + chunk;
        f8_v_voff[i] = static_cast<uint32_t>(row * vstride_p) + chunk;
      }
    } else {
      const uint32_t row = lane >> 4;
#pragma unroll
      for (int i = 0; i < 4; ++i)
        k_voff[i] = static_cast<uint32_t>(row * kstride_p) + (((lane & 15U) ^ (4 * i + row)) << 4);
#pragma unroll
      for (int i = 0; i < 2; ++i)
        v_voff[i] = static_cast<uint32_t>(row * vstride_p) + (((lane & 15U) ^ (((4 * i + row) & 7U) << 1)) << 4);
    }
  }

  // One step's K and V (and nothing else) into a stage.
  __device__ __forceinline__ void issue(uint8_t* stage, uint32_t blk, uint32_t t0) const {
    const uint64_t kb = row_base(kbase, kstride_b, kstride_p, blk, t0);
    const uint64_t vb = row_base(vbase, vstride_b, vstride_p, blk, t0);
    if constexpr (kRot) {
#pragma unroll
      for (int i = 0; i < kRotDma; ++i) vm_load16_lds_sv<kNtKV>(w_voff[i], kb, stage + i * 1024);
#pragma unroll
      for (int i = 0; i < kRotDma; ++i)
        vm_load16_lds_sv<kNtKV>(w_voff[kRotDma + i], vb, stage + (kFp8 ? kF8TileBytes : kVOff) + i * 1024);
    } else if constexpr (kF8Narrow) {
      vm_load16_lds_sv<kNtKV>(f8_k_voff[0], kb, stage);
      vm_load16_lds_sv<kNtKV>(f8_v_voff[0], vb, stage + kF8TileBytes);
    } else if constexpr (kF8Wide) {
#pragma unroll
      for (int i = 0; i < 4; ++i) vm_load16_lds_sv<kNtKV>(w_voff[i], kb + 4 * i * kstride_p, stage + i * 1024);
#pragma unroll
      for (int i = 0; i < 4; ++i)
        vm_load16_lds_sv<kNtKV>(w_voff[4 + i], vb + 4 * i * vstride_p, stage + kF8TileBytes + i * 1024);
    } else if constexpr (kWide) {
#pragma unroll
      for (int i = 0; i < 8; ++i) vm_load16_lds_sv<kNtKV>(w_voff[i], kb + 2 * i * kstride_p, stage + i * 1024);
#pragma unroll
      for (int i = 0; i < 8; ++i) vm_load16_lds_sv<kNtKV>(w_voff[8 + i], vb + 2 * i * vstride_p, stage + kVOff + i * 1024);
    } else if (kNarrow) {
#pragma unroll
      for (int i = 0; i < 2; ++i) vm_load16_lds_sv<kNtKV>(f8_k_voff[i], kb + 8 * i * kstride_p, stage + i * 1024);
#pragma unroll
      for (int i = 0; i < 2; ++i)
        vm_load16_lds_sv<kNtKV>(f8_v_voff[i], vb + 8 * i * vstride_p, stage + kVOff + i * 1024);
    } else if (kFp8) {
#pragma unroll
      for (int i = 0; i < 2; ++i) vm_load16_lds_sv<kNtKV>(f8_k_voff[i], kb + 8 * i * kstride_p, stage + i * 1024);
#pragma unroll
      for (int i = 0; i < 2; ++i)
        vm_load16_lds_sv<kNtKV>(f8_v_voff[i], vb + 8 * i * vstride_p, stage + kF8TileBytes + i * 1024);
    } else {
#pragma unroll
      for (int i = 0; i < 4; ++i) vm_load16_lds_sv<kNtKV>(k_voff[i], kb + 4 * i * kstride_p, stage + i * 1024);
#pragma unroll
      for (int i = 0; i < 4; ++i) vm_load16_lds_sv<kNtKV>(v_voff[i & 1], vb + 4 * i * vstride_p, stage + kVOff + i * 1024);
    }
  }

  // MFMA A operand kc of token c. 16-bit: dims kc*32 + g*8 .. +7. FP8: dims
  // (kc >> 1)*64 + g*16 + ((kc ^ g) & 1)*8 .. +7, converted (Q uses the same
  // dims); the half depends on g so that the two lane groups served together
  // read different banks.
  __device__ __forceinline__ vec8 k_operand(const uint8_t* stage, int kc) const {
    if constexpr (kF8Rot) {
      const uint32_t chunk = (static_cast<uint32_t>(kc) >> 1) * 4 + g;  // FP8 chunk of 16 dims
      const uint2 w = *reinterpret_cast<const uint2*>(stage + c * kD + (chunk < kSrcChunks ? chunk : 0U) * 16 +
                                                      ((kc ^ g) & 1U) * 8);
      if (chunk >= kSrcChunks) return vec8{};  // dims past the head size
      return Ops::from_fp8(w.x, w.y);
    } else if constexpr (kRot) {
      const uint32_t chunk = static_cast<uint32_t>(kc) * 4 + g;
      const uint32_t slot = rot_slot(c, chunk < kRowChunks ? chunk : 0U);
      const vec8 k = *reinterpret_cast<const vec8*>(stage + c * kPitch + slot * 16);
      if constexpr (kRowChunks % 4 != 0) {
        if (chunk >= kRowChunks) return vec8{};  // dims past the head size
      }
      return k;
    } else if (kNarrow) {
      const uint32_t chunk = (static_cast<uint32_t>(kc) * 4 + g) ^ ((c >> 1) & 7U);
      return *reinterpret_cast<const vec8*>(stage + c * kPitch + chunk * 16);
    } else if (kFp8) {
      const uint32_t swz = kF8Wide ? (c & 15U) : kF8Narrow ? ((c >> 2) & 3U) : ((c >> 1) & 7U);
      const uint32_t chunk = ((static_cast<uint32_t>(kc) >> 1) * 4 + g) ^ swz;
      const uint2 w = *reinterpret_cast<const uint2*>(stage + c * kD + chunk * 16 + ((kc ^ g) & 1U) * 8);
      return Ops::from_fp8(w.x, w.y);
    } else {
      const uint32_t chunk = (static_cast<uint32_t>(kc) * 4 + g) ^ c;
      return *reinterpret_cast<const vec8*>(stage + c * kPitch + chunk * 16);
    }
  }

  __device__ __forceinline__ void qk(const uint8_t* stage, f32x4 (&z)[kHT]) const {
    vec8 kop[kKc];
#pragma unroll
    for (int kc = 0; kc < kKc; ++kc) kop[kc] = k_operand(stage, kc);
#pragma unroll
    for (int ht = 0; ht < kHT; ++ht) {
      z[ht] = f32x4{0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
      for (int kc = 0; kc < kKc; ++kc) z[ht] = Ops::mma(kop[kc], qb[ht][kc], z[ht]);
    }
  }

  // FP8 V bytes of a stage -> the wave's swizzled 16-bit V tile (rows past
  // the sequence end become zero). Head sizes 64 and 128: lane handles kD / 4
  // bytes of token lane >> 2; head size 256: lane handles four 16-byte chunks
  // of token lane & 15. 16-byte LDS reads are served 16 lanes at a time over 256 bytes
  // of banks, 16-byte writes 8 lanes at a time over 128 bytes; the row
  // mapping, the V swizzle and the order of each lane's two stores (the
  // `up` lanes store the upper 16-bit chunk first) keep every read and every
  // store free of bank conflicts.
  __device__ __forceinline__ void stage_v_fp8(const uint8_t* stage, uint8_t* tile, uint32_t t0) const {
    if constexpr (kF8Rot) {
      // Rows of 5, 6 or 7 FP8 chunks: lanes take chunks by flat index.
#pragma unroll
      for (uint32_t it = 0; it < (kStep * kSrcChunks + 63) / 64; ++it) {
        const uint32_t idx = it * 64U + lane;
        if (idx < kStep * kSrcChunks) {
          const uint32_t t = idx / kSrcChunks, lc = idx % kSrcChunks;
          const u32x4 raw = *reinterpret_cast<const u32x4*>(stage + kF8TileBytes + t * kD + lc * 16);
          const u32x4 w = t0 + t < len ? raw : u32x4{0U, 0U, 0U, 0U};
          const pv8 lo = PvOps::from_fp8(w[0], w[1]), hi = PvOps::from_fp8(w[2], w[3]);
          // Lanes 4..7 of each eight store their upper chunk first, which
          // spreads each store's eight lanes over distinct bank quarters.
          const uint32_t up = (lane >> 2) & 1U;
          *reinterpret_cast<pv8*>(tile + vt_off(t, 2 * lc + up)) = up ? hi : lo;
          *reinterpret_cast<pv8*>(tile + vt_off(t, 2 * lc + 1 - up)) = up ? lo : hi;
        }
      }
      return;
    }
    constexpr uint32_t kLaneChunks = kD / 64;  // 16-byte FP8 chunks per lane
    const uint32_t t = kF8Wide ? (lane & 15U) : (lane >> 2);
    const uint32_t q = kF8Wide ? (lane >> 4) : (lane & 3U);
    const bool live = t0 + t < len;
    const uint8_t* vrow = stage + kF8TileBytes + t * kD;
    const uint32_t up = kF8Wide ? ((t >> 2) & 1U) : kF8Narrow ? (lane & 1U) : ((lane >> 1) & 1U);
    const uint32_t swz = kF8Wide ? (t & 15U) : kF8Narrow ? ((t >> 2) & 3U) : ((t >> 1) & 7U);
#pragma unroll
    for (uint32_t h = 0; h < kLaneChunks; ++h) {
      // Logical 16-byte chunk of the FP8 row: head size 256 interleaves the
      // four lane groups (q, q + 4, q + 8, q + 12), which measured free of
      // read conflicts where q * 4 + h read 16 conflict cycles per step.
      const uint32_t lc = kF8Wide ? q + 4U * h : q * kLaneChunks + h;
      const u32x4 raw = *reinterpret_cast<const u32x4*>(vrow + ((lc ^ swz) << 4));
      const u32x4 w = live ? raw : u32x4{0U, 0U, 0U, 0U};
      // 16-bit chunks 2 lc and 2 lc + 1 (8 dims each).
      const pv8 lo = PvOps::from_fp8(w[0], w[1]), hi = PvOps::from_fp8(w[2], w[3]);
      const uint32_t ch = lc * 2;
      *reinterpret_cast<pv8*>(tile + vtile_off<kPitch>(t, ch + up)) = up ? hi : lo;
      *reinterpret_cast<pv8*>(tile + vtile_off<kPitch>(t, ch + 1 - up)) = up ? lo : hi;
    }
  }

  // Tile rows of tokens past the sequence end (possible only in its last
  // step) may hold unwritten cache slots: zero them so P = 0 meets a finite V.
  __device__ __forceinline__ void zero_dead_rows(uint8_t* tile, uint32_t t0) const {
    if (t0 + kStep <= len) return;  // uniform
    const uint32_t t = lane >> 2;   // 4 lanes per row, kPitch / 4 bytes each
    if (t0 + t >= len) {
      uint8_t* part = tile + t * kPitch + (lane & 3U) * (kPitch / 4);
      if constexpr ((kPitch / 4) % 16 == 0) {
        u32x4* row = reinterpret_cast<u32x4*>(part);
#pragma unroll
        for (uint32_t i = 0; i < kPitch / 64; ++i) row[i] = u32x4{0U, 0U, 0U, 0U};
      } else {  // 40- or 56-byte quarters (head sizes 80, 112): 8-byte stores
        uint2* row = reinterpret_cast<uint2*>(part);
#pragma unroll
        for (uint32_t i = 0; i < kPitch / 32; ++i) row[i] = make_uint2(0U, 0U);
      }
    }
  }

  __device__ __forceinline__ void softmax_pv(f32x4 (&s)[kHT], uint32_t t0, const uint8_t* tile) {
    typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));
    pv4 pb[kHT], pr[kHT];
#pragma unroll
    for (int ht = 0; ht < kHT; ++ht) {
      float cmax = -INFINITY;
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const float v = t0 + 4 * g + r < p1 ? s[ht][r] * sl2 : -INFINITY;
        s[ht][r] = v;
        cmax = fmaxf(cmax, v);
      }
      cmax = fmaxf(cmax, __shfl_xor(cmax, 16, 64));
      cmax = fmaxf(cmax, __shfl_xor(cmax, 32, 64));
      const float mn = fmaxf(m[ht], cmax);  // finite: every step has a valid token
      // Rescale only when some head's maximum moved (exact; usually skipped).
      if (__builtin_amdgcn_ballot_w64(mn > m[ht]) != 0) {
        const float alpha = __builtin_amdgcn_exp2f(m[ht] - mn);
        lsum[ht] *= alpha;
#pragma unroll
        for (int dt = 0; dt < kDt; ++dt) acc[ht][dt] *= alpha;
        m[ht] = mn;
      }
      float p[4];
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        p[r] = __builtin_amdgcn_exp2f(s[ht][r] - m[ht]);
        lsum[ht] += p[r];
      }
      const uint32_t w0 = PvOps::pack2(p[0], p[1]), w1 = PvOps::pack2(p[2], p[3]);
      pb[ht] = __builtin_bit_cast(pv4, u32x2{w0, w1});
      if constexpr (PvOps::kSplitP)
        pr[ht] = __builtin_bit_cast(pv4, u32x2{PvOps::rest2(p[0], p[1], w0), PvOps::rest2(p[2], p[3], w1)});
    }
    const uint32_t k = c >> 2, q = c & 3U;
    lds_u8* base = (lds_u8*)tile;
#pragma unroll
    for (uint32_t dt = 0; dt < kDt; ++dt) {
      const uint32_t off = vt_off(4 * g + k, 2 * dt + (q >> 1)) + (q & 1U) * 8;
      const s16x4 va = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_s16x4*)(base + off));
#pragma unroll
      for (int ht = 0; ht < kHT; ++ht) {
        if constexpr (PvOps::kSplitP) {
          // One K = 32 MFMA: K index 8g + r pairs token 4g + r with hi, 8g + 4 + r
          // with its remainder lo; the V operand repeats the lane's four tokens.
          typedef short s16x8 __attribute__((ext_vector_type(8)));
          const s16x4 v4 = __builtin_bit_cast(s16x4, va);
          const s16x4 h4 = __builtin_bit_cast(s16x4, pb[ht]), l4 = __builtin_bit_cast(s16x4, pr[ht]);
          const s16x8 a8 = __builtin_shufflevector(v4, v4, 0, 1, 2, 3, 0, 1, 2, 3);
          const s16x8 b8 = __builtin_shufflevector(h4, l4, 0, 1, 2, 3, 4, 5, 6, 7);
          acc[ht][dt] = PvOps::mma(__builtin_bit_cast(pv8, a8), __builtin_bit_cast(pv8, b8), acc[ht][dt]);
        } else {
          acc[ht][dt] = PvOps::mma16(__builtin_bit_cast(pv4, va), pb[ht], acc[ht][dt]);
        }
      }
    }
  }
};

// Per-wave timeline of the streaming kernels, compiled only into profiling
// builds (-DLOOM_HIP_WAVE_TRACE, attnarc_amd/wave_trace.py): each wave of an
// item records its start and end (s_memrealtime, 100 MHz), XCC and hardware
// IDs, and the item. The record of wave slot i of a launch goes to entry i.
#ifdef LOOM_HIP_WAVE_TRACE
struct WaveRecord {
  unsigned long long t0, t1;
  uint32_t xcc, hw_id, seq, part, kvh, tokens;
};
constexpr uint32_t kWaveRecords = 1U << 16;
__device__ WaveRecord g_wave_records[kWaveRecords];

struct WaveStamp {
  uint32_t slot;
  unsigned long long t0;
  uint32_t seq = 0, part = 0, kvh = 0, tokens = 0;
  __device__ ~WaveStamp() {
    const unsigned long long t1 = __builtin_amdgcn_s_memrealtime();
    uint32_t xcc, hw;
    asm volatile("s_getreg_b32 %0, hwreg(HW_REG_XCC_ID)" : "=s"(xcc));
    asm volatile("s_getreg_b32 %0, hwreg(HW_REG_HW_ID)" : "=s"(hw));
    if ((threadIdx.x & 63U) == 0 && slot < kWaveRecords && tokens != 0)
      g_wave_records[slot] = WaveRecord{t0, t1, xcc, hw, seq, part, kvh, tokens};
  }
};
#define LOOM_WAVE_STAMP(slot) WaveStamp wave_stamp{(slot), __builtin_amdgcn_s_memrealtime()}
// Times at which a wave starts its step loop (its Q and first steps' K/V have
// arrived) and reaches 1/4, 1/2 and 3/4 of its steps (record of the same
// wave slot; the slot is the wave's index in the launch).
__device__ unsigned long long g_wave_marks[kWaveRecords][4];
// Time a wave spends waiting for its step loads, per quarter of its steps.
__device__ unsigned long long g_wave_stall[kWaveRecords][4];
#define LOOM_WAVE_STALL_DECL unsigned long long wave_stall[4] = {0ULL, 0ULL, 0ULL, 0ULL}
#define LOOM_WAVE_STALL(step, total, wait_stmt)                                               \
  do {                                                                                        \
    const unsigned long long w0 = __builtin_amdgcn_s_memrealtime();                          \
    wait_stmt;                                                                                \
    const unsigned long long w1 = __builtin_amdgcn_s_memrealtime();                          \
    const uint32_t quarter = min(4U * (step) / max((total), 1U), 3U);                        \
    _Pragma("unroll") for (uint32_t q = 0; q < 4; ++q) if (q == quarter) wave_stall[q] += w1 - w0; \
  } while (0)
#define LOOM_WAVE_STALL_STORE                                                                 \
  do {                                                                                        \
    const uint32_t wave_slot = blockIdx.x * (blockDim.x >> 6) + (threadIdx.x >> 6);          \
    if ((threadIdx.x & 63U) == 0 && wave_slot < kWaveRecords)                                 \
      _Pragma("unroll") for (uint32_t q = 0; q < 4; ++q) g_wave_stall[wave_slot][q] = wave_stall[q]; \
  } while (0)
#define LOOM_WAVE_MARK(n, stride, total)                                                      \
  do {                                                                                        \
    const uint32_t wave_slot = blockIdx.x * (blockDim.x >> 6) + (threadIdx.x >> 6);          \
    _Pragma("unroll") for (uint32_t q = 0; q < 4; ++q) {                                      \
      const uint32_t target = q * (total) / 4U;                                               \
      if (target >= (n) && target < (n) + (stride) && (threadIdx.x & 63U) == 0 &&             \
          wave_slot < kWaveRecords)                                                           \
        g_wave_marks[wave_slot][q] = __builtin_amdgcn_s_memrealtime();                       \
    }                                                                                         \
  } while (0)
#define LOOM_WAVE_ITEM(a, item)                                                                            \
  do {                                                                                                     \
    wave_stamp.seq = (item).seq;                                                                           \
    wave_stamp.part = (item).part;                                                                         \
    wave_stamp.kvh = (item).kvh;                                                                           \
    wave_stamp.tokens = (item).valid ? min((item).len - (item).part * (a).partition_tokens, (a).partition_tokens) : 0U; \
  } while (0)
#else
#define LOOM_WAVE_STAMP(slot) \
  do {                        \
  } while (0)
#define LOOM_WAVE_ITEM(a, item) \
  do {                          \
  } while (0)
#define LOOM_WAVE_MARK(n, stride, total) \
  do {                                   \
  } while (0)
#define LOOM_WAVE_STALL_DECL \
  do {                       \
  } while (0)
#define LOOM_WAVE_STALL(step, total, wait_stmt) wait_stmt
#define LOOM_WAVE_STALL_STORE \
  do {                        \
  } while (0)
#endif

// Work-item schedule of the streaming kernel. The grid has one workgroup per
// (sequence, partition, KV head) slot; slots are handed out so that every full
// partition comes first and the shorter last partitions of the sequences come
// after them (longest-first, which shortens the tail of a ragged batch), with
// empty slots at the end. Pairs (sequence, partition) are numbered in sequence
// order inside each class and the KV head varies fastest, so the heads of one
// block are read close together in time. Every wave of the workgroup computes
// the same (wave-uniform) answer from the sequence lengths.
struct WorkItem {
  uint32_t seq, part, kvh, len;
  bool valid;
  // schedule_item: the first 64 sequences do not all hold the same number
  // of full partitions (a ragged batch)
  bool uneven = false;
};

__device__ __forceinline__ uint32_t wave_inclusive_sum(uint32_t x, uint32_t lane) {
#pragma unroll
  for (uint32_t d = 1; d < 64; d <<= 1) {
    const uint32_t t = __shfl_up(x, d, 64);
    if (lane >= d) x += t;
  }
  return x;
}

typedef uint32_t u32x16 __attribute__((ext_vector_type(16)));

// Lengths of sequences c0 .. c0 + 63, lane i holding sequence c0 + i (zero
// past the end). They are read through the scalar cache with bounds-checked
// buffer loads: a wave that has just started would wait far longer for a
// vector load queued behind the running waves' KV traffic.
__device__ __forceinline__ uint32_t lengths_chunk(const DecodeArgs& a, uint32_t c0, uint32_t lane) {
  const uint64_t base = reinterpret_cast<uint64_t>(a.sequence_lengths);
  typedef uint32_t u32x4s __attribute__((ext_vector_type(4)));
  const u32x4s rsrc = {static_cast<uint32_t>(base), static_cast<uint32_t>(base >> 32) & 0xFFFFU, a.sequences * 4U,
                       0x00020000U};
  u32x16 w0, w1, w2, w3;
  // The loads and their wait in one statement: the words are asm outputs
  // only once they have arrived, so no register copy or spill can read them
  // early.
  asm volatile(
      "s_buffer_load_dwordx16 %0, %4, %5\n\t"
      "s_buffer_load_dwordx16 %1, %4, %6\n\t"
      "s_buffer_load_dwordx16 %2, %4, %7\n\t"
      "s_buffer_load_dwordx16 %3, %4, %8\n\t"
      "s_waitcnt lgkmcnt(0)"
      : "=&s"(w0), "=&s"(w1), "=&s"(w2), "=&s"(w3)
      : "s"(rsrc), "s"(c0 * 4U), "s"(c0 * 4U + 64U), "s"(c0 * 4U + 128U), "s"(c0 * 4U + 192U)
      : "memory");
  uint32_t v = 0;
#pragma unroll
  for (int i = 0; i < 16; ++i) {
    asm("v_writelane_b32 %0, %1, %2" : "+v"(v) : "s"(w0[i]), "n"(i));
    asm("v_writelane_b32 %0, %1, %2" : "+v"(v) : "s"(w1[i]), "n"(16 + i));
    asm("v_writelane_b32 %0, %1, %2" : "+v"(v) : "s"(w2[i]), "n"(32 + i));
    asm("v_writelane_b32 %0, %1, %2" : "+v"(v) : "s"(w3[i]), "n"(48 + i));
  }
  return c0 + lane < a.sequences ? v : 0U;
}

__device__ __forceinline__ WorkItem schedule_item(const DecodeArgs& a, uint32_t bid) {
  WorkItem it{0, 0, 0, 0, false};
  const uint32_t lane = threadIdx.x & 63U;
  const uint32_t pt = a.partition_tokens;
  it.kvh = bid % a.kv_heads;
  const uint32_t pair = bid / a.kv_heads;
  // Odd (sequence, partition) pairs swap the halves of the KV heads: the
  // dispatcher deals workgroups to the XCDs in turn, and with the head
  // varying fastest each XCD would otherwise read the same half of every
  // token row (the XCDs holding the second half finished up to 15 us later;
  // C3 call 205.2 -> 204.8 us). XOR with kv_heads / 2 is a permutation of
  // the heads only when kv_heads is a power of two (6 heads would map 4 to 7).
  if (a.kv_heads >= 2 && (a.kv_heads & (a.kv_heads - 1U)) == 0 && (pair & 1U)) it.kvh ^= a.kv_heads / 2;
  // Class 0: full partitions (len / pt per sequence); class 1: one partial
  // last partition per sequence whose length is not a multiple of pt.
  uint32_t before = 0;  // pairs of earlier classes and chunks
#pragma unroll 1
  for (int cls = 0; cls < 2; ++cls) {
#pragma unroll 1
    for (uint32_t c0 = 0; c0 < a.sequences; c0 += 64) {
      // A length past the launch's partitions (a caller breaking the
      // max_sequence_length contract) is clamped to them, so no item
      // addresses a state or a table entry outside its sequence's share.
      const uint32_t len = static_cast<uint32_t>(min(static_cast<uint64_t>(lengths_chunk(a, c0, lane)),
                                                     static_cast<uint64_t>(a.parts) * pt));
      const uint32_t full = len / pt;
      if (cls == 0 && c0 == 0)
        it.uneven = __builtin_amdgcn_ballot_w64(lane < a.sequences && full != __builtin_amdgcn_readfirstlane(full)) != 0;
      const uint32_t n = cls == 0 ? full : (len % pt != 0 ? 1U : 0U);
      const uint32_t incl = wave_inclusive_sum(n, lane);
      const uint32_t total = __builtin_amdgcn_readlane(incl, 63);
      if (pair < before + total) {
        const uint32_t r = pair - before;
        const uint64_t hit = __builtin_amdgcn_ballot_w64(incl > r);
        const uint32_t src = static_cast<uint32_t>(__builtin_ctzll(hit));
        it.seq = c0 + src;
        it.len = __builtin_amdgcn_readlane(len, src);
        it.part = cls == 0 ? r - (__builtin_amdgcn_readlane(incl, src) - __builtin_amdgcn_readlane(n, src))
                           : __builtin_amdgcn_readlane(full, src);
        it.valid = true;
        return it;
      }
      before += total;
    }
  }
  return it;
}

// Schedule of the two-partition workgroups (decode_stream_group_kernel
// with kPair): unit `unit` is (sequence, pair of partitions 2j and 2j + 1,
// group of `heads` adjacent KV heads), numbered as schedule_item numbers its
// items (every full pair first, then each sequence's last, shorter pair;
// the head group varies fastest). Wave w of the workgroup takes KV head
// w % heads of the group and partition 2j + w / heads. valid is false for a
// partition past its sequence's end (only 2j + 1 can be); len is 0 for a
// unit past the schedule's end (the grid is sized for the longest sequence).
__device__ __forceinline__ WorkItem pair_item(const DecodeArgs& a, uint32_t unit, uint32_t heads, uint32_t wave) {
  WorkItem it{0, 0, 0, 0, false};
  const uint32_t lane = threadIdx.x & 63U;
  const uint32_t pt2 = 2U * a.partition_tokens;
  const uint32_t groups = a.kv_heads / heads;
  const uint32_t hg = unit % groups;
  const uint32_t pair = unit / groups;
  uint32_t before = 0;
#pragma unroll 1
  for (int cls = 0; cls < 2; ++cls) {
#pragma unroll 1
    for (uint32_t c0 = 0; c0 < a.sequences; c0 += 64) {
      const uint32_t len = static_cast<uint32_t>(min(static_cast<uint64_t>(lengths_chunk(a, c0, lane)),
                                                     static_cast<uint64_t>(a.parts) * a.partition_tokens));
      const uint32_t full = len / pt2;
      const uint32_t n = cls == 0 ? full : (len % pt2 != 0 ? 1U : 0U);
      const uint32_t incl = wave_inclusive_sum(n, lane);
      const uint32_t total = __builtin_amdgcn_readlane(incl, 63);
      if (pair < before + total) {
        const uint32_t r = pair - before;
        const uint64_t hit = __builtin_amdgcn_ballot_w64(incl > r);
        const uint32_t src = static_cast<uint32_t>(__builtin_ctzll(hit));
        const uint32_t j = cls == 0 ? r - (__builtin_amdgcn_readlane(incl, src) - __builtin_amdgcn_readlane(n, src))
                                    : __builtin_amdgcn_readlane(full, src);
        it.seq = c0 + src;
        it.len = __builtin_amdgcn_readlane(len, src);
        it.kvh = hg * heads + wave % heads;
        it.part = 2U * j + wave / heads;
        it.valid = it.part * a.partition_tokens < it.len;
        return it;
      }
      before += total;
    }
  }
  return it;
}

// One wave's result for its KV head's query group: the normalised output
// (and LSE) when the sequence is one partition, else the partition's
// partial output (F32 sum) and (m, l) in the split-K workspace. Lane (g, c) holds dims
// dt*16 + 4g .. +3 of head c; only lanes of live heads call this.
template <typename QE, bool kNt = false, typename Dec>
__device__ __forceinline__ void store_wave_result(const DecodeArgs& a, const Dec& dec, int ht, uint32_t seq,
                                                  uint32_t head0, uint32_t part, float v_scale, float l) {
  constexpr uint32_t D = Dec::kDt * 16;
  const uint64_t row = static_cast<uint64_t>(seq) * a.query_heads + head0 + dec.c;
  if (a.parts == 1) {
    const float inv = v_scale / l;
    uint16_t* o = static_cast<uint16_t*>(a.output) + row * D + 4 * dec.g;
#pragma unroll
    for (int dt = 0; dt < Dec::kDt; ++dt) {
      uint32_t w0 = QE::from_f(dec.acc[ht][dt][0] * inv) | (static_cast<uint32_t>(QE::from_f(dec.acc[ht][dt][1] * inv)) << 16);
      uint32_t w1 = QE::from_f(dec.acc[ht][dt][2] * inv) | (static_cast<uint32_t>(QE::from_f(dec.acc[ht][dt][3] * inv)) << 16);
      *reinterpret_cast<uint2*>(o + dt * 16) = make_uint2(w0, w1);
    }
    if (a.lse != nullptr && dec.g == 0) a.lse[row] = (dec.m[ht] + log2f(l)) * kLn2;
  } else {
    const uint64_t state = state_of(a, row, part);
#pragma unroll
    for (int dt = 0; dt < Dec::kDt; ++dt) put_partial4<kNt>(a, state * D + 4 * dec.g + dt * 16, dec.acc[ht][dt], v_scale);
    if (dec.g == 0) {
      a.ws_ml[state * 2] = dec.m[ht];
      a.ws_ml[state * 2 + 1] = l;
    }
  }
}


// Merge state of one lane: the running maximum M (log2 units), the sum L
// and dims 4c .. 4c + 3 of the weighted partial sums.
struct MergeState {
  float m, l;
  f32x4 o;
};

// Combines two merge states by the log-sum-exp identity (a state without
// partitions has m = -inf and weight 0).
__device__ __forceinline__ MergeState merge_combine(const MergeState& x, const MergeState& y) {
  const float m = fmaxf(x.m, y.m);
  const float fx = isfinite(x.m) ? exp2f(x.m - m) : 0.0f;
  const float fy = isfinite(y.m) ? exp2f(y.m - m) : 0.0f;
  return MergeState{m, x.l * fx + y.l * fy, x.o * fx + y.o * fy};
}

// One wave's merge of the partitions first, first + stride, ... (below n)
// of the row whose partition 0 is state s0 (partition p: state s0 + p *
// query_heads), Dv = kD (64, 128 or 256) F32 partial rows, 16-byte aligned.
// Lane (q, c) reads dims 4c .. 4c + 3 of every kQ-th of those partitions, kB
// loads in flight per batch (one batch covers kQ * kB partitions), keeping
// its own running state; the kQ lane groups are then combined, so every
// lane c of the wave returns dims 4c .. 4c + 3 of the wave's state.
template <uint32_t kD, uint32_t kB = 8>
__device__ __forceinline__ MergeState merge_partitions(const DecodeArgs& a, uint64_t s0, uint32_t n, uint32_t first,
                                                       uint32_t stride) {
  constexpr uint32_t kL = kD / 4;   // lanes per partial row (16 bytes each)
  constexpr uint32_t kQ = 64 / kL;  // partitions per load instruction
  const uint32_t lane = threadIdx.x & 63U;
  const uint32_t c = lane % kL, q = lane / kL;
  const uint64_t ss = a.query_heads;
  const float* os = a.ws_o + s0 * kD + 4 * c;
  const float* ml = a.ws_ml + s0 * 2;
  const uint32_t mine = n > first ? (n - first + stride - 1) / stride : 0U;  // this wave's partitions
  MergeState st{-INFINITY, 0.0f, f32x4{0.0f, 0.0f, 0.0f, 0.0f}};
  for (uint32_t b0 = 0; b0 < mine; b0 += kQ * kB) {
    f32x4 ov[kB];
    float2 pm[kB];
#pragma unroll
    for (uint32_t i = 0; i < kB; ++i) {
      const uint32_t k = b0 + q + kQ * i;
      const uint64_t at = static_cast<uint64_t>(k < mine ? first + k * stride : first) * ss;  // past the end: re-read
      ov[i] = *reinterpret_cast<const f32x4*>(os + at * kD);
      pm[i] = *reinterpret_cast<const float2*>(ml + at * 2);
    }
    float mb = st.m;
#pragma unroll
    for (uint32_t i = 0; i < kB; ++i) {
      if (b0 + q + kQ * i >= mine) pm[i] = make_float2(-INFINITY, 0.0f);
      mb = fmaxf(mb, pm[i].x);
    }
    const float r = isfinite(st.m) ? exp2f(st.m - mb) : 0.0f;
    st.l *= r;
    st.o *= r;
    st.m = mb;
#pragma unroll
    for (uint32_t i = 0; i < kB; ++i) {
      const float f = isfinite(pm[i].x) ? exp2f(pm[i].x - st.m) : 0.0f;
      st.l = fmaf(pm[i].y, f, st.l);
      st.o += ov[i] * f;
    }
  }
#pragma unroll
  for (uint32_t off = kL; off < 64; off <<= 1) {
    MergeState other;
    other.m = __shfl_xor(st.m, off, 64);
    other.l = __shfl_xor(st.l, off, 64);
#pragma unroll
    for (int j = 0; j < 4; ++j) other.o[j] = __shfl_xor(st.o[j], off, 64);
    st = merge_combine(st, other);
  }
  return st;
}

// Writes a merged row: output dims 4c .. 4c + 3 from lanes c < Dv / 4 of
// the calling wave, and the LSE (natural log) from lane 0.
template <typename QE, uint32_t kD>
__device__ __forceinline__ void merge_store_row(const DecodeArgs& a, uint64_t row, const MergeState& st) {
  const uint32_t lane = threadIdx.x & 63U;
  if (lane < kD / 4) {
    const float inv = 1.0f / st.l;
    if constexpr (std::is_same<QE, F32Elem>::value) {
      *reinterpret_cast<f32x4*>(static_cast<float*>(a.output) + row * kD + 4 * lane) = st.o * inv;
    } else {
      const uint32_t w0 = QE::from_f(st.o[0] * inv) | (static_cast<uint32_t>(QE::from_f(st.o[1] * inv)) << 16);
      const uint32_t w1 = QE::from_f(st.o[2] * inv) | (static_cast<uint32_t>(QE::from_f(st.o[3] * inv)) << 16);
      *reinterpret_cast<uint2*>(static_cast<uint16_t*>(a.output) + row * kD + 4 * lane) = make_uint2(w0, w1);
    }
  }
  if (lane == 0 && a.lse != nullptr) a.lse[row] = (st.m + log2f(st.l)) * kLn2;
}


// The state of a wave's item (head c of lane (g, c): maximum m, sum l, and
// dims dt * 16 + 4g .. + 3 of O) in LDS at `tile`, lane by lane, for the
// wave that merges it (pair_combine). An empty item publishes m = -inf,
// l = 0.
template <typename Dec>
__device__ __forceinline__ void pair_publish(uint8_t* tile, float m, float l, const f32x4 (&acc)[Dec::kDt]) {
  static_assert(Dec::kWaveBytes >= Dec::kDt * 1024 + 512, "the state fits the wave's stages");
  const uint32_t lane = threadIdx.x & 63U;
  f32x4* o = reinterpret_cast<f32x4*>(tile);
#pragma unroll
  for (int dt = 0; dt < Dec::kDt; ++dt) o[dt * 64 + lane] = acc[dt];  // lane-linear: no bank conflicts
  reinterpret_cast<float2*>(tile + Dec::kDt * 1024)[lane] = make_float2(m, l);
}

template <typename Dec>
__device__ __forceinline__ void pair_publish_empty(uint8_t* tile) {
  f32x4 zero[Dec::kDt];
#pragma unroll
  for (int dt = 0; dt < Dec::kDt; ++dt) zero[dt] = f32x4{0.0f, 0.0f, 0.0f, 0.0f};
  pair_publish<Dec>(tile, -INFINITY, 0.0f, zero);
}

// Folds the partner's published state into this wave's (m, l, O) by the
// log-sum-exp identity; this wave's item holds tokens, so m is finite.
template <typename Dec>
__device__ __forceinline__ void pair_combine(const uint8_t* tile, float& m, float& l, f32x4 (&acc)[Dec::kDt]) {
  const uint32_t lane = threadIdx.x & 63U;
  const float2 ml = reinterpret_cast<const float2*>(tile + Dec::kDt * 1024)[lane];
  const float mn = fmaxf(m, ml.x);
  const float fa = __builtin_amdgcn_exp2f(m - mn);
  const float fb = isfinite(ml.x) ? __builtin_amdgcn_exp2f(ml.x - mn) : 0.0f;
  const f32x4* o = reinterpret_cast<const f32x4*>(tile);
#pragma unroll
  for (int dt = 0; dt < Dec::kDt; ++dt) acc[dt] = acc[dt] * fa + o[dt * 64 + lane] * fb;
  l = l * fa + ml.y * fb;
  m = mn;
}

// One work item of the streaming kernel, from its first loads to its
// partial-state stores. `tiles` holds kSplit waves' LDS (Dec::kWaveBytes
// each); after the step loop the same memory holds each wave's O (16 heads x
// 128 dims F32 = 8 KiB) for the cross-wave reduction.
template <typename QE, bool kFp8, int kSplit, int kHT = 1, uint32_t kD = kDim,
          int kS = kFp8 ? kStreamStagesFp8 : kStreamStages, int kNt = -1, bool kPair = false>
__device__ __forceinline__ void stream_item(const DecodeArgs& a, uint8_t* tiles, const WorkItem& item,
                                            bool preloaded = false, const uint32_t* first_blocks = nullptr,
                                            uint8_t* partner = nullptr) {
  static_assert(kHT == 1 || kSplit == 1, "two head tiles run one wave per item");
  using Dec = StreamDecoder<QE, kFp8, kHT, kD, kS, kNt>;
  using vec8 = typename Dec::vec8;
  constexpr int S = Dec::kStages;
  const uint32_t kvh = item.kvh;
  const uint32_t part = item.part;
  const uint32_t seq = item.seq;
  const uint32_t len = item.len;
  const uint32_t p0 = part * a.partition_tokens;
  static_assert(Dec::kWaveBytes >= 16 * (kD + 4) * sizeof(float),
                "the cross-wave reduction reuses the stages");

  Dec dec(a);
  dec.lane = threadIdx.x & 63U;
  dec.g = dec.lane >> 4;
  dec.c = dec.lane & 15U;
  dec.len = len;
  dec.p1 = min(p0 + a.partition_tokens, len);
  dec.last_block = (len - 1U) >> a.block_shift;
  dec.table = a.block_tables + static_cast<uint64_t>(seq) * a.max_blocks;
  constexpr uint32_t es = Dec::kElem;
  dec.kstride_b = a.k_block * es;
  dec.vstride_b = a.v_block * es;
  dec.kstride_p = a.k_page * es;
  dec.vstride_p = a.v_page * es;
  dec.kbase = reinterpret_cast<uint64_t>(a.key_cache) + static_cast<uint64_t>(kvh) * a.k_head * es;
  dec.vbase = reinterpret_cast<uint64_t>(a.value_cache) + static_cast<uint64_t>(kvh) * a.v_head * es;
  dec.init_offsets();
  const uint32_t wave = kSplit == 1 ? 0U : __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  uint8_t* tw = tiles + wave * Dec::kWaveBytes;

  float k_scale = 1.0f, v_scale = 1.0f;
  if (kFp8) {
    k_scale = a.key_scales[kvh * a.scale_stride];
    v_scale = a.value_scales[kvh * a.scale_stride];
  }
  dec.sl2 = a.score_scale_log2 * k_scale;

  // Steps of this partition: step k covers [p0 + 16k, p0 + 16k + 16); wave
  // w takes steps w, w + kSplit, ... Block-table reads past the wave's last
  // step are clamped onto it; no K/V load is issued past it.
  const uint32_t nst = (dec.p1 - p0 + kStep - 1) / kStep;
  const uint32_t my_n = nst > wave ? (nst - wave + kSplit - 1) / kSplit : 0;
  const uint32_t st = kSplit * kStep;
  const uint32_t t_first = p0 + wave * kStep;
  const uint32_t t_last = t_first + (my_n > 0 ? my_n - 1 : 0) * st;

#pragma unroll
  for (int ht = 0; ht < kHT; ++ht) {
    dec.m[ht] = -INFINITY;
    dec.lsum[ht] = 0.0f;
#pragma unroll
    for (int dt = 0; dt < Dec::kDt; ++dt) dec.acc[ht][dt] = f32x4{0.0f, 0.0f, 0.0f, 0.0f};
  }

  if (my_n > 0) {
    // Block IDs run S steps ahead of the loads that use them.
    uint8_t* tl[S];
    uint32_t nx[S];
    uint32_t bk[S];
#pragma unroll
    for (int i = 0; i < S; ++i) tl[i] = tw + i * Dec::kStageBytes;
    if (preloaded) {
      // The block IDs of steps 0 .. 2S - 1, loaded with the item's length.
#pragma unroll
      for (int i = 0; i < S; ++i) {
        bk[i] = first_blocks[i];
        nx[i] = first_blocks[S + i];
      }
    } else {
#pragma unroll
      for (int i = 0; i < S; ++i) bk[i] = dec.block_of(min(t_first + i * st, t_last));
#pragma unroll
      for (int i = 0; i < S; ++i) nx[i] = dec.block_of(min(t_first + (S + i) * st, t_last));
    }
#pragma unroll
    for (int i = 0; i < S; ++i) scalar_ready(bk[i]);
#pragma unroll
    for (int i = 0; i < S; ++i) {
      if (i < my_n) dec.issue(tl[i], bk[i], t_first + i * st);
    }
    // Q is loaded after the first steps' K/V and waited for together with
    // them, so a wave's start costs one memory round trip, not two.
    {
      u32x4 qw[kHT][Dec::kKc];
#pragma unroll
      for (int ht = 0; ht < kHT; ++ht) {
        const uint32_t h = min(ht * 16U + dec.c, a.group - 1U);  // rows >= group are zeroed below
        const uint16_t* qrow = static_cast<const uint16_t*>(a.query) +
                               (static_cast<uint64_t>(seq) * a.query_heads + kvh * a.group + h) * kD;
#pragma unroll
        for (int kc = 0; kc < Dec::kKc; ++kc) {
          const uint32_t dim = kFp8 ? ((kc >> 1) * 64 + dec.g * 16 + ((kc ^ dec.g) & 1U) * 8) : (kc * 32 + dec.g * 8);
          vm_load16(qw[ht][kc], qrow + (dim < kD ? dim : 0U));  // dims past the head size are zeroed below
        }
      }
      asm volatile("s_waitcnt vmcnt(0)" : : : "memory");
#pragma unroll
      for (int ht = 0; ht < kHT; ++ht) {
#pragma unroll
        for (int kc = 0; kc < Dec::kKc; ++kc) asm volatile("" : "+v"(qw[ht][kc]));  // loaded: the wait above was vmcnt(0)
      }
#pragma unroll
      for (int ht = 0; ht < kHT; ++ht) {
        const bool live = ht * 16U + dec.c < a.group;
#pragma unroll
        for (int kc = 0; kc < Dec::kKc; ++kc) {
          const uint32_t dim = kFp8 ? ((kc >> 1) * 64 + dec.g * 16 + ((kc ^ dec.g) & 1U) * 8) : (kc * 32 + dec.g * 8);
          const bool in_row = dim < kD;
          dec.qb[ht][kc] = __builtin_bit_cast(vec8, live && in_row ? qw[ht][kc] : u32x4{0U, 0U, 0U, 0U});
        }
      }
    }
    LOOM_WAVE_STALL_DECL;
    for (uint32_t n = 0; n < my_n; n += S) {
      LOOM_WAVE_MARK(n, S, my_n);
#pragma unroll
      for (int i = 0; i < S; ++i) {
        if (n + i < my_n) {
          const uint32_t t0 = t_first + (n + i) * st;
          uint8_t* vtile = kFp8 ? tw + Dec::kVTileOff : tl[i] + Dec::kVOff;
          // this step's loads; the later steps' (up to S - 1) stay in flight
          LOOM_WAVE_STALL(n + i, my_n, (vm_wait_dma_later<Dec::kDmaPerStep, S - 1>(my_n - 1 - (n + i))));
          scalar_ready(nx[i]);
          if (kFp8) {
            dec.stage_v_fp8(tl[i], vtile, t0);
          } else {
            dec.zero_dead_rows(vtile, t0);
          }
          wave_fence_lds();
          f32x4 sc[kHT];
          dec.qk(tl[i], sc);
          dec.softmax_pv(sc, t0, vtile);
          wait_lds_reads();
          // No load past the item's last step: such a load would re-read
          // rows nobody consumes, and the wave's exit would wait for it.
          if (n + i + S < my_n) dec.issue(tl[i], nx[i], t0 + S * st);
          wave_fence_lds();
          nx[i] = dec.block_of(min(t0 + 2 * S * st, t_last));
        }
      }
    }
    asm volatile("s_waitcnt vmcnt(0)" : : : "memory");
    LOOM_WAVE_STALL_STORE;
  }

  float lt[kHT];
#pragma unroll
  for (int ht = 0; ht < kHT; ++ht) {
    float l = dec.lsum[ht];
    l += __shfl_xor(l, 16, 64);
    l += __shfl_xor(l, 32, 64);
    lt[ht] = l;
  }
  if constexpr (kPair) {
    // Two partitions of one KV head per workgroup (pair_item): the odd one
    // hands its state to the even one through its own LDS, which combines
    // them and stores one state for the pair.
    static_assert(kSplit == 1 && kHT == 1, "pairs run one wave per item");
    if (partner == nullptr) {
      pair_publish<Dec>(tiles, dec.m[0], lt[0], dec.acc[0]);
      __syncthreads();
      return;
    }
    __syncthreads();
    pair_combine<Dec>(partner, dec.m[0], lt[0], dec.acc[0]);
    DecodeArgs pairs = a;
    pairs.parts = (a.parts + 1U) / 2U;  // the states are per pair of partitions
    if (dec.c < a.group) store_wave_result<QE, kFp8 && Dec::kNtKV>(pairs, dec, 0, seq, kvh * a.group, part / 2U, v_scale, lt[0]);
    return;
  }
  if (kSplit == 1) {
#pragma unroll
    for (int ht = 0; ht < kHT; ++ht) {
      if (ht * 16U + dec.c < a.group) store_wave_result<QE, kFp8 && Dec::kNtKV>(a, dec, ht, seq, kvh * a.group + ht * 16U, part, v_scale, lt[ht]);
    }
    return;
  }

  // Several waves split the partition (one head tile): reduce through LDS.
  const uint32_t h = dec.c;
  const float l = lt[0];
  // Rows padded by 16 bytes: the eight lanes of one 16-byte store then fall
  // in distinct bank quarters.
  constexpr uint32_t kRedPitch = kD + 4;
  float (*red_o)[16][kRedPitch] = reinterpret_cast<float (*)[16][kRedPitch]>(tiles);
  __shared__ float red_ml[kSplit][16][2];
  __syncthreads();  // every wave is done with its V tiles
  if (dec.g == 0) {
    red_ml[wave][h][0] = dec.m[0];
    red_ml[wave][h][1] = l;
  }
#pragma unroll
  for (int dt = 0; dt < Dec::kDt; ++dt) *reinterpret_cast<f32x4*>(&red_o[wave][h][dt * 16 + 4 * dec.g]) = dec.acc[0][dt];
  __syncthreads();
  const uint32_t heads = min(a.group, 16U);
  for (uint32_t idx = threadIdx.x; idx < heads * kD; idx += kSplit * 64) {
    const uint32_t hl = idx / kD, d = idx % kD;
    float M = -INFINITY;
#pragma unroll
    for (int w = 0; w < kSplit; ++w) M = fmaxf(M, red_ml[w][hl][0]);
    float L = 0.0f, O = 0.0f;
#pragma unroll
    for (int w = 0; w < kSplit; ++w) {
      const float f = exp2f(red_ml[w][hl][0] - M);
      L = fmaf(red_ml[w][hl][1], f, L);
      O = fmaf(red_o[w][hl][d], f, O);
    }
    O *= v_scale;
    const uint64_t row = static_cast<uint64_t>(seq) * a.query_heads + kvh * a.group + hl;
    if (a.parts == 1) {
      static_cast<uint16_t*>(a.output)[row * kD + d] = QE::from_f(O / L);
      if (a.lse != nullptr && d == 0) a.lse[row] = (M + log2f(L)) * kLn2;
    } else {
      const uint64_t state = state_of(a, row, part);
      put_partial(a, state * kD + d, O);
      if (d == 0) {
        a.ws_ml[state * 2] = M;
        a.ws_ml[state * 2 + 1] = L;
      }
    }
  }
}

// Workgroup barrier after this wave's LDS operations have completed. Unlike
// __syncthreads it leaves outstanding global loads (the DMA pipeline) alone;
// the clobber keeps the compiler from moving LDS accesses across it.
__device__ __forceinline__ void lds_barrier() { asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" : : : "memory"); }

// Pipeline stages shared by the waves of a wide-group workgroup (16-bit: 8 KiB
// each; FP8: 4 KiB, plus one converted V tile per wave).
constexpr int kSharedStages = 4;

// One work item of a group of 33-128 query heads: kWaves waves, wave w
// computing heads 32 w .. 32 w + 31 with two head tiles, from a ring of K/V
// stages that all waves share. Wave 0 issues every step's DMA. One barrier
// per step, after wave 0's wait for the step's stage, both publishes that
// stage and shows that every wave has finished the previous step, whose
// stage wave 0 then refills (S - 1 steps ahead). The waves have the same
// steps, so all of them reach every barrier.
template <typename QE, bool kFp8, int kWaves, uint32_t kD, int kHTW = 2>
__device__ __forceinline__ void stream_item_shared(const DecodeArgs& a, uint8_t* tiles, const WorkItem& item) {
  using Dec = StreamDecoder<QE, kFp8, kHTW, kD>;
  using vec8 = typename Dec::vec8;
  constexpr int S = kSharedStages;
  const uint32_t kvh = item.kvh, part = item.part, seq = item.seq, len = item.len;
  const uint32_t p0 = part * a.partition_tokens;
  const uint32_t wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const uint32_t h0 = wave * 16U * kHTW;

  Dec dec(a);
  dec.lane = threadIdx.x & 63U;
  dec.g = dec.lane >> 4;
  dec.c = dec.lane & 15U;
  dec.len = len;
  dec.p1 = min(p0 + a.partition_tokens, len);
  dec.last_block = (len - 1U) >> a.block_shift;
  dec.table = a.block_tables + static_cast<uint64_t>(seq) * a.max_blocks;
  constexpr uint32_t es = Dec::kElem;
  dec.kstride_b = a.k_block * es;
  dec.vstride_b = a.v_block * es;
  dec.kstride_p = a.k_page * es;
  dec.vstride_p = a.v_page * es;
  dec.kbase = reinterpret_cast<uint64_t>(a.key_cache) + static_cast<uint64_t>(kvh) * a.k_head * es;
  dec.vbase = reinterpret_cast<uint64_t>(a.value_cache) + static_cast<uint64_t>(kvh) * a.v_head * es;
  dec.init_offsets();
  uint8_t* vconv = tiles + S * Dec::kStageBytes + wave * (kStep * Dec::kPitch);  // FP8: this wave's 16-bit V

  float k_scale = 1.0f, v_scale = 1.0f;
  if (kFp8) {
    k_scale = a.key_scales[kvh * a.scale_stride];
    v_scale = a.value_scales[kvh * a.scale_stride];
  }
  dec.sl2 = a.score_scale_log2 * k_scale;
#pragma unroll
  for (int ht = 0; ht < kHTW; ++ht) {
    dec.m[ht] = -INFINITY;
    dec.lsum[ht] = 0.0f;
#pragma unroll
    for (int dt = 0; dt < Dec::kDt; ++dt) dec.acc[ht][dt] = f32x4{0.0f, 0.0f, 0.0f, 0.0f};
  }

  const uint32_t nst = (dec.p1 - p0 + kStep - 1) / kStep;  // >= 1: the item holds tokens
  const uint32_t t_last = p0 + (nst - 1) * kStep;
  // nx[j]: block of the next step that wave 0 loads into stage j (table
  // reads past the item's last step are clamped onto it; no K/V load is
  // issued past it).
  uint32_t nx[S];
  if (wave == 0) {
    uint32_t bk[S - 1];
#pragma unroll
    for (int i = 0; i < S - 1; ++i) bk[i] = dec.block_of(min(p0 + i * kStep, t_last));
#pragma unroll
    for (int i = 0; i < S - 1; ++i) nx[i] = dec.block_of(min(p0 + (S + i) * kStep, t_last));
    nx[S - 1] = dec.block_of(min(p0 + (S - 1) * kStep, t_last));
#pragma unroll
    for (int i = 0; i < S - 1; ++i) scalar_ready(bk[i]);
#pragma unroll
    for (int i = 0; i < S - 1; ++i) {
      if (i < nst) dec.issue(tiles + i * Dec::kStageBytes, bk[i], p0 + i * kStep);
    }
  }
  {
    u32x4 qw[kHTW][Dec::kKc];
#pragma unroll
    for (int ht = 0; ht < kHTW; ++ht) {
      const uint32_t h = min(h0 + ht * 16U + dec.c, a.group - 1U);  // rows >= group are zeroed below
      const uint16_t* qrow = static_cast<const uint16_t*>(a.query) +
                             (static_cast<uint64_t>(seq) * a.query_heads + kvh * a.group + h) * kD;
#pragma unroll
      for (int kc = 0; kc < Dec::kKc; ++kc) {
        const uint32_t dim = kFp8 ? ((kc >> 1) * 64 + dec.g * 16 + ((kc ^ dec.g) & 1U) * 8) : (kc * 32 + dec.g * 8);
        vm_load16(qw[ht][kc], qrow + dim);
      }
    }
    asm volatile("s_waitcnt vmcnt(0)" : : : "memory");
#pragma unroll
    for (int ht = 0; ht < kHTW; ++ht) {
#pragma unroll
      for (int kc = 0; kc < Dec::kKc; ++kc) asm volatile("" : "+v"(qw[ht][kc]));  // loaded: the wait above was vmcnt(0)
    }
#pragma unroll
    for (int ht = 0; ht < kHTW; ++ht) {
      const bool live = h0 + ht * 16U + dec.c < a.group;
#pragma unroll
      for (int kc = 0; kc < Dec::kKc; ++kc)
        dec.qb[ht][kc] = __builtin_bit_cast(vec8, live ? qw[ht][kc] : u32x4{0U, 0U, 0U, 0U});
    }
  }

  LOOM_WAVE_STALL_DECL;
  for (uint32_t n = 0; n < nst; n += S) {
    if (wave == 0) LOOM_WAVE_MARK(n, S, nst);
#pragma unroll
    for (int i = 0; i < S; ++i) {
      if (n + i < nst) {
        const uint32_t t0 = p0 + (n + i) * kStep;
        uint8_t* stage = tiles + i * Dec::kStageBytes;
        const int j = (i + S - 1) % S;  // the stage of the previous step
        if (wave == 0) {
          // this step's loads; the later steps' (up to S - 2) stay in flight
          LOOM_WAVE_STALL(n + i, nst, (vm_wait_dma_later<Dec::kDmaPerStep, S - 2>(nst - 1 - (n + i))));
          if (!kFp8) dec.zero_dead_rows(stage + Dec::kVOff, t0);
        }
        lds_barrier();  // this step's stage is in LDS; every wave is done with the previous one
        if (wave == 0) {
          scalar_ready(nx[j]);
          if (n + i + S - 1 < nst) dec.issue(tiles + j * Dec::kStageBytes, nx[j], t0 + (S - 1) * kStep);
          nx[j] = dec.block_of(min(t0 + (2 * S - 1) * kStep, t_last));
        }
        uint8_t* vtile = kFp8 ? vconv : stage + Dec::kVOff;
        if (kFp8) {
          dec.stage_v_fp8(stage, vtile, t0);
          wave_fence_lds();
        }
        f32x4 sc[kHTW];
        dec.qk(stage, sc);
        dec.softmax_pv(sc, t0, vtile);
      }
    }
  }
  if (wave == 0) {
    asm volatile("s_waitcnt vmcnt(0)" : : : "memory");
    LOOM_WAVE_STALL_STORE;
  }

#pragma unroll
  for (int ht = 0; ht < kHTW; ++ht) {
    float l = dec.lsum[ht];
    l += __shfl_xor(l, 16, 64);
    l += __shfl_xor(l, 32, 64);
    if (h0 + ht * 16U + dec.c < a.group)
      store_wave_result<QE>(a, dec, ht, seq, kvh * a.group + h0 + ht * 16U, part, v_scale, l);
  }
}

// Item bid in index order (KV head fastest, then partition, then sequence;
// valid = false for a partition past its sequence's end), with the block IDs
// of the item's first kN steps loaded together with its length. preloaded
// tells whether they are the ones the item uses: a partition with fewer than
// kN steps, or a sequence ending inside step kN - 1, takes the ordinary
// loads. Volatile constant-address-space scalar loads: the compiler issues
// them here, unconditionally and in order, and waits for them before any use
// or copy.
template <int kN>
__device__ __forceinline__ WorkItem direct_item(const DecodeArgs& a, uint32_t bid, uint32_t (&first)[kN],
                                                bool& preloaded) {
  WorkItem item{0, 0, bid % a.kv_heads, 0, false};
  const uint32_t pair = bid / a.kv_heads;
  item.seq = pair / a.parts;
  item.part = pair % a.parts;
  preloaded = false;
  if (item.seq >= a.sequences) return item;
  using ConstWord = const volatile __attribute__((address_space(4))) int32_t;
  const ConstWord* row = (const ConstWord*)(a.block_tables + static_cast<uint64_t>(item.seq) * a.max_blocks);
  const ConstWord* lens = (const ConstWord*)a.sequence_lengths;
  const uint32_t p0 = item.part * a.partition_tokens;
  const uint32_t t_end = p0 + a.partition_tokens - kStep;  // steps past the last one clamp onto it
  uint32_t at[kN];
#pragma unroll
  for (int i = 0; i < kN; ++i) at[i] = min(min(p0 + i * kStep, t_end) >> a.block_shift, a.max_blocks - 1U);
  item.len = static_cast<uint32_t>(lens[item.seq]);  // first: its address needs nothing loaded
  item.len = static_cast<uint32_t>(min(static_cast<uint64_t>(item.len),
                                       static_cast<uint64_t>(a.parts) * a.partition_tokens));
#pragma unroll
  for (int i = 0; i < kN; ++i) first[i] = static_cast<uint32_t>(row[at[i]]);
  if (p0 >= item.len) return item;
  item.valid = true;
  preloaded = min(a.partition_tokens, item.len - p0) > (kN - 1) * kStep;
  return item;
}

template <typename QE, bool kFp8, int kSplit, int kHT = 1, uint32_t kD = kDim, int kNt = -1>
__global__ __launch_bounds__(kSplit * 64) __attribute__((amdgpu_waves_per_eu(2)))
void decode_stream_kernel(DecodeArgs a) {
  constexpr int kS = kFp8 ? kStreamStagesFp8 : kStreamStages;
  using Dec = StreamDecoder<QE, kFp8, kHT, kD, kS, kNt>;
  __shared__ __attribute__((aligned(16))) uint8_t tiles[kSplit * Dec::kWaveBytes];
  LOOM_WAVE_STAMP(blockIdx.x * kSplit + (threadIdx.x >> 6));
  const WorkItem item = schedule_item(a, blockIdx.x);
  LOOM_WAVE_ITEM(a, item);
  if (!item.valid) return;  // uniform across the workgroup
  stream_item<QE, kFp8, kSplit, kHT, kD, kS, kNt>(a, tiles, item);
}

// kGroup consecutive work items per workgroup, one wave each and independent
// (the single-wave path has no workgroup barrier). With the KV head varying
// fastest in the schedule, a workgroup holds adjacent heads of one
// (sequence, partition): their rows of each block share pages and are
// requested from one CU at about the same time, which the memory system
// serves faster than the same rows requested from CUs on different XCDs.
constexpr int kStreamGroup = 4;
// Pipeline stages of the grouped kernel's 16-bit waves.
constexpr int kStreamGroupStages = 2;
// FP8 caches (rows half as long, stages half as large): eight items per
// workgroup, which covers all heads of a token row or block when Hkv = 8.
// Measured against four: C4 210 -> 205.6 us, head size 64 112.6 -> 108.5,
// 96 169.7 -> 164.4, 112 104.8 -> 98.6; 16-bit caches measured 1% slower
// with eight (head size 64) and 6% slower at head size 128 (one workgroup of
// 128 KiB per CU). With non-temporal K/V loads and partial stores, four
// against eight: C4 decode 189.4-189.9 against 189.6-190.1 us (the same);
// head size 96 82.9-84.2 against 79.9-80.3, 112 89.7-90.2 against 84.9-85.3
// (eight faster). Head size 128 with more than two partitions takes four-item
// workgroups that fold pairs of partitions instead (pair_eligible).
constexpr int kStreamGroupFp8 = 8;

// kDirect: items in index order (KV head fastest, then partition, then
// sequence) instead of the longest-first schedule, for the library's own
// split of small grids, where one round of items covers the launch. The
// item is known from the index, so its length and its first 2S block IDs
// are loaded together: the wave starts after two memory round trips, not
// three. (Compiler-visible scalar loads: the compiler waits for them before
// any use or copy.)
// Wave priority rising with the workgroup's place in the grid (s_setprio
// 0-3): of the waves on one CU, those dispatched later, which run the
// schedule's last and shortest items, get the issue slots first, so the
// launch's tail is shorter. kSteep: 1 from half the grid, 2 from three
// quarters, 3 from seven eighths; else one step per quarter. The grouped
// kernel applies it only to ragged batches (WorkItem::uneven): where every
// item is the same length the later workgroups starve the earlier ones on
// their CUs (B=64 x 4096 tokens, Hq 32 / Hkv 8: head size 128 175.5 ->
// 186.7 us per call, 96 187.1 -> 200.5, 112 171.8 -> 185.3). Measured (call
// us, A/B pairs on one box): C3 205.3 -> 204.2 with quarter steps, 205.0 ->
// 204.5 steep against quarter steps, 205.5 -> 204.5 steep on ragged batches
// only; wide groups (B=64, 16384 tokens, quarter
// steps) BF16 48/1 126.5 -> 124.1, FP8 64/1 127.0 -> 125.1, where steep steps
// measured C5 +2.5 and BF16 48/1 +1.5, but FP8 two-tile waves gain from them
// (64/1 124.7 -> 118.7, 128/1 at 8192 tokens 110.2 -> 108.7; FP8 48/1 on
// one-tile waves +1.3). The FP8 two-partition workgroups
// measured 0.9 us slower with it (C4) and keep the default priority.
template <bool kSteep>
__device__ __forceinline__ void rise_priority_with_dispatch() {
  if constexpr (kSteep) {
    const uint32_t e = blockIdx.x * 8U / gridDim.x;
    if (e >= 7) __builtin_amdgcn_s_setprio(3);
    else if (e >= 6) __builtin_amdgcn_s_setprio(2);
    else if (e >= 4) __builtin_amdgcn_s_setprio(1);
  } else {
    const uint32_t q = blockIdx.x * 4U / gridDim.x;
    if (q == 1) __builtin_amdgcn_s_setprio(1);
    else if (q == 2) __builtin_amdgcn_s_setprio(2);
    else if (q == 3) __builtin_amdgcn_s_setprio(3);
  }
}

template <typename QE, bool kFp8, int kGroup, uint32_t kD = kDim, int kNt = -1, bool kDirect = false,
          bool kPair = false>
__global__ __launch_bounds__(kGroup * 64) __attribute__((amdgpu_waves_per_eu(2)))
void decode_stream_group_kernel(DecodeArgs a) {
  constexpr int kGroupStages = kFp8 ? kStreamStagesFp8 : kStreamGroupStages;
  using Dec = StreamDecoder<QE, kFp8, 1, kD, kGroupStages, kNt>;
  __shared__ __attribute__((aligned(16))) uint8_t tiles[kGroup * Dec::kWaveBytes];
  const uint32_t wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  LOOM_WAVE_STAMP(blockIdx.x * kGroup + wave);
  if constexpr (kPair) {
    // kGroup / 2 adjacent KV heads x two consecutive partitions: waves
    // w and w + kGroup / 2 hold the same head's partitions 2j and 2j + 1 and
    // leave one merged state (pair_publish / pair_combine).
    constexpr uint32_t kHeads = kGroup / 2;
    const WorkItem item = pair_item(a, blockIdx.x, kHeads, wave);
    if (item.len == 0) return;  // a unit past the schedule's end: uniform across the workgroup
    LOOM_WAVE_ITEM(a, item);
    uint8_t* own = tiles + wave * Dec::kWaveBytes;
    if (wave >= kHeads) {
      if (!item.valid) {  // the sequence ends in partition 2j
        pair_publish_empty<Dec>(own);
        __syncthreads();
        return;
      }
      stream_item<QE, kFp8, 1, 1, kD, kGroupStages, kNt, true>(a, own, item);
    } else {
      stream_item<QE, kFp8, 1, 1, kD, kGroupStages, kNt, true>(a, own, item, false, nullptr,
                                                               tiles + (wave + kHeads) * Dec::kWaveBytes);
    }
    return;
  } else if constexpr (kDirect) {
    uint32_t first[2 * kGroupStages];
    bool preloaded = false;
    const WorkItem item = direct_item<2 * kGroupStages>(a, blockIdx.x * kGroup + wave, first, preloaded);
    if (!item.valid) return;  // per wave: nothing below waits on the other waves
    LOOM_WAVE_ITEM(a, item);
    stream_item<QE, kFp8, 1, 1, kD, kGroupStages, kNt>(a, tiles + wave * Dec::kWaveBytes, item, preloaded, first);
  } else {
    const WorkItem item = schedule_item(a, blockIdx.x * kGroup + wave);
    if (item.uneven) rise_priority_with_dispatch<true>();
    LOOM_WAVE_ITEM(a, item);
    if (!item.valid) return;  // per wave: nothing below waits on the other waves
    stream_item<QE, kFp8, 1, 1, kD, kGroupStages, kNt>(a, tiles + wave * Dec::kWaveBytes, item);
  }
}


// Groups of 17-128 query heads: one workgroup of waves of 16 or 32 heads each
// (kHTW head tiles of 16) per work item (stream_item_shared), so that each K/V
// row is read from HBM once into LDS for all of the group's heads.
template <typename QE, bool kFp8, int kWaves, uint32_t kD = kDim, int kHTW = 2>
__global__ __launch_bounds__(kWaves * 64) __attribute__((amdgpu_waves_per_eu(2)))
void decode_stream_heads_kernel(DecodeArgs a) {
  using Dec = StreamDecoder<QE, kFp8, kHTW, kD>;
  __shared__ __attribute__((aligned(16)))
  uint8_t tiles[kSharedStages * Dec::kStageBytes + (kFp8 ? kWaves * kStep * Dec::kPitch : 0)];
  rise_priority_with_dispatch<kFp8 && kHTW == 2>();
  LOOM_WAVE_STAMP(blockIdx.x * kWaves + (threadIdx.x >> 6));
  const WorkItem item = schedule_item(a, blockIdx.x);
  if (threadIdx.x < 64) LOOM_WAVE_ITEM(a, item);  // one record per item: the waves share its K/V reads
  if (!item.valid) return;  // uniform across the workgroup
  stream_item_shared<QE, kFp8, kWaves, kD, kHTW>(a, tiles, item);
}

// ---------------------------------------------------------------------------
// Split-K merge kernels (the log-sum-exp identity of
// paged_decode_attention.cu:780-852), launched after the decode kernel when
// the decode launch does not merge its own partitions. Only the
// min(ceil(len / partition_tokens), parts) partitions that hold tokens are
// read. Partial outputs are F32 sums O_p weighted by f_p = 2^(m_p - M).
// ---------------------------------------------------------------------------
constexpr uint32_t kMergeThreads = 256;
constexpr uint32_t kMergeRowsPerGroup = kMergeThreads / 64;
constexpr uint32_t kMergeRowParts = 32;  // largest kParts instantiated

__device__ __forceinline__ uint32_t merge_parts(const DecodeArgs& a, uint32_t seq) {
  const uint32_t len = static_cast<uint32_t>(a.sequence_lengths[seq]);
  return static_cast<uint32_t>(min((static_cast<uint64_t>(len) + a.partition_tokens - 1) / a.partition_tokens,
                                   static_cast<uint64_t>(a.parts)));
}

// At most kParts partitions, any value head size: one wave per (sequence,
// query head) row, four rows per workgroup, no barriers. Every load of the
// row (m, l of lane p; two output dims of all partitions per lane) is issued
// before any result is needed, so a row costs one memory round trip; the
// factors f_p are broadcast with readlane.
template <typename QE, uint32_t kParts>
__global__ __launch_bounds__(kMergeThreads) void merge_kernel(DecodeArgs a, uint32_t rows) {
  using QT = typename QE::T;
  const uint32_t lane = threadIdx.x & 63U;
  const uint32_t row = blockIdx.x * kMergeRowsPerGroup + __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  if (row >= rows) return;
  const uint32_t n = min(merge_parts(a, row / a.query_heads), kParts);
  const uint64_t s0 = state_of(a, row, 0);
  const uint64_t sstride = a.query_heads;
  const float* ml = a.ws_ml + s0 * 2;
  const uint32_t Dv = a.value_head_size;
  const float* os = a.ws_o + s0 * Dv;
  QT* out = static_cast<QT*>(a.output) + static_cast<uint64_t>(row) * Dv;

  const float mp = lane < n ? ml[2 * sstride * lane] : -INFINITY;
  const float lp = lane < n ? ml[2 * sstride * lane + 1] : 0.0f;
  for (uint32_t d0 = 0; d0 < Dv; d0 += 128) {
    const uint32_t d = d0 + 2 * lane;
    float v0[kParts], v1[kParts];
#pragma unroll
    for (uint32_t j = 0; j < kParts; ++j) {
      const float* src = os + static_cast<uint64_t>(j) * sstride * Dv + d;
      v0[j] = j < n && d < Dv ? src[0] : 0.0f;
      v1[j] = j < n && d + 1 < Dv ? src[1] : 0.0f;
    }
    const float M = wave_max_dpp(mp);
    // A partition without tokens would hold m = -inf and contributes nothing.
    const float f = isfinite(mp) ? exp2f(mp - M) : 0.0f;
    const float L = wave_sum_dpp(lp * f);
    float o0 = 0.0f, o1 = 0.0f;
#pragma unroll
    for (uint32_t j = 0; j < kParts; ++j) {
      const float fj = __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, f), j));
      o0 = fmaf(v0[j], fj, o0);
      o1 = fmaf(v1[j], fj, o1);
    }
    const float inv = 1.0f / L;
    if (d < Dv) out[d] = QE::from_f(o0 * inv);
    if (d + 1 < Dv) out[d + 1] = QE::from_f(o1 * inv);
    if (d0 == 0 && lane == 0 && a.lse != nullptr) a.lse[row] = (M + log2f(L)) * kLn2;
  }
}

// Many partitions, any value head size: one workgroup of 256 threads per
// row. Factors f_p go to LDS; then wave w accumulates partitions p = w mod 4
// for 2 dims per lane (unrolled for loads in flight), and the four partial
// sums are added in LDS.
constexpr uint32_t kMergeWaves = kMergeThreads / 64;
constexpr uint32_t kMergeWindow = 2048;
constexpr uint32_t kMergeDimsPerPass = 128;

template <typename QE>
__global__ __launch_bounds__(kMergeThreads) void merge_wide_kernel(DecodeArgs a) {
  using QT = typename QE::T;
  __shared__ float factor[kMergeWindow];
  __shared__ float red[kMergeWaves];
  __shared__ float part[kMergeWaves][kMergeDimsPerPass];
  const uint32_t row = blockIdx.x;
  const uint32_t n = merge_parts(a, row / a.query_heads);
  const uint64_t s0 = state_of(a, row, 0);
  const uint64_t sstride = a.query_heads;
  const float* ml = a.ws_ml + s0 * 2;
  const uint32_t Dv = a.value_head_size;
  const uint64_t pstride = sstride * Dv;  // elements between partitions' partial outputs
  const float* os = a.ws_o + s0 * Dv;
  const uint32_t tid = threadIdx.x;
  const uint32_t lane = tid & 63U;
  const uint32_t wave = tid >> 6;

  float M = -INFINITY;
  for (uint32_t p = tid; p < n; p += kMergeThreads) M = fmaxf(M, ml[2 * sstride * p]);
#pragma unroll
  for (int off = 32; off > 0; off >>= 1) M = fmaxf(M, __shfl_xor(M, off, 64));
  if (lane == 0) red[wave] = M;
  __syncthreads();
  M = red[0];
#pragma unroll
  for (uint32_t w = 1; w < kMergeWaves; ++w) M = fmaxf(M, red[w]);
  __syncthreads();

  float Lp = 0.0f;
  for (uint32_t p = tid; p < n; p += kMergeThreads)
    Lp = fmaf(ml[2 * sstride * p + 1], exp2f(ml[2 * sstride * p] - M), Lp);
#pragma unroll
  for (int off = 32; off > 0; off >>= 1) Lp += __shfl_xor(Lp, off, 64);
  if (lane == 0) red[wave] = Lp;
  __syncthreads();
  float L = 0.0f;
#pragma unroll
  for (uint32_t w = 0; w < kMergeWaves; ++w) L += red[w];
  const float inv = 1.0f / L;

  for (uint32_t d0 = 0; d0 < Dv; d0 += kMergeDimsPerPass) {
    const uint32_t d_a = d0 + lane, d_b = d0 + 64 + lane;
    auto pair = [&](const float* o, float& va, float& vb) {
      va = d_a < Dv ? o[d_a] : 0.0f;
      vb = d_b < Dv ? o[d_b] : 0.0f;
    };
    float acc_a = 0.0f, acc_b = 0.0f;
    for (uint32_t w0 = 0; w0 < n; w0 += kMergeWindow) {
      const uint32_t wn = min(kMergeWindow, n - w0);
      __syncthreads();
      for (uint32_t p = tid; p < wn; p += kMergeThreads) factor[p] = exp2f(ml[2 * sstride * (w0 + p)] - M);
      __syncthreads();
      uint32_t p = wave;
      for (; p + 3 * kMergeWaves < wn; p += 4 * kMergeWaves) {
        const float* o0 = os + static_cast<uint64_t>(w0 + p) * pstride;
        const float* o1 = o0 + kMergeWaves * pstride;
        const float* o2 = o1 + kMergeWaves * pstride;
        const float* o3 = o2 + kMergeWaves * pstride;
        float a0, b0, a1, b1, a2, b2, a3, b3;
        pair(o0, a0, b0);
        pair(o1, a1, b1);
        pair(o2, a2, b2);
        pair(o3, a3, b3);
        const float f0 = factor[p], f1 = factor[p + kMergeWaves];
        const float f2 = factor[p + 2 * kMergeWaves], f3 = factor[p + 3 * kMergeWaves];
        acc_a = fmaf(a0, f0, acc_a);
        acc_b = fmaf(b0, f0, acc_b);
        acc_a = fmaf(a1, f1, acc_a);
        acc_b = fmaf(b1, f1, acc_b);
        acc_a = fmaf(a2, f2, acc_a);
        acc_b = fmaf(b2, f2, acc_b);
        acc_a = fmaf(a3, f3, acc_a);
        acc_b = fmaf(b3, f3, acc_b);
      }
      for (; p < wn; p += kMergeWaves) {
        const float* o0 = os + static_cast<uint64_t>(w0 + p) * pstride;
        float a0, b0;
        pair(o0, a0, b0);
        acc_a = fmaf(a0, factor[p], acc_a);
        acc_b = fmaf(b0, factor[p], acc_b);
      }
    }
    part[wave][d_a - d0] = acc_a;
    part[wave][d_b - d0] = acc_b;
    __syncthreads();
    if (tid < kMergeDimsPerPass && d0 + tid < Dv) {
      float O = 0.0f;
#pragma unroll
      for (uint32_t w = 0; w < kMergeWaves; ++w) O += part[w][tid];
      static_cast<QT*>(a.output)[static_cast<uint64_t>(row) * Dv + d0 + tid] = QE::from_f(O * inv);
    }
    __syncthreads();
  }
  if (tid == 0 && a.lse != nullptr) a.lse[row] = (M + log2f(L)) * kLn2;
}

// Value head size 64, 128 or 256 with 16-byte aligned partial rows, any
// partition count: kW waves per row, each loading 16-byte pieces of its
// partitions (w, w + kW, ...) in batches of kB per lane. With kW = 1 a
// workgroup holds four independent rows; otherwise one row, merged in two
// stages of the log-sum-exp identity (the two-stage merge of long contexts):
//   Stage 1 (registers, merge_partitions): each wave's own running state
//     over its partitions, its lane groups then combined.
//   Stage 2 (LDS, one barrier): wave 0 combines the kW wave states.
// The launch picks kW and kB so that one batch covers the row's partitions.
template <typename QE, uint32_t kD, uint32_t kW, uint32_t kB>
__global__ __launch_bounds__(kW == 1 ? 256 : kW * 64) void merge_rows_kernel(DecodeArgs a, uint32_t rows) {
  constexpr uint32_t kRowsPerGroup = kW == 1 ? 4 : 1;
  __shared__ float wave_ml[kW][2];
  __shared__ f32x4 wave_o[kW][kD / 4];
  const uint32_t wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const uint32_t lane = threadIdx.x & 63U;
  const uint32_t row = kW == 1 ? blockIdx.x * kRowsPerGroup + wave : blockIdx.x;
  if (row >= rows) return;  // kW == 1 only: whole workgroups otherwise
  const uint32_t n = merge_parts(a, row / a.query_heads);
  const uint32_t w = kW == 1 ? 0U : wave;
  const MergeState st = merge_partitions<kD, kB>(a, state_of(a, row, 0), n, w, kW);
  if constexpr (kW == 1) {
    merge_store_row<QE, kD>(a, row, st);
  } else {
    if (lane < kD / 4) wave_o[wave][lane] = st.o;
    if (lane == 0) {
      wave_ml[wave][0] = st.m;
      wave_ml[wave][1] = st.l;
    }
    __syncthreads();
    if (wave != 0) return;
    MergeState total = st;
#pragma unroll
    for (uint32_t v = 1; v < kW; ++v)
      total = merge_combine(total, MergeState{wave_ml[v][0], wave_ml[v][1],
                                              lane < kD / 4 ? wave_o[v][lane] : f32x4{0.0f, 0.0f, 0.0f, 0.0f}});
    merge_store_row<QE, kD>(a, row, total);
  }
}

// ---------------------------------------------------------------------------
// Host side: error reporting, telemetry, validation, planning, launch.
// ---------------------------------------------------------------------------
thread_local std::string g_last_error;
thread_local const char* g_last_family = "";
thread_local const char* g_last_kernel = "";  // decode kernel of the last successful call
thread_local const char* g_launch_kernel = "";  // decode kernel of the launch in progress
thread_local bool g_launch_pairs = false;       // that launch leaves one state per two partitions
thread_local uint32_t g_last_internal_split = 0;
std::atomic<uint64_t> g_decode_launches{0};
std::atomic<uint64_t> g_rope_launches{0};

int fail(int status, const char* message) {
  g_last_error = message;
  return status;
}

constexpr int kTimedKernels = 3;  // LOOM_HIP_KERNEL_DECODE, _MERGE, _ROPE

struct TimingState {
  std::mutex mu;
  std::atomic<bool> enabled{false};
  std::vector<std::pair<hipEvent_t, hipEvent_t>> pending[kTimedKernels];
  double total_ms[kTimedKernels] = {};
  uint64_t launches[kTimedKernels] = {};
};

TimingState& timing() {
  static TimingState* state = new TimingState();
  return *state;
}

struct TimedLaunch {
  hipEvent_t start = nullptr, stop = nullptr;
  int kernel;
  hipStream_t stream;
  TimedLaunch(int k, hipStream_t s) : kernel(k), stream(s) {
    TimingState& t = timing();
    std::lock_guard<std::mutex> lock(t.mu);
    if (!t.enabled) return;
    if (hipEventCreate(&start) != hipSuccess || hipEventCreate(&stop) != hipSuccess) {
      start = stop = nullptr;
      return;
    }
    (void)hipEventRecord(start, stream);
  }
  ~TimedLaunch() {
    if (start == nullptr) return;
    (void)hipEventRecord(stop, stream);
    TimingState& t = timing();
    std::lock_guard<std::mutex> lock(t.mu);
    t.pending[kernel].emplace_back(start, stop);
  }
};

enum DTypeCode : uint32_t { kF32 = LOOM_HIP_F32, kF16 = LOOM_HIP_F16, kBf16 = LOOM_HIP_BF16 };

struct Problem {
  uint32_t dtype;
  const void* query;
  const void* key_cache;
  const void* value_cache;
  const float* key_scales;
  const float* value_scales;
  const int32_t* block_tables;
  const int32_t* sequence_lengths;
  void* output;
  float* lse;
  float* workspace;
  uint64_t workspace_elements;
  uint32_t sequences, query_heads, kv_heads, head_size, value_head_size;
  uint32_t num_blocks, block_size, cache_encoding, scale_stride;
  uint64_t k_block, k_page, k_head, v_block, v_page, v_head;
  uint32_t max_blocks_per_sequence, max_sequence_length;
  uint32_t partition_tokens;  // 0 = one partition per sequence
  float scale;
  bool static_workspace;  // split-K states go to the library's per-device array
  bool direct_schedule = false;  // split inside the library: items in index order
};

size_t elem_size(uint32_t dtype) { return dtype == kF32 ? 4 : 2; }

size_t cache_elem_size(const Problem& p) {
  return p.cache_encoding == LOOM_HIP_KV_CACHE_FP8_E4M3 ? 1 : elem_size(p.dtype);
}

bool mul_ok(uint64_t a, uint64_t b, uint64_t* out) {
  if (a != 0 && b > std::numeric_limits<uint64_t>::max() / a) return false;
  *out = a * b;
  return true;
}

uint64_t parts_for(uint32_t max_len, uint32_t partition_tokens) {
  if (partition_tokens == 0 || partition_tokens >= max_len) return 1;
  return (static_cast<uint64_t>(max_len) + partition_tokens - 1) / partition_tokens;
}

bool is_pow2(uint32_t v) { return v != 0 && (v & (v - 1)) == 0; }

// Byte span [lo, hi) of the elements a cache view can address.
bool cache_span(const Problem& p, bool key, uint64_t* bytes) {
  const uint64_t dim = key ? p.head_size : p.value_head_size;
  const uint64_t sb = key ? p.k_block : p.v_block;
  const uint64_t sp = key ? p.k_page : p.v_page;
  const uint64_t sh = key ? p.k_head : p.v_head;
  uint64_t a, b, c, total;
  if (!mul_ok(p.num_blocks - 1ULL, sb, &a) || !mul_ok(p.block_size - 1ULL, sp, &b) ||
      !mul_ok(p.kv_heads - 1ULL, sh, &c))
    return false;
  total = a + b;
  if (total < a) return false;
  if (total + c < total) return false;
  total += c;
  if (total + dim < total) return false;
  total += dim;
  return mul_ok(total, cache_elem_size(p), bytes);
}

bool overlaps(const void* a, uint64_t abytes, const void* b, uint64_t bbytes) {
  if (a == nullptr || b == nullptr || abytes == 0 || bbytes == 0) return false;
  const uintptr_t a0 = reinterpret_cast<uintptr_t>(a), b0 = reinterpret_cast<uintptr_t>(b);
  return a0 < b0 + bbytes && b0 < a0 + abytes;
}

// Host validation (paged_decode_attention.cu:999-1049 without the 1024
// context cap, plus the extension fields). Returns LOOM_HIP_SUCCESS or the
// status to report, with the thread-local message set.
int validate(const Problem& p) {
  if (p.dtype != kF32 && p.dtype != kF16 && p.dtype != kBf16)
    return fail(LOOM_HIP_INVALID_ARGUMENT, "unknown dtype code");
  if (p.query == nullptr || p.key_cache == nullptr || p.value_cache == nullptr ||
      p.block_tables == nullptr || p.sequence_lengths == nullptr || p.output == nullptr)
    return fail(LOOM_HIP_INVALID_ARGUMENT, "paged decode pointers must be non-null");
  if (p.sequences == 0 || p.query_heads == 0 || p.kv_heads == 0 || p.head_size == 0 ||
      p.value_head_size == 0 || p.num_blocks == 0 || p.block_size == 0 ||
      p.max_blocks_per_sequence == 0 || p.max_sequence_length == 0)
    return fail(LOOM_HIP_INVALID_ARGUMENT, "paged decode dimensions must be non-zero");
  if (p.query_heads % p.kv_heads != 0)
    return fail(LOOM_HIP_INVALID_ARGUMENT, "query head count must be divisible by KV head count");
  if (!std::isfinite(p.scale) || p.scale <= 0.0f)
    return fail(LOOM_HIP_INVALID_ARGUMENT, "attention scale must be finite and positive");
  if (static_cast<uint64_t>(p.max_sequence_length) >
      static_cast<uint64_t>(p.block_size) * p.max_blocks_per_sequence)
    return fail(LOOM_HIP_INVALID_ARGUMENT,
                "maximum sequence length exceeds block-table capacity");
  uint64_t tmp;
  if (!mul_ok(static_cast<uint64_t>(p.sequences) * p.query_heads, p.head_size, &tmp) ||
      !mul_ok(static_cast<uint64_t>(p.sequences) * p.query_heads, p.value_head_size, &tmp) ||
      !mul_ok(static_cast<uint64_t>(p.num_blocks) * p.block_size, static_cast<uint64_t>(p.kv_heads) * p.head_size, &tmp) ||
      !mul_ok(static_cast<uint64_t>(p.num_blocks) * p.block_size, static_cast<uint64_t>(p.kv_heads) * p.value_head_size, &tmp))
    return fail(LOOM_HIP_INVALID_ARGUMENT, "paged decode element count overflows");
  if (static_cast<uint64_t>(p.sequences) * p.query_heads >
      static_cast<uint64_t>(std::numeric_limits<int>::max()))
    return fail(LOOM_HIP_INVALID_ARGUMENT, "sequences * query_heads exceeds the launch grid");
  if (p.cache_encoding != LOOM_HIP_KV_CACHE_NATIVE && p.cache_encoding != LOOM_HIP_KV_CACHE_FP8_E4M3)
    return fail(LOOM_HIP_INVALID_ARGUMENT, "unknown K/V cache encoding");
  if (p.cache_encoding == LOOM_HIP_KV_CACHE_FP8_E4M3) {
    if (p.key_scales == nullptr || p.value_scales == nullptr)
      return fail(LOOM_HIP_INVALID_ARGUMENT, "FP8 K/V caches require key and value scales");
    if (p.scale_stride > 1)
      return fail(LOOM_HIP_INVALID_ARGUMENT, "scale_stride must be 0 (per tensor) or 1 (per KV head)");
  } else if (p.key_scales != nullptr || p.value_scales != nullptr || p.scale_stride != 0) {
    return fail(LOOM_HIP_INVALID_ARGUMENT, "native K/V caches take no scales");
  }
  if (p.k_block == 0 || p.k_page == 0 || p.k_head == 0 || p.v_block == 0 || p.v_page == 0 ||
      p.v_head == 0)
    return fail(LOOM_HIP_INVALID_ARGUMENT, "cache strides must be non-zero");
  uint64_t kbytes, vbytes;
  if (!cache_span(p, true, &kbytes) || !cache_span(p, false, &vbytes))
    return fail(LOOM_HIP_INVALID_ARGUMENT, "cache strides overflow the address space");

  const uint64_t parts = parts_for(p.max_sequence_length, p.partition_tokens);
  uint64_t need = 0;
  if (parts > 1) {
    need = static_cast<uint64_t>(p.sequences) * p.query_heads * parts * (p.value_head_size + 2ULL);
  }
  if (p.static_workspace) {
    if (need > LOOM_HIP_STATIC_WORKSPACE_ELEMENTS)
      return fail(LOOM_HIP_UNSUPPORTED,
                  "split-K states exceed the static workspace (LOOM_HIP_STATIC_WORKSPACE_ELEMENTS F32 elements)");
  } else if (need == 0) {
    if (p.workspace != nullptr || p.workspace_elements != 0)
      return fail(LOOM_HIP_INVALID_ARGUMENT,
                  "this shape uses a single partition; the workspace must be null with zero elements");
  } else if (p.workspace == nullptr || p.workspace_elements < need) {
    return fail(LOOM_HIP_INVALID_ARGUMENT, "split-K workspace is missing or too small");
  }

  // Output, LSE and workspace must not alias any input or each other
  // (the byte-range rule of the reference bridge, cuda/mod.rs:119-153).
  const uint64_t qbytes = static_cast<uint64_t>(p.sequences) * p.query_heads * p.head_size * elem_size(p.dtype);
  const uint64_t obytes = static_cast<uint64_t>(p.sequences) * p.query_heads * p.value_head_size * elem_size(p.dtype);
  const uint64_t tbytes = static_cast<uint64_t>(p.sequences) * p.max_blocks_per_sequence * 4;
  const uint64_t lbytes = static_cast<uint64_t>(p.sequences) * 4;
  const uint64_t lsebytes = p.lse ? static_cast<uint64_t>(p.sequences) * p.query_heads * 4 : 0;
  const uint64_t wbytes = p.workspace ? p.workspace_elements * 4 : 0;
  const uint64_t sbytes = p.scale_stride ? static_cast<uint64_t>(p.kv_heads) * 4 : 4;
  struct Region { const void* ptr; uint64_t bytes; };
  const Region inputs[] = {
      {p.query, qbytes}, {p.key_cache, kbytes}, {p.value_cache, vbytes},
      {p.block_tables, tbytes}, {p.sequence_lengths, lbytes},
      {p.key_scales, p.key_scales ? sbytes : 0}, {p.value_scales, p.value_scales ? sbytes : 0}};
  const Region outputs[] = {{p.output, obytes}, {p.lse, lsebytes}, {p.workspace, wbytes}};
  for (const Region& o : outputs) {
    for (const Region& i : inputs) {
      if (overlaps(o.ptr, o.bytes, i.ptr, i.bytes))
        return fail(LOOM_HIP_INVALID_ARGUMENT, "output, LSE and workspace must not overlap the inputs");
    }
  }
  for (int i = 0; i < 3; ++i) {
    for (int j = i + 1; j < 3; ++j) {
      if (overlaps(outputs[i].ptr, outputs[i].bytes, outputs[j].ptr, outputs[j].bytes))
        return fail(LOOM_HIP_INVALID_ARGUMENT, "output, LSE and workspace must not overlap each other");
    }
  }
  return LOOM_HIP_SUCCESS;
}

bool aligned16(const void* ptr) { return (reinterpret_cast<uintptr_t>(ptr) & 15U) == 0; }

// The matrix-core kernels store the output four 16-bit elements at a time
// with 8-byte stores, (m, l) pairs as 8 bytes and partial rows four F32
// elements at a time with 16-byte stores.
bool stores_aligned8(const Problem& p) {
  const auto a8 = [](const void* ptr) { return (reinterpret_cast<uintptr_t>(ptr) & 7U) == 0; };
  if (!a8(p.output)) return false;
  const uint64_t parts = parts_for(p.max_sequence_length, p.partition_tokens);
  if (parts == 1 || p.workspace == nullptr) return true;
  const float* ws_o = p.workspace + static_cast<uint64_t>(p.sequences) * p.query_heads * parts * 2;
  return a8(p.workspace) && aligned16(ws_o);
}

// Shape-level eligibility of the matrix-core kernel.
bool mfma_shape(uint32_t dtype, uint32_t head_size, uint32_t value_head_size,
                uint32_t query_heads, uint32_t kv_heads, uint32_t block_size) {
  return (dtype == kF16 || dtype == kBf16) && head_size == kDim && value_head_size == kDim &&
         query_heads / kv_heads <= 32 && is_pow2(block_size);
}

bool mfma_eligible(const Problem& p) {
  if (!mfma_shape(p.dtype, p.head_size, p.value_head_size, p.query_heads, p.kv_heads, p.block_size))
    return false;
  const uint64_t es = cache_elem_size(p);
  const uint64_t strides[] = {p.k_block, p.k_page, p.k_head, p.v_block, p.v_page, p.v_head};
  for (uint64_t s : strides) {
    if ((s * es) % 16 != 0) return false;
  }
  return aligned16(p.query) && aligned16(p.key_cache) && aligned16(p.value_cache) && stores_aligned8(p);
}

uint32_t log2u(uint32_t v) {
  uint32_t r = 0;
  while ((1U << r) < v) ++r;
  return r;
}

// Launches merge_rows_kernel with kW waves per row (four rows per workgroup
// at kW = 1) and kB loads per lane: the smallest shape whose one batch
// covers `parts` partitions (kQ = 256 / kD partitions per load), else 8
// waves of 8-load batches.
template <typename QE, uint32_t kD>
void launch_merge_rows(const DecodeArgs& args, uint32_t rows, hipStream_t stream) {
  constexpr uint32_t kQ = 256 / kD;
  const uint32_t parts = args.parts;
  const dim3 quad((rows + 3) / 4), one(rows);
  if (parts <= kQ * 2) {
    hipLaunchKernelGGL((merge_rows_kernel<QE, kD, 1, 2>), quad, dim3(256), 0, stream, args, rows);
  } else if (parts <= kQ * 4) {
    hipLaunchKernelGGL((merge_rows_kernel<QE, kD, 1, 4>), quad, dim3(256), 0, stream, args, rows);
  } else if (parts <= kQ * 8) {
    hipLaunchKernelGGL((merge_rows_kernel<QE, kD, 1, 8>), quad, dim3(256), 0, stream, args, rows);
  } else if (parts <= kQ * 8 * 4) {
    hipLaunchKernelGGL((merge_rows_kernel<QE, kD, 4, 8>), one, dim3(256), 0, stream, args, rows);
  } else {
    hipLaunchKernelGGL((merge_rows_kernel<QE, kD, 8, 8>), one, dim3(512), 0, stream, args, rows);
  }
}

template <typename QE>
int launch_merge(const DecodeArgs& args, uint32_t rows, hipStream_t stream) {
  TimedLaunch timed(LOOM_HIP_KERNEL_MERGE, stream);
  const dim3 grid((rows + kMergeRowsPerGroup - 1) / kMergeRowsPerGroup);
  const uint32_t dv = args.value_head_size;
  const bool rows_aligned = reinterpret_cast<uintptr_t>(args.ws_o) % 16 == 0 &&
                            reinterpret_cast<uintptr_t>(args.ws_ml) % 8 == 0;
  if (rows_aligned && dv == 64) {
    launch_merge_rows<QE, 64>(args, rows, stream);
  } else if (rows_aligned && dv == 128) {
    launch_merge_rows<QE, 128>(args, rows, stream);
  } else if (rows_aligned && dv == 256) {
    launch_merge_rows<QE, 256>(args, rows, stream);
  } else if (args.parts <= 8) {
    hipLaunchKernelGGL((merge_kernel<QE, 8>), grid, dim3(kMergeThreads), 0, stream, args, rows);
  } else if (args.parts <= 16) {
    hipLaunchKernelGGL((merge_kernel<QE, 16>), grid, dim3(kMergeThreads), 0, stream, args, rows);
  } else if (args.parts <= kMergeRowParts) {
    hipLaunchKernelGGL((merge_kernel<QE, kMergeRowParts>), grid, dim3(kMergeThreads), 0, stream, args, rows);
  } else {
    hipLaunchKernelGGL(merge_wide_kernel<QE>, dim3(rows), dim3(kMergeThreads), 0, stream, args);
  }
  return hipGetLastError() == hipSuccess ? LOOM_HIP_SUCCESS : LOOM_HIP_LAUNCH_ERROR;
}

template <typename QE, bool kFp8, int kHT, int kWaves>
int launch_mfma(const DecodeArgs& args, uint64_t grid, hipStream_t stream) {
  TimedLaunch timed(LOOM_HIP_KERNEL_DECODE, stream);
  g_launch_kernel = "decode_mfma_kernel";
  hipLaunchKernelGGL((decode_mfma_kernel<QE, kFp8, kHT, kWaves>), dim3(static_cast<uint32_t>(grid)),
                     dim3(kWaves * 64), 0, stream, args);
  return hipGetLastError() == hipSuccess ? LOOM_HIP_SUCCESS : LOOM_HIP_LAUNCH_ERROR;
}

template <typename QE, bool kFp8, int kHT>
int launch_mfma_waves(const DecodeArgs& args, uint64_t grid, uint32_t chunks, hipStream_t stream) {
  // One wave per workgroup up to 32 chunks per partition, four beyond (a
  // long single partition would otherwise leave most CUs idle).
  return chunks <= 32 ? launch_mfma<QE, kFp8, kHT, 1>(args, grid, stream)
                      : launch_mfma<QE, kFp8, kHT, 4>(args, grid, stream);
}

// FP8 caches at head size 128 pre-merge pairs of partitions in the
// workgroup when the call is split (more than two partitions, so the states
// halve): four-item workgroups of two adjacent KV heads x two partitions
// (the KV heads divide into twos) leave one state per pair of partitions.
// One state per pair halves the split-K state bytes written, which cost far
// more than their share of the traffic: on C3 the F32 state stores (10.5 MB,
// 0.9% of the bytes) cost the decode kernel 17 us of 205 (188 us with the
// stores sent to 32 KiB of L2-resident lines). Measured (C4 call us):
// eight-item workgroups of four heads x two partitions 201.8 -> 198.4
// against one state per partition; four-item workgroups of two heads x two
// partitions then 199.6 -> 194.7 (three pairs; kernel trace 199.1 -> 190.0:
// three 48 KiB workgroups per CU, where one 96 KiB workgroup per CU ran the
// launch as four synchronous rounds that dipped at every turnover). 16-bit
// caches keep one state per partition: two heads x two partitions measured
// C3 205.5 -> 206.9 us, the loss of four adjacent heads outweighing the
// halved writes. FP8 at other head sizes neither (call us, pairs against
// none, B=64, Hq 32 / Hkv 8, 512-token partitions, NHD): head size 64 117.1
// against 115.3, 80 134.2 against 132.7, 96 131.2 against 129.3, 112 105.5
// against 104.4.
bool pair_eligible(const DecodeArgs& a, int group, bool fp8) {
  return fp8 && a.head_size == kDim && a.parts > 2 && group >= 4 && a.kv_heads % static_cast<uint32_t>(group / 2) == 0;
}

template <typename QE, bool kFp8, uint32_t kD = kDim, int kGroup = kStreamGroup, int kNt = -1, bool kDirect = false>
int launch_stream_group(const DecodeArgs& args, uint64_t items, hipStream_t stream) {
  TimedLaunch timed(LOOM_HIP_KERNEL_DECODE, stream);
  g_launch_kernel = "decode_stream_group_kernel";
  // Pair workgroups exist only as FP8 four-item workgroups at head size 128
  // (pair_eligible); other instantiations do not compile the pair path.
  constexpr bool kMayPair = kFp8 && kGroup == 4 && kD == kDim && !kDirect;
  g_launch_pairs = kMayPair && pair_eligible(args, kGroup, kFp8);
  if constexpr (kMayPair) {
    if (g_launch_pairs) {
      // one workgroup per (sequence, pair of partitions, group of kGroup / 2 KV heads)
      const uint64_t units = (args.parts + 1ULL) / 2ULL * args.sequences * (args.kv_heads / (kGroup / 2));
      hipLaunchKernelGGL((decode_stream_group_kernel<QE, kFp8, kGroup, kD, kNt, false, true>),
                         dim3(static_cast<uint32_t>(units)), dim3(kGroup * 64), 0, stream, args);
      return hipGetLastError() == hipSuccess ? LOOM_HIP_SUCCESS : LOOM_HIP_LAUNCH_ERROR;
    }
  }
  {
    const uint64_t groups = (items + kGroup - 1) / kGroup;
    hipLaunchKernelGGL((decode_stream_group_kernel<QE, kFp8, kGroup, kD, kNt, kDirect>),
                       dim3(static_cast<uint32_t>(groups)), dim3(kGroup * 64), 0, stream, args);
  }
  return hipGetLastError() == hipSuccess ? LOOM_HIP_SUCCESS : LOOM_HIP_LAUNCH_ERROR;
}

template <typename QE, bool kFp8, int kSplit, int kHT = 1, uint32_t kD = kDim, int kNt = -1>
int launch_stream(const DecodeArgs& args, uint64_t grid, hipStream_t stream) {
  TimedLaunch timed(LOOM_HIP_KERNEL_DECODE, stream);
  g_launch_kernel = "decode_stream_kernel";
  hipLaunchKernelGGL((decode_stream_kernel<QE, kFp8, kSplit, kHT, kD, kNt>), dim3(static_cast<uint32_t>(grid)),
                     dim3(kSplit * 64), 0, stream, args);
  return hipGetLastError() == hipSuccess ? LOOM_HIP_SUCCESS : LOOM_HIP_LAUNCH_ERROR;
}

// Head sizes 80, 96 and 112 (16-bit cache, one head tile): the launch shapes
// of head size 128.
template <typename QE, bool kFp8, uint32_t kD, int kNt = -1>
int launch_stream_rot_nt(const DecodeArgs& args, uint64_t grid, uint32_t steps, hipStream_t stream) {
  if (grid >= 4096 || (grid >= 1024 && steps >= 8))
    return launch_stream_group<QE, kFp8, kD, kFp8 ? kStreamGroupFp8 : kStreamGroup, kNt>(args, grid, stream);
  if (steps < 8) return launch_stream<QE, kFp8, 1, 1, kD, kNt>(args, grid, stream);
  return launch_stream<QE, kFp8, 4, 1, kD, kNt>(args, grid, stream);
}

// Rows that are not whole 128-byte lines take the non-temporal hint only
// when each KV head's token rows are contiguous (dense_rows: HND).
template <typename QE, bool kFp8, uint32_t kD>
int launch_stream_rot(const DecodeArgs& args, uint64_t grid, uint32_t steps, bool dense_rows, hipStream_t stream) {
  return dense_rows ? launch_stream_rot_nt<QE, kFp8, kD, 1>(args, grid, steps, stream)
                    : launch_stream_rot_nt<QE, kFp8, kD>(args, grid, steps, stream);
}

// The streaming kernel needs steps that stay inside one block (power-of-two
// block size >= 16, partitions starting on multiples of 16), at most 32 query
// heads per KV head (two 16-head tiles per wave), and per-lane byte offsets
// (15 pages + one row) that fit in 31 bits.
bool stream_eligible(const Problem& p, uint64_t parts, uint32_t group) {
  if (group > 32 || p.block_size < kStep) return false;
  if (parts > 1 && p.partition_tokens % kStep != 0) return false;
  const uint64_t es = cache_elem_size(p);
  const uint64_t limit = 1ULL << 31;
  return 15 * p.k_page * es + 256 < limit && 15 * p.v_page * es + 256 < limit;
}

// Head size 64 on the streaming kernel: 16-bit queries, native or FP8 cache,
// D = Dv = 64, power-of-two blocks, 16-byte aligned bases and strides, and the
// streaming kernel's own step and offset conditions.
bool narrow_shape(uint32_t dtype, uint32_t cache_encoding, uint32_t head_size, uint32_t value_head_size,
                  uint32_t query_heads, uint32_t kv_heads, uint32_t block_size) {
  return (dtype == kF16 || dtype == kBf16) && cache_encoding <= LOOM_HIP_KV_CACHE_FP8_E4M3 && head_size == 64 &&
         value_head_size == 64 && query_heads / kv_heads <= 32 && is_pow2(block_size) && block_size >= kStep;
}

// Head size 256 with a 16-bit or FP8 cache: as head size 64, with at most 16
// query heads per KV head (one head tile per wave).
bool wide_shape(uint32_t dtype, uint32_t cache_encoding, uint32_t head_size, uint32_t value_head_size,
                uint32_t query_heads, uint32_t kv_heads, uint32_t block_size) {
  return (dtype == kF16 || dtype == kBf16) && cache_encoding <= LOOM_HIP_KV_CACHE_FP8_E4M3 && head_size == 256 &&
         value_head_size == 256 && query_heads / kv_heads <= 16 && is_pow2(block_size) && block_size >= kStep;
}

// Head size 96 with a 16-bit cache (192-byte rows), at most 16 query heads per
// KV head.
bool rot_shape(uint32_t dtype, uint32_t cache_encoding, uint32_t head_size, uint32_t value_head_size,
               uint32_t query_heads, uint32_t kv_heads, uint32_t block_size) {
  return (dtype == kF16 || dtype == kBf16) && cache_encoding <= LOOM_HIP_KV_CACHE_FP8_E4M3 &&
         (head_size == 80 || head_size == 96 || head_size == 112) && value_head_size == head_size &&
         query_heads / kv_heads <= 16 && is_pow2(block_size) && block_size >= kStep;
}

// Groups of 33-128 query heads at head size 64 or 128, native or FP8 cache:
// the streaming kernel with one wave per 16 or 32 heads of the group.
bool heads_shape(uint32_t dtype, uint32_t cache_encoding, uint32_t head_size, uint32_t value_head_size,
                 uint32_t query_heads, uint32_t kv_heads, uint32_t block_size) {
  const uint32_t group = query_heads / kv_heads;
  return (dtype == kF16 || dtype == kBf16) && cache_encoding <= LOOM_HIP_KV_CACHE_FP8_E4M3 &&
         (head_size == 64 || head_size == kDim) && value_head_size == head_size && group > 32 && group <= 128 &&
         is_pow2(block_size) && block_size >= kStep;
}

bool heads_stream_eligible(const Problem& p, uint64_t parts) {
  if (!heads_shape(p.dtype, p.cache_encoding, p.head_size, p.value_head_size, p.query_heads, p.kv_heads,
                   p.block_size))
    return false;
  const uint64_t es = cache_elem_size(p);
  const uint64_t strides[] = {p.k_block, p.k_page, p.k_head, p.v_block, p.v_page, p.v_head};
  for (uint64_t st : strides) {
    if ((st * es) % 16 != 0) return false;
  }
  if (parts > 1 && p.partition_tokens % kStep != 0) return false;
  const uint64_t limit = 1ULL << 31;
  return aligned16(p.query) && aligned16(p.key_cache) && aligned16(p.value_cache) && stores_aligned8(p) &&
         15 * p.k_page * es + 256 < limit && 15 * p.v_page * es + 256 < limit;
}

template <typename QE, bool kFp8, uint32_t kD>
int launch_stream_heads(const DecodeArgs& args, uint64_t items, uint32_t group, hipStream_t stream) {
  using Dec = StreamDecoder<QE, kFp8, 2, kD>;
  TimedLaunch timed(LOOM_HIP_KERNEL_DECODE, stream);
  static_assert(4 * Dec::kWaveBytes <= 64 * 1024, "four waves' stages fit in 64 KiB of LDS");
  const dim3 grid(static_cast<uint32_t>(items));
  g_launch_kernel = "decode_stream_heads_kernel";
  // One head tile per wave for 16-bit caches up to 64 heads (BF16 PV splits
  // probabilities into hi + lo, two MFMAs per tile; F16 48/1 and 64/1 gain
  // 3.5 us as well), and for FP8 groups of up to 48 heads, whose second wave
  // would otherwise hold a half-empty tile. Decode us, two-tile waves ->
  // one-tile waves (B=64, 16384 tokens, 512-token partitions): BF16 48/1
  // 120.4 -> 109.7, 64/1 124.5 -> 112.9, head size 64 48/1 62.2 -> 56.0;
  // FP8 48/1 102.8 -> 98.3, FP8 64/1 105.6 -> 107.1 (kept on two tiles).
  if ((!kFp8 && group <= 64) || group <= 48) {
    if (group <= 48)
      hipLaunchKernelGGL((decode_stream_heads_kernel<QE, kFp8, 3, kD, 1>), grid, dim3(192), 0, stream, args);
    else
      hipLaunchKernelGGL((decode_stream_heads_kernel<QE, kFp8, 4, kD, 1>), grid, dim3(256), 0, stream, args);
    return hipGetLastError() == hipSuccess ? LOOM_HIP_SUCCESS : LOOM_HIP_LAUNCH_ERROR;
  }
  // 16-bit caches with groups of 97-128: seven or eight one-tile waves (BF16
  // 128/1, 8192 tokens: 93.3 -> 88.4 us). Groups of 65-96 stay on three two-tile
  // waves: six one-tile waves took 102 us against 70.
  if (!kFp8 && group > 96) {
    // ceil(group / 16) waves, so that every wave holds a live head
    if (group <= 112)
      hipLaunchKernelGGL((decode_stream_heads_kernel<QE, kFp8, 7, kD, 1>), grid, dim3(448), 0, stream, args);
    else
      hipLaunchKernelGGL((decode_stream_heads_kernel<QE, kFp8, 8, kD, 1>), grid, dim3(512), 0, stream, args);
    return hipGetLastError() == hipSuccess ? LOOM_HIP_SUCCESS : LOOM_HIP_LAUNCH_ERROR;
  }
  if (group <= 64) {
    hipLaunchKernelGGL((decode_stream_heads_kernel<QE, kFp8, 2, kD>), grid, dim3(128), 0, stream, args);
  } else if (group <= 96) {
    hipLaunchKernelGGL((decode_stream_heads_kernel<QE, kFp8, 3, kD>), grid, dim3(192), 0, stream, args);
  } else {
    hipLaunchKernelGGL((decode_stream_heads_kernel<QE, kFp8, 4, kD>), grid, dim3(256), 0, stream, args);
  }
  return hipGetLastError() == hipSuccess ? LOOM_HIP_SUCCESS : LOOM_HIP_LAUNCH_ERROR;
}

// Groups of 17-32 query heads as two waves of 16 heads on one shared ring of
// K/V stages (decode_stream_heads_kernel with one head tile per wave). With
// PV taking BF16 probabilities as hi + lo, a wave holding both head tiles
// became bound by its own MFMA and softmax chain at ~3 waves per CU: C5
// decode 74.7 us as one wave per item, 70.2 us as two.
template <typename QE, bool kFp8, uint32_t kD>
int launch_stream_heads2(const DecodeArgs& args, uint64_t items, hipStream_t stream) {
  TimedLaunch timed(LOOM_HIP_KERNEL_DECODE, stream);
  g_launch_kernel = "decode_stream_heads_kernel";
  hipLaunchKernelGGL((decode_stream_heads_kernel<QE, kFp8, 2, kD, 1>), dim3(static_cast<uint32_t>(items)), dim3(128), 0,
                     stream, args);
  return hipGetLastError() == hipSuccess ? LOOM_HIP_SUCCESS : LOOM_HIP_LAUNCH_ERROR;
}

bool narrow_stream_eligible(const Problem& p, uint64_t parts, uint32_t group) {
  if (!narrow_shape(p.dtype, p.cache_encoding, p.head_size, p.value_head_size, p.query_heads, p.kv_heads,
                    p.block_size) &&
      !rot_shape(p.dtype, p.cache_encoding, p.head_size, p.value_head_size, p.query_heads, p.kv_heads,
                 p.block_size) &&
      !wide_shape(p.dtype, p.cache_encoding, p.head_size, p.value_head_size, p.query_heads, p.kv_heads,
                  p.block_size))
    return false;
  const uint64_t es = cache_elem_size(p);
  const uint64_t strides[] = {p.k_block, p.k_page, p.k_head, p.v_block, p.v_page, p.v_head};
  for (uint64_t st : strides) {
    if ((st * es) % 16 != 0) return false;
  }
  return aligned16(p.query) && aligned16(p.key_cache) && aligned16(p.value_cache) && stores_aligned8(p) &&
         stream_eligible(p, parts, group);
}


template <typename QE, typename CE, bool kVecK, uint32_t kDvl, bool kQLds, uint32_t kH>
int launch_vector_kernel(const DecodeArgs& args, uint64_t grid, hipStream_t stream) {
  g_launch_kernel = "decode_vector_kernel";
  TimedLaunch timed(LOOM_HIP_KERNEL_DECODE, stream);
  hipLaunchKernelGGL((decode_vector_kernel<QE, CE, kVecK, kDvl, kQLds, kH>), dim3(static_cast<uint32_t>(grid)),
                     dim3(kVecThreads), 0, stream, args);
  return hipGetLastError() == hipSuccess ? LOOM_HIP_SUCCESS : LOOM_HIP_LAUNCH_ERROR;
}

// 16-byte K vectors need the head size, every K stride and the cache base to
// be multiples of 16 bytes.
template <typename CE>
bool vector_k_aligned(const DecodeArgs& args) {
  constexpr uint64_t kW = 16 / sizeof(typename CE::T);
  return args.head_size % kW == 0 && args.k_block % kW == 0 && args.k_page % kW == 0 &&
         args.k_head % kW == 0 && reinterpret_cast<uintptr_t>(args.key_cache) % 16 == 0;
}

// The general kernel's common path: 16-byte K vectors and the query in LDS.
// It is compiled per value dims per lane (sized to Dv) and per heads class;
// every other shape takes 256-dim value tiles and 8-head workgroups.
template <typename CE>
bool vector_common_path(const DecodeArgs& args) {
  return vector_k_aligned<CE>(args) && args.head_size <= kVecQLds;
}

template <typename CE>
uint32_t vector_dims_per_lane(const DecodeArgs& args) {
  return vector_common_path<CE>(args) ? vec_dims_per_lane(args.value_head_size) : 4;
}

template <typename QE, typename CE, uint32_t kDvl>
int launch_vector_heads(const DecodeArgs& args, uint64_t grid, hipStream_t stream) {
  const uint32_t g = args.group < kVecHeads ? args.group : kVecHeads;
  if (g == 1) return launch_vector_kernel<QE, CE, true, kDvl, true, 1>(args, grid, stream);
  if (g == 2) return launch_vector_kernel<QE, CE, true, kDvl, true, 2>(args, grid, stream);
  if (g <= 4) return launch_vector_kernel<QE, CE, true, kDvl, true, 4>(args, grid, stream);
  return launch_vector_kernel<QE, CE, true, kDvl, true, 8>(args, grid, stream);
}

template <typename QE, typename CE>
int launch_vector(const DecodeArgs& args, uint64_t grid, hipStream_t stream) {
  if (args.head_size > kVecQLds) {
    return vector_k_aligned<CE>(args) ? launch_vector_kernel<QE, CE, true, 4, false, 8>(args, grid, stream)
                                      : launch_vector_kernel<QE, CE, false, 4, false, 8>(args, grid, stream);
  }
  if (!vector_k_aligned<CE>(args)) return launch_vector_kernel<QE, CE, false, 4, true, 8>(args, grid, stream);
  switch (vector_dims_per_lane<CE>(args)) {
    case 1: return launch_vector_heads<QE, CE, 1>(args, grid, stream);
    case 2: return launch_vector_heads<QE, CE, 2>(args, grid, stream);
    default: return launch_vector_heads<QE, CE, 4>(args, grid, stream);
  }
}

template <typename QE>
int run_typed(const Problem& p, hipStream_t stream) {
  const uint64_t parts = parts_for(p.max_sequence_length, p.partition_tokens);
  const uint32_t partition_tokens = parts > 1 ? p.partition_tokens : p.max_sequence_length;
  const uint32_t group = p.query_heads / p.kv_heads;
  const bool fp8 = p.cache_encoding == LOOM_HIP_KV_CACHE_FP8_E4M3;

  DecodeArgs args{};
  args.query = p.query;
  args.key_cache = p.key_cache;
  args.value_cache = p.value_cache;
  args.key_scales = fp8 ? p.key_scales : nullptr;
  args.value_scales = fp8 ? p.value_scales : nullptr;
  args.block_tables = p.block_tables;
  args.sequence_lengths = p.sequence_lengths;
  args.output = p.output;
  args.lse = p.lse;
  if (parts > 1) {
    args.ws_ml = p.workspace;
    args.ws_o = p.workspace + static_cast<uint64_t>(p.sequences) * p.query_heads * parts * 2;
  }
  args.k_block = p.k_block;
  args.k_page = p.k_page;
  args.k_head = p.k_head;
  args.v_block = p.v_block;
  args.v_page = p.v_page;
  args.v_head = p.v_head;
  args.sequences = p.sequences;
  args.query_heads = p.query_heads;
  args.kv_heads = p.kv_heads;
  args.group = group;
  args.head_size = p.head_size;
  args.value_head_size = p.value_head_size;
  args.block_size = p.block_size;
  args.block_shift = log2u(p.block_size);
  args.max_blocks = p.max_blocks_per_sequence;
  args.partition_tokens = partition_tokens;
  args.parts = static_cast<uint32_t>(parts);
  args.scale_stride = p.scale_stride;
  args.score_scale_log2 = p.scale * kLog2e;
  g_launch_kernel = "";
  g_launch_pairs = false;

  int status = LOOM_HIP_SUCCESS;
  bool use_narrow = false, use_mfma = false, use_heads = false;
  if constexpr (!std::is_same<QE, F32Elem>::value) {
    use_heads = heads_stream_eligible(p, parts);
    use_narrow = !use_heads && narrow_stream_eligible(p, parts, group);
    use_mfma = !use_heads && !use_narrow && mfma_eligible(p);
  }
  if (use_heads) {
    if constexpr (!std::is_same<QE, F32Elem>::value) {
      const uint64_t grid = parts * p.kv_heads * static_cast<uint64_t>(p.sequences);
      if (grid > static_cast<uint64_t>(std::numeric_limits<int>::max()))
        return fail(LOOM_HIP_UNSUPPORTED, "paged decode grid exceeds the launch limit");
      args.grid_y = p.kv_heads;
      if (p.head_size == 64) {
        status = fp8 ? launch_stream_heads<QE, true, 64>(args, grid, group, stream)
                     : launch_stream_heads<QE, false, 64>(args, grid, group, stream);
      } else {
        status = fp8 ? launch_stream_heads<QE, true, kDim>(args, grid, group, stream)
                     : launch_stream_heads<QE, false, kDim>(args, grid, group, stream);
      }
    }
  } else if (use_narrow) {
    if constexpr (!std::is_same<QE, F32Elem>::value) {
      // Head size 64 or 256, native or FP8 cache: the streaming kernel, in the
      // launch shapes of the head-size-128 path below.
      const uint64_t grid = parts * p.kv_heads * static_cast<uint64_t>(p.sequences);
      if (grid > static_cast<uint64_t>(std::numeric_limits<int>::max()))
        return fail(LOOM_HIP_UNSUPPORTED, "paged decode grid exceeds the launch limit");
      args.grid_y = p.kv_heads;
      const uint32_t steps = (partition_tokens + kStep - 1) / kStep;
      // Each KV head's token rows contiguous (HND): steps cover whole lines.
      const bool dense_rows = p.k_page == p.head_size && p.v_page == p.value_head_size;
      if (p.head_size == 80) {
        status = fp8 ? launch_stream_rot<QE, true, 80>(args, grid, steps, dense_rows, stream)
                     : launch_stream_rot<QE, false, 80>(args, grid, steps, dense_rows, stream);
      } else if (p.head_size == 96) {
        status = fp8 ? launch_stream_rot<QE, true, 96>(args, grid, steps, dense_rows, stream)
                     : launch_stream_rot<QE, false, 96>(args, grid, steps, dense_rows, stream);
      } else if (p.head_size == 112) {
        status = fp8 ? launch_stream_rot<QE, true, 112>(args, grid, steps, dense_rows, stream)
                     : launch_stream_rot<QE, false, 112>(args, grid, steps, dense_rows, stream);
      } else if (p.head_size == 256) {
        // 32 KiB of LDS per wave: two items per grouped workgroup, and the
        // 4-wave split (129 KiB, one workgroup per CU) only for grids under
        // 4 items per CU (measured: 1024-2048 items ran 11-15% faster as
        // one wave per item; 128 items 1.6x slower).
        if (grid >= 4096) {
          status = fp8 ? launch_stream_group<QE, true, 256, 2>(args, grid, stream)
                       : launch_stream_group<QE, false, 256, 2>(args, grid, stream);
        } else if (grid >= 1024 || steps < 8) {
          status = fp8 ? launch_stream<QE, true, 1, 1, 256>(args, grid, stream)
                       : launch_stream<QE, false, 1, 1, 256>(args, grid, stream);
        } else {
          status = fp8 ? launch_stream<QE, true, 4, 1, 256>(args, grid, stream)
                       : launch_stream<QE, false, 4, 1, 256>(args, grid, stream);
        }
      } else if (group > 16) {
        status = fp8 ? launch_stream_heads2<QE, true, 64>(args, grid, stream)
                     : launch_stream_heads2<QE, false, 64>(args, grid, stream);
      } else if (grid >= 4096 || (grid >= 1024 && steps >= 8)) {
        status = fp8 ? (dense_rows ? launch_stream_group<QE, true, 64, kStreamGroupFp8, 1>(args, grid, stream)
                                   : launch_stream_group<QE, true, 64, kStreamGroupFp8>(args, grid, stream))
                     : launch_stream_group<QE, false, 64>(args, grid, stream);
      } else if (steps < 8) {
        status = fp8 ? (dense_rows ? launch_stream<QE, true, 1, 1, 64, 1>(args, grid, stream)
                                   : launch_stream<QE, true, 1, 1, 64>(args, grid, stream))
                     : launch_stream<QE, false, 1, 1, 64>(args, grid, stream);
      } else {
        status = fp8 ? (dense_rows ? launch_stream<QE, true, 4, 1, 64, 1>(args, grid, stream)
                                   : launch_stream<QE, true, 4, 1, 64>(args, grid, stream))
                     : launch_stream<QE, false, 4, 1, 64>(args, grid, stream);
      }
    }
  } else if (use_mfma) {
    if constexpr (!std::is_same<QE, F32Elem>::value) {
    const uint64_t grid = parts * p.kv_heads * static_cast<uint64_t>(p.sequences);
    if (grid > static_cast<uint64_t>(std::numeric_limits<int>::max()))
      return fail(LOOM_HIP_UNSUPPORTED, "paged decode grid exceeds the launch limit");
    args.grid_y = p.kv_heads;
    const uint32_t chunks = (partition_tokens + kChunk - 1) / kChunk;
    const uint32_t steps = (partition_tokens + kStep - 1) / kStep;
    if (stream_eligible(p, parts, group)) {
      // One wave per item, four items (adjacent KV heads) per workgroup, for
      // grids of 4096 items or more, and from 1024 items (4 per CU) when
      // partitions have at least 8 steps (measured 10% faster there than the
      // 4-wave split). Smaller grids split each partition over 4 waves when
      // that leaves at least 2 steps per wave, else run one wave per
      // workgroup: there the number of CUs in use matters more than
      // co-locating heads. (16-wave groups measured slower: they add no CUs,
      // only contention within one.)
      if (group > 16) {
        status = fp8 ? launch_stream_heads2<QE, true, kDim>(args, grid, stream)
                     : launch_stream_heads2<QE, false, kDim>(args, grid, stream);
      } else if (grid >= 4096 || (grid >= 1024 && steps >= 8)) {
        // The library's own split runs its items in index order with each
        // item's first block IDs loaded alongside its length (C2 decode
        // 18.3-18.5 -> 17.5-17.7 us).
        status = fp8 && pair_eligible(args, 4, true)
                                      ? launch_stream_group<QE, true, kDim, 4>(args, grid, stream)
                 : fp8                ? launch_stream_group<QE, true, kDim, kStreamGroupFp8>(args, grid, stream)
                 : p.direct_schedule ? launch_stream_group<QE, false, kDim, kStreamGroup, -1, true>(args, grid, stream)
                                     : launch_stream_group<QE, false>(args, grid, stream);
      } else if (steps < 8) {
        status = fp8 ? launch_stream<QE, true, 1>(args, grid, stream) : launch_stream<QE, false, 1>(args, grid, stream);
      } else {
        status = fp8 ? launch_stream<QE, true, 4>(args, grid, stream) : launch_stream<QE, false, 4>(args, grid, stream);
      }
    } else if (group > 16) {
      status = fp8 ? launch_mfma_waves<QE, true, 2>(args, grid, chunks, stream)
                   : launch_mfma_waves<QE, false, 2>(args, grid, chunks, stream);
    } else {
      status = fp8 ? launch_mfma_waves<QE, true, 1>(args, grid, chunks, stream)
                   : launch_mfma_waves<QE, false, 1>(args, grid, chunks, stream);
    }
    }
  } else {
    const uint64_t n_hc = (group + kVecHeads - 1) / kVecHeads;
    const uint64_t dv_tile = 64ULL * (fp8 ? vector_dims_per_lane<Fp8Elem>(args) : vector_dims_per_lane<QE>(args));
    const uint64_t n_dvt = (p.value_head_size + dv_tile - 1) / dv_tile;
    const uint64_t gy = static_cast<uint64_t>(p.kv_heads) * n_hc * n_dvt;
    const uint64_t grid = parts * gy * p.sequences;
    if (gy > std::numeric_limits<uint32_t>::max() ||
        grid > static_cast<uint64_t>(std::numeric_limits<int>::max()))
      return fail(LOOM_HIP_UNSUPPORTED, "paged decode grid exceeds the launch limit");
    args.grid_y = static_cast<uint32_t>(gy);
    status = fp8 ? launch_vector<QE, Fp8Elem>(args, grid, stream)
                 : launch_vector<QE, QE>(args, grid, stream);
  }
  if (status != LOOM_HIP_SUCCESS) return fail(status, "decode kernel launch failed");
  g_last_family = use_heads || use_narrow ? "mfma-stream"
                  : use_mfma             ? (stream_eligible(p, parts, group) ? "mfma-stream" : "mfma")
                                         : "vector";
  if (parts > 1) {
    DecodeArgs merge = args;
    if (g_launch_pairs) {  // one state per two partitions
      merge.parts = (args.parts + 1U) / 2U;
      merge.partition_tokens = 2U * args.partition_tokens;
    }
    status = launch_merge<QE>(merge, p.sequences * p.query_heads, stream);
    if (status != LOOM_HIP_SUCCESS) return fail(status, "merge kernel launch failed");
  }
  return LOOM_HIP_SUCCESS;
}

int device_available() {
  int count = 0;
  if (hipGetDeviceCount(&count) != hipSuccess || count <= 0) {
    (void)hipGetLastError();
    return fail(LOOM_HIP_UNAVAILABLE, "no HIP device is available");
  }
  return LOOM_HIP_SUCCESS;
}

// Split-K scratch of the no-allocation entry point: one array per device,
// resident from module load until the process ends. Host code never uses the
// array's name as an address: the per-device address comes from
// hipGetSymbolAddress, called once per device with that device current.
__device__ __align__(256) float scratch[LOOM_HIP_STATIC_WORKSPACE_ELEMENTS];

constexpr int kMaxScratchDevices = 64;
std::mutex g_scratch_mu;
float* g_scratch_ptr[kMaxScratchDevices] = {};

int scratch_address(hipStream_t stream, float** out) {
  int dev = -1;
  if (hipGetDevice(&dev) != hipSuccess) {
    (void)hipGetLastError();
    return fail(LOOM_HIP_UNAVAILABLE, "no current HIP device");
  }
  // The array's address is the current device's; the launch stream must be
  // on that device too (the null, legacy and per-thread handles always are).
  if (stream != nullptr && stream != hipStreamLegacy && stream != hipStreamPerThread) {
    hipDevice_t stream_dev = -1;
    if (hipStreamGetDevice(stream, &stream_dev) != hipSuccess) {
      (void)hipGetLastError();
      return fail(LOOM_HIP_INVALID_ARGUMENT, "the stream's device cannot be queried");
    }
    if (stream_dev != dev)
      return fail(LOOM_HIP_INVALID_ARGUMENT, "no-allocation calls need the stream on the current device");
  }
  if (dev < 0 || dev >= kMaxScratchDevices)
    return fail(LOOM_HIP_UNSUPPORTED, "device ordinal beyond the static workspace table");
  std::lock_guard<std::mutex> lock(g_scratch_mu);
  if (g_scratch_ptr[dev] == nullptr) {
    void* ptr = nullptr;
    if (hipGetSymbolAddress(&ptr, HIP_SYMBOL(scratch)) != hipSuccess || ptr == nullptr) {
      (void)hipGetLastError();
      return fail(LOOM_HIP_LAUNCH_ERROR, "hipGetSymbolAddress of the static workspace failed");
    }
    g_scratch_ptr[dev] = static_cast<float*>(ptr);
  }
  *out = g_scratch_ptr[dev];
  return LOOM_HIP_SUCCESS;
}

// Internal split of single-partition calls. A call whose (sequence, KV head)
// items cannot fill the CUs (C2's 64 items put 4 waves on each of 64 of the
// 256 CUs, and 64 CUs pull at most ~3.1 TB/s) is run as a split-K call with
// partial states in a library-held slot, then merged into the caller's
// output: the caller still passes no workspace. The slots are one static
// array per device, kPoolSlots slots of kPoolSlotElements F32 elements
// (64 MiB per device, resident until the process ends). The first
// kPoolSlots streams that make such a call on a device each own one slot
// until the process ends; calls on one stream use its slot in stream order,
// so no call waits for another and no event is recorded (an event record
// after every call measured 3 us per call on C2, 1 us without its system
// fence). A stream handle names a live stream object: a handle can only come
// back after its stream was destroyed and its work drained, so a reused
// handle inherits an idle slot. Calls from further streams, from
// hipStreamPerThread (one handle for many streams), under stream capture (a
// graph would keep the slot's address), or made while the environment
// variable LOOM_HIP_INTERNAL_SPLIT is "0" run as one partition per item.
constexpr int kPoolSlots = 4;
constexpr uint64_t kPoolSlotElements = 4ULL * 1024ULL * 1024ULL;
__device__ __align__(256) float split_pool[kPoolSlots * kPoolSlotElements];

struct DevicePool {
  float* base = nullptr;
  bool unavailable = false;
  int owners = 0;
  hipStream_t owner[kPoolSlots] = {};
};

std::mutex g_pool_mu;
DevicePool g_pool[kMaxScratchDevices];

uint32_t split_k_partition_tokens(uint32_t sequences, uint32_t query_heads, uint32_t kv_heads,
                                  uint32_t head_size, uint32_t value_head_size,
                                  uint32_t max_sequence_length);

// Partition size of the internal split, or 0 when the call stays whole: the
// split entry points' policy (fewer items than CUs) for contexts of at least
// 2048 tokens, with partitions doubled until a sequence has at most 256 and
// the states fit one slot. Measured as whole calls (us, one partition against
// the split): 16 items x 1024 tokens 15.2 against 17.0 (the merge launch
// costs more than the split gains), C2's 64 x 2048 28.2 against 20.4,
// 64 x 8192 99.6 against 53.7, 4 MQA items x 32768 1423 against 30.0.
uint32_t internal_partition_tokens(const Problem& p) {
  if (p.max_sequence_length < 2048) return 0;
  uint64_t t = split_k_partition_tokens(p.sequences, p.query_heads, p.kv_heads, p.head_size, p.value_head_size,
                                        p.max_sequence_length);
  if (t == 0) return 0;
  const uint64_t len = p.max_sequence_length;
  const uint64_t row = static_cast<uint64_t>(p.sequences) * p.query_heads * (p.value_head_size + 2ULL);
  while (t < len && ((len + t - 1) / t > 256 || row * ((len + t - 1) / t) > kPoolSlotElements)) t *= 2;
  const uint64_t parts = (len + t - 1) / t;
  if (parts < 2 || row * parts > kPoolSlotElements) return 0;
  return static_cast<uint32_t>(t);
}

bool internal_split_enabled() {
  const char* v = getenv("LOOM_HIP_INTERNAL_SPLIT");
  return v == nullptr || strcmp(v, "0") != 0;
}

// The slot of `stream` on the current device, claiming a free one on the
// stream's first call (claim = false: only whether it has or would get one,
// non-null then); nullptr when the call runs as one partition.
float* stream_slot(hipStream_t stream, bool claim = true) {
  if (stream == hipStreamPerThread) return nullptr;
  int dev = -1;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= kMaxScratchDevices) {
    (void)hipGetLastError();
    return nullptr;
  }
  hipStreamCaptureStatus capture = hipStreamCaptureStatusNone;
  if (hipStreamIsCapturing(stream, &capture) != hipSuccess) {
    (void)hipGetLastError();
    return nullptr;
  }
  if (capture != hipStreamCaptureStatusNone) return nullptr;
  if (stream != nullptr && stream != hipStreamLegacy) {
    hipDevice_t stream_dev = -1;
    if (hipStreamGetDevice(stream, &stream_dev) != hipSuccess || stream_dev != dev) {
      (void)hipGetLastError();
      return nullptr;
    }
  }
  std::lock_guard<std::mutex> lock(g_pool_mu);
  DevicePool& pool = g_pool[dev];
  if (pool.unavailable) return nullptr;
  if (pool.base == nullptr) {
    void* ptr = nullptr;
    if (hipGetSymbolAddress(&ptr, HIP_SYMBOL(split_pool)) != hipSuccess || ptr == nullptr) {
      (void)hipGetLastError();
      pool.unavailable = true;
      return nullptr;
    }
    pool.base = static_cast<float*>(ptr);
  }
  int pick = -1;
  for (int i = 0; i < pool.owners && pick < 0; ++i)
    if (pool.owner[i] == stream) pick = i;
  if (pick < 0) {
    if (pool.owners == kPoolSlots) return nullptr;
    if (!claim) return pool.base;
    pick = pool.owners++;
    pool.owner[pick] = stream;
  }
  return pool.base + static_cast<uint64_t>(pick) * kPoolSlotElements;
}

int run(Problem p, void* stream) {
  int status = validate(p);
  if (status != LOOM_HIP_SUCCESS) return status;
  status = device_available();
  if (status != LOOM_HIP_SUCCESS) return status;
  if (p.static_workspace) {
    const uint64_t parts = parts_for(p.max_sequence_length, p.partition_tokens);
    if (parts > 1) {
      status = scratch_address(static_cast<hipStream_t>(stream), &p.workspace);
      if (status != LOOM_HIP_SUCCESS) return status;
      p.workspace_elements = LOOM_HIP_STATIC_WORKSPACE_ELEMENTS;
    }
  }
  hipStream_t s = static_cast<hipStream_t>(stream);
  uint32_t internal = 0;
  if (!p.static_workspace && parts_for(p.max_sequence_length, p.partition_tokens) == 1) {
    const uint32_t t = internal_partition_tokens(p);
    float* slot = t != 0 && internal_split_enabled() ? stream_slot(s) : nullptr;
    if (slot != nullptr) {
      p.partition_tokens = t;
      p.workspace = slot;
      p.workspace_elements = kPoolSlotElements;
      p.direct_schedule = true;
      internal = t;
    }
  }
  switch (p.dtype) {
    case kF32: status = run_typed<F32Elem>(p, s); break;
    case kF16: status = run_typed<F16Elem>(p, s); break;
    default: status = run_typed<Bf16Elem>(p, s); break;
  }
  if (status == LOOM_HIP_SUCCESS) {
    g_last_internal_split = internal;
    g_last_kernel = g_launch_kernel;
    g_decode_launches.fetch_add(1, std::memory_order_relaxed);
  }
  return status;
}

// Split-K policy of the reference-compatible split entry points. The shape
// splits when there are fewer (sequence, KV head) work items than the 256
// CUs and the context reaches 512 tokens: partitions of at least 64 tokens
// (a multiple of 32), sized so that the grid reaches about 1024 items.
// Measured as whole calls (us, by partition size): 64 items x 2048 tokens
// 64: 22.3, 128: 20.4, 256: 21.4; 64 x 8192 256: 55.1, 512: 53.7; from 256
// items (x 2048-4096 tokens) every split measured 1-3% slower than none.
uint32_t split_k_partition_tokens(uint32_t sequences, uint32_t query_heads, uint32_t kv_heads,
                                  uint32_t head_size, uint32_t value_head_size,
                                  uint32_t max_sequence_length) {
  if (sequences == 0 || query_heads == 0 || kv_heads == 0 || head_size == 0 ||
      value_head_size == 0 || max_sequence_length == 0 || query_heads % kv_heads != 0)
    return 0;
  const uint64_t work = static_cast<uint64_t>(sequences) * kv_heads;
  if (work >= 256 || max_sequence_length < 512) return 0;
  const uint64_t want_parts = (1024 + work - 1) / work;
  uint64_t tokens = (max_sequence_length + want_parts - 1) / want_parts;
  tokens = ((tokens + kChunk - 1) / kChunk) * kChunk;
  if (tokens < 64) tokens = 64;
  if (parts_for(max_sequence_length, static_cast<uint32_t>(tokens)) < 2) return 0;
  return static_cast<uint32_t>(tokens);
}

Problem base_problem(uint32_t dtype, const void* query, const void* key_cache,
                     const void* value_cache, const int32_t* block_tables,
                     const int32_t* sequence_lengths, void* output, uint32_t sequences,
                     uint32_t query_heads, uint32_t kv_heads, uint32_t head_size,
                     uint32_t value_head_size, uint32_t num_blocks, uint32_t block_size,
                     uint64_t key_block_stride, uint64_t value_block_stride,
                     uint32_t max_blocks_per_sequence, uint32_t max_sequence_length, float scale) {
  Problem p{};
  p.dtype = dtype;
  p.query = query;
  p.key_cache = key_cache;
  p.value_cache = value_cache;
  p.block_tables = block_tables;
  p.sequence_lengths = sequence_lengths;
  p.output = output;
  p.sequences = sequences;
  p.query_heads = query_heads;
  p.kv_heads = kv_heads;
  p.head_size = head_size;
  p.value_head_size = value_head_size;
  p.num_blocks = num_blocks;
  p.block_size = block_size;
  p.cache_encoding = LOOM_HIP_KV_CACHE_NATIVE;
  p.k_block = key_block_stride;
  p.k_page = static_cast<uint64_t>(kv_heads) * head_size;
  p.k_head = head_size;
  p.v_block = value_block_stride;
  p.v_page = static_cast<uint64_t>(kv_heads) * value_head_size;
  p.v_head = value_head_size;
  p.max_blocks_per_sequence = max_blocks_per_sequence;
  p.max_sequence_length = max_sequence_length;
  p.scale = scale;
  return p;
}

// The base ABI requires block strides of at least one dense NHD block
// (paged_decode_attention.cu:1034-1049).
int check_block_strides(const Problem& p) {
  const uint64_t kb = static_cast<uint64_t>(p.block_size) * p.kv_heads * p.head_size;
  const uint64_t vb = static_cast<uint64_t>(p.block_size) * p.kv_heads * p.value_head_size;
  if (p.k_block < kb || p.v_block < vb)
    return fail(LOOM_HIP_INVALID_ARGUMENT, "cache block stride is smaller than one dense NHD block");
  return LOOM_HIP_SUCCESS;
}

int run_base(Problem p, void* stream) {
  if (p.block_size != 0 && p.kv_heads != 0) {
    int status = check_block_strides(p);
    if (status != LOOM_HIP_SUCCESS) return status;
  }
  return run(p, stream);
}

int run_split_k(Problem p, float* workspace, uint64_t workspace_elements, void* stream) {
  const uint32_t tokens = split_k_partition_tokens(p.sequences, p.query_heads, p.kv_heads,
                                                   p.head_size, p.value_head_size,
                                                   p.max_sequence_length);
  if (tokens == 0)
    return fail(LOOM_HIP_INVALID_ARGUMENT, "paged decode shape does not select the split-K path");
  if (workspace == nullptr)
    return fail(LOOM_HIP_INVALID_ARGUMENT, "split-K workspace must be non-null");
  p.partition_tokens = tokens;
  p.workspace = workspace;
  p.workspace_elements = workspace_elements;
  if (p.block_size != 0 && p.kv_heads != 0) {
    int status = check_block_strides(p);
    if (status != LOOM_HIP_SUCCESS) return status;
  }
  return run(p, stream);
}

Problem extended_problem(uint32_t dtype, const void* query, const void* key_cache,
                         const void* value_cache, const float* key_scales,
                         const float* value_scales, const int32_t* block_tables,
                         const int32_t* sequence_lengths, void* output, float* lse,
                         float* workspace, uint64_t workspace_elements, uint32_t sequences,
                         uint32_t query_heads, uint32_t kv_heads, uint32_t head_size,
                         uint32_t value_head_size, uint32_t num_blocks, uint32_t block_size,
                         uint32_t cache_encoding, uint32_t scale_stride, uint64_t kb, uint64_t kp,
                         uint64_t kh, uint64_t vb, uint64_t vp, uint64_t vh,
                         uint32_t max_blocks_per_sequence, uint32_t max_sequence_length,
                         uint32_t partition_tokens, float scale) {
  Problem p{};
  p.dtype = dtype;
  p.query = query;
  p.key_cache = key_cache;
  p.value_cache = value_cache;
  p.key_scales = key_scales;
  p.value_scales = value_scales;
  p.block_tables = block_tables;
  p.sequence_lengths = sequence_lengths;
  p.output = output;
  p.lse = lse;
  p.workspace = workspace;
  p.workspace_elements = workspace_elements;
  p.sequences = sequences;
  p.query_heads = query_heads;
  p.kv_heads = kv_heads;
  p.head_size = head_size;
  p.value_head_size = value_head_size;
  p.num_blocks = num_blocks;
  p.block_size = block_size;
  p.cache_encoding = cache_encoding;
  p.scale_stride = scale_stride;
  p.k_block = kb;
  p.k_page = kp;
  p.k_head = kh;
  p.v_block = vb;
  p.v_page = vp;
  p.v_head = vh;
  p.max_blocks_per_sequence = max_blocks_per_sequence;
  p.max_sequence_length = max_sequence_length;
  p.partition_tokens = partition_tokens;
  p.scale = scale;
  return p;
}

}  // namespace

namespace loom_hip_detail {

int fail(int status, const char* message) { return ::fail(status, message); }

int device_available() { return ::device_available(); }

void count_launch(uint32_t operation) {
  if (operation == LOOM_HIP_PAGED_DECODE_ATTENTION) g_decode_launches.fetch_add(1, std::memory_order_relaxed);
  if (operation == LOOM_HIP_ROPE_PAGED_KV_WRITE) g_rope_launches.fetch_add(1, std::memory_order_relaxed);
}

KernelTimer::KernelTimer(int kernel, void* stream)
    : impl_(timing().enabled.load(std::memory_order_relaxed)
                ? new TimedLaunch(kernel, static_cast<hipStream_t>(stream))
                : nullptr) {}

KernelTimer::~KernelTimer() { delete static_cast<TimedLaunch*>(impl_); }

}  // namespace loom_hip_detail

// ===========================================================================
// C ABI
// ===========================================================================
extern "C" {

const char* loom_hip_status_string(int status) {
  switch (status) {
    case LOOM_HIP_SUCCESS: return "success";
    case LOOM_HIP_INVALID_ARGUMENT: return "invalid argument";
    case LOOM_HIP_UNSUPPORTED: return "unsupported";
    case LOOM_HIP_LAUNCH_ERROR: return "HIP launch error";
    case LOOM_HIP_UNAVAILABLE: return "HIP unavailable";
    default: return "unknown Loom HIP status";
  }
}

const char* loom_hip_backend_name(void) { return "loom-hip"; }

uint32_t loom_hip_abi_version(void) { return 1; }

const char* loom_hip_last_error_message(void) { return g_last_error.c_str(); }

const char* loom_hip_last_kernel_family(void) { return g_last_family; }

uint32_t loom_hip_last_internal_partition_tokens(void) { return g_last_internal_split; }

const char* loom_hip_last_kernel_name(void) { return g_last_kernel; }

int loom_hip_paged_decode_attention_plan(uint32_t dtype, uint32_t sequences, uint32_t query_heads, uint32_t kv_heads,
                                         uint32_t head_size, uint32_t value_head_size, uint32_t max_sequence_length,
                                         uint32_t partition_tokens, void* stream, uint32_t* run_partition_tokens,
                                         uint32_t* internal_split) {
  if (run_partition_tokens == nullptr || internal_split == nullptr)
    return fail(LOOM_HIP_INVALID_ARGUMENT, "plan outputs must be non-null");
  if (dtype > kBf16 || sequences == 0 || query_heads == 0 || kv_heads == 0 || head_size == 0 ||
      value_head_size == 0 || max_sequence_length == 0 || query_heads % kv_heads != 0)
    return fail(LOOM_HIP_INVALID_ARGUMENT, "plan shape is invalid");
  *internal_split = 0;
  *run_partition_tokens = parts_for(max_sequence_length, partition_tokens) > 1 ? partition_tokens : 0;
  if (*run_partition_tokens != 0) return LOOM_HIP_SUCCESS;
  Problem p{};
  p.sequences = sequences;
  p.query_heads = query_heads;
  p.kv_heads = kv_heads;
  p.head_size = head_size;
  p.value_head_size = value_head_size;
  p.max_sequence_length = max_sequence_length;
  const uint32_t t = internal_partition_tokens(p);
  if (t != 0 && internal_split_enabled() && device_available() == LOOM_HIP_SUCCESS &&
      stream_slot(static_cast<hipStream_t>(stream), false) != nullptr) {
    *run_partition_tokens = t;
    *internal_split = 1;
  }
  return LOOM_HIP_SUCCESS;
}

int loom_hip_launch_count(uint32_t operation, uint64_t* count) {
  if ((operation != LOOM_HIP_PAGED_DECODE_ATTENTION && operation != LOOM_HIP_ROPE_PAGED_KV_WRITE) ||
      count == nullptr)
    return fail(LOOM_HIP_INVALID_ARGUMENT, "unknown operator id or null count");
  *count = (operation == LOOM_HIP_PAGED_DECODE_ATTENTION ? g_decode_launches : g_rope_launches)
               .load(std::memory_order_relaxed);
  return LOOM_HIP_SUCCESS;
}

int loom_hip_reset_launch_count(uint32_t operation) {
  if (operation == LOOM_HIP_ROPE_PAGED_KV_WRITE) {
    g_rope_launches.store(0, std::memory_order_relaxed);
    return LOOM_HIP_SUCCESS;
  }
  if (operation != LOOM_HIP_PAGED_DECODE_ATTENTION)
    return fail(LOOM_HIP_INVALID_ARGUMENT, "unknown operator id");
  g_decode_launches.store(0, std::memory_order_relaxed);
  return LOOM_HIP_SUCCESS;
}

int loom_hip_kernel_timing_enable(uint32_t enable) {
  TimingState& t = timing();
  std::lock_guard<std::mutex> lock(t.mu);
  t.enabled = enable != 0;
  for (int k = 0; k < kTimedKernels; ++k) {
    for (auto& e : t.pending[k]) {
      (void)hipEventSynchronize(e.second);
      (void)hipEventDestroy(e.first);
      (void)hipEventDestroy(e.second);
    }
    t.pending[k].clear();
    t.total_ms[k] = 0.0;
    t.launches[k] = 0;
  }
  return LOOM_HIP_SUCCESS;
}

int loom_hip_kernel_timing_read(uint32_t kernel, double* total_ms, uint64_t* launches) {
  if (kernel >= static_cast<uint32_t>(kTimedKernels) || total_ms == nullptr || launches == nullptr)
    return fail(LOOM_HIP_INVALID_ARGUMENT, "unknown kernel id or null output");
  TimingState& t = timing();
  std::lock_guard<std::mutex> lock(t.mu);
  for (auto& e : t.pending[kernel]) {
    float ms = 0.0f;
    if (hipEventSynchronize(e.second) == hipSuccess &&
        hipEventElapsedTime(&ms, e.first, e.second) == hipSuccess) {
      t.total_ms[kernel] += ms;
      t.launches[kernel] += 1;
    }
    (void)hipEventDestroy(e.first);
    (void)hipEventDestroy(e.second);
  }
  t.pending[kernel].clear();
  *total_ms = t.total_ms[kernel];
  *launches = t.launches[kernel];
  return LOOM_HIP_SUCCESS;
}

int loom_hip_paged_decode_attention_supports(
    uint32_t dtype, uint32_t cache_encoding, uint32_t sequences, uint32_t query_heads,
    uint32_t kv_heads, uint32_t head_size, uint32_t value_head_size, uint32_t num_blocks,
    uint32_t block_size, uint32_t max_blocks_per_sequence, uint32_t max_sequence_length,
    float scale, const char** reason, const char** kernel_family) {
  const char* why = "supported";
  int status = LOOM_HIP_SUCCESS;
  if (dtype != kF32 && dtype != kF16 && dtype != kBf16) {
    status = LOOM_HIP_UNSUPPORTED;
    why = "HIP paged decode attention supports F32, FP16 and BF16 queries";
  } else if (cache_encoding > LOOM_HIP_KV_CACHE_FP8_E4M3) {
    status = LOOM_HIP_UNSUPPORTED;
    why = "HIP paged decode attention supports native and FP8 E4M3 K/V caches";
  } else if (sequences == 0 || query_heads == 0 || kv_heads == 0 || head_size == 0 ||
             value_head_size == 0 || num_blocks == 0 || block_size == 0 ||
             max_blocks_per_sequence == 0 || max_sequence_length == 0) {
    status = LOOM_HIP_INVALID_ARGUMENT;
    why = "paged decode dimensions must be non-zero";
  } else if (query_heads % kv_heads != 0) {
    status = LOOM_HIP_INVALID_ARGUMENT;
    why = "query head count must be divisible by KV head count";
  } else if (!std::isfinite(scale) || scale <= 0.0f) {
    status = LOOM_HIP_INVALID_ARGUMENT;
    why = "attention scale must be finite and positive";
  } else if (static_cast<uint64_t>(max_sequence_length) >
             static_cast<uint64_t>(block_size) * max_blocks_per_sequence) {
    status = LOOM_HIP_INVALID_ARGUMENT;
    why = "maximum sequence length exceeds block-table capacity";
  } else if (static_cast<uint64_t>(sequences) * query_heads >
             static_cast<uint64_t>(std::numeric_limits<int>::max())) {
    status = LOOM_HIP_UNSUPPORTED;
    why = "paged decode shape exceeds the HIP launch grid";
  }
  if (reason != nullptr) *reason = why;
  if (kernel_family != nullptr) {
    *kernel_family = status != LOOM_HIP_SUCCESS ? ""
                     : narrow_shape(dtype, cache_encoding, head_size, value_head_size, query_heads, kv_heads,
                                    block_size) ||
                               wide_shape(dtype, cache_encoding, head_size, value_head_size, query_heads, kv_heads,
                                          block_size) ||
                               rot_shape(dtype, cache_encoding, head_size, value_head_size, query_heads, kv_heads,
                                         block_size) ||
                               heads_shape(dtype, cache_encoding, head_size, value_head_size, query_heads, kv_heads,
                                           block_size)
                         ? "mfma-stream"
                     : !mfma_shape(dtype, head_size, value_head_size, query_heads, kv_heads, block_size)
                         ? "vector"
                         : (query_heads / kv_heads <= 32 && block_size >= kStep) ? "mfma-stream"
                                                                                  : "mfma";
  }
  return status;
}

int loom_hip_paged_decode_attention_f32(
    const float* query, const float* key_cache, const float* value_cache,
    const int32_t* block_tables, const int32_t* sequence_lengths, float* output,
    uint32_t sequences, uint32_t query_heads, uint32_t kv_heads, uint32_t head_size,
    uint32_t value_head_size, uint32_t num_blocks, uint32_t block_size,
    uint64_t key_block_stride, uint64_t value_block_stride, uint32_t max_blocks_per_sequence,
    uint32_t max_sequence_length, float scale, void* stream) {
  return run_base(base_problem(kF32, query, key_cache, value_cache, block_tables,
                               sequence_lengths, output, sequences, query_heads, kv_heads,
                               head_size, value_head_size, num_blocks, block_size,
                               key_block_stride, value_block_stride, max_blocks_per_sequence,
                               max_sequence_length, scale),
                  stream);
}

int loom_hip_paged_decode_attention_f16(
    const uint16_t* query, const uint16_t* key_cache, const uint16_t* value_cache,
    const int32_t* block_tables, const int32_t* sequence_lengths, uint16_t* output,
    uint32_t sequences, uint32_t query_heads, uint32_t kv_heads, uint32_t head_size,
    uint32_t value_head_size, uint32_t num_blocks, uint32_t block_size,
    uint64_t key_block_stride, uint64_t value_block_stride, uint32_t max_blocks_per_sequence,
    uint32_t max_sequence_length, float scale, void* stream) {
  return run_base(base_problem(kF16, query, key_cache, value_cache, block_tables,
                               sequence_lengths, output, sequences, query_heads, kv_heads,
                               head_size, value_head_size, num_blocks, block_size,
                               key_block_stride, value_block_stride, max_blocks_per_sequence,
                               max_sequence_length, scale),
                  stream);
}

int loom_hip_paged_decode_attention_bf16(
    const uint16_t* query, const uint16_t* key_cache, const uint16_t* value_cache,
    const int32_t* block_tables, const int32_t* sequence_lengths, uint16_t* output,
    uint32_t sequences, uint32_t query_heads, uint32_t kv_heads, uint32_t head_size,
    uint32_t value_head_size, uint32_t num_blocks, uint32_t block_size,
    uint64_t key_block_stride, uint64_t value_block_stride, uint32_t max_blocks_per_sequence,
    uint32_t max_sequence_length, float scale, void* stream) {
  return run_base(base_problem(kBf16, query, key_cache, value_cache, block_tables,
                               sequence_lengths, output, sequences, query_heads, kv_heads,
                               head_size, value_head_size, num_blocks, block_size,
                               key_block_stride, value_block_stride, max_blocks_per_sequence,
                               max_sequence_length, scale),
                  stream);
}

uint64_t loom_hip_paged_decode_attention_split_k_workspace_elements(
    uint32_t sequences, uint32_t query_heads, uint32_t kv_heads, uint32_t head_size,
    uint32_t value_head_size, uint32_t max_sequence_length) {
  const uint32_t tokens = split_k_partition_tokens(sequences, query_heads, kv_heads, head_size,
                                                   value_head_size, max_sequence_length);
  if (tokens == 0) return 0;
  return static_cast<uint64_t>(sequences) * query_heads * parts_for(max_sequence_length, tokens) *
         (value_head_size + 2ULL);
}

int loom_hip_paged_decode_attention_split_k_f32(
    const float* query, const float* key_cache, const float* value_cache,
    const int32_t* block_tables, const int32_t* sequence_lengths, float* output,
    float* workspace, uint64_t workspace_elements, uint32_t sequences, uint32_t query_heads,
    uint32_t kv_heads, uint32_t head_size, uint32_t value_head_size, uint32_t num_blocks,
    uint32_t block_size, uint64_t key_block_stride, uint64_t value_block_stride,
    uint32_t max_blocks_per_sequence, uint32_t max_sequence_length, float scale,
    void* stream) {
  return run_split_k(base_problem(kF32, query, key_cache, value_cache, block_tables,
                                  sequence_lengths, output, sequences, query_heads, kv_heads,
                                  head_size, value_head_size, num_blocks, block_size,
                                  key_block_stride, value_block_stride, max_blocks_per_sequence,
                                  max_sequence_length, scale),
                     workspace, workspace_elements, stream);
}

int loom_hip_paged_decode_attention_split_k_f16(
    const uint16_t* query, const uint16_t* key_cache, const uint16_t* value_cache,
    const int32_t* block_tables, const int32_t* sequence_lengths, uint16_t* output,
    float* workspace, uint64_t workspace_elements, uint32_t sequences, uint32_t query_heads,
    uint32_t kv_heads, uint32_t head_size, uint32_t value_head_size, uint32_t num_blocks,
    uint32_t block_size, uint64_t key_block_stride, uint64_t value_block_stride,
    uint32_t max_blocks_per_sequence, uint32_t max_sequence_length, float scale,
    void* stream) {
  return run_split_k(base_problem(kF16, query, key_cache, value_cache, block_tables,
                                  sequence_lengths, output, sequences, query_heads, kv_heads,
                                  head_size, value_head_size, num_blocks, block_size,
                                  key_block_stride, value_block_stride, max_blocks_per_sequence,
                                  max_sequence_length, scale),
                     workspace, workspace_elements, stream);
}

int loom_hip_paged_decode_attention_split_k_bf16(
    const uint16_t* query, const uint16_t* key_cache, const uint16_t* value_cache,
    const int32_t* block_tables, const int32_t* sequence_lengths, uint16_t* output,
    float* workspace, uint64_t workspace_elements, uint32_t sequences, uint32_t query_heads,
    uint32_t kv_heads, uint32_t head_size, uint32_t value_head_size, uint32_t num_blocks,
    uint32_t block_size, uint64_t key_block_stride, uint64_t value_block_stride,
    uint32_t max_blocks_per_sequence, uint32_t max_sequence_length, float scale,
    void* stream) {
  return run_split_k(base_problem(kBf16, query, key_cache, value_cache, block_tables,
                                  sequence_lengths, output, sequences, query_heads, kv_heads,
                                  head_size, value_head_size, num_blocks, block_size,
                                  key_block_stride, value_block_stride, max_blocks_per_sequence,
                                  max_sequence_length, scale),
                     workspace, workspace_elements, stream);
}

uint64_t loom_hip_paged_decode_attention_extended_workspace_elements(
    uint32_t sequences, uint32_t query_heads, uint32_t value_head_size,
    uint32_t max_sequence_length, uint32_t partition_tokens) {
  if (max_sequence_length == 0) return 0;
  const uint64_t parts = parts_for(max_sequence_length, partition_tokens);
  if (parts <= 1) return 0;
  return static_cast<uint64_t>(sequences) * query_heads * parts * (value_head_size + 2ULL);
}

int loom_hip_paged_decode_attention_extended_f32(
    const float* query, const void* key_cache, const void* value_cache, const float* key_scales,
    const float* value_scales, const int32_t* block_tables, const int32_t* sequence_lengths,
    float* output, float* lse, float* workspace, uint64_t workspace_elements,
    uint32_t sequences, uint32_t query_heads, uint32_t kv_heads, uint32_t head_size,
    uint32_t value_head_size, uint32_t num_blocks, uint32_t block_size,
    uint32_t cache_encoding, uint32_t scale_stride, uint64_t key_block_stride,
    uint64_t key_page_stride, uint64_t key_head_stride, uint64_t value_block_stride,
    uint64_t value_page_stride, uint64_t value_head_stride, uint32_t max_blocks_per_sequence,
    uint32_t max_sequence_length, uint32_t partition_tokens, float scale, void* stream) {
  return run(extended_problem(kF32, query, key_cache, value_cache, key_scales, value_scales,
                              block_tables, sequence_lengths, output, lse, workspace,
                              workspace_elements, sequences, query_heads, kv_heads, head_size,
                              value_head_size, num_blocks, block_size, cache_encoding,
                              scale_stride, key_block_stride, key_page_stride, key_head_stride,
                              value_block_stride, value_page_stride, value_head_stride,
                              max_blocks_per_sequence, max_sequence_length, partition_tokens,
                              scale),
             stream);
}

int loom_hip_paged_decode_attention_extended_f16(
    const uint16_t* query, const void* key_cache, const void* value_cache,
    const float* key_scales, const float* value_scales, const int32_t* block_tables,
    const int32_t* sequence_lengths, uint16_t* output, float* lse, float* workspace,
    uint64_t workspace_elements, uint32_t sequences, uint32_t query_heads, uint32_t kv_heads,
    uint32_t head_size, uint32_t value_head_size, uint32_t num_blocks, uint32_t block_size,
    uint32_t cache_encoding, uint32_t scale_stride, uint64_t key_block_stride,
    uint64_t key_page_stride, uint64_t key_head_stride, uint64_t value_block_stride,
    uint64_t value_page_stride, uint64_t value_head_stride, uint32_t max_blocks_per_sequence,
    uint32_t max_sequence_length, uint32_t partition_tokens, float scale, void* stream) {
  return run(extended_problem(kF16, query, key_cache, value_cache, key_scales, value_scales,
                              block_tables, sequence_lengths, output, lse, workspace,
                              workspace_elements, sequences, query_heads, kv_heads, head_size,
                              value_head_size, num_blocks, block_size, cache_encoding,
                              scale_stride, key_block_stride, key_page_stride, key_head_stride,
                              value_block_stride, value_page_stride, value_head_stride,
                              max_blocks_per_sequence, max_sequence_length, partition_tokens,
                              scale),
             stream);
}

int loom_hip_paged_decode_attention_extended_bf16(
    const uint16_t* query, const void* key_cache, const void* value_cache,
    const float* key_scales, const float* value_scales, const int32_t* block_tables,
    const int32_t* sequence_lengths, uint16_t* output, float* lse, float* workspace,
    uint64_t workspace_elements, uint32_t sequences, uint32_t query_heads, uint32_t kv_heads,
    uint32_t head_size, uint32_t value_head_size, uint32_t num_blocks, uint32_t block_size,
    uint32_t cache_encoding, uint32_t scale_stride, uint64_t key_block_stride,
    uint64_t key_page_stride, uint64_t key_head_stride, uint64_t value_block_stride,
    uint64_t value_page_stride, uint64_t value_head_stride, uint32_t max_blocks_per_sequence,
    uint32_t max_sequence_length, uint32_t partition_tokens, float scale, void* stream) {
  return run(extended_problem(kBf16, query, key_cache, value_cache, key_scales, value_scales,
                              block_tables, sequence_lengths, output, lse, workspace,
                              workspace_elements, sequences, query_heads, kv_heads, head_size,
                              value_head_size, num_blocks, block_size, cache_encoding,
                              scale_stride, key_block_stride, key_page_stride, key_head_stride,
                              value_block_stride, value_page_stride, value_head_stride,
                              max_blocks_per_sequence, max_sequence_length, partition_tokens,
                              scale),
             stream);
}

int loom_hip_paged_decode_attention_extended_no_alloc(
    uint32_t dtype, const void* query, const void* key_cache, const void* value_cache,
    const float* key_scales, const float* value_scales, const int32_t* block_tables,
    const int32_t* sequence_lengths, void* output, float* lse, uint32_t sequences,
    uint32_t query_heads, uint32_t kv_heads, uint32_t head_size, uint32_t value_head_size,
    uint32_t num_blocks, uint32_t block_size, uint32_t cache_encoding, uint32_t scale_stride,
    uint64_t key_block_stride, uint64_t key_page_stride, uint64_t key_head_stride,
    uint64_t value_block_stride, uint64_t value_page_stride, uint64_t value_head_stride,
    uint32_t max_blocks_per_sequence, uint32_t max_sequence_length, uint32_t partition_tokens,
    float scale, void* stream) {
  Problem p = extended_problem(dtype, query, key_cache, value_cache, key_scales, value_scales,
                               block_tables, sequence_lengths, output, lse, nullptr, 0, sequences,
                               query_heads, kv_heads, head_size, value_head_size, num_blocks,
                               block_size, cache_encoding, scale_stride, key_block_stride,
                               key_page_stride, key_head_stride, value_block_stride,
                               value_page_stride, value_head_stride, max_blocks_per_sequence,
                               max_sequence_length, partition_tokens, scale);
  p.static_workspace = true;
  return run(p, stream);
}

}  // extern "C"

#ifdef LOOM_HIP_WAVE_TRACE
// Profiling builds only (not part of the ABI): copies the wave records of the
// launches so far to host memory and clears them.
extern "C" int loom_hip_wave_trace_read(void* host, uint64_t bytes) {
  const uint64_t n = bytes < sizeof(g_wave_records) ? bytes : sizeof(g_wave_records);
  if (hipMemcpyFromSymbol(host, HIP_SYMBOL(g_wave_records), n, 0, hipMemcpyDeviceToHost) != hipSuccess) return 1;
  static WaveRecord zero[1024];
  for (uint64_t off = 0; off < sizeof(g_wave_records); off += sizeof(zero))
    if (hipMemcpyToSymbol(HIP_SYMBOL(g_wave_records), zero, sizeof(zero), off, hipMemcpyHostToDevice) != hipSuccess)
      return 1;
  return 0;
}

// The loop-start and quarter marks of the same wave slots (four u64 per slot); not cleared
// (every traced wave with steps overwrites its own).
extern "C" int loom_hip_wave_trace_marks_read(void* host, uint64_t bytes) {
  const uint64_t n = bytes < sizeof(g_wave_marks) ? bytes : sizeof(g_wave_marks);
  return hipMemcpyFromSymbol(host, HIP_SYMBOL(g_wave_marks), n, 0, hipMemcpyDeviceToHost) == hipSuccess ? 0 : 1;
}

// Per quarter of its steps, the time each wave slot spent waiting for step
// loads (four u64 per slot, 100 MHz ticks); not cleared either.
extern "C" int loom_hip_wave_trace_stall_read(void* host, uint64_t bytes) {
  const uint64_t n = bytes < sizeof(g_wave_stall) ? bytes : sizeof(g_wave_stall);
  return hipMemcpyFromSymbol(host, HIP_SYMBOL(g_wave_stall), n, 0, hipMemcpyDeviceToHost) == hipSuccess ? 0 : 1;
}
#endif

