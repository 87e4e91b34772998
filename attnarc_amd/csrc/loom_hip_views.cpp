// Tensor-view front end of the checked bridge (include/loom_hip_views.h).
//
// Each operator's tensor contract is data: a table with one row per operand
// (rank, accepted element types, layout class, named dimensions and the
// message for each kind of violation) and a short list of rules that relate
// several operands or scalars. `apply` walks the table one aspect at a time
// (placement, element types, ranks, extents, named dimensions, layouts) and
// then the rules, and reports the first violation. The rules restate what
// the reference's adapters check (python/csrc/attention.cpp:5-88,
// python/csrc/rope_kv.cpp:37-150) without the 1024-token decode cap; the
// messages are the reference's texts, which callers and tests match.
//
// Views that pass are marshalled into the element-count spans and strides of
// the checked bridge (loom_hip_bridge.cpp), which repeats the Loom contract
// and adds exact span, alignment and alias checks before it launches.

#include "../../include/loom_hip_views.h"

#include <cmath>
#include <cstdint>
#include <limits>
#include <string>

#include "../../include/loom_hip_bridge.h"

namespace {

thread_local std::string g_views_error;

using View = loom_hip_tensor_view;

int violation(const char* message) {
  g_views_error = message;
  return LOOM_HIP_VIEWS_CONTRACT;
}

int bridge_failure(int status) {
  g_views_error = std::string(loom_hip_bridge_last_error_message()) + " (status " + std::to_string(status) + ")";
  return LOOM_HIP_VIEWS_BRIDGE;
}

constexpr uint32_t bit(uint32_t dtype) { return 1U << dtype; }
constexpr uint32_t kFloats = bit(LOOM_HIP_VIEW_F32) | bit(LOOM_HIP_VIEW_F16) | bit(LOOM_HIP_VIEW_BF16);
constexpr uint32_t kFp8Bytes = bit(LOOM_HIP_VIEW_U8) | bit(LOOM_HIP_VIEW_FP8_E4M3FN);
// Marker in Operand::types: the element type of operand 0 (alone or with others).
constexpr uint32_t kSameAsFirst = 1U << 31;

enum class Layout : uint8_t {
  kAny,
  kContiguous,  // row-major dense (strides of extent-1 dimensions are free)
  kDenseNhd,    // [blocks, block_size, heads, dim]: only the block stride may leave gaps
  kUnitInner,   // unit innermost stride, positive outer strides
};

// One operand of an operator contract. `dims` names each dimension: an
// upper-case letter is a shared extent (its first appearance binds it, later
// appearances must equal it), a digit is a required extent, '.' is free.
struct Operand {
  uint32_t rank;            // 0: any rank
  uint32_t types;           // accepted element types (bit set, kSameAsFirst)
  Layout layout;
  const char* dims;
  bool positive;            // every extent must be > 0
  const char* rank_msg;
  const char* type_msg;
  const char* layout_msg;
  const char* extent_msg;   // for `positive`
  const char* dim_msg[LOOM_HIP_VIEW_MAX_RANK];  // per dimension, on a mismatch
};

// Bound extents of the named dimensions ('A'..'Z').
struct Extents {
  int64_t v[26];
  bool bound[26] = {};
  int64_t operator[](char name) const { return v[name - 'A']; }
};

struct Contract {
  const Operand* operands;
  uint32_t count;
  const char* gpu_msg;      // operand 0 must be on a GPU
  const char* device_msg;   // every operand on operand 0's device
};

uint64_t element_bytes(uint32_t dtype) {
  switch (dtype) {
    case LOOM_HIP_VIEW_F32: case LOOM_HIP_VIEW_I32: return 4;
    case LOOM_HIP_VIEW_F16: case LOOM_HIP_VIEW_BF16: return 2;
    case LOOM_HIP_VIEW_U8: case LOOM_HIP_VIEW_FP8_E4M3FN: return 1;
    case LOOM_HIP_VIEW_I64: return 8;
    default: return 0;
  }
}

int64_t numel(const View& t) {
  int64_t n = 1;
  for (uint32_t d = 0; d < t.rank; ++d) n *= t.sizes[d];
  return n;
}

bool laid_out(const View& t, Layout layout) {
  switch (layout) {
    case Layout::kAny: return true;
    case Layout::kContiguous: {
      int64_t expect = 1;
      for (uint32_t d = t.rank; d-- > 0;) {
        if (t.sizes[d] != 1 && t.strides[d] != expect) return false;
        expect *= t.sizes[d];
      }
      return true;
    }
    case Layout::kDenseNhd:
      return t.rank == 4 && t.strides[3] == 1 && t.strides[2] == t.sizes[3] &&
             t.strides[1] == t.sizes[2] * t.sizes[3] && t.strides[0] >= t.sizes[1] * t.sizes[2] * t.sizes[3];
    case Layout::kUnitInner:
      if (t.rank == 0 || t.strides[t.rank - 1] != 1) return false;
      for (uint32_t d = 0; d + 1 < t.rank; ++d)
        if (t.strides[d] <= 0) return false;
      return true;
  }
  return false;
}

// Elements from the first addressed element to one past the last, over the
// listed dimensions (all when dims is null); 0 for an empty view or on overflow.
uint64_t span_elements(const View& t, const uint32_t* dims = nullptr, uint32_t ndims = 0) {
  if (numel(t) <= 0) return 0;
  uint64_t span = 1;
  const uint32_t n = dims ? ndims : t.rank;
  for (uint32_t i = 0; i < n; ++i) {
    const uint32_t d = dims ? dims[i] : i;
    if (t.strides[d] < 0) return 0;
    const auto extent = static_cast<uint64_t>(t.sizes[d] - 1);
    const auto stride = static_cast<uint64_t>(t.strides[d]);
    if (extent != 0 && stride > (std::numeric_limits<uint64_t>::max() - span) / extent) return 0;
    span += extent * stride;
  }
  return span;
}

bool storage_overlaps(const View& a, const View& b) {
  const uint64_t an = span_elements(a) * element_bytes(a.dtype);
  const uint64_t bn = span_elements(b) * element_bytes(b.dtype);
  if (an == 0 || bn == 0) return false;
  const auto a0 = reinterpret_cast<uintptr_t>(a.data), b0 = reinterpret_cast<uintptr_t>(b.data);
  return a0 < b0 + bn && b0 < a0 + an;
}

bool fits_u32(int64_t v) { return v > 0 && v <= static_cast<int64_t>(std::numeric_limits<uint32_t>::max()); }

// Walks the operand table; on success `ext` holds the named extents.
int apply(const Contract& c, const View* v, uint32_t present, Extents* ext) {
  if (v[0].device_index < 0) return violation(c.gpu_msg);
  for (uint32_t i = 1; i < present; ++i)
    if (v[i].device_index != v[0].device_index) return violation(c.device_msg);
  for (uint32_t i = 0; i < present; ++i) {
    const Operand& o = c.operands[i];
    uint32_t ok = o.types & ~kSameAsFirst;
    if (o.types & kSameAsFirst) ok |= bit(v[0].dtype);
    if (v[i].dtype > 30 || !(ok & bit(v[i].dtype))) return violation(o.type_msg);
  }
  for (uint32_t i = 0; i < present; ++i) {
    const Operand& o = c.operands[i];
    if (v[i].rank > LOOM_HIP_VIEW_MAX_RANK || (o.rank != 0 && v[i].rank != o.rank)) return violation(o.rank_msg);
  }
  for (uint32_t i = 0; i < present; ++i) {
    const Operand& o = c.operands[i];
    if (!o.positive) continue;
    for (uint32_t d = 0; d < v[i].rank; ++d)
      if (v[i].sizes[d] <= 0) return violation(o.extent_msg);
  }
  for (uint32_t i = 0; i < present; ++i) {
    const Operand& o = c.operands[i];
    for (uint32_t d = 0; o.dims != nullptr && o.dims[d] != '\0'; ++d) {
      const char name = o.dims[d];
      const int64_t size = v[i].sizes[d];
      if (name >= '0' && name <= '9') {
        if (size != name - '0') return violation(o.dim_msg[d]);
      } else if (name >= 'A' && name <= 'Z') {
        const int k = name - 'A';
        if (!ext->bound[k]) {
          ext->bound[k] = true;
          ext->v[k] = size;
        } else if (ext->v[k] != size) {
          return violation(o.dim_msg[d]);
        }
      }
    }
  }
  for (uint32_t i = 0; i < present; ++i) {
    const Operand& o = c.operands[i];
    if (!laid_out(v[i], o.layout)) return violation(o.layout_msg);
  }
  return LOOM_HIP_VIEWS_OK;
}

// ---------------------------------------------------------------------------
// Paged decode: query, key_cache, value_cache, block_tables, sequence_lengths, output.
// Named extents: B sequences, H query heads, D head size, N blocks, S block
// size, K KV heads, V value head size, M table width.
// ---------------------------------------------------------------------------

constexpr const char* kDecodeRank =
    "Loom paged decode requires rank-3 query/output, rank-4 K/V caches, rank-2 block tables, and rank-1 "
    "sequence lengths";
constexpr const char* kDecodeLayout =
    "Loom paged decode requires contiguous query/output/metadata and dense-inner NHD caches with an optional "
    "block stride";
constexpr const char* kDecodePositive = "Loom paged decode dimensions must be positive";
constexpr const char* kDecodeShare = "Loom paged decode data tensors must share a dtype";
constexpr const char* kDecodeMeta = "Loom paged decode metadata must use int32";
constexpr const char* kDecodeBatch = "Loom paged decode metadata batch dimensions must match query";
constexpr const char* kDecodePrefix = "Loom paged decode K/V cache prefixes must match";
constexpr const char* kDecodeOut = "Loom paged decode output must have shape [B, Hq, Dv]";

const Operand kDecodeOperands[6] = {
    {3, kFloats, Layout::kContiguous, "BHD", true, kDecodeRank,
     "Loom paged decode supports F32, FP16, and BF16 native caches", kDecodeLayout, kDecodePositive, {}},
    {4, kSameAsFirst, Layout::kDenseNhd, "NSKD", true, kDecodeRank, kDecodeShare, kDecodeLayout, kDecodePositive,
     {nullptr, nullptr, nullptr, "Loom paged decode Q/K head sizes must match"}},
    {4, kSameAsFirst, Layout::kDenseNhd, "NSKV", true, kDecodeRank, kDecodeShare, kDecodeLayout, kDecodePositive,
     {kDecodePrefix, kDecodePrefix, kDecodePrefix, nullptr}},
    {2, bit(LOOM_HIP_VIEW_I32), Layout::kContiguous, "BM", true, kDecodeRank, kDecodeMeta, kDecodeLayout,
     kDecodeBatch, {kDecodeBatch, nullptr}},
    {1, bit(LOOM_HIP_VIEW_I32), Layout::kContiguous, "B", true, kDecodeRank, kDecodeMeta, kDecodeLayout,
     kDecodeBatch, {kDecodeBatch}},
    {3, kSameAsFirst, Layout::kContiguous, "BHV", true, kDecodeRank, kDecodeShare, kDecodeLayout, kDecodeOut,
     {kDecodeOut, kDecodeOut, kDecodeOut}},
};

const Contract kDecode = {kDecodeOperands, 6, "Loom paged decode query must be on a GPU",
                          "Loom paged decode tensors must be on one GPU device"};

int check_decode(const View* v, uint32_t present, int64_t max_len, double scale, bool check_scale, Extents* e) {
  if (v == nullptr || (present != 5 && present != 6)) return violation("Loom paged decode takes 5 or 6 views");
  int status = apply(kDecode, v, present, e);
  if (status != LOOM_HIP_VIEWS_OK) return status;
  const Extents& x = *e;
  if (x['H'] % x['K'] != 0) return violation("Loom paged decode query heads must be divisible by KV heads");
  if (max_len <= 0 || max_len > x['M'] * x['S'])
    return violation("Loom paged decode max_sequence_length must be within table capacity");
  if (check_scale && !(std::isfinite(scale) && scale > 0.0))
    return violation("Loom paged decode scale must be finite and positive");
  if (present == 6) {
    for (uint32_t i = 0; i < 5; ++i)
      if (storage_overlaps(v[5], v[i])) return violation("Loom paged decode output storage must not overlap inputs");
  }
  for (const char n : {'B', 'H', 'K', 'D', 'V', 'N', 'S', 'M'})
    if (!fits_u32(x[n])) return violation("Loom paged decode shape exceeds the HIP ABI");
  if (!fits_u32(max_len)) return violation("Loom paged decode shape exceeds the HIP ABI");
  if (x['B'] > std::numeric_limits<int32_t>::max() / x['H'])
    return violation("Loom paged decode grid exceeds the HIP ABI");
  return LOOM_HIP_VIEWS_OK;
}

// ---------------------------------------------------------------------------
// RoPE + paged-KV write: query, key, value, positions, cos_sin_cache,
// kv_cache, key_scales, value_scales, slot_mapping. Named extents: T tokens,
// H query heads, D head size, K KV heads, P max position, R rotary dims, N
// blocks, S block size.
// ---------------------------------------------------------------------------

constexpr const char* kRopeRank3 = "Loom RoPE+paged-KV Q/K/V must have rank 3";
constexpr const char* kRopeShare = "Loom RoPE+paged-KV Q/K/V and cos/sin cache must share a dtype";
constexpr const char* kRopeTokens = "Loom RoPE+paged-KV Q/K/V token counts must match";
constexpr const char* kRopeSources =
    "Loom RoPE+paged-KV sources require unit dim stride and positive token/head strides; metadata must be "
    "contiguous";
constexpr const char* kRopeInt64 = "Loom RoPE+paged-KV positions and slot mapping must be int64";
constexpr const char* kRopeCover =
    "Loom RoPE positions must cover every token and slot_mapping must not exceed the padded token count";
constexpr const char* kRopeCosSin =
    "Loom RoPE+paged-KV cos/sin cache must be [max_position, even rotary_dim <= head_size]";
constexpr const char* kRopeCacheShape =
    "Loom paged K/V cache must have shape [blocks, 2, block_size, kv_heads, head_size]";
constexpr const char* kRopeCacheShare = "Loom packed K/V cache and K/V sources must share head count and head size";
constexpr const char* kRopeScales =
    "Loom paged K/V cache scales must be contiguous float32 tensors with one element or one element per KV head";

const Operand kRopeOperands[9] = {
    {3, kFloats, Layout::kUnitInner, "THD", true, kRopeRank3, "Loom RoPE+paged-KV supports F32, FP16, and BF16 sources",
     kRopeSources, "Loom RoPE+paged-KV query must be non-empty", {}},
    {3, kSameAsFirst, Layout::kUnitInner, "TKD", true, kRopeRank3, kRopeShare, kRopeSources,
     "Loom RoPE+paged-KV K/V head counts must match",
     {kRopeTokens, nullptr, "Loom RoPE+paged-KV Q/K head sizes must match"}},
    {3, kSameAsFirst, Layout::kUnitInner, "TKD", true, kRopeRank3, kRopeShare, kRopeSources,
     "Loom RoPE+paged-KV value head size must be positive",
     {kRopeTokens, "Loom RoPE+paged-KV K/V head counts must match", kRopeCacheShare}},
    {1, bit(LOOM_HIP_VIEW_I64), Layout::kContiguous, "T", false, kRopeCover, kRopeInt64, kRopeSources, nullptr,
     {kRopeCover}},
    {2, kSameAsFirst, Layout::kContiguous, "PR", true, kRopeCosSin, kRopeShare, kRopeSources, kRopeCosSin, {}},
    {5, kSameAsFirst | kFp8Bytes, Layout::kAny, "N2SKD", true, kRopeCacheShape,
     "Loom paged K/V cache must use the source dtype or uint8 FP8 E4M3 storage", nullptr, kRopeCacheShape,
     {nullptr, kRopeCacheShape, nullptr, kRopeCacheShare, kRopeCacheShare}},
    {0, bit(LOOM_HIP_VIEW_F32), Layout::kContiguous, nullptr, false, kRopeScales, kRopeScales, kRopeScales, nullptr, {}},
    {0, bit(LOOM_HIP_VIEW_F32), Layout::kContiguous, nullptr, false, kRopeScales, kRopeScales, kRopeScales, nullptr, {}},
    {1, bit(LOOM_HIP_VIEW_I64), Layout::kContiguous, nullptr, false, kRopeCover, kRopeInt64, kRopeSources, nullptr, {}},
};

const Contract kRope = {kRopeOperands, 9, "Loom RoPE+paged-KV query must be on a GPU",
                        "Loom RoPE+paged-KV tensors must be on one GPU device"};

int check_rope(const View* v, Extents* e) {
  if (v == nullptr) return violation("Loom RoPE+paged-KV takes 9 views");
  int status = apply(kRope, v, 9, e);
  if (status != LOOM_HIP_VIEWS_OK) return status;
  const Extents& x = *e;
  const View& kv = v[5];
  const int64_t scales = numel(v[6]);
  if (scales != numel(v[7]) || (scales != 1 && scales != x['K'])) return violation(kRopeScales);
  if (numel(v[8]) > x['T']) return violation(kRopeCover);
  if (x['R'] % 2 != 0 || x['R'] > x['D']) return violation(kRopeCosSin);
  if (kv.strides[4] != 1 || kv.strides[0] <= 0 || kv.strides[1] <= 0 || kv.strides[2] <= 0 || kv.strides[3] <= 0)
    return violation("Loom packed K/V cache requires unit element stride and positive block/KV/page/head strides");
  // One half (K or V) of a block spans `half` elements; the halves and the
  // blocks must not interleave.
  const uint32_t inner[] = {2, 3, 4};
  const uint64_t half = span_elements(kv, inner, 3);
  const auto kv_stride = static_cast<uint64_t>(kv.strides[1]);
  const auto block_stride = static_cast<uint64_t>(kv.strides[0]);
  if (half == 0 || kv_stride < half || block_stride < kv_stride || block_stride - kv_stride < half)
    return violation("Loom packed K/V cache partitions must not overlap");
  for (const char n : {'T', 'H', 'K', 'D', 'R', 'P', 'N', 'S'})
    if (!fits_u32(x[n])) return violation("Loom RoPE+paged-KV shape exceeds the HIP ABI");
  if (!fits_u32(v[2].sizes[2]) || x['T'] > std::numeric_limits<int32_t>::max())
    return violation("Loom RoPE+paged-KV shape exceeds the HIP ABI");
  return LOOM_HIP_VIEWS_OK;
}

uint32_t u32(int64_t v) { return static_cast<uint32_t>(v); }
uint64_t u64(int64_t v) { return static_cast<uint64_t>(v); }

}  // namespace

extern "C" {

const char* loom_hip_views_last_error_message(void) { return g_views_error.c_str(); }

int loom_hip_views_paged_decode_check(const loom_hip_tensor_view* views, uint32_t count,
                                      int64_t max_sequence_length, double scale) {
  Extents e;
  return check_decode(views, count, max_sequence_length, scale, count == 6, &e);
}

int loom_hip_views_paged_decode_workspace_elements(const loom_hip_tensor_view* views,
                                                   int64_t max_sequence_length, double scale,
                                                   uint64_t* workspace_elements) {
  if (workspace_elements == nullptr) return violation("Loom paged decode workspace count pointer is null");
  *workspace_elements = 0;
  Extents e;
  int status = check_decode(views, 6, max_sequence_length, scale, true, &e);
  if (status != LOOM_HIP_VIEWS_OK) return status;
  status = loom_hip_bridge_paged_decode_workspace_elements(
      views[0].dtype, u32(e['B']), u32(e['H']), u32(e['K']), u32(e['D']), u32(e['V']), u32(e['N']), u32(e['S']),
      u32(e['M']), u32(max_sequence_length), static_cast<float>(scale), workspace_elements);
  return status == LOOM_HIP_BRIDGE_SUCCESS ? LOOM_HIP_VIEWS_OK : bridge_failure(status);
}

int loom_hip_views_paged_decode_attention(const loom_hip_tensor_view* views, int64_t max_sequence_length,
                                          double scale, float* workspace, uint64_t workspace_elements,
                                          void* stream) {
  Extents e;
  int status = check_decode(views, 6, max_sequence_length, scale, true, &e);
  if (status != LOOM_HIP_VIEWS_OK) return status;
  const View &q = views[0], &k = views[1], &v = views[2], &tables = views[3], &lens = views[4], &out = views[5];
  status = loom_hip_bridge_paged_decode_attention(
      q.dtype, q.data, span_elements(q), k.data, span_elements(k), v.data, span_elements(v),
      static_cast<const int32_t*>(tables.data), span_elements(tables), static_cast<const int32_t*>(lens.data),
      span_elements(lens), const_cast<void*>(out.data), span_elements(out), workspace, workspace_elements,
      u32(e['B']), u32(e['H']), u32(e['K']), u32(e['D']), u32(e['V']), u32(e['N']), u32(e['S']),
      u64(k.strides[0]), u64(v.strides[0]), u32(e['M']), u32(max_sequence_length), static_cast<float>(scale),
      stream);
  return status == LOOM_HIP_BRIDGE_SUCCESS ? LOOM_HIP_VIEWS_OK : bridge_failure(status);
}

int loom_hip_views_rope_paged_kv_check(const loom_hip_tensor_view* views) {
  Extents e;
  return check_rope(views, &e);
}

int loom_hip_views_rope_paged_kv_write(const loom_hip_tensor_view* views, uint32_t is_neox, void* stream) {
  Extents e;
  int status = check_rope(views, &e);
  if (status != LOOM_HIP_VIEWS_OK) return status;
  const View &q = views[0], &k = views[1], &v = views[2], &pos = views[3], &cs = views[4], &kv = views[5];
  const View &ks = views[6], &vs = views[7], &slots = views[8];
  const bool fp8 = kv.dtype == LOOM_HIP_VIEW_U8 || kv.dtype == LOOM_HIP_VIEW_FP8_E4M3FN;
  // K is half 0 of each block, V half 1: the V view starts one half-stride in.
  auto* k_cache = static_cast<uint8_t*>(const_cast<void*>(kv.data));
  uint8_t* v_cache = k_cache + u64(kv.strides[1]) * element_bytes(kv.dtype);
  const uint32_t view_dims[] = {0, 2, 3, 4};
  const uint64_t view_span = span_elements(kv, view_dims, 4);
  const uint64_t block = u64(kv.strides[0]), page = u64(kv.strides[2]), head = u64(kv.strides[3]);
  status = loom_hip_bridge_rope_paged_kv_write(
      q.dtype, fp8 ? LOOM_HIP_BRIDGE_KV_CACHE_FP8_E4M3 : LOOM_HIP_BRIDGE_KV_CACHE_NATIVE, const_cast<void*>(q.data),
      span_elements(q), const_cast<void*>(k.data), span_elements(k), v.data, span_elements(v),
      static_cast<const int64_t*>(pos.data), u64(numel(pos)), cs.data, u64(numel(cs)), k_cache, view_span, v_cache,
      view_span, static_cast<const float*>(ks.data), u64(numel(ks)), static_cast<const float*>(vs.data),
      u64(numel(vs)), static_cast<const int64_t*>(slots.data), u64(numel(slots)), u32(e['T']), u32(numel(slots)),
      u32(e['H']), u32(e['K']), u32(e['D']), u32(v.sizes[2]), u32(e['R']), u32(e['P']), u32(e['N']), u32(e['S']),
      u64(q.strides[0]), u64(q.strides[1]), u64(k.strides[0]), u64(k.strides[1]), u64(v.strides[0]),
      u64(v.strides[1]), block, page, head, block, page, head, is_neox ? 1U : 0U, stream);
  return status == LOOM_HIP_BRIDGE_SUCCESS ? LOOM_HIP_VIEWS_OK : bridge_failure(status);
}

}  // extern "C"
