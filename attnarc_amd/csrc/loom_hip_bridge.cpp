// Checked C bridge over the loom-hip kernels (include/loom_hip_bridge.h).
//
// The reference bridge is Rust (crates/loom-cuda-bridge/src/cuda/mod.rs,
// attention_bridge.rs, rope_kv_bridge.rs) over the safe loom-cuda layer
// (attention_dispatch.rs, rope_kv_dispatch.rs, layout.rs). This is the same
// sequence of checks in host C++, ending in a call of the unchecked loom_hip
// entry points of include/loom_hip.h. Messages follow the reference's
// Display texts so that callers matching on them keep working; the
// "invalid operator contract: " prefix is CudaExecutorError::InvalidContract's
// (loom-cuda/src/lib.rs:41-48).

#include "loom_hip_bridge.h"

#include <atomic>
#include <cmath>
#include <cstdint>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <initializer_list>
#include <string>
#include <utility>
#include <vector>

#include "loom_hip.h"

namespace {

constexpr uint32_t kOperatorCount = 11;
std::atomic<uint64_t> g_launches[kOperatorCount];

thread_local std::string g_last_error = "no bridge error has been recorded";

// A failed check: bridge status plus the message recorded for the caller.
struct Failure {
  int status;
  std::string message;
};

using Result = std::pair<bool, Failure>;  // (ok, failure if !ok)

Result ok() { return {true, Failure{LOOM_HIP_BRIDGE_SUCCESS, std::string()}}; }

Result contract(const std::string& message) {
  return {false, Failure{LOOM_HIP_BRIDGE_INVALID_ARGUMENT, "invalid operator contract: " + message}};
}

#define BRIDGE_TRY(expr)          \
  do {                            \
    Result r_ = (expr);           \
    if (!r_.first) return r_;     \
  } while (0)

int finish(const Result& r) {
  if (r.first) return LOOM_HIP_BRIDGE_SUCCESS;
  g_last_error = r.second.message;
  return r.second.status;
}

std::string u64s(uint64_t v) { return std::to_string(v); }

// Rust's Display for f32: the shortest digits that read back to the same
// value, written positionally (no exponent), "NaN", "inf", "-inf".
std::string rust_f32(float v) {
  if (std::isnan(v)) return "NaN";
  if (std::isinf(v)) return v > 0 ? "inf" : "-inf";
  if (v == 0.0f) return std::signbit(v) ? "-0" : "0";
  char buf[64];
  int prec = 0;
  for (; prec < 9; ++prec) {
    std::snprintf(buf, sizeof(buf), "%.*e", prec, static_cast<double>(v));
    if (std::strtof(buf, nullptr) == v) break;
  }
  std::snprintf(buf, sizeof(buf), "%.*e", prec, static_cast<double>(v));
  std::string s(buf);
  const bool neg = s[0] == '-';
  if (neg) s.erase(0, 1);
  const size_t e = s.find('e');
  const int exp10 = std::atoi(s.c_str() + e + 1);
  std::string digits;
  for (size_t i = 0; i < e; ++i)
    if (s[i] != '.') digits.push_back(s[i]);
  while (digits.size() > 1 && digits.back() == '0') digits.pop_back();
  std::string out;
  const int point = exp10 + 1;  // digits before the decimal point
  if (point <= 0) {
    out = "0." + std::string(static_cast<size_t>(-point), '0') + digits;
  } else if (static_cast<size_t>(point) >= digits.size()) {
    out = digits + std::string(static_cast<size_t>(point) - digits.size(), '0');
  } else {
    out = digits.substr(0, static_cast<size_t>(point)) + "." + digits.substr(static_cast<size_t>(point));
  }
  return neg ? "-" + out : out;
}

// ---------------------------------------------------------------------------
// Regions (cuda/mod.rs:84-230)
// ---------------------------------------------------------------------------

struct Range {
  uintptr_t start = 0, end = 0;
};

bool overlap(Range a, Range b) { return a.start < b.end && b.start < a.end; }

Result byte_range(const void* p, uint64_t elements, size_t elem_size, size_t align, const char* name, Range* out) {
  if (p == nullptr) return contract(std::string(name) + " pointer is null");
  if (elements == 0) return contract(std::string(name) + " region is empty");
  if (reinterpret_cast<uintptr_t>(p) % align != 0)
    return contract(std::string(name) + " pointer is not aligned to " + u64s(align) + " bytes");
  if (elements > UINT64_MAX / elem_size) return contract(std::string(name) + " byte size overflows usize");
  const uint64_t bytes = elements * elem_size;
  const uintptr_t start = reinterpret_cast<uintptr_t>(p);
  if (start > UINTPTR_MAX - bytes) return contract(std::string(name) + " address range overflows usize");
  *out = Range{start, start + static_cast<uintptr_t>(bytes)};
  return ok();
}

Result disjoint_from(const char* target_name, Range target,
                     std::initializer_list<std::pair<const char*, Range>> others, const char* op) {
  for (const auto& o : others)
    if (overlap(target, o.second))
      return contract(std::string(op) + " regions " + target_name + " and " + o.first + " must not overlap");
  return ok();
}

// Two views of one packed allocation (e.g. Q, K, V as column slices of one
// QKV row) may share bytes only if they step through memory with the same
// outer stride and their dense inner spans do not meet (mod.rs:161-231).
// `dense_inner` is 0 when the view's inner span is not dense.
Result disjoint_or_dense_packed(const char* left_name, Range left, uint64_t left_outer, uint64_t left_dense_inner,
                                const char* right_name, Range right, uint64_t right_outer,
                                uint64_t right_dense_inner, size_t elem_size, const char* op) {
  if (!overlap(left, right)) return ok();
  if (left_dense_inner == 0 || right_dense_inner == 0)
    return contract(std::string(op) + " regions " + left_name + " and " + right_name +
                    " overlap without a dense packed layout");
  if (left_outer != right_outer)
    return contract(std::string(op) + " packed regions " + left_name + " and " + right_name +
                    " must share an outer stride");
  if (left_outer > UINT64_MAX / elem_size) return contract(std::string(op) + " packed outer stride overflows usize");
  const uint64_t outer = left_outer * elem_size;
  const uint64_t lbytes = left_dense_inner * elem_size, rbytes = right_dense_inner * elem_size;
  const bool left_first = left.start <= right.start;
  const char* earlier_name = left_first ? left_name : right_name;
  const char* later_name = left_first ? right_name : left_name;
  const Range earlier = left_first ? left : right, later = left_first ? right : left;
  const uint64_t earlier_inner = left_first ? lbytes : rbytes, later_inner = left_first ? rbytes : lbytes;
  const uint64_t offset = later.start - earlier.start;
  if (offset > UINT64_MAX - later_inner) return contract(std::string(op) + " packed inner span overflows usize");
  if (offset >= outer || earlier_inner > offset || offset + later_inner > outer)
    return contract(std::string(op) + " logical elements in packed regions " + earlier_name + " and " + later_name +
                    " overlap");
  return ok();
}

// ---------------------------------------------------------------------------
// Strided layouts (loom-cuda layout.rs:18-62)
// ---------------------------------------------------------------------------

bool mul_ok(uint64_t a, uint64_t b, uint64_t* out) {
  if (a != 0 && b > UINT64_MAX / a) return false;
  *out = a * b;
  return true;
}

bool add_ok(uint64_t a, uint64_t b, uint64_t* out) {
  if (a > UINT64_MAX - b) return false;
  *out = a + b;
  return true;
}

// Storage span: width + sum (size - 1) * stride.
Result strided_span(std::initializer_list<std::pair<uint64_t, uint64_t>> dims, uint64_t width, const char* name,
                    uint64_t* out) {
  if (width == 0) return contract(std::string(name) + " contiguous width must be positive");
  uint64_t span = width;
  for (const auto& d : dims) {
    if (d.first == 0 || d.second == 0) return contract(std::string(name) + " dimensions and strides must be positive");
    uint64_t t;
    if (!mul_ok(d.first - 1, d.second, &t) || !add_ok(span, t, &span))
      return contract(std::string(name) + " storage span overflows usize");
  }
  *out = span;
  return ok();
}

// No two logical elements share an address: sorted by stride, every stride
// reaches past the span of the dimensions inside it.
Result non_overlapping(std::vector<std::pair<uint64_t, uint64_t>> dims, uint64_t width, const char* name) {
  dims.insert(dims.begin(), {width, 1});
  for (size_t i = 1; i < dims.size(); ++i)  // stable insertion sort by stride
    for (size_t j = i; j > 0 && dims[j].second < dims[j - 1].second; --j) std::swap(dims[j], dims[j - 1]);
  uint64_t occupied = 1;
  for (const auto& d : dims) {
    if (d.first == 0 || d.second == 0) return contract(std::string(name) + " dimensions and strides must be positive");
    if (d.first == 1) continue;
    if (d.second < occupied) return contract(std::string(name) + " layout overlaps itself");
    uint64_t t;
    if (!mul_ok(d.first - 1, d.second, &t) || !add_ok(occupied, t, &occupied))
      return contract(std::string(name) + " storage span overflows usize");
  }
  return ok();
}

Result require_len(uint64_t actual, uint64_t expected, const char* name) {
  if (actual != expected)
    return contract(std::string(name) + " has " + u64s(actual) + " elements, expected " + u64s(expected));
  return ok();
}

// ---------------------------------------------------------------------------
// Status of the unchecked library -> bridge status
// ---------------------------------------------------------------------------

Result from_core(int status) {
  if (status == LOOM_HIP_SUCCESS) return ok();
  const std::string msg = loom_hip_last_error_message();
  if (status == LOOM_HIP_UNAVAILABLE) return {false, Failure{LOOM_HIP_BRIDGE_UNAVAILABLE, msg}};
  if (status == LOOM_HIP_LAUNCH_ERROR)
    return {false, Failure{LOOM_HIP_BRIDGE_LAUNCH_ERROR,
                           "HIP kernel submission failed with status " + std::to_string(status) + ": " + msg}};
  return contract(msg);  // INVALID_ARGUMENT, UNSUPPORTED
}

Result elem_info(uint32_t dtype, size_t* size) {
  if (dtype == LOOM_HIP_BRIDGE_F32) {
    *size = 4;
  } else if (dtype == LOOM_HIP_BRIDGE_F16 || dtype == LOOM_HIP_BRIDGE_BF16) {
    *size = 2;
  } else {
    return contract("unknown bridge dtype code " + u64s(dtype));
  }
  return ok();
}

// ---------------------------------------------------------------------------
// Paged decode attention (attention_bridge.rs, attention_dispatch.rs)
// ---------------------------------------------------------------------------

struct DecodeShape {
  uint32_t sequences, query_heads, kv_heads, head_size, value_head_size;
  uint32_t num_blocks, block_size, max_blocks_per_sequence, max_sequence_length;
  float scale;
};

// PagedDecodeAttentionSpec::new (attention.rs:34-98).
Result decode_spec(const DecodeShape& s) {
  if (s.sequences == 0 || s.query_heads == 0 || s.kv_heads == 0 || s.head_size == 0 || s.value_head_size == 0 ||
      s.num_blocks == 0 || s.block_size == 0 || s.max_blocks_per_sequence == 0 || s.max_sequence_length == 0)
    return contract("tensor dimensions must be non-zero");
  if (s.query_heads % s.kv_heads != 0)
    return contract("query head count " + u64s(s.query_heads) + " must be divisible by KV head count " +
                    u64s(s.kv_heads));
  if (!std::isfinite(s.scale) || s.scale <= 0.0f)
    return contract("attention scale must be finite and positive, got " + rust_f32(s.scale));
  // Products of u32 values fit u64 up to three factors; four-factor products are checked.
  uint64_t t;
  if (!mul_ok(static_cast<uint64_t>(s.num_blocks) * s.block_size, static_cast<uint64_t>(s.kv_heads) * s.head_size,
              &t) ||
      !mul_ok(static_cast<uint64_t>(s.num_blocks) * s.block_size,
              static_cast<uint64_t>(s.kv_heads) * s.value_head_size, &t))
    return contract("tensor element count overflowed");
  const uint64_t capacity = static_cast<uint64_t>(s.max_blocks_per_sequence) * s.block_size;
  if (s.max_sequence_length > capacity)
    return contract("maximum sequence length " + u64s(s.max_sequence_length) + " exceeds block-table capacity " +
                    u64s(capacity));
  return ok();
}

Result decode_workspace(const DecodeShape& s, uint64_t* elements) {
  *elements = loom_hip_paged_decode_attention_split_k_workspace_elements(
      s.sequences, s.query_heads, s.kv_heads, s.head_size, s.value_head_size, s.max_sequence_length);
  return ok();
}

template <typename Fn>
int guarded(Fn&& fn) {
  try {
    return finish(fn());
  } catch (...) {
    g_last_error = "C++ exception was contained at the Loom HIP bridge";
    return LOOM_HIP_BRIDGE_LAUNCH_ERROR;
  }
}

}  // namespace

extern "C" {

uint32_t loom_hip_bridge_abi_version(void) { return 2; }

const char* loom_hip_bridge_last_error_message(void) { return g_last_error.c_str(); }

int loom_hip_bridge_launch_count(uint32_t operation, uint64_t* count) {
  return guarded([&]() -> Result {
    if (operation >= kOperatorCount) return contract("unknown bridge operator code " + u64s(operation));
    if (count == nullptr || reinterpret_cast<uintptr_t>(count) % alignof(uint64_t) != 0)
      return contract("launch-count output pointer is null or misaligned");
    *count = g_launches[operation].load(std::memory_order_relaxed);
    return ok();
  });
}

int loom_hip_bridge_reset_launch_count(uint32_t operation) {
  return guarded([&]() -> Result {
    if (operation >= kOperatorCount) return contract("unknown bridge operator code " + u64s(operation));
    g_launches[operation].store(0, std::memory_order_relaxed);
    return ok();
  });
}

int loom_hip_bridge_paged_decode_workspace_elements(uint32_t dtype, uint32_t sequences, uint32_t query_heads,
                                                    uint32_t kv_heads, uint32_t head_size, uint32_t value_head_size,
                                                    uint32_t num_blocks, uint32_t block_size,
                                                    uint32_t max_blocks_per_sequence, uint32_t max_sequence_length,
                                                    float scale, uint64_t* workspace_elements) {
  return guarded([&]() -> Result {
    if (workspace_elements == nullptr || reinterpret_cast<uintptr_t>(workspace_elements) % alignof(uint64_t) != 0)
      return contract("workspace-size output pointer is null or misaligned");
    size_t es;
    BRIDGE_TRY(elem_info(dtype, &es));
    const DecodeShape s{sequences,  query_heads,           kv_heads, head_size, value_head_size, num_blocks,
                        block_size, max_blocks_per_sequence, max_sequence_length, scale};
    BRIDGE_TRY(decode_spec(s));
    uint64_t n;
    BRIDGE_TRY(decode_workspace(s, &n));
    *workspace_elements = n;
    return ok();
  });
}

int loom_hip_bridge_paged_decode_attention(
    uint32_t dtype, const void* query, uint64_t query_elements, const void* key_cache, uint64_t key_cache_elements,
    const void* value_cache, uint64_t value_cache_elements, const int32_t* block_tables,
    uint64_t block_table_elements, const int32_t* sequence_lengths, uint64_t sequence_length_elements, void* output,
    uint64_t output_elements, float* workspace, uint64_t workspace_elements, uint32_t sequences,
    uint32_t query_heads, uint32_t kv_heads, uint32_t head_size, uint32_t value_head_size, uint32_t num_blocks,
    uint32_t block_size, uint64_t key_block_stride, uint64_t value_block_stride, uint32_t max_blocks_per_sequence,
    uint32_t max_sequence_length, float scale, void* stream) {
  return guarded([&]() -> Result {
    size_t es;
    BRIDGE_TRY(elem_info(dtype, &es));
    const DecodeShape s{sequences,  query_heads,           kv_heads, head_size, value_head_size, num_blocks,
                        block_size, max_blocks_per_sequence, max_sequence_length, scale};
    BRIDGE_TRY(decode_spec(s));
    // PagedDecodeLayout::new (layout.rs:115-143).
    const uint64_t k_block = static_cast<uint64_t>(block_size) * kv_heads * head_size;
    const uint64_t v_block = static_cast<uint64_t>(block_size) * kv_heads * value_head_size;
    if (key_block_stride < k_block) return contract("paged key block stride is smaller than one dense NHD block");
    if (value_block_stride < v_block) return contract("paged value block stride is smaller than one dense NHD block");
    uint64_t expected_ws;
    BRIDGE_TRY(decode_workspace(s, &expected_ws));
    if (workspace_elements != expected_ws)
      return contract("paged decode workspace has " + u64s(workspace_elements) + " F32 elements, expected " +
                      u64s(expected_ws));
    if (expected_ws == 0 && workspace != nullptr) return contract("base paged decode requires a null workspace pointer");
    if (expected_ws != 0 && workspace == nullptr) return contract("split-K paged decode requires a workspace pointer");

    Range rq, rk, rv, rt, rl, ro;
    BRIDGE_TRY(byte_range(query, query_elements, es, es, "paged decode query", &rq));
    BRIDGE_TRY(byte_range(key_cache, key_cache_elements, es, es, "paged decode key cache", &rk));
    BRIDGE_TRY(byte_range(value_cache, value_cache_elements, es, es, "paged decode value cache", &rv));
    BRIDGE_TRY(byte_range(block_tables, block_table_elements, 4, 4, "paged decode block tables", &rt));
    BRIDGE_TRY(byte_range(sequence_lengths, sequence_length_elements, 4, 4, "paged decode sequence lengths", &rl));
    BRIDGE_TRY(byte_range(output, output_elements, es, es, "paged decode output", &ro));
    BRIDGE_TRY(disjoint_from("output", ro,
                             {{"query", rq}, {"key cache", rk}, {"value cache", rv}, {"block tables", rt},
                              {"sequence lengths", rl}},
                             "paged decode"));
    if (expected_ws != 0) {
      Range rw;
      BRIDGE_TRY(byte_range(workspace, workspace_elements, 4, 4, "paged decode split-K workspace", &rw));
      BRIDGE_TRY(disjoint_from("workspace", rw,
                               {{"query", rq}, {"key cache", rk}, {"value cache", rv}, {"block tables", rt},
                                {"sequence lengths", rl}, {"output", ro}},
                               "paged decode"));
    }
    // validate_buffers (attention_dispatch.rs:457-478): exact storage spans.
    BRIDGE_TRY(require_len(query_elements, static_cast<uint64_t>(sequences) * query_heads * head_size,
                           "paged decode query"));
    BRIDGE_TRY(require_len(key_cache_elements, (static_cast<uint64_t>(num_blocks) - 1) * key_block_stride + k_block,
                           "paged decode key cache"));
    BRIDGE_TRY(require_len(value_cache_elements,
                           (static_cast<uint64_t>(num_blocks) - 1) * value_block_stride + v_block,
                           "paged decode value cache"));
    BRIDGE_TRY(require_len(block_table_elements, static_cast<uint64_t>(sequences) * max_blocks_per_sequence,
                           "paged decode block tables"));
    BRIDGE_TRY(require_len(sequence_length_elements, sequences, "paged decode sequence lengths"));
    BRIDGE_TRY(require_len(output_elements, static_cast<uint64_t>(sequences) * query_heads * value_head_size,
                           "paged decode output"));

    int status;
    using u16 = uint16_t;
    const auto* q16 = static_cast<const u16*>(query);
    const auto* k16 = static_cast<const u16*>(key_cache);
    const auto* v16 = static_cast<const u16*>(value_cache);
    auto* o16 = static_cast<u16*>(output);
    const auto* q32 = static_cast<const float*>(query);
    const auto* k32 = static_cast<const float*>(key_cache);
    const auto* v32 = static_cast<const float*>(value_cache);
    auto* o32 = static_cast<float*>(output);
#define LOOM_BASE_ARGS                                                                                          \
  block_tables, sequence_lengths
#define LOOM_SHAPE_ARGS                                                                                         \
  sequences, query_heads, kv_heads, head_size, value_head_size, num_blocks, block_size, key_block_stride,      \
      value_block_stride, max_blocks_per_sequence, max_sequence_length, scale, stream
    if (expected_ws == 0) {
      if (dtype == LOOM_HIP_BRIDGE_F32)
        status = loom_hip_paged_decode_attention_f32(q32, k32, v32, LOOM_BASE_ARGS, o32, LOOM_SHAPE_ARGS);
      else if (dtype == LOOM_HIP_BRIDGE_F16)
        status = loom_hip_paged_decode_attention_f16(q16, k16, v16, LOOM_BASE_ARGS, o16, LOOM_SHAPE_ARGS);
      else
        status = loom_hip_paged_decode_attention_bf16(q16, k16, v16, LOOM_BASE_ARGS, o16, LOOM_SHAPE_ARGS);
    } else {
      if (dtype == LOOM_HIP_BRIDGE_F32)
        status = loom_hip_paged_decode_attention_split_k_f32(q32, k32, v32, LOOM_BASE_ARGS, o32, workspace,
                                                             workspace_elements, LOOM_SHAPE_ARGS);
      else if (dtype == LOOM_HIP_BRIDGE_F16)
        status = loom_hip_paged_decode_attention_split_k_f16(q16, k16, v16, LOOM_BASE_ARGS, o16, workspace,
                                                             workspace_elements, LOOM_SHAPE_ARGS);
      else
        status = loom_hip_paged_decode_attention_split_k_bf16(q16, k16, v16, LOOM_BASE_ARGS, o16, workspace,
                                                              workspace_elements, LOOM_SHAPE_ARGS);
    }
#undef LOOM_BASE_ARGS
#undef LOOM_SHAPE_ARGS
    BRIDGE_TRY(from_core(status));
    g_launches[LOOM_HIP_BRIDGE_PAGED_DECODE_ATTENTION].fetch_add(1, std::memory_order_relaxed);
    return ok();
  });
}

int loom_hip_bridge_rope_paged_kv_write(
    uint32_t dtype, uint32_t cache_encoding, void* query, uint64_t query_elements, void* key, uint64_t key_elements,
    const void* value, uint64_t value_elements, const int64_t* positions, uint64_t position_elements,
    const void* cos_sin_cache, uint64_t cos_sin_cache_elements, void* key_cache, uint64_t key_cache_elements,
    void* value_cache, uint64_t value_cache_elements, const float* key_scales, uint64_t key_scale_elements,
    const float* value_scales, uint64_t value_scale_elements, const int64_t* slot_mapping,
    uint64_t slot_mapping_elements, uint32_t tokens, uint32_t cache_tokens, uint32_t query_heads, uint32_t kv_heads,
    uint32_t head_size, uint32_t value_head_size, uint32_t rotary_dim, uint32_t max_position, uint32_t num_blocks,
    uint32_t block_size, uint64_t query_token_stride, uint64_t query_head_stride, uint64_t key_token_stride,
    uint64_t source_key_head_stride, uint64_t value_token_stride, uint64_t source_value_head_stride,
    uint64_t key_block_stride, uint64_t key_page_stride, uint64_t key_head_stride, uint64_t value_block_stride,
    uint64_t value_page_stride, uint64_t value_cache_head_stride, uint32_t is_neox, void* stream) {
  return guarded([&]() -> Result {
    const char* op = "RoPE+paged-KV";
    size_t es;
    BRIDGE_TRY(elem_info(dtype, &es));
    if (is_neox > 1) return contract("RoPE style flag must be 0 or 1");
    // RotaryEmbeddingSpec::new (rope_kv.rs:69-112).
    if (tokens == 0 || query_heads == 0 || kv_heads == 0 || head_size == 0 || max_position == 0)
      return contract("tensor dimensions must be non-zero");
    if (rotary_dim == 0 || rotary_dim % 2 != 0 || rotary_dim > head_size)
      return contract("rotary dimension must be non-zero, even, and no larger than head size; got rotary_dim=" +
                      u64s(rotary_dim) + ", head_size=" + u64s(head_size));
    // Scale tensors: same length, one value or one per KV head (rope_kv_bridge.rs:84-112).
    if (key_scale_elements != value_scale_elements)
      return contract("paged K/V cache scale tensors must have the same length");
    if (key_scale_elements != 1 && key_scale_elements != kv_heads)
      return contract("paged K/V cache scales must contain one value or one value per KV head");
    if (cache_encoding != LOOM_HIP_BRIDGE_KV_CACHE_NATIVE && cache_encoding != LOOM_HIP_BRIDGE_KV_CACHE_FP8_E4M3)
      return contract("unsupported paged K/V cache encoding");
    const bool fp8 = cache_encoding == LOOM_HIP_BRIDGE_KV_CACHE_FP8_E4M3;
    // RopePagedKvWriteSpec::new (rope_kv.rs:177-211).
    if (value_head_size == 0 || num_blocks == 0 || block_size == 0)
      return contract("tensor dimensions must be non-zero");
    uint64_t t;
    const uint64_t slots = static_cast<uint64_t>(num_blocks) * block_size;
    if (!mul_ok(slots, static_cast<uint64_t>(kv_heads) * head_size, &t) ||
        !mul_ok(slots, static_cast<uint64_t>(kv_heads) * value_head_size, &t))
      return contract("tensor element count overflowed");
    // RopePagedKvLayout::new (layout.rs:221-287).
    if (cache_tokens == 0 || cache_tokens > tokens)
      return contract("RoPE+paged-KV cache token count must be in [1, tokens]");
    BRIDGE_TRY(non_overlapping({{tokens, query_token_stride}, {query_heads, query_head_stride}}, head_size,
                               "RoPE query"));
    BRIDGE_TRY(non_overlapping({{tokens, key_token_stride}, {kv_heads, source_key_head_stride}}, head_size,
                               "RoPE key"));
    BRIDGE_TRY(non_overlapping({{tokens, value_token_stride}, {kv_heads, source_value_head_stride}},
                               value_head_size, "RoPE value"));
    BRIDGE_TRY(non_overlapping({{num_blocks, key_block_stride}, {block_size, key_page_stride},
                                {kv_heads, key_head_stride}},
                               head_size, "paged key cache"));
    BRIDGE_TRY(non_overlapping({{num_blocks, value_block_stride}, {block_size, value_page_stride},
                                {kv_heads, value_cache_head_stride}},
                               value_head_size, "paged value cache"));

    // Regions (rope_kv_bridge.rs:149-324).
    const size_t ce = fp8 ? 1 : es;
    Range rq, rk, rv, rp, rc, rkc, rvc, rks, rvs, rs;
    BRIDGE_TRY(byte_range(query, query_elements, es, es, "RoPE query", &rq));
    BRIDGE_TRY(byte_range(key, key_elements, es, es, "RoPE key", &rk));
    BRIDGE_TRY(byte_range(value, value_elements, es, es, "RoPE value", &rv));
    BRIDGE_TRY(byte_range(positions, position_elements, 8, 8, "RoPE positions", &rp));
    BRIDGE_TRY(byte_range(cos_sin_cache, cos_sin_cache_elements, es, es, "RoPE cos/sin cache", &rc));
    BRIDGE_TRY(byte_range(key_cache, key_cache_elements, ce, ce, fp8 ? "paged FP8 key cache" : "paged key cache", &rkc));
    BRIDGE_TRY(byte_range(value_cache, value_cache_elements, ce, ce,
                          fp8 ? "paged FP8 value cache" : "paged value cache", &rvc));
    BRIDGE_TRY(byte_range(key_scales, key_scale_elements, 4, 4, "paged key cache scales", &rks));
    BRIDGE_TRY(byte_range(value_scales, value_scale_elements, 4, 4, "paged value cache scales", &rvs));
    BRIDGE_TRY(byte_range(slot_mapping, slot_mapping_elements, 8, 8, "paged slot mapping", &rs));

    const uint64_t dq = query_head_stride == head_size ? static_cast<uint64_t>(query_heads) * head_size : 0;
    const uint64_t dk = source_key_head_stride == head_size ? static_cast<uint64_t>(kv_heads) * head_size : 0;
    const uint64_t dv =
        source_value_head_stride == value_head_size ? static_cast<uint64_t>(kv_heads) * value_head_size : 0;
    BRIDGE_TRY(disjoint_or_dense_packed("query", rq, query_token_stride, dq, "key", rk, key_token_stride, dk, es, op));
    BRIDGE_TRY(
        disjoint_or_dense_packed("query", rq, query_token_stride, dq, "value", rv, value_token_stride, dv, es, op));
    BRIDGE_TRY(disjoint_or_dense_packed("key", rk, key_token_stride, dk, "value", rv, value_token_stride, dv, es, op));

    uint64_t kblock_span, vblock_span;
    BRIDGE_TRY(strided_span({{block_size, key_page_stride}, {kv_heads, key_head_stride}}, head_size,
                            "paged key cache block", &kblock_span));
    BRIDGE_TRY(strided_span({{block_size, value_page_stride}, {kv_heads, value_cache_head_stride}}, value_head_size,
                            "paged value cache block", &vblock_span));
    const uint64_t k_dense = static_cast<uint64_t>(block_size) * kv_heads * head_size;
    const uint64_t v_dense = static_cast<uint64_t>(block_size) * kv_heads * value_head_size;
    BRIDGE_TRY(disjoint_or_dense_packed("key cache", rkc, key_block_stride, kblock_span == k_dense ? k_dense : 0,
                                        "value cache", rvc, value_block_stride, vblock_span == v_dense ? v_dense : 0,
                                        ce, op));
    const std::initializer_list<std::pair<const char*, Range>> metadata_and_caches = {
        {"positions", rp},     {"cos/sin cache", rc}, {"key cache", rkc},   {"value cache", rvc},
        {"key scales", rks},   {"value scales", rvs}, {"slot mapping", rs}};
    BRIDGE_TRY(disjoint_from("query", rq, metadata_and_caches, op));
    BRIDGE_TRY(disjoint_from("key", rk, metadata_and_caches, op));
    BRIDGE_TRY(disjoint_from("key cache", rkc,
                             {{"value", rv}, {"positions", rp}, {"cos/sin cache", rc}, {"key scales", rks},
                              {"value scales", rvs}, {"slot mapping", rs}},
                             op));
    BRIDGE_TRY(disjoint_from("value cache", rvc,
                             {{"value", rv}, {"positions", rp}, {"cos/sin cache", rc}, {"key scales", rks},
                              {"value scales", rvs}, {"slot mapping", rs}},
                             op));

    // validate_buffers (rope_kv_dispatch.rs:520-560): exact storage spans.
    uint64_t need;
    BRIDGE_TRY(strided_span({{tokens, query_token_stride}, {query_heads, query_head_stride}}, head_size, "RoPE query",
                            &need));
    BRIDGE_TRY(require_len(query_elements, need, "RoPE query"));
    BRIDGE_TRY(strided_span({{tokens, key_token_stride}, {kv_heads, source_key_head_stride}}, head_size, "RoPE key",
                            &need));
    BRIDGE_TRY(require_len(key_elements, need, "RoPE key"));
    BRIDGE_TRY(strided_span({{tokens, value_token_stride}, {kv_heads, source_value_head_stride}}, value_head_size,
                            "RoPE value", &need));
    BRIDGE_TRY(require_len(value_elements, need, "RoPE value"));
    BRIDGE_TRY(require_len(position_elements, tokens, "RoPE positions"));
    BRIDGE_TRY(require_len(cos_sin_cache_elements, static_cast<uint64_t>(max_position) * rotary_dim,
                           "RoPE cos/sin cache"));
    uint64_t kc_need, vc_need;
    if (!mul_ok(static_cast<uint64_t>(num_blocks) - 1, key_block_stride, &kc_need) ||
        !add_ok(kc_need, kblock_span, &kc_need))
      return contract("paged key cache storage span overflows usize");
    if (!mul_ok(static_cast<uint64_t>(num_blocks) - 1, value_block_stride, &vc_need) ||
        !add_ok(vc_need, vblock_span, &vc_need))
      return contract("paged value cache storage span overflows usize");
    BRIDGE_TRY(require_len(key_cache_elements, kc_need, "paged key cache"));
    BRIDGE_TRY(require_len(value_cache_elements, vc_need, "paged value cache"));
    BRIDGE_TRY(require_len(slot_mapping_elements, cache_tokens, "paged slot mapping"));

    const uint32_t scale_stride = key_scale_elements == 1 ? 0U : 1U;
    int status;
    if (dtype == LOOM_HIP_BRIDGE_F32) {
      status = loom_hip_rope_paged_kv_write_f32(
          static_cast<float*>(query), static_cast<float*>(key), static_cast<const float*>(value), positions,
          static_cast<const float*>(cos_sin_cache), key_cache, value_cache, key_scales, value_scales, slot_mapping,
          tokens, cache_tokens, query_heads, kv_heads, head_size, value_head_size, rotary_dim, max_position,
          num_blocks, block_size, cache_encoding, scale_stride, query_token_stride, query_head_stride,
          key_token_stride, source_key_head_stride, value_token_stride, source_value_head_stride, key_block_stride,
          key_page_stride, key_head_stride, value_block_stride, value_page_stride, value_cache_head_stride, is_neox,
          stream);
    } else {
      auto fn = dtype == LOOM_HIP_BRIDGE_F16 ? loom_hip_rope_paged_kv_write_f16 : loom_hip_rope_paged_kv_write_bf16;
      status = fn(static_cast<uint16_t*>(query), static_cast<uint16_t*>(key), static_cast<const uint16_t*>(value),
                  positions, static_cast<const uint16_t*>(cos_sin_cache), key_cache, value_cache, key_scales,
                  value_scales, slot_mapping, tokens, cache_tokens, query_heads, kv_heads, head_size,
                  value_head_size, rotary_dim, max_position, num_blocks, block_size, cache_encoding, scale_stride,
                  query_token_stride, query_head_stride, key_token_stride, source_key_head_stride,
                  value_token_stride, source_value_head_stride, key_block_stride, key_page_stride, key_head_stride,
                  value_block_stride, value_page_stride, value_cache_head_stride, is_neox, stream);
    }
    BRIDGE_TRY(from_core(status));
    g_launches[LOOM_HIP_BRIDGE_ROPE_PAGED_KV_WRITE].fetch_add(1, std::memory_order_relaxed);
    return ok();
  });
}

}  // extern "C"
