// CPU oracle for paged MQA/GQA decode attention.
//
// TEST INFRASTRUCTURE ONLY. This library is the checker that the HIP path is
// compared against. Only tests/, __graft_entry__.smoke() and the cpu_baseline
// leg of bench.py may load it; the product library never links or calls it.
//
// It restates the Loom Kernels Rust contract and CPU reference:
//   - PagedDecodeAttentionSpec::new      crates/loom-kernels/src/attention.rs:34-98
//   - paged_decode_attention_reference   crates/loom-kernels/src/attention.rs:270-357
//   - validate_buffers                   crates/loom-kernels/src/attention.rs:359-402
//   - attention_score / cache_offset     crates/loom-kernels/src/attention.rs:404-426
//   - ContractError + Display            crates/loom-kernels/src/contract.rs:80-301
//   - require_len                        crates/loom-kernels/src/contract.rs:321-335
//   - fp8_e4m3fn_to_f32 / _from_f32      crates/loom-kernels/src/quantization.rs:13-56
//   - KvCacheEncoding scale elements     crates/loom-kernels/src/rope_kv.rs:19-46
//   - validate_kv_scales                 crates/loom-kernels/src/rope_kv.rs:654-667
//   - split-K merge math                 crates/loom-cuda-sys/cuda/src/paged_decode_attention.cu:780-852
// F16/BF16 <-> F32 follow the `half` crate 2.7.1 (Cargo.lock:130-131), which
// is not vendored in the reference: IEEE-754 round-to-nearest-even with NaN
// kept quiet. Tie behaviour is checked against torch's own casts in tests.
//
// Extensions beyond the reference oracle (the reference decode contract has
// no FP8 KV, HND strides, LSE or partition states) are separate functions:
// oracle_paged_decode_attention_ext, oracle_partition_states and
// oracle_merge_states. They keep the reference loop order and F64
// accumulation.

#include <cmath>
#include <cstdint>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <limits>
#include <vector>

#include "oracle.h"

namespace {

enum DType : int32_t { kF32 = 0, kF16 = 1, kBf16 = 2, kFp8E4M3Fn = 3 };

// ContractError variants used by the paged decode path (contract.rs:80-164).
enum ErrorKind : int32_t {
  kOk = 0,
  kZeroDimension = 1,
  kElementCountOverflow = 2,
  kInvalidScale = 3,
  kHeadCountNotDivisible = 4,
  kSequenceLengthOutOfBounds = 5,
  kMaxSequenceLengthOutOfBounds = 6,
  kBlockIdOutOfBounds = 7,
  kLengthMismatch = 8,
  kUnsupportedDType = 9,
};

const char* dtype_debug_name(int32_t dtype) {
  switch (dtype) {
    case kF32: return "F32";
    case kF16: return "F16";
    case kBf16: return "Bf16";
    case kFp8E4M3Fn: return "Fp8E4M3Fn";
    default: return "Unknown";
  }
}

}  // namespace


namespace {

void set_error(OracleError* err, int32_t kind) {
  if (err == nullptr) return;
  std::memset(err, 0, sizeof(*err));
  err->kind = kind;
}

// Rust's `{}` for f32 prints the shortest round-trip decimal; "%g" with
// enough digits is close enough for messages (the tests compare fields).
void format_f32(char* out, size_t n, float v) {
  if (std::isnan(v)) { std::snprintf(out, n, "NaN"); return; }
  if (std::isinf(v)) { std::snprintf(out, n, v > 0 ? "inf" : "-inf"); return; }
  char buf[64];
  for (int prec = 1; prec <= 9; ++prec) {
    std::snprintf(buf, sizeof(buf), "%.*g", prec, static_cast<double>(v));
    if (std::strtof(buf, nullptr) == v) break;
  }
  std::snprintf(out, n, "%s", buf);
}

// Display impl, contract.rs:166-301 (attention variants only).
void render_message(OracleError* e, int32_t dtype_for_unsupported) {
  char f[64];
  switch (e->kind) {
    case kOk: std::snprintf(e->message, sizeof(e->message), "ok"); break;
    case kZeroDimension:
      std::snprintf(e->message, sizeof(e->message), "tensor dimensions must be non-zero");
      break;
    case kElementCountOverflow:
      std::snprintf(e->message, sizeof(e->message), "tensor element count overflowed");
      break;
    case kInvalidScale:
      format_f32(f, sizeof(f), e->fvalue);
      std::snprintf(e->message, sizeof(e->message),
                    "attention scale must be finite and positive, got %s", f);
      break;
    case kHeadCountNotDivisible:
      std::snprintf(e->message, sizeof(e->message),
                    "query head count %llu must be divisible by KV head count %llu",
                    (unsigned long long)e->a, (unsigned long long)e->b);
      break;
    case kSequenceLengthOutOfBounds:
      std::snprintf(e->message, sizeof(e->message),
                    "sequence length %lld for sequence %llu is outside [1, %llu]",
                    (long long)e->value, (unsigned long long)e->a, (unsigned long long)e->b);
      break;
    case kMaxSequenceLengthOutOfBounds:
      std::snprintf(e->message, sizeof(e->message),
                    "maximum sequence length %llu exceeds block-table capacity %llu",
                    (unsigned long long)e->a, (unsigned long long)e->b);
      break;
    case kBlockIdOutOfBounds:
      std::snprintf(e->message, sizeof(e->message),
                    "physical block ID %lld for sequence %llu, logical block %llu is outside [0, %llu)",
                    (long long)e->value, (unsigned long long)e->a, (unsigned long long)e->b,
                    (unsigned long long)e->c);
      break;
    case kLengthMismatch:
      std::snprintf(e->message, sizeof(e->message),
                    "%s length mismatch: expected %llu, got %llu", e->buffer,
                    (unsigned long long)e->a, (unsigned long long)e->b);
      break;
    case kUnsupportedDType:
      std::snprintf(e->message, sizeof(e->message),
                    "CPU reference does not support dtype %s",
                    dtype_debug_name(dtype_for_unsupported));
      break;
    default:
      std::snprintf(e->message, sizeof(e->message), "unknown error");
  }
}

bool checked_mul(uint64_t a, uint64_t b, uint64_t* out) {
  if (a != 0 && b > std::numeric_limits<uint64_t>::max() / a) return false;
  *out = a * b;
  return true;
}

bool checked_product(std::initializer_list<uint64_t> dims) {
  uint64_t p = 1;
  for (uint64_t d : dims) {
    if (!checked_mul(p, d, &p)) return false;
  }
  return true;
}

// ---- element conversions ------------------------------------------------

inline float bits_to_f32(uint32_t bits) {
  float f;
  std::memcpy(&f, &bits, 4);
  return f;
}
inline uint32_t f32_to_bits(float f) {
  uint32_t b;
  std::memcpy(&b, &f, 4);
  return b;
}

inline float bf16_to_f32(uint16_t h) { return bits_to_f32(static_cast<uint32_t>(h) << 16); }

// Round-to-nearest-even F32 -> BF16; NaN stays a quiet NaN with its sign.
inline uint16_t f32_to_bf16(float f) {
  uint32_t x = f32_to_bits(f);
  if ((x & 0x7fffffffU) > 0x7f800000U) {
    return static_cast<uint16_t>((x >> 16) | 0x0040U);
  }
  uint32_t lsb = (x >> 16) & 1U;
  uint32_t rounded = x + 0x7fffU + lsb;
  return static_cast<uint16_t>(rounded >> 16);
}

inline float f16_to_f32(uint16_t h) {
  uint32_t sign = static_cast<uint32_t>(h & 0x8000U) << 16;
  uint32_t exp = (h >> 10) & 0x1fU;
  uint32_t man = h & 0x3ffU;
  if (exp == 0) {
    if (man == 0) return bits_to_f32(sign);
    // subnormal: man * 2^-24
    float v = static_cast<float>(man) * std::ldexp(1.0f, -24);
    return (sign != 0U) ? -v : v;
  }
  if (exp == 0x1fU) {
    return bits_to_f32(sign | 0x7f800000U | (man << 13));
  }
  return bits_to_f32(sign | ((exp + 112U) << 23) | (man << 13));
}

// Round-to-nearest-even F32 -> F16 with overflow to infinity, gradual
// underflow and quiet NaN.
inline uint16_t f32_to_f16(float f) {
  uint32_t x = f32_to_bits(f);
  uint16_t sign = static_cast<uint16_t>((x >> 16) & 0x8000U);
  uint32_t ax = x & 0x7fffffffU;
  if (ax > 0x7f800000U) {
    return static_cast<uint16_t>(sign | 0x7e00U | ((ax >> 13) & 0x3ffU));
  }
  if (ax >= 0x477ff000U) {  // >= 65520 rounds to infinity
    return static_cast<uint16_t>(sign | 0x7c00U);
  }
  if (ax >= 0x38800000U) {  // normal half range (>= 2^-14)
    uint32_t lsb = (ax >> 13) & 1U;
    uint32_t r = ax + 0xfffU + lsb;
    return static_cast<uint16_t>(sign | ((r >> 13) - (112U << 10)));
  }
  if (ax < 0x33000000U) {  // < 2^-25: rounds to zero (2^-25 is a tie -> even 0)
    return sign;
  }
  // subnormal half: value = m * 2^-24 with m in [0, 1024]
  uint32_t e = ax >> 23;
  uint32_t mant = (ax & 0x7fffffU) | 0x800000U;
  uint32_t shift = 126U - e;  // in [14, 24]
  uint32_t half_m = mant >> shift;
  uint32_t rem = mant & ((1U << shift) - 1U);
  uint32_t halfway = 1U << (shift - 1U);
  if (rem > halfway || (rem == halfway && (half_m & 1U))) half_m += 1U;
  return static_cast<uint16_t>(sign | half_m);
}

// quantization.rs:13-29
inline float fp8_e4m3fn_to_f32(uint8_t bits) {
  uint8_t magnitude = bits & 0x7f;
  float sign = (bits & 0x80) == 0 ? 1.0f : -1.0f;
  if (magnitude == 0x7f) {
    return std::copysign(std::numeric_limits<float>::quiet_NaN(), sign);
  }
  int exponent = magnitude >> 3;
  int mantissa = magnitude & 0x07;
  float value;
  if (exponent == 0) {
    value = static_cast<float>(mantissa) * std::ldexp(1.0f, -9);
  } else {
    value = (1.0f + static_cast<float>(mantissa) / 8.0f) * std::ldexp(1.0f, exponent - 7);
  }
  return sign * value;
}

// quantization.rs:32-56 (brute-force RNE with finite saturation)
inline uint8_t fp8_e4m3fn_from_f32(float value) {
  uint8_t sign = std::signbit(value) ? 0x80 : 0x00;
  if (std::isnan(value)) return sign | 0x7f;
  float magnitude = std::fabs(value);
  if (magnitude >= 448.0f) return sign | 0x7e;
  uint8_t best_bits = 0;
  float best_distance = std::numeric_limits<float>::infinity();
  for (int candidate = 0; candidate <= 0x7e; ++candidate) {
    float decoded = fp8_e4m3fn_to_f32(static_cast<uint8_t>(candidate));
    float distance = std::fabs(decoded - magnitude);
    if (distance < best_distance ||
        (distance == best_distance && (candidate & 1) == 0 && (best_bits & 1) != 0)) {
      best_bits = static_cast<uint8_t>(candidate);
      best_distance = distance;
    }
  }
  return sign | best_bits;
}

inline float load_elem(const void* base, uint64_t index, int32_t dtype) {
  switch (dtype) {
    case kF32: return static_cast<const float*>(base)[index];
    case kF16: return f16_to_f32(static_cast<const uint16_t*>(base)[index]);
    case kBf16: return bf16_to_f32(static_cast<const uint16_t*>(base)[index]);
    case kFp8E4M3Fn: return fp8_e4m3fn_to_f32(static_cast<const uint8_t*>(base)[index]);
  }
  return 0.0f;
}

inline void store_elem(void* base, uint64_t index, int32_t dtype, float v) {
  switch (dtype) {
    case kF32: static_cast<float*>(base)[index] = v; break;
    case kF16: static_cast<uint16_t*>(base)[index] = f32_to_f16(v); break;
    case kBf16: static_cast<uint16_t*>(base)[index] = f32_to_bf16(v); break;
    default: break;
  }
}

// ---- spec --------------------------------------------------------------

// PagedDecodeAttentionSpec::new, attention.rs:34-98
int32_t spec_new(uint64_t sequences, uint64_t query_heads, uint64_t kv_heads,
                 uint64_t head_size, uint64_t value_head_size, uint64_t num_blocks,
                 uint64_t block_size, uint64_t max_blocks_per_sequence,
                 uint64_t max_sequence_length, float scale, int32_t dtype,
                 OracleSpec* out, OracleError* err) {
  set_error(err, kOk);
  if (sequences == 0 || query_heads == 0 || kv_heads == 0 || head_size == 0 ||
      value_head_size == 0 || num_blocks == 0 || block_size == 0 ||
      max_blocks_per_sequence == 0 || max_sequence_length == 0) {
    set_error(err, kZeroDimension);
    return kZeroDimension;
  }
  if (query_heads % kv_heads != 0) {
    set_error(err, kHeadCountNotDivisible);
    err->a = query_heads;
    err->b = kv_heads;
    return kHeadCountNotDivisible;
  }
  if (!std::isfinite(scale) || scale <= 0.0f) {
    set_error(err, kInvalidScale);
    err->fvalue = scale;
    return kInvalidScale;
  }
  if (!checked_product({sequences, query_heads, head_size}) ||
      !checked_product({sequences, query_heads, value_head_size}) ||
      !checked_product({num_blocks, block_size, kv_heads, head_size}) ||
      !checked_product({num_blocks, block_size, kv_heads, value_head_size}) ||
      !checked_product({sequences, max_blocks_per_sequence})) {
    set_error(err, kElementCountOverflow);
    return kElementCountOverflow;
  }
  uint64_t capacity;
  if (!checked_mul(max_blocks_per_sequence, block_size, &capacity)) {
    set_error(err, kElementCountOverflow);
    return kElementCountOverflow;
  }
  if (max_sequence_length > capacity) {
    set_error(err, kMaxSequenceLengthOutOfBounds);
    err->a = max_sequence_length;
    err->b = capacity;
    return kMaxSequenceLengthOutOfBounds;
  }
  out->sequences = sequences;
  out->query_heads = query_heads;
  out->kv_heads = kv_heads;
  out->head_size = head_size;
  out->value_head_size = value_head_size;
  out->num_blocks = num_blocks;
  out->block_size = block_size;
  out->max_blocks_per_sequence = max_blocks_per_sequence;
  out->max_sequence_length = max_sequence_length;
  out->scale = scale;
  out->dtype = dtype;
  return kOk;
}

int32_t require_len(const char* buffer, uint64_t actual, uint64_t expected, OracleError* err) {
  if (actual == expected) return kOk;
  set_error(err, kLengthMismatch);
  std::snprintf(err->buffer, sizeof(err->buffer), "%s", buffer);
  err->a = expected;
  err->b = actual;
  return kLengthMismatch;
}

// Metadata half of validate_buffers, attention.rs:380-401: every sequence
// length in [1, max_sequence_length] and every active block ID in
// [0, num_blocks). Negative sentinels in inactive table slots are allowed.
int32_t validate_metadata(const int64_t* block_tables, const int64_t* sequence_lengths,
                          const OracleSpec& s, OracleError* err) {
  for (uint64_t sequence = 0; sequence < s.sequences; ++sequence) {
    int64_t length = sequence_lengths[sequence];
    if (length <= 0 || static_cast<uint64_t>(length) > s.max_sequence_length) {
      set_error(err, kSequenceLengthOutOfBounds);
      err->a = sequence;
      err->b = s.max_sequence_length;
      err->value = length;
      return kSequenceLengthOutOfBounds;
    }
    uint64_t active_blocks = (static_cast<uint64_t>(length) + s.block_size - 1) / s.block_size;
    uint64_t table_offset = sequence * s.max_blocks_per_sequence;
    for (uint64_t logical_block = 0; logical_block < active_blocks; ++logical_block) {
      int64_t block_id = block_tables[table_offset + logical_block];
      if (block_id < 0 || static_cast<uint64_t>(block_id) >= s.num_blocks) {
        set_error(err, kBlockIdOutOfBounds);
        err->a = sequence;
        err->b = logical_block;
        err->c = s.num_blocks;
        err->value = block_id;
        return kBlockIdOutOfBounds;
      }
    }
  }
  return kOk;
}

// Physical row of (sequence, position, kv_head) in element units.
// Dense NHD (attention.rs:413-426) is block_stride = bs*Hkv*D,
// page_stride = Hkv*D, head_stride = D.
struct CacheStrides {
  uint64_t block;
  uint64_t page;
  uint64_t head;
};

inline uint64_t cache_row(uint64_t sequence, uint64_t position, uint64_t kv_head,
                          const int64_t* block_tables, const OracleSpec& s,
                          const CacheStrides& st) {
  uint64_t logical_block = position / s.block_size;
  uint64_t block_offset = position % s.block_size;
  uint64_t table_offset = sequence * s.max_blocks_per_sequence;
  uint64_t physical_block = static_cast<uint64_t>(block_tables[table_offset + logical_block]);
  return physical_block * st.block + block_offset * st.page + kv_head * st.head;
}

struct CacheView {
  const void* data;
  int32_t dtype;      // element type of the stored bytes
  const float* scales;  // nullptr for native caches
  uint32_t scale_stride;
  CacheStrides strides;
};

inline float cache_value(const CacheView& c, uint64_t index, uint64_t kv_head) {
  float v = load_elem(c.data, index, c.dtype);
  if (c.scales != nullptr) v = v * c.scales[kv_head * c.scale_stride];
  return v;
}

// attention_score, attention.rs:404-411: F64 dot of F32-widened elements,
// times the F32 scale widened to F64.
inline double attention_score(const void* query, uint64_t q_off, int32_t q_dtype,
                              const CacheView& key, uint64_t k_off, uint64_t kv_head,
                              uint64_t head_size, float scale) {
  double sum = 0.0;
  for (uint64_t d = 0; d < head_size; ++d) {
    sum += static_cast<double>(load_elem(query, q_off + d, q_dtype)) *
           static_cast<double>(cache_value(key, k_off + d, kv_head));
  }
  return sum * static_cast<double>(scale);
}

// Loop body of paged_decode_attention_reference, attention.rs:292-355, over
// one (sequence, query head). Two passes: F64 max, then F64 exp-weights and
// weighted value sums in position order. Returns the denominator and max.
void attend_one(const void* query, int32_t q_dtype, const CacheView& key,
                const CacheView& value, const int64_t* block_tables,
                uint64_t sequence, uint64_t sequence_length, uint64_t query_head,
                const OracleSpec& s, uint64_t position_begin, uint64_t position_end,
                double* maximum_out, double* denominator_out, double* accumulator) {
  uint64_t queries_per_kv = s.query_heads / s.kv_heads;
  uint64_t kv_head = query_head / queries_per_kv;
  uint64_t q_off = (sequence * s.query_heads + query_head) * s.head_size;
  (void)sequence_length;

  double maximum = -std::numeric_limits<double>::infinity();
  for (uint64_t position = position_begin; position < position_end; ++position) {
    uint64_t k_off = cache_row(sequence, position, kv_head, block_tables, s, key.strides);
    maximum = std::fmax(maximum,
                        attention_score(query, q_off, q_dtype, key, k_off, kv_head,
                                        s.head_size, s.scale));
  }
  double denominator = 0.0;
  for (uint64_t d = 0; d < s.value_head_size; ++d) accumulator[d] = 0.0;
  for (uint64_t position = position_begin; position < position_end; ++position) {
    uint64_t k_off = cache_row(sequence, position, kv_head, block_tables, s, key.strides);
    double weight = std::exp(attention_score(query, q_off, q_dtype, key, k_off, kv_head,
                                             s.head_size, s.scale) -
                             maximum);
    denominator += weight;
    uint64_t v_off = cache_row(sequence, position, kv_head, block_tables, s, value.strides);
    for (uint64_t d = 0; d < s.value_head_size; ++d) {
      accumulator[d] += weight * static_cast<double>(cache_value(value, v_off + d, kv_head));
    }
  }
  *maximum_out = maximum;
  *denominator_out = denominator;
}

}  // namespace

extern "C" {

int32_t oracle_spec_new(uint64_t sequences, uint64_t query_heads, uint64_t kv_heads,
                        uint64_t head_size, uint64_t value_head_size, uint64_t num_blocks,
                        uint64_t block_size, uint64_t max_blocks_per_sequence,
                        uint64_t max_sequence_length, float scale, int32_t dtype,
                        OracleSpec* out, OracleError* err) {
  int32_t rc = spec_new(sequences, query_heads, kv_heads, head_size, value_head_size,
                        num_blocks, block_size, max_blocks_per_sequence,
                        max_sequence_length, scale, dtype, out, err);
  if (err != nullptr) render_message(err, dtype);
  return rc;
}

// paged_decode_attention_{f32,f16,bf16}_reference -> the generic reference,
// attention.rs:169-357. `expected_dtype` selects the element type of every
// buffer (F32 = 0, F16 = 1, BF16 = 2). Buffer lengths are passed so that
// require_len (contract.rs:321-335) is restated exactly. The output is left
// untouched on any error.
int32_t oracle_paged_decode_attention_reference(
    const void* query, uint64_t query_len, const void* key_cache, uint64_t key_len,
    const void* value_cache, uint64_t value_len, const int64_t* block_tables,
    uint64_t block_tables_len, const int64_t* sequence_lengths, uint64_t lengths_len,
    void* output, uint64_t output_len, const OracleSpec* spec, int32_t expected_dtype,
    OracleError* err) {
  set_error(err, kOk);
  const OracleSpec& s = *spec;
  int32_t rc = kOk;
  if (s.dtype != expected_dtype) {
    set_error(err, kUnsupportedDType);
    rc = kUnsupportedDType;
  }
  if (rc == kOk) rc = require_len("query", query_len, s.sequences * s.query_heads * s.head_size, err);
  if (rc == kOk)
    rc = require_len("key_cache", key_len, s.num_blocks * s.block_size * s.kv_heads * s.head_size, err);
  if (rc == kOk)
    rc = require_len("value_cache", value_len,
                     s.num_blocks * s.block_size * s.kv_heads * s.value_head_size, err);
  if (rc == kOk)
    rc = require_len("block_tables", block_tables_len, s.sequences * s.max_blocks_per_sequence, err);
  if (rc == kOk) rc = require_len("sequence_lengths", lengths_len, s.sequences, err);
  if (rc == kOk)
    rc = require_len("output", output_len, s.sequences * s.query_heads * s.value_head_size, err);
  if (rc == kOk) rc = validate_metadata(block_tables, sequence_lengths, s, err);
  if (rc != kOk) {
    render_message(err, s.dtype);
    return rc;
  }

  CacheView key{key_cache, expected_dtype, nullptr, 0,
                {s.block_size * s.kv_heads * s.head_size, s.kv_heads * s.head_size, s.head_size}};
  CacheView value{value_cache, expected_dtype, nullptr, 0,
                  {s.block_size * s.kv_heads * s.value_head_size, s.kv_heads * s.value_head_size,
                   s.value_head_size}};
  std::vector<double> accumulator(s.value_head_size);
  for (uint64_t sequence = 0; sequence < s.sequences; ++sequence) {
    uint64_t length = static_cast<uint64_t>(sequence_lengths[sequence]);
    for (uint64_t query_head = 0; query_head < s.query_heads; ++query_head) {
      double maximum, denominator;
      attend_one(query, expected_dtype, key, value, block_tables, sequence, length, query_head,
                 s, 0, length, &maximum, &denominator, accumulator.data());
      uint64_t o_off = (sequence * s.query_heads + query_head) * s.value_head_size;
      for (uint64_t d = 0; d < s.value_head_size; ++d) {
        store_elem(output, o_off + d, expected_dtype,
                   static_cast<float>(accumulator[d] / denominator));
      }
    }
  }
  render_message(err, s.dtype);
  return kOk;
}

// Extension oracle: the same two-pass F64 algorithm over
//   - query/output of dtype `spec->dtype` (F32/F16/BF16),
//   - K/V caches that are either native (`cache_encoding` 0, same dtype as
//     the query) or OCP FP8 E4M3FN bytes (`cache_encoding` 1) reconstructed
//     as fp8_e4m3fn_to_f32(byte) * scale[kv_head * scale_stride]
//     (docs/design/fp8-kv-cache.md:42-48, rope_kv.rs:19-46),
//   - explicit element strides (block, page, head) for each cache so both
//     NHD and HND views are expressible (layout.rs:204-333 template),
//   - optional LSE per (sequence, query head) = max + ln(denominator), in
//     natural-log units of the scaled scores, computed in F64.
// Caller-side storage lengths are not re-checked here (the C-ABI validates
// spans); metadata and scales are validated before the output is written.
int32_t oracle_paged_decode_attention_ext(
    const void* query, const void* key_cache, const void* value_cache,
    int32_t cache_encoding, const float* key_scales, const float* value_scales,
    uint32_t scale_stride, const int64_t* block_tables, const int64_t* sequence_lengths,
    void* output, double* lse, const OracleSpec* spec, uint64_t key_block_stride,
    uint64_t key_page_stride, uint64_t key_head_stride, uint64_t value_block_stride,
    uint64_t value_page_stride, uint64_t value_head_stride, OracleError* err) {
  set_error(err, kOk);
  const OracleSpec& s = *spec;
  if (s.dtype != kF32 && s.dtype != kF16 && s.dtype != kBf16) {
    set_error(err, kUnsupportedDType);
    render_message(err, s.dtype);
    return kUnsupportedDType;
  }
  if (cache_encoding != 0 && cache_encoding != 1) {
    set_error(err, kUnsupportedDType);
    render_message(err, s.dtype);
    return kUnsupportedDType;
  }
  if (cache_encoding == 1) {
    uint64_t n = scale_stride == 0 ? 1 : s.kv_heads;
    for (uint64_t i = 0; i < n; ++i) {
      for (const float* sc : {key_scales, value_scales}) {
        if (!std::isfinite(sc[i]) || sc[i] <= 0.0f) {
          set_error(err, kInvalidScale);
          err->fvalue = sc[i];
          render_message(err, s.dtype);
          return kInvalidScale;
        }
      }
    }
  }
  int32_t rc = validate_metadata(block_tables, sequence_lengths, s, err);
  if (rc != kOk) {
    render_message(err, s.dtype);
    return rc;
  }
  int32_t cache_dtype = cache_encoding == 1 ? kFp8E4M3Fn : s.dtype;
  CacheView key{key_cache, cache_dtype, cache_encoding == 1 ? key_scales : nullptr,
                scale_stride, {key_block_stride, key_page_stride, key_head_stride}};
  CacheView value{value_cache, cache_dtype, cache_encoding == 1 ? value_scales : nullptr,
                  scale_stride, {value_block_stride, value_page_stride, value_head_stride}};
  std::vector<double> accumulator(s.value_head_size);
  for (uint64_t sequence = 0; sequence < s.sequences; ++sequence) {
    uint64_t length = static_cast<uint64_t>(sequence_lengths[sequence]);
    for (uint64_t query_head = 0; query_head < s.query_heads; ++query_head) {
      double maximum, denominator;
      attend_one(query, s.dtype, key, value, block_tables, sequence, length, query_head, s, 0,
                 length, &maximum, &denominator, accumulator.data());
      uint64_t row = sequence * s.query_heads + query_head;
      for (uint64_t d = 0; d < s.value_head_size; ++d) {
        store_elem(output, row * s.value_head_size + d, s.dtype,
                   static_cast<float>(accumulator[d] / denominator));
      }
      if (lse != nullptr) lse[row] = maximum + std::log(denominator);
    }
  }
  return kOk;
}

// Per-partition softmax states of the extension oracle: for every
// (sequence, query head, partition p) with partition p covering positions
// [p*partition_tokens, min((p+1)*partition_tokens, length)), writes
//   m[row*max_parts + p] = F64 max of the partition's scores,
//   l[...]               = sum of exp(score - m),
//   o[(row*max_parts + p)*Dv + d] = sum of exp(score - m) * v[d].
// Partitions past the end of a sequence get (m, l, o) = (-inf, 0, 0), the
// empty-split convention of paged_decode_attention.cu:553-575.
int32_t oracle_partition_states(
    const void* query, const void* key_cache, const void* value_cache,
    int32_t cache_encoding, const float* key_scales, const float* value_scales,
    uint32_t scale_stride, const int64_t* block_tables, const int64_t* sequence_lengths,
    const OracleSpec* spec, uint64_t key_block_stride, uint64_t key_page_stride,
    uint64_t key_head_stride, uint64_t value_block_stride, uint64_t value_page_stride,
    uint64_t value_head_stride, uint64_t partition_tokens, uint64_t max_parts, double* m,
    double* l, double* o, OracleError* err) {
  set_error(err, kOk);
  const OracleSpec& s = *spec;
  int32_t rc = validate_metadata(block_tables, sequence_lengths, s, err);
  if (rc != kOk) {
    render_message(err, s.dtype);
    return rc;
  }
  int32_t cache_dtype = cache_encoding == 1 ? kFp8E4M3Fn : s.dtype;
  CacheView key{key_cache, cache_dtype, cache_encoding == 1 ? key_scales : nullptr,
                scale_stride, {key_block_stride, key_page_stride, key_head_stride}};
  CacheView value{value_cache, cache_dtype, cache_encoding == 1 ? value_scales : nullptr,
                  scale_stride, {value_block_stride, value_page_stride, value_head_stride}};
  for (uint64_t sequence = 0; sequence < s.sequences; ++sequence) {
    uint64_t length = static_cast<uint64_t>(sequence_lengths[sequence]);
    for (uint64_t query_head = 0; query_head < s.query_heads; ++query_head) {
      uint64_t row = sequence * s.query_heads + query_head;
      for (uint64_t p = 0; p < max_parts; ++p) {
        uint64_t idx = row * max_parts + p;
        uint64_t begin = p * partition_tokens;
        uint64_t end = begin + partition_tokens < length ? begin + partition_tokens : length;
        double* acc = o + idx * s.value_head_size;
        if (begin >= length) {
          m[idx] = -std::numeric_limits<double>::infinity();
          l[idx] = 0.0;
          for (uint64_t d = 0; d < s.value_head_size; ++d) acc[d] = 0.0;
          continue;
        }
        attend_one(query, s.dtype, key, value, block_tables, sequence, length, query_head, s,
                   begin, end, &m[idx], &l[idx], acc);
      }
    }
  }
  return kOk;
}

// Stable log-sum-exp merge of partition states (paged_decode_attention.cu:
// 780-852, in F64): M = max_p m_p; f_p = isfinite(m_p) ? exp(m_p - M) : 0;
// out = sum_p o_p f_p / sum_p l_p f_p; lse = M + ln(sum_p l_p f_p).
void oracle_merge_states(const double* m, const double* l, const double* o, uint64_t rows,
                         uint64_t max_parts, uint64_t value_head_size, double* out,
                         double* lse) {
  std::vector<double> factor(max_parts);
  for (uint64_t row = 0; row < rows; ++row) {
    double global_maximum = -std::numeric_limits<double>::infinity();
    for (uint64_t p = 0; p < max_parts; ++p) global_maximum = std::fmax(global_maximum, m[row * max_parts + p]);
    double denominator = 0.0;
    for (uint64_t p = 0; p < max_parts; ++p) {
      double mp = m[row * max_parts + p];
      factor[p] = std::isfinite(mp) ? std::exp(mp - global_maximum) : 0.0;
      denominator += l[row * max_parts + p] * factor[p];
    }
    for (uint64_t d = 0; d < value_head_size; ++d) {
      double acc = 0.0;
      for (uint64_t p = 0; p < max_parts; ++p) {
        acc += o[(row * max_parts + p) * value_head_size + d] * factor[p];
      }
      out[row * value_head_size + d] = acc / denominator;
    }
    if (lse != nullptr) lse[row] = global_maximum + std::log(denominator);
  }
}

// ---- element helpers exported for the tests -----------------------------

float oracle_fp8_e4m3fn_to_f32(uint8_t bits) { return fp8_e4m3fn_to_f32(bits); }
uint8_t oracle_fp8_e4m3fn_from_f32(float value) { return fp8_e4m3fn_from_f32(value); }
uint16_t oracle_f32_to_bf16(float value) { return f32_to_bf16(value); }
float oracle_bf16_to_f32(uint16_t bits) { return bf16_to_f32(bits); }
uint16_t oracle_f32_to_f16(float value) { return f32_to_f16(value); }
float oracle_f16_to_f32(uint16_t bits) { return f16_to_f32(bits); }

void oracle_fp8_encode_array(const float* src, uint8_t* dst, uint64_t n) {
  for (uint64_t i = 0; i < n; ++i) dst[i] = fp8_e4m3fn_from_f32(src[i]);
}
void oracle_bf16_encode_array(const float* src, uint16_t* dst, uint64_t n) {
  for (uint64_t i = 0; i < n; ++i) dst[i] = f32_to_bf16(src[i]);
}
void oracle_f16_encode_array(const float* src, uint16_t* dst, uint64_t n) {
  for (uint64_t i = 0; i < n; ++i) dst[i] = f32_to_f16(src[i]);
}

}  // extern "C"
