// CPU oracle for fused RoPE + paged K/V cache writes.
//
// TEST INFRASTRUCTURE ONLY. This is the checker that the HIP write kernel is
// compared against. Only tests/, __graft_entry__.smoke() and the bench's CPU
// baseline may load it; the product library never links or calls it.
//
// It restates crates/loom-kernels/src/rope_kv.rs:
//   RotaryEmbeddingSpec::new                 rope_kv.rs:66-113
//   RopePagedKvWriteSpec::new                rope_kv.rs:176-211
//   KvCacheEncoding::scale_elements          rope_kv.rs:37-46
//   rotary_embedding_reference               rope_kv.rs:499-511
//   rope_paged_kv_write_reference            rope_kv.rs:513-563
//   rope_paged_kv_write_fp8_e4m3_reference   rope_kv.rs:565-631
//   validate_rope_paged_kv_buffers           rope_kv.rs:633-652
//   validate_kv_scales                       rope_kv.rs:654-667
//   validate_rotary_buffers                  rope_kv.rs:669-698
//   validate_slot_mapping                    rope_kv.rs:700-724
//   apply_validated_rotary_embedding         rope_kv.rs:726-757
//   apply_rotary_to_head                     rope_kv.rs:759-777
// and the ContractError messages of contract.rs:184-214. Arithmetic is F32
// with no fused multiply-add (the Makefile builds with -ffp-contract=off), as
// Rust evaluates `first * cosine - second * sine`. Element conversions are the
// ones of paged_decode_oracle.cpp (half 2.7.1 semantics, OCP FP8 E4M3FN).

#include <cmath>
#include <cstdint>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <limits>
#include <unordered_map>

#include "oracle.h"

namespace {

constexpr int32_t kF32 = 0, kF16 = 1, kBf16 = 2, kFp8E4M3Fn = 3;
constexpr int32_t kNeoX = 0, kInterleaved = 1;
constexpr int32_t kNative = 0, kFp8Cache = 1;
constexpr int32_t kPerTensor = 0, kPerHead = 1;

const char* dtype_name(int32_t dtype) {
  switch (dtype) {
    case kF32: return "F32";
    case kF16: return "F16";
    case kBf16: return "Bf16";
    case kFp8E4M3Fn: return "Fp8E4M3Fn";
    default: return "Unknown";
  }
}

void clear(OracleError* e, int32_t kind) {
  if (e == nullptr) return;
  std::memset(e, 0, sizeof(*e));
  e->kind = kind;
}

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

// ContractError Display for the variants this oracle raises.
int32_t fail(OracleError* e, int32_t kind, uint64_t a, uint64_t b, uint64_t c, int64_t value, float fvalue,
             const char* buffer, int32_t dtype) {
  if (e == nullptr) return kind;
  clear(e, kind);
  e->a = a;
  e->b = b;
  e->c = c;
  e->value = value;
  e->fvalue = fvalue;
  if (buffer != nullptr) std::snprintf(e->buffer, sizeof(e->buffer), "%s", buffer);
  char f[64];
  switch (kind) {
    case ORACLE_ZERO_DIMENSION:
      std::snprintf(e->message, sizeof(e->message), "tensor dimensions must be non-zero");
      break;
    case ORACLE_ELEMENT_COUNT_OVERFLOW:
      std::snprintf(e->message, sizeof(e->message), "tensor element count overflowed");
      break;
    case ORACLE_INVALID_ROTARY_DIMENSION:
      std::snprintf(e->message, sizeof(e->message),
                    "rotary dimension must be non-zero, even, and no larger than head size; got rotary_dim=%llu, "
                    "head_size=%llu",
                    (unsigned long long)a, (unsigned long long)b);
      break;
    case ORACLE_POSITION_OUT_OF_BOUNDS:
      std::snprintf(e->message, sizeof(e->message), "position %lld for token %llu is outside [0, %llu)",
                    (long long)value, (unsigned long long)a, (unsigned long long)b);
      break;
    case ORACLE_SLOT_OUT_OF_BOUNDS:
      std::snprintf(e->message, sizeof(e->message), "cache slot %lld for token %llu is outside [0, %llu)",
                    (long long)value, (unsigned long long)a, (unsigned long long)b);
      break;
    case ORACLE_DUPLICATE_SLOT:
      std::snprintf(e->message, sizeof(e->message), "cache slot %llu is assigned to both token %llu and token %llu",
                    (unsigned long long)c, (unsigned long long)a, (unsigned long long)b);
      break;
    case ORACLE_LENGTH_MISMATCH:
      std::snprintf(e->message, sizeof(e->message), "%s length mismatch: expected %llu, got %llu", e->buffer,
                    (unsigned long long)a, (unsigned long long)b);
      break;
    case ORACLE_INVALID_SCALE:
      format_f32(f, sizeof(f), fvalue);
      std::snprintf(e->message, sizeof(e->message), "attention scale must be finite and positive, got %s", f);
      break;
    case ORACLE_UNSUPPORTED_DTYPE:
      std::snprintf(e->message, sizeof(e->message), "CPU reference does not support dtype %s", dtype_name(dtype));
      break;
    default:
      std::snprintf(e->message, sizeof(e->message), "unknown error");
  }
  return kind;
}

bool mul_ok(uint64_t a, uint64_t b, uint64_t* out) {
  if (a != 0 && b > std::numeric_limits<uint64_t>::max() / a) return false;
  *out = a * b;
  return true;
}

// Storage element access: `data` holds F32 or 16-bit values (the spec dtype).
float load(const void* data, uint64_t i, int32_t dtype) {
  if (dtype == kF32) return static_cast<const float*>(data)[i];
  const uint16_t bits = static_cast<const uint16_t*>(data)[i];
  return dtype == kF16 ? oracle_f16_to_f32(bits) : oracle_bf16_to_f32(bits);
}

void store(void* data, uint64_t i, int32_t dtype, float v) {
  if (dtype == kF32) {
    static_cast<float*>(data)[i] = v;
  } else {
    static_cast<uint16_t*>(data)[i] = dtype == kF16 ? oracle_f32_to_f16(v) : oracle_f32_to_bf16(v);
  }
}

uint64_t elem_bytes(int32_t dtype) { return dtype == kF32 ? 4 : 2; }

}  // namespace

extern "C" {

struct OracleRotarySpec {
  uint64_t tokens;
  uint64_t query_heads;
  uint64_t key_heads;
  uint64_t head_size;
  uint64_t rotary_dim;
  uint64_t max_position;
  int32_t dtype;
  int32_t style;  // 0 = NeoX, 1 = Interleaved
};

struct OracleRopeWriteSpec {
  OracleRotarySpec rotary;
  uint64_t value_head_size;
  uint64_t num_blocks;
  uint64_t block_size;
  int32_t encoding;     // 0 = native, 1 = FP8 E4M3FN
  int32_t granularity;  // FP8 scales: 0 = per tensor, 1 = per KV head
};

// RotaryEmbeddingSpec::new (rope_kv.rs:66-113).
int32_t oracle_rotary_spec_new(uint64_t tokens, uint64_t query_heads, uint64_t key_heads, uint64_t head_size,
                               uint64_t rotary_dim, uint64_t max_position, int32_t dtype, int32_t style,
                               OracleRotarySpec* out, OracleError* err) {
  clear(err, ORACLE_OK);
  if (tokens == 0 || query_heads == 0 || key_heads == 0 || head_size == 0 || max_position == 0)
    return fail(err, ORACLE_ZERO_DIMENSION, 0, 0, 0, 0, 0.f, nullptr, 0);
  if (rotary_dim == 0 || rotary_dim % 2 != 0 || rotary_dim > head_size)
    return fail(err, ORACLE_INVALID_ROTARY_DIMENSION, rotary_dim, head_size, 0, 0, 0.f, nullptr, 0);
  uint64_t t;
  if (!mul_ok(tokens, query_heads, &t) || !mul_ok(t, head_size, &t) || !mul_ok(tokens, key_heads, &t) ||
      !mul_ok(t, head_size, &t) || !mul_ok(max_position, rotary_dim, &t))
    return fail(err, ORACLE_ELEMENT_COUNT_OVERFLOW, 0, 0, 0, 0, 0.f, nullptr, 0);
  *out = OracleRotarySpec{tokens, query_heads, key_heads, head_size, rotary_dim, max_position, dtype, style};
  return ORACLE_OK;
}

// RopePagedKvWriteSpec::new (rope_kv.rs:176-211).
int32_t oracle_rope_write_spec_new(const OracleRotarySpec* rotary, uint64_t value_head_size, uint64_t num_blocks,
                                   uint64_t block_size, int32_t encoding, int32_t granularity,
                                   OracleRopeWriteSpec* out, OracleError* err) {
  clear(err, ORACLE_OK);
  if (value_head_size == 0 || num_blocks == 0 || block_size == 0)
    return fail(err, ORACLE_ZERO_DIMENSION, 0, 0, 0, 0, 0.f, nullptr, 0);
  uint64_t t;
  if (!mul_ok(rotary->tokens, rotary->key_heads, &t) || !mul_ok(t, value_head_size, &t) ||
      !mul_ok(num_blocks, block_size, &t) || !mul_ok(t, rotary->key_heads, &t) || !mul_ok(t, rotary->head_size, &t) ||
      !mul_ok(num_blocks, block_size, &t) || !mul_ok(t, rotary->key_heads, &t) || !mul_ok(t, value_head_size, &t))
    return fail(err, ORACLE_ELEMENT_COUNT_OVERFLOW, 0, 0, 0, 0, 0.f, nullptr, 0);
  *out = OracleRopeWriteSpec{*rotary, value_head_size, num_blocks, block_size, encoding, granularity};
  return ORACLE_OK;
}

uint64_t oracle_rope_scale_elements(const OracleRopeWriteSpec* spec) {
  if (spec->encoding == kNative) return 0;
  return spec->granularity == kPerTensor ? 1 : spec->rotary.key_heads;
}

}  // extern "C"

namespace {

int32_t require_len(OracleError* err, const char* name, uint64_t actual, uint64_t expected) {
  if (actual != expected) return fail(err, ORACLE_LENGTH_MISMATCH, expected, actual, 0, 0, 0.f, name, 0);
  return ORACLE_OK;
}

// validate_rotary_buffers (rope_kv.rs:669-698).
int32_t validate_rotary(const OracleRotarySpec& s, int32_t expected_dtype, uint64_t qlen, uint64_t klen,
                        const int64_t* positions, uint64_t plen, uint64_t clen, OracleError* err) {
  if (s.dtype != expected_dtype) return fail(err, ORACLE_UNSUPPORTED_DTYPE, 0, 0, 0, 0, 0.f, nullptr, s.dtype);
  int32_t st;
  if ((st = require_len(err, "query", qlen, s.tokens * s.query_heads * s.head_size))) return st;
  if ((st = require_len(err, "key", klen, s.tokens * s.key_heads * s.head_size))) return st;
  if ((st = require_len(err, "positions", plen, s.tokens))) return st;
  if ((st = require_len(err, "cos_sin_cache", clen, s.max_position * s.rotary_dim))) return st;
  for (uint64_t t = 0; t < s.tokens; ++t) {
    const int64_t p = positions[t];
    if (p < 0 || static_cast<uint64_t>(p) >= s.max_position)
      return fail(err, ORACLE_POSITION_OUT_OF_BOUNDS, t, s.max_position, 0, p, 0.f, nullptr, 0);
  }
  return ORACLE_OK;
}

// validate_slot_mapping (rope_kv.rs:700-724): bounds, then first duplicate in token order.
int32_t validate_slots(const int64_t* slots, uint64_t n, uint64_t capacity, OracleError* err) {
  std::unordered_map<uint64_t, uint64_t> owners;
  for (uint64_t t = 0; t < n; ++t) {
    const int64_t slot = slots[t];
    if (slot < 0) continue;
    if (static_cast<uint64_t>(slot) >= capacity)
      return fail(err, ORACLE_SLOT_OUT_OF_BOUNDS, t, capacity, 0, slot, 0.f, nullptr, 0);
    auto it = owners.find(static_cast<uint64_t>(slot));
    if (it != owners.end())
      return fail(err, ORACLE_DUPLICATE_SLOT, it->second, t, static_cast<uint64_t>(slot), 0, 0.f, nullptr, 0);
    owners.emplace(static_cast<uint64_t>(slot), t);
  }
  return ORACLE_OK;
}

// apply_rotary_to_head (rope_kv.rs:759-777): F32 products and sums, no fusion.
void rotate_head(void* data, uint64_t off, const void* cos_sin, uint64_t row, const OracleRotarySpec& s) {
  const uint64_t half = s.rotary_dim / 2;
  for (uint64_t pair = 0; pair < half; ++pair) {
    const uint64_t i1 = s.style == kNeoX ? pair : pair * 2;
    const uint64_t i2 = s.style == kNeoX ? pair + half : pair * 2 + 1;
    const float first = load(data, off + i1, s.dtype);
    const float second = load(data, off + i2, s.dtype);
    const float cosine = load(cos_sin, row + pair, s.dtype);
    const float sine = load(cos_sin, row + half + pair, s.dtype);
    const float a = first * cosine;
    const float b = second * sine;
    const float c = second * cosine;
    const float d = first * sine;
    store(data, off + i1, s.dtype, a - b);
    store(data, off + i2, s.dtype, c + d);
  }
}

// apply_validated_rotary_embedding (rope_kv.rs:726-757).
void rotate_all(void* query, void* key, const int64_t* positions, const void* cos_sin, const OracleRotarySpec& s) {
  for (uint64_t t = 0; t < s.tokens; ++t) {
    const uint64_t row = static_cast<uint64_t>(positions[t]) * s.rotary_dim;
    for (uint64_t h = 0; h < s.query_heads; ++h) rotate_head(query, (t * s.query_heads + h) * s.head_size, cos_sin, row, s);
    for (uint64_t h = 0; h < s.key_heads; ++h) rotate_head(key, (t * s.key_heads + h) * s.head_size, cos_sin, row, s);
  }
}

}  // namespace

extern "C" {

// rotary_embedding_reference (rope_kv.rs:499-511). Buffer lengths are in
// elements; query/key are mutated only on success.
int32_t oracle_rotary_embedding(void* query, uint64_t qlen, void* key, uint64_t klen, const int64_t* positions,
                                uint64_t plen, const void* cos_sin, uint64_t clen, const OracleRotarySpec* spec,
                                int32_t expected_dtype, OracleError* err) {
  clear(err, ORACLE_OK);
  const int32_t st = validate_rotary(*spec, expected_dtype, qlen, klen, positions, plen, clen, err);
  if (st) return st;
  rotate_all(query, key, positions, cos_sin, *spec);
  return ORACLE_OK;
}

// rope_paged_kv_write_reference / rope_paged_kv_write_fp8_e4m3_reference
// (rope_kv.rs:513-631) on contiguous NHD caches [num_blocks, block_size,
// key_heads, dim]: elements of the spec dtype (native) or FP8 bytes. Scales
// are ignored for native caches. Nothing is mutated on error.
int32_t oracle_rope_paged_kv_write(void* query, uint64_t qlen, void* key, uint64_t klen, const void* value,
                                   uint64_t vlen, const int64_t* positions, uint64_t plen, const void* cos_sin,
                                   uint64_t clen, void* key_cache, uint64_t kclen, void* value_cache, uint64_t vclen,
                                   const int64_t* slots, uint64_t slen, const float* key_scales, uint64_t kslen,
                                   const float* value_scales, uint64_t vslen, const OracleRopeWriteSpec* spec,
                                   int32_t expected_dtype, OracleError* err) {
  clear(err, ORACLE_OK);
  const OracleRotarySpec& r = spec->rotary;
  // The reference has one entry per encoding (rope_kv.rs:525-527, 580-585);
  // here the spec's encoding selects it.
  if (spec->encoding != kNative && spec->encoding != kFp8Cache)
    return fail(err, ORACLE_UNSUPPORTED_DTYPE, 0, 0, 0, 0, 0.f, nullptr, r.dtype);
  int32_t st = validate_rotary(r, expected_dtype, qlen, klen, positions, plen, clen, err);
  if (st) return st;
  const uint64_t slots_cap = spec->num_blocks * spec->block_size;
  if ((st = require_len(err, "value", vlen, r.tokens * r.key_heads * spec->value_head_size))) return st;
  if ((st = require_len(err, "key_cache", kclen, slots_cap * r.key_heads * r.head_size))) return st;
  if ((st = require_len(err, "value_cache", vclen, slots_cap * r.key_heads * spec->value_head_size))) return st;
  if ((st = require_len(err, "slot_mapping", slen, r.tokens))) return st;
  if ((st = validate_slots(slots, slen, slots_cap, err))) return st;
  const bool fp8 = spec->encoding == kFp8Cache;
  if (fp8) {
    const uint64_t n = oracle_rope_scale_elements(spec);
    if ((st = require_len(err, "key_scales", kslen, n))) return st;
    if ((st = require_len(err, "value_scales", vslen, n))) return st;
    for (uint64_t i = 0; i < 2 * n; ++i) {
      const float v = i < n ? key_scales[i] : value_scales[i - n];
      if (!std::isfinite(v) || v <= 0.0f) return fail(err, ORACLE_INVALID_SCALE, 0, 0, 0, 0, v, nullptr, 0);
    }
  }

  rotate_all(query, key, positions, cos_sin, r);

  const uint64_t D = r.head_size, Dv = spec->value_head_size, H = r.key_heads;
  for (uint64_t t = 0; t < r.tokens; ++t) {
    if (slots[t] < 0) continue;
    const uint64_t slot = static_cast<uint64_t>(slots[t]);
    for (uint64_t h = 0; h < H; ++h) {
      const uint64_t sk = (t * H + h) * D, tk = (slot * H + h) * D;
      const uint64_t sv = (t * H + h) * Dv, tv = (slot * H + h) * Dv;
      if (!fp8) {
        std::memcpy(static_cast<uint8_t*>(key_cache) + tk * elem_bytes(r.dtype),
                    static_cast<const uint8_t*>(key) + sk * elem_bytes(r.dtype), D * elem_bytes(r.dtype));
        std::memcpy(static_cast<uint8_t*>(value_cache) + tv * elem_bytes(r.dtype),
                    static_cast<const uint8_t*>(value) + sv * elem_bytes(r.dtype), Dv * elem_bytes(r.dtype));
      } else {
        const uint64_t si = spec->granularity == kPerTensor ? 0 : h;
        const float ks = key_scales[si], vs = value_scales[si];
        for (uint64_t d = 0; d < D; ++d)
          static_cast<uint8_t*>(key_cache)[tk + d] = oracle_fp8_e4m3fn_from_f32(load(key, sk + d, r.dtype) / ks);
        for (uint64_t d = 0; d < Dv; ++d)
          static_cast<uint8_t*>(value_cache)[tv + d] = oracle_fp8_e4m3fn_from_f32(load(value, sv + d, r.dtype) / vs);
      }
    }
  }
  return ORACLE_OK;
}

}  // extern "C"
