// Shared declarations of the CPU oracle library (test infrastructure only:
// loaded by tests/, __graft_entry__.smoke() and the bench's CPU baseline, never
// by the product library).

#ifndef LOOM_ORACLE_H_
#define LOOM_ORACLE_H_

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

// ContractError variants (crates/loom-kernels/src/contract.rs:80-164) the
// oracle reports; numbering is this library's own.
enum {
  ORACLE_OK = 0,
  ORACLE_ZERO_DIMENSION = 1,
  ORACLE_ELEMENT_COUNT_OVERFLOW = 2,
  ORACLE_INVALID_SCALE = 3,
  ORACLE_HEAD_COUNT_NOT_DIVISIBLE = 4,
  ORACLE_SEQUENCE_LENGTH_OUT_OF_BOUNDS = 5,
  ORACLE_MAX_SEQUENCE_LENGTH_OUT_OF_BOUNDS = 6,
  ORACLE_BLOCK_ID_OUT_OF_BOUNDS = 7,
  ORACLE_LENGTH_MISMATCH = 8,
  ORACLE_UNSUPPORTED_DTYPE = 9,
  ORACLE_INVALID_ROTARY_DIMENSION = 10,
  ORACLE_POSITION_OUT_OF_BOUNDS = 11,
  ORACLE_SLOT_OUT_OF_BOUNDS = 12,
  ORACLE_DUPLICATE_SLOT = 13,
};

struct OracleSpec {
  uint64_t sequences;
  uint64_t query_heads;
  uint64_t kv_heads;
  uint64_t head_size;
  uint64_t value_head_size;
  uint64_t num_blocks;
  uint64_t block_size;
  uint64_t max_blocks_per_sequence;
  uint64_t max_sequence_length;
  float scale;
  int32_t dtype;
};

struct OracleError {
  int32_t kind;
  uint64_t a;  // first usize field of the variant
  uint64_t b;  // second usize field
  uint64_t c;  // third usize field
  int64_t value;  // i64 field (length / block_id / position / slot)
  float fvalue;   // f32 field (scale)
  char buffer[32];
  char message[256];
};

float oracle_fp8_e4m3fn_to_f32(uint8_t bits);
uint8_t oracle_fp8_e4m3fn_from_f32(float value);
uint16_t oracle_f32_to_bf16(float value);
float oracle_bf16_to_f32(uint16_t bits);
uint16_t oracle_f32_to_f16(float value);
float oracle_f16_to_f32(uint16_t bits);

#ifdef __cplusplus
}
#endif

#endif  // LOOM_ORACLE_H_
