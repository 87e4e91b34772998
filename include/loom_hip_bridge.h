#ifndef LOOM_HIP_BRIDGE_H_
#define LOOM_HIP_BRIDGE_H_

/*
 * Checked C bridge over the loom-hip kernels: the MI355X counterpart of
 * crates/loom-cuda-bridge/include/loom_cuda_bridge.h for the two operators
 * this library implements (RoPE + paged-KV write and paged decode attention).
 *
 * Every buffer arrives with its element count. Before any launch the bridge
 * validates the Loom Kernels contract (attention.rs:34-98, rope_kv.rs:69-211),
 * the strided layouts (loom-cuda layout.rs:107-333), exact storage spans,
 * pointer alignment, and that no written region aliases another region
 * (attention_bridge.rs:71-200, rope_kv_bridge.rs:17-372). Failures return a
 * status and leave a thread-local message; successes count per operator.
 * Pointers are HIP device pointers; `stream` is a hipStream_t (null = the
 * default stream).
 */

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* loom_cuda_bridge.h:10-15 */
enum loom_hip_bridge_status {
  LOOM_HIP_BRIDGE_SUCCESS = 0,
  LOOM_HIP_BRIDGE_INVALID_ARGUMENT = 1,
  LOOM_HIP_BRIDGE_LAUNCH_ERROR = 2,
  LOOM_HIP_BRIDGE_UNAVAILABLE = 3,
};

/* loom_cuda_bridge.h:17-21 */
enum loom_hip_bridge_dtype {
  LOOM_HIP_BRIDGE_F32 = 0,
  LOOM_HIP_BRIDGE_F16 = 1,
  LOOM_HIP_BRIDGE_BF16 = 2,
};

/* loom_cuda_bridge.h:23-26 */
enum loom_hip_bridge_kv_cache_encoding {
  LOOM_HIP_BRIDGE_KV_CACHE_NATIVE = 0,
  LOOM_HIP_BRIDGE_KV_CACHE_FP8_E4M3 = 1,
};

/*
 * Operator ids of loom_cuda_bridge.h:28-40. Only ROPE_PAGED_KV_WRITE and
 * PAGED_DECODE_ATTENTION have entry points here; the other ids stay valid for
 * the telemetry calls and always read 0.
 */
enum loom_hip_bridge_operator {
  LOOM_HIP_BRIDGE_RMS_NORM = 0,
  LOOM_HIP_BRIDGE_ADD_RMS_NORM = 1,
  LOOM_HIP_BRIDGE_RMS_NORM_DYNAMIC_FP8 = 2,
  LOOM_HIP_BRIDGE_SILU_AND_MUL = 3,
  LOOM_HIP_BRIDGE_SILU_AND_MUL_DYNAMIC_FP8 = 4,
  LOOM_HIP_BRIDGE_ROPE_PAGED_KV_WRITE = 5,
  LOOM_HIP_BRIDGE_GREEDY_SAMPLE_LOGPROBS = 6,
  LOOM_HIP_BRIDGE_SELECTED_TOKEN_LOGPROBS = 7,
  LOOM_HIP_BRIDGE_MIN_P_FILTER = 8,
  LOOM_HIP_BRIDGE_PAGED_DECODE_ATTENTION = 9,
  LOOM_HIP_BRIDGE_GREEDY_SPECULATIVE_VERIFY = 10,
};

/* loom_cuda_bridge_abi_version (cuda/mod.rs:719-723): 2. */
uint32_t loom_hip_bridge_abi_version(void);

/* loom_cuda_bridge_last_error_message (cuda/mod.rs:725-731). */
const char* loom_hip_bridge_last_error_message(void);

/* loom_cuda_bridge_launch_count / _reset_launch_count (cuda/mod.rs:733-774). */
int loom_hip_bridge_launch_count(uint32_t operation, uint64_t* count);
int loom_hip_bridge_reset_launch_count(uint32_t operation);

/*
 * loom_cuda_bridge_rope_paged_kv_write (loom_cuda_bridge.h:99-118,
 * rope_kv_bridge.rs:374-515). Element counts are the storage spans of the
 * strided views; cache_tokens must be in [1, tokens]. Scale tensors are
 * always passed (one element, or one per KV head); native caches ignore
 * their values.
 */
int loom_hip_bridge_rope_paged_kv_write(
    uint32_t dtype, uint32_t cache_encoding, void* query,
    uint64_t query_elements, void* key, uint64_t key_elements,
    const void* value, uint64_t value_elements, const int64_t* positions,
    uint64_t position_elements, const void* cos_sin_cache,
    uint64_t cos_sin_cache_elements, void* key_cache,
    uint64_t key_cache_elements, void* value_cache,
    uint64_t value_cache_elements, const float* key_scales,
    uint64_t key_scale_elements, const float* value_scales,
    uint64_t value_scale_elements, const int64_t* slot_mapping,
    uint64_t slot_mapping_elements, uint32_t tokens, uint32_t cache_tokens,
    uint32_t query_heads, uint32_t kv_heads, uint32_t head_size,
    uint32_t value_head_size, uint32_t rotary_dim, uint32_t max_position,
    uint32_t num_blocks, uint32_t block_size, uint64_t query_token_stride,
    uint64_t query_head_stride, uint64_t key_token_stride,
    uint64_t source_key_head_stride, uint64_t value_token_stride,
    uint64_t source_value_head_stride, uint64_t key_block_stride,
    uint64_t key_page_stride, uint64_t key_head_stride,
    uint64_t value_block_stride, uint64_t value_page_stride,
    uint64_t value_cache_head_stride, uint32_t is_neox, void* stream);

/*
 * loom_cuda_bridge_paged_decode_workspace_elements (loom_cuda_bridge.h:120-126,
 * attention_bridge.rs:203-249): the exact F32 workspace the decode call
 * below requires (0 = the single-partition path).
 */
int loom_hip_bridge_paged_decode_workspace_elements(
    uint32_t dtype, uint32_t sequences, uint32_t query_heads,
    uint32_t kv_heads, uint32_t head_size, uint32_t value_head_size,
    uint32_t num_blocks, uint32_t block_size,
    uint32_t max_blocks_per_sequence, uint32_t max_sequence_length,
    float scale, uint64_t* workspace_elements);

/*
 * loom_cuda_bridge_paged_decode_attention (loom_cuda_bridge.h:128-140,
 * attention_bridge.rs:251-347). A null, zero-length workspace selects the
 * single-partition path when the sizing call returns 0; otherwise exactly
 * that many elements select split-K. Dense-inner NHD caches with a block
 * stride of at least one dense block.
 */
int loom_hip_bridge_paged_decode_attention(
    uint32_t dtype, const void* query, uint64_t query_elements,
    const void* key_cache, uint64_t key_cache_elements,
    const void* value_cache, uint64_t value_cache_elements,
    const int32_t* block_tables, uint64_t block_table_elements,
    const int32_t* sequence_lengths, uint64_t sequence_length_elements,
    void* output, uint64_t output_elements, float* workspace,
    uint64_t workspace_elements, uint32_t sequences, uint32_t query_heads,
    uint32_t kv_heads, uint32_t head_size, uint32_t value_head_size,
    uint32_t num_blocks, uint32_t block_size, uint64_t key_block_stride,
    uint64_t value_block_stride, uint32_t max_blocks_per_sequence,
    uint32_t max_sequence_length, float scale, void* stream);

#ifdef __cplusplus
}  /* extern "C" */
#endif

#endif  /* LOOM_HIP_BRIDGE_H_ */
