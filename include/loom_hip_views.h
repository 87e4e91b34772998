#ifndef LOOM_HIP_VIEWS_H_
#define LOOM_HIP_VIEWS_H_

/*
 * Tensor-view front end of the checked bridge, shared by every framework
 * binding (the torch Stable-ABI adapter and the ctypes operators).
 *
 * A framework describes each operand once as a loom_hip_tensor_view (data
 * pointer, device, element type, sizes and element strides). The library then
 * applies the operator's tensor contract, which it holds as data: one entry
 * per operand (rank, element types, layout class, named dimensions) and one
 * message per rule category. The contract is the one the reference's
 * framework adapters enforce (python/csrc/attention.cpp:5-88 for paged
 * decode, python/csrc/rope_kv.cpp:37-150 for the RoPE + paged-KV write)
 * without the 1024-token decode context cap; the error texts are the
 * reference's. A view set that passes is translated to the element-count
 * spans and strides of include/loom_hip_bridge.h and submitted through that
 * bridge, whose own span, alignment and alias checks then apply.
 *
 * These entry points have no one-to-one counterpart in the reference: they
 * replace the per-framework check-and-marshal code of its adapters.
 */

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* Element types a view may carry. */
enum loom_hip_view_dtype {
  LOOM_HIP_VIEW_F32 = 0,
  LOOM_HIP_VIEW_F16 = 1,
  LOOM_HIP_VIEW_BF16 = 2,
  LOOM_HIP_VIEW_U8 = 3,
  LOOM_HIP_VIEW_FP8_E4M3FN = 4,
  LOOM_HIP_VIEW_I32 = 5,
  LOOM_HIP_VIEW_I64 = 6,
  LOOM_HIP_VIEW_OTHER = 255,
};

#define LOOM_HIP_VIEW_MAX_RANK 5

/* One operand. device_index is the GPU ordinal, or -1 for host memory. */
typedef struct loom_hip_tensor_view {
  const void* data;
  int32_t device_index;
  uint32_t dtype;
  uint32_t rank;
  int64_t sizes[LOOM_HIP_VIEW_MAX_RANK];
  int64_t strides[LOOM_HIP_VIEW_MAX_RANK];
} loom_hip_tensor_view;

/* Results of the view entry points. */
enum loom_hip_views_status {
  LOOM_HIP_VIEWS_OK = 0,
  LOOM_HIP_VIEWS_CONTRACT = 1, /* the views break the operator contract */
  LOOM_HIP_VIEWS_BRIDGE = 2,   /* the bridge refused the call or the launch failed */
};

/* Thread-local text of the last failure on this thread: the contract rule's
 * message, or for LOOM_HIP_VIEWS_BRIDGE the bridge's message and status. */
const char* loom_hip_views_last_error_message(void);

/*
 * Paged decode views, in this order: query [B, Hq, D], key_cache and
 * value_cache [blocks, block_size, Hkv, D|Dv] (dense inner NHD, any block
 * stride of at least one dense block), block_tables [B, max_blocks] int32,
 * sequence_lengths [B] int32, output [B, Hq, Dv]. With count 5 (no output)
 * only the rules on the inputs apply: the capability predicate of
 * python/src/loom_kernels/ops/attention.py:29-96.
 */
int loom_hip_views_paged_decode_check(const loom_hip_tensor_view* views,
                                      uint32_t count,
                                      int64_t max_sequence_length,
                                      double scale);

/* The exact F32 split-K workspace the launch below needs (0: none). */
int loom_hip_views_paged_decode_workspace_elements(
    const loom_hip_tensor_view* views, int64_t max_sequence_length,
    double scale, uint64_t* workspace_elements);

/* Check, then submit through loom_hip_bridge_paged_decode_attention. */
int loom_hip_views_paged_decode_attention(const loom_hip_tensor_view* views,
                                          int64_t max_sequence_length,
                                          double scale, float* workspace,
                                          uint64_t workspace_elements,
                                          void* stream);

/*
 * RoPE + paged-KV write views, in this order: query [T, Hq, D], key
 * [T, Hkv, D], value [T, Hkv, D], positions [T] int64, cos_sin_cache
 * [max_position, rotary_dim], kv_cache [blocks, 2, block_size, Hkv, D]
 * (source dtype, or uint8 FP8 E4M3 bytes), key_scales and value_scales
 * (F32, 1 or Hkv elements), slot_mapping [<= T] int64.
 */
int loom_hip_views_rope_paged_kv_check(const loom_hip_tensor_view* views);

/* Check, then submit through loom_hip_bridge_rope_paged_kv_write. */
int loom_hip_views_rope_paged_kv_write(const loom_hip_tensor_view* views,
                                       uint32_t is_neox, void* stream);

#ifdef __cplusplus
}  /* extern "C" */
#endif

#endif  /* LOOM_HIP_VIEWS_H_ */
