#ifndef LOOM_HIP_H_
#define LOOM_HIP_H_

/*
 * loom-hip: MI355X (gfx950) launch ABI for paged MQA/GQA decode attention.
 *
 * Drop-in replacement for the paged-decode part of the Loom Kernels internal
 * CUDA launch ABI (crates/loom-cuda-sys/cuda/include/loom_cuda.h). Every
 * reference entry point keeps its argument list, argument meaning, integer
 * widths and status codes; `void* stream` is a hipStream_t (null = the
 * default stream). Launches are asynchronous on that stream, allocate
 * nothing and never synchronize the host.
 *
 * Differences from the reference kernels, all widening the accepted set:
 *   - no 1024-token context cap (the reference's kMaxContext,
 *     paged_decode_attention.cu:29); the contract and CPU oracle never had
 *     one (crates/loom-kernels/src/attention.rs:34-98);
 *   - the split-K policy is MI355X's own (fixed-size partitions merged by a
 *     stable log-sum-exp kernel) and is not limited to batch <= 8.
 * Extensions (no reference counterpart in the decode ABI; vocabulary taken
 * from the reference's RoPE+KV-write ABI, loom_cuda.h:252-318):
 *   - FP8 E4M3FN K/V caches with static per-tensor or per-KV-head scales,
 *   - explicit block/page/head element strides (NHD and HND views),
 *   - an optional F32 log-sum-exp output per (sequence, query head),
 *   - a caller-chosen split-K partition size.
 *
 * Metadata (block tables, sequence lengths) is trusted on the device exactly
 * as in the reference: active sequence lengths must lie in
 * [1, max_sequence_length] and active block IDs in [0, num_blocks).
 */

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* Status codes: loom_cuda.h:10-16. */
enum LoomHipStatus {
  LOOM_HIP_SUCCESS = 0,
  LOOM_HIP_INVALID_ARGUMENT = 1,
  LOOM_HIP_UNSUPPORTED = 2,
  LOOM_HIP_LAUNCH_ERROR = 3,
  LOOM_HIP_UNAVAILABLE = 4,
};

/* K/V cache encodings: loom_cuda.h:18-21 (LoomCudaKvCacheEncoding). */
enum LoomHipKvCacheEncoding {
  LOOM_HIP_KV_CACHE_NATIVE = 0,
  LOOM_HIP_KV_CACHE_FP8_E4M3 = 1,
};

/* Element types of query/output: loom_cuda_bridge.h:17-21. */
enum LoomHipDType {
  LOOM_HIP_F32 = 0,
  LOOM_HIP_F16 = 1,
  LOOM_HIP_BF16 = 2,
};

/* Operator ids for launch telemetry: loom_cuda_bridge.h:28-40. */
enum LoomHipOperator {
  LOOM_HIP_ROPE_PAGED_KV_WRITE = 5,
  LOOM_HIP_PAGED_DECODE_ATTENTION = 9,
};

/* Kernel ids for loom_hip_kernel_timing_read. */
enum LoomHipKernel {
  LOOM_HIP_KERNEL_DECODE = 0, /* per-(sequence, KV head, partition) kernel */
  LOOM_HIP_KERNEL_MERGE = 1,  /* split-K log-sum-exp merge kernel */
  LOOM_HIP_KERNEL_ROPE = 2,   /* fused RoPE + paged-KV write kernel */
};

/* Replaces loom_cuda_status_string (rms_norm.cu:170-185). */
const char* loom_hip_status_string(int status);

/*
 * Base paged decode attention. Replaces loom_cuda_paged_decode_attention_
 * {f32,f16,bf16} (loom_cuda.h:182-212; definitions paged_decode_attention.cu:
 * 1168-1210). Query/output are contiguous [sequences, query_heads, dim];
 * K/V caches have dense inner NHD [block_size, kv_heads, dim] dimensions and
 * an explicit element stride between blocks (separate caches or vLLM's
 * interleaved [blocks, 2, block_size, kv_heads, dim] storage). F16/BF16 data
 * is passed as uint16_t bit patterns. No caller workspace: a (sequence, KV
 * head) is reduced inside one workgroup, except for small grids with long
 * contexts, which the library splits over a slot of its own (see
 * loom_hip_last_internal_partition_tokens).
 */
int loom_hip_paged_decode_attention_f32(
    const float* query, const float* key_cache, const float* value_cache,
    const int32_t* block_tables, const int32_t* sequence_lengths,
    float* output, uint32_t sequences, uint32_t query_heads,
    uint32_t kv_heads, uint32_t head_size, uint32_t value_head_size,
    uint32_t num_blocks, uint32_t block_size, uint64_t key_block_stride,
    uint64_t value_block_stride, uint32_t max_blocks_per_sequence,
    uint32_t max_sequence_length, float scale, void* stream);

int loom_hip_paged_decode_attention_f16(
    const uint16_t* query, const uint16_t* key_cache,
    const uint16_t* value_cache, const int32_t* block_tables,
    const int32_t* sequence_lengths, uint16_t* output, uint32_t sequences,
    uint32_t query_heads, uint32_t kv_heads, uint32_t head_size,
    uint32_t value_head_size, uint32_t num_blocks, uint32_t block_size,
    uint64_t key_block_stride, uint64_t value_block_stride,
    uint32_t max_blocks_per_sequence, uint32_t max_sequence_length,
    float scale, void* stream);

int loom_hip_paged_decode_attention_bf16(
    const uint16_t* query, const uint16_t* key_cache,
    const uint16_t* value_cache, const int32_t* block_tables,
    const int32_t* sequence_lengths, uint16_t* output, uint32_t sequences,
    uint32_t query_heads, uint32_t kv_heads, uint32_t head_size,
    uint32_t value_head_size, uint32_t num_blocks, uint32_t block_size,
    uint64_t key_block_stride, uint64_t value_block_stride,
    uint32_t max_blocks_per_sequence, uint32_t max_sequence_length,
    float scale, void* stream);

/*
 * Split-K workspace sizing. Replaces loom_cuda_paged_decode_attention_split_
 * k_workspace_elements (loom_cuda.h:219-222; paged_decode_attention.cu:
 * 1156-1166). Returns zero when the shape should use the base entry points
 * (enough (sequence, KV head) work to fill the GPU, or a context too short to
 * split); otherwise the F32 element count of the caller-owned workspace.
 */
uint64_t loom_hip_paged_decode_attention_split_k_workspace_elements(
    uint32_t sequences, uint32_t query_heads, uint32_t kv_heads,
    uint32_t head_size, uint32_t value_head_size,
    uint32_t max_sequence_length);

/*
 * Split-K paged decode attention. Replaces loom_cuda_paged_decode_attention_
 * split_k_{f32,f16,bf16} (loom_cuda.h:224-250; paged_decode_attention.cu:
 * 1212-1276). `workspace` must hold at least the element count returned by
 * the sizing function for the same shape, which must be non-zero.
 */
int loom_hip_paged_decode_attention_split_k_f32(
    const float* query, const float* key_cache, const float* value_cache,
    const int32_t* block_tables, const int32_t* sequence_lengths,
    float* output, float* workspace, uint64_t workspace_elements,
    uint32_t sequences, uint32_t query_heads, uint32_t kv_heads,
    uint32_t head_size, uint32_t value_head_size, uint32_t num_blocks,
    uint32_t block_size, uint64_t key_block_stride,
    uint64_t value_block_stride, uint32_t max_blocks_per_sequence,
    uint32_t max_sequence_length, float scale, void* stream);

int loom_hip_paged_decode_attention_split_k_f16(
    const uint16_t* query, const uint16_t* key_cache,
    const uint16_t* value_cache, const int32_t* block_tables,
    const int32_t* sequence_lengths, uint16_t* output, float* workspace,
    uint64_t workspace_elements, uint32_t sequences, uint32_t query_heads,
    uint32_t kv_heads, uint32_t head_size, uint32_t value_head_size,
    uint32_t num_blocks, uint32_t block_size, uint64_t key_block_stride,
    uint64_t value_block_stride, uint32_t max_blocks_per_sequence,
    uint32_t max_sequence_length, float scale, void* stream);

int loom_hip_paged_decode_attention_split_k_bf16(
    const uint16_t* query, const uint16_t* key_cache,
    const uint16_t* value_cache, const int32_t* block_tables,
    const int32_t* sequence_lengths, uint16_t* output, float* workspace,
    uint64_t workspace_elements, uint32_t sequences, uint32_t query_heads,
    uint32_t kv_heads, uint32_t head_size, uint32_t value_head_size,
    uint32_t num_blocks, uint32_t block_size, uint64_t key_block_stride,
    uint64_t value_block_stride, uint32_t max_blocks_per_sequence,
    uint32_t max_sequence_length, float scale, void* stream);

/*
 * Extended entry points (no reference counterpart in the decode ABI; they
 * replace nothing and add FP8 KV, strides, LSE and fixed partitions).
 *
 * Workspace for the extended entry points: returns B*Hq*P*(Dv+2) F32
 * elements with P = ceil(max_sequence_length / partition_tokens), or zero
 * when P <= 1 or partition_tokens == 0 (single partition, no workspace).
 */
uint64_t loom_hip_paged_decode_attention_extended_workspace_elements(
    uint32_t sequences, uint32_t query_heads, uint32_t value_head_size,
    uint32_t max_sequence_length, uint32_t partition_tokens);

/*
 * Query/output are contiguous [sequences, query_heads, dim] of the entry
 * point's dtype. The caches are logical [num_blocks, block_size, kv_heads,
 * dim] views with unit dim stride and the given block/page/head element
 * strides: NHD is (bs*Hkv*D, Hkv*D, D), HND is (Hkv*bs*D, D, bs*D).
 * cache_encoding NATIVE: cache elements have the query dtype and the scale
 * pointers must be null. FP8_E4M3: cache elements are OCP E4M3FN bytes and
 * the logical value is fp8_to_f32(byte) * scale[kv_head * scale_stride]
 * (scale_stride 0 = per tensor, 1 = per KV head; scales finite, > 0).
 * `lse` (nullable) receives [sequences, query_heads] F32 natural-log
 * log-sum-exp of the scaled scores. partition_tokens == 0 means one
 * partition per sequence. The workspace must be null with zero elements when
 * the sizing function returns 0, and hold at least that many otherwise.
 */
int loom_hip_paged_decode_attention_extended_f32(
    const float* query, const void* key_cache, const void* value_cache,
    const float* key_scales, const float* value_scales,
    const int32_t* block_tables, const int32_t* sequence_lengths,
    float* output, float* lse, float* workspace, uint64_t workspace_elements,
    uint32_t sequences, uint32_t query_heads, uint32_t kv_heads,
    uint32_t head_size, uint32_t value_head_size, uint32_t num_blocks,
    uint32_t block_size, uint32_t cache_encoding, uint32_t scale_stride,
    uint64_t key_block_stride, uint64_t key_page_stride,
    uint64_t key_head_stride, uint64_t value_block_stride,
    uint64_t value_page_stride, uint64_t value_head_stride,
    uint32_t max_blocks_per_sequence, uint32_t max_sequence_length,
    uint32_t partition_tokens, float scale, void* stream);

int loom_hip_paged_decode_attention_extended_f16(
    const uint16_t* query, const void* key_cache, const void* value_cache,
    const float* key_scales, const float* value_scales,
    const int32_t* block_tables, const int32_t* sequence_lengths,
    uint16_t* output, float* lse, float* workspace,
    uint64_t workspace_elements, uint32_t sequences, uint32_t query_heads,
    uint32_t kv_heads, uint32_t head_size, uint32_t value_head_size,
    uint32_t num_blocks, uint32_t block_size, uint32_t cache_encoding,
    uint32_t scale_stride, uint64_t key_block_stride,
    uint64_t key_page_stride, uint64_t key_head_stride,
    uint64_t value_block_stride, uint64_t value_page_stride,
    uint64_t value_head_stride, uint32_t max_blocks_per_sequence,
    uint32_t max_sequence_length, uint32_t partition_tokens, float scale,
    void* stream);

int loom_hip_paged_decode_attention_extended_bf16(
    const uint16_t* query, const void* key_cache, const void* value_cache,
    const float* key_scales, const float* value_scales,
    const int32_t* block_tables, const int32_t* sequence_lengths,
    uint16_t* output, float* lse, float* workspace,
    uint64_t workspace_elements, uint32_t sequences, uint32_t query_heads,
    uint32_t kv_heads, uint32_t head_size, uint32_t value_head_size,
    uint32_t num_blocks, uint32_t block_size, uint32_t cache_encoding,
    uint32_t scale_stride, uint64_t key_block_stride,
    uint64_t key_page_stride, uint64_t key_head_stride,
    uint64_t value_block_stride, uint64_t value_page_stride,
    uint64_t value_head_stride, uint32_t max_blocks_per_sequence,
    uint32_t max_sequence_length, uint32_t partition_tokens, float scale,
    void* stream);

/*
 * No-allocation variant of loom_hip_paged_decode_attention_extended_*. It has
 * no counterpart in the reference: it is for callers that cannot allocate
 * device memory (code under HIP graph capture, serving loops, harnesses that
 * forbid hipMalloc). `dtype` is a LoomHipDType; every other argument means
 * what it means for the extended entry point of that dtype, and the results
 * are the same. The split-K partial states go to a static array of
 * LOOM_HIP_STATIC_WORKSPACE_ELEMENTS F32 elements (64 MiB) that the library
 * holds on each device it runs on until the process ends. A call whose
 * states need more (the extended sizing function's count) returns
 * LOOM_HIP_UNSUPPORTED before launching anything. Nothing is allocated,
 * freed or cleared by the call. The array used is the current device's, so
 * `stream` must belong to the current device (LOOM_HIP_INVALID_ARGUMENT
 * otherwise). All calls on one device share that device's array: calls that
 * may overlap in time on one device (different streams, or different threads
 * without ordering) race and must not be issued.
 */
#define LOOM_HIP_STATIC_WORKSPACE_ELEMENTS (16ULL * 1024ULL * 1024ULL)

int loom_hip_paged_decode_attention_extended_no_alloc(
    uint32_t dtype, const void* query, const void* key_cache,
    const void* value_cache, const float* key_scales,
    const float* value_scales, const int32_t* block_tables,
    const int32_t* sequence_lengths, void* output, float* lse,
    uint32_t sequences, uint32_t query_heads, uint32_t kv_heads,
    uint32_t head_size, uint32_t value_head_size, uint32_t num_blocks,
    uint32_t block_size, uint32_t cache_encoding, uint32_t scale_stride,
    uint64_t key_block_stride, uint64_t key_page_stride,
    uint64_t key_head_stride, uint64_t value_block_stride,
    uint64_t value_page_stride, uint64_t value_head_stride,
    uint32_t max_blocks_per_sequence, uint32_t max_sequence_length,
    uint32_t partition_tokens, float scale, void* stream);

/*
 * Capability query. Replaces the PagedDecodeAttention arms of
 * CudaBackend::supports (crates/loom-cuda/src/cuda_backend.rs:112-134,
 * attention_dispatch.rs:330-344). Reports without launching work. Returns
 * LOOM_HIP_SUCCESS when the shape is executable, LOOM_HIP_UNSUPPORTED or
 * LOOM_HIP_INVALID_ARGUMENT otherwise, with a static reason in *reason
 * (nullable). *kernel_family (nullable) receives "mfma-stream" for the
 * 16-token matrix-core kernel (at most 16 query heads per KV head, block size
 * >= 16), "mfma" for the 32-token matrix-core kernel or "vector" for the
 * general kernel. A call whose partition size is not a multiple of 16 moves
 * from "mfma-stream" to "mfma"; one whose strides or pointers are not 16-byte
 * aligned moves to "vector".
 */
int loom_hip_paged_decode_attention_supports(
    uint32_t dtype, uint32_t cache_encoding, uint32_t sequences,
    uint32_t query_heads, uint32_t kv_heads, uint32_t head_size,
    uint32_t value_head_size, uint32_t num_blocks, uint32_t block_size,
    uint32_t max_blocks_per_sequence, uint32_t max_sequence_length,
    float scale, const char** reason, const char** kernel_family);

/*
 * Fused rotary embedding + paged K/V cache write. Replaces
 * loom_cuda_rope_paged_kv_write_{f32,f16,bf16} (loom_cuda.h:252-318) with the
 * same argument list and meaning (contract: crates/loom-kernels/src/
 * rope_kv.rs:513-631). Q [tokens, query_heads, head_size] and K
 * [tokens, kv_heads, head_size] are rotated in place over the first
 * rotary_dim dims (is_neox 1: pairs (p, p + rotary_dim/2); 0: (2p, 2p+1))
 * with cos/sin from cos_sin_cache[position, 0:rotary_dim/2 | rotary_dim/2:].
 * For token < cache_tokens with 0 <= slot_mapping[token] < num_blocks *
 * block_size, the rotated K row and the V row [value_head_size] are stored at
 * block = slot / block_size, page = slot % block_size through the cache
 * block/page/head element strides. cache_encoding FP8_E4M3 stores
 * e4m3fn(x / scale[kv_head * scale_stride]) (round to nearest even, finite
 * saturation); native stores the element type. Tokens with a position
 * outside [0, max_position) are not touched. All strides are in elements.
 */
int loom_hip_rope_paged_kv_write_f32(
    float* query, float* key, const float* value, const int64_t* positions,
    const float* cos_sin_cache, void* key_cache, void* value_cache,
    const float* key_scales, const float* value_scales,
    const int64_t* slot_mapping, uint32_t tokens, uint32_t cache_tokens,
    uint32_t query_heads, uint32_t kv_heads, uint32_t head_size,
    uint32_t value_head_size, uint32_t rotary_dim, uint32_t max_position,
    uint32_t num_blocks, uint32_t block_size, uint32_t cache_encoding,
    uint32_t scale_stride, uint64_t query_token_stride,
    uint64_t query_head_stride, uint64_t key_token_stride,
    uint64_t key_head_stride, uint64_t value_token_stride,
    uint64_t value_head_stride, uint64_t key_cache_block_stride,
    uint64_t key_cache_page_stride, uint64_t key_cache_head_stride,
    uint64_t value_cache_block_stride, uint64_t value_cache_page_stride,
    uint64_t value_cache_head_stride, uint32_t is_neox, void* stream);

int loom_hip_rope_paged_kv_write_f16(
    uint16_t* query, uint16_t* key, const uint16_t* value,
    const int64_t* positions, const uint16_t* cos_sin_cache, void* key_cache,
    void* value_cache, const float* key_scales, const float* value_scales,
    const int64_t* slot_mapping, uint32_t tokens, uint32_t cache_tokens,
    uint32_t query_heads, uint32_t kv_heads, uint32_t head_size,
    uint32_t value_head_size, uint32_t rotary_dim, uint32_t max_position,
    uint32_t num_blocks, uint32_t block_size, uint32_t cache_encoding,
    uint32_t scale_stride, uint64_t query_token_stride,
    uint64_t query_head_stride, uint64_t key_token_stride,
    uint64_t key_head_stride, uint64_t value_token_stride,
    uint64_t value_head_stride, uint64_t key_cache_block_stride,
    uint64_t key_cache_page_stride, uint64_t key_cache_head_stride,
    uint64_t value_cache_block_stride, uint64_t value_cache_page_stride,
    uint64_t value_cache_head_stride, uint32_t is_neox, void* stream);

int loom_hip_rope_paged_kv_write_bf16(
    uint16_t* query, uint16_t* key, const uint16_t* value,
    const int64_t* positions, const uint16_t* cos_sin_cache, void* key_cache,
    void* value_cache, const float* key_scales, const float* value_scales,
    const int64_t* slot_mapping, uint32_t tokens, uint32_t cache_tokens,
    uint32_t query_heads, uint32_t kv_heads, uint32_t head_size,
    uint32_t value_head_size, uint32_t rotary_dim, uint32_t max_position,
    uint32_t num_blocks, uint32_t block_size, uint32_t cache_encoding,
    uint32_t scale_stride, uint64_t query_token_stride,
    uint64_t query_head_stride, uint64_t key_token_stride,
    uint64_t key_head_stride, uint64_t value_token_stride,
    uint64_t value_head_stride, uint64_t key_cache_block_stride,
    uint64_t key_cache_page_stride, uint64_t key_cache_head_stride,
    uint64_t value_cache_block_stride, uint64_t value_cache_page_stride,
    uint64_t value_cache_head_stride, uint32_t is_neox, void* stream);

/* Backend name, as CudaBackend::name() = "loom-cuda" (cuda_backend.rs:43). */
const char* loom_hip_backend_name(void);

/* ABI version (loom-cuda-bridge reports 2, cuda/mod.rs:720-724). */
uint32_t loom_hip_abi_version(void);

/*
 * Thread-local message describing the last failed call on this thread
 * (replaces loom_cuda_bridge_last_error_message, cuda/mod.rs:726-731).
 */
const char* loom_hip_last_error_message(void);

/*
 * Kernel family ("mfma-stream", "mfma" or "vector", the names of
 * loom_hip_paged_decode_attention_supports) that the last successful paged
 * decode call on this thread launched; "" before the first. No reference
 * counterpart: a diagnostic for tests and profiling, since the family also
 * depends on pointer and stride alignment and the partition size, which the
 * capability query does not see.
 */
const char* loom_hip_last_kernel_family(void);

/*
 * Partition size (tokens) of the internal split that the last successful
 * paged decode call on this thread ran, or 0 when it ran as the caller asked.
 * Single-partition calls (no caller workspace) whose (sequence, KV head)
 * items cannot fill the GPU and whose context reaches 2048 tokens are split
 * with their partial states in a library-held slot: a static array per
 * device of 4 slots x 16 MiB, resident until the process ends. The first 4
 * streams that make such a call on a device each keep one slot (calls on one
 * stream use it in stream order). Calls from other streams, from
 * hipStreamPerThread, under stream capture, and all calls while the
 * environment variable LOOM_HIP_INTERNAL_SPLIT is "0" run as one partition.
 * No reference counterpart: a diagnostic.
 */
uint32_t loom_hip_last_internal_partition_tokens(void);

/*
 * Plan of a paged decode call on `stream`, without launching anything:
 * *run_partition_tokens is the partition size the call would run with
 * (partition_tokens itself for a split call; for a single-partition call,
 * the internal split's size when the call would take it, else 0), and
 * *internal_split is 1 when that size comes from the internal split. A
 * single-partition call takes the internal split when its (sequence, KV
 * head) items cannot fill the GPU, its context reaches 2048 tokens, the
 * environment variable LOOM_HIP_INTERNAL_SPLIT is not "0", and `stream` owns
 * one of the library's 4 slots or a free slot remains (the query does not
 * claim one; hipStreamPerThread and capturing streams never take a slot).
 * Library-held state behind this: split_pool, a static device array of
 * 4 slots x 16 MiB per device, and the no-allocation entry point's 64 MiB
 * array, both resident from module load until the process ends (128 MiB of
 * HBM per device). No reference counterpart: the reference keeps no state
 * beyond counters and the last error (cuda/mod.rs:45-52).
 */
int loom_hip_paged_decode_attention_plan(uint32_t dtype, uint32_t sequences,
                                         uint32_t query_heads, uint32_t kv_heads,
                                         uint32_t head_size, uint32_t value_head_size,
                                         uint32_t max_sequence_length,
                                         uint32_t partition_tokens, void* stream,
                                         uint32_t* run_partition_tokens,
                                         uint32_t* internal_split);

/*
 * Name of the decode kernel that the last successful paged decode call on
 * this thread launched ("decode_stream_group_kernel", "decode_stream_kernel",
 * "decode_stream_heads_kernel", "decode_mfma_kernel" or
 * "decode_vector_kernel"); "" before the first. No reference counterpart: a
 * diagnostic for profiling (the kernel a rocprof trace names).
 */
const char* loom_hip_last_kernel_name(void);

/*
 * Relaxed atomic launch counters (replace loom_cuda_bridge_launch_count /
 * _reset_launch_count, cuda/mod.rs:733-774). One successful decode call
 * counts once regardless of how many kernels it launches.
 */
int loom_hip_launch_count(uint32_t operation, uint64_t* count);
int loom_hip_reset_launch_count(uint32_t operation);

/*
 * Per-kernel timing for profiling (no reference counterpart). When enabled,
 * every launch is bracketed by events on the launch stream; reading
 * synchronizes the recorded events and returns the accumulated milliseconds
 * and launch count since the last reset. Enabling resets the totals.
 */
int loom_hip_kernel_timing_enable(uint32_t enable);
int loom_hip_kernel_timing_read(uint32_t kernel, double* total_ms,
                                uint64_t* launches);

#ifdef __cplusplus
}  /* extern "C" */
#endif

#endif  /* LOOM_HIP_H_ */
