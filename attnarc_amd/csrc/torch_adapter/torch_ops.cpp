// Schema of the `loom_kernels` operators this library implements (the
// paged-decode and RoPE+KV subset of python/csrc/torch_ops.cpp, identical
// signatures) and the bridge telemetry ops (python/csrc/telemetry.cpp).
#include <limits>

#include "common.h"

STABLE_TORCH_LIBRARY(loom_kernels, library) {
  library.def(
      "paged_decode_attention(Tensor query, Tensor key_cache, Tensor value_cache, Tensor block_tables, "
      "Tensor sequence_lengths, Tensor(a!) output, int max_sequence_length, float scale) -> ()");
  library.def(
      "rope_paged_kv_write_(Tensor(a!) query, Tensor(b!) key, Tensor value, Tensor positions, "
      "Tensor cos_sin_cache, Tensor(c!) kv_cache, Tensor key_scales, Tensor value_scales, Tensor slot_mapping, "
      "bool is_neox) -> ()");
  library.def("bridge_abi_version() -> int");
  library.def("bridge_launch_count(int operation) -> int");
  library.def("reset_bridge_launch_count(int operation) -> ()");
}

namespace loom_hip::torch_adapter {

namespace {

void check_bridge_status(int status, const char* operation) {
  STD_TORCH_CHECK(status == LOOM_HIP_BRIDGE_SUCCESS, "Loom HIP ", operation,
                  " bridge failed: ", loom_hip_bridge_last_error_message(), " (status ", status, ")");
}

}  // namespace

int64_t bridge_abi_version() { return static_cast<int64_t>(loom_hip_bridge_abi_version()); }

int64_t bridge_launch_count(int64_t operation) {
  STD_TORCH_CHECK(operation >= 0 && operation <= LOOM_HIP_BRIDGE_GREEDY_SPECULATIVE_VERIFY,
                  "Loom bridge operator id is out of range");
  uint64_t count = 0;
  check_bridge_status(loom_hip_bridge_launch_count(static_cast<uint32_t>(operation), &count), "telemetry query");
  STD_TORCH_CHECK(count <= static_cast<uint64_t>(std::numeric_limits<int64_t>::max()),
                  "Loom bridge launch count exceeds int64");
  return static_cast<int64_t>(count);
}

void reset_bridge_launch_count(int64_t operation) {
  STD_TORCH_CHECK(operation >= 0 && operation <= LOOM_HIP_BRIDGE_GREEDY_SPECULATIVE_VERIFY,
                  "Loom bridge operator id is out of range");
  check_bridge_status(loom_hip_bridge_reset_launch_count(static_cast<uint32_t>(operation)), "telemetry reset");
}

}  // namespace loom_hip::torch_adapter

STABLE_TORCH_LIBRARY_IMPL(loom_kernels, CompositeExplicitAutograd, library) {
  library.impl("bridge_abi_version", TORCH_BOX(&loom_hip::torch_adapter::bridge_abi_version));
  library.impl("bridge_launch_count", TORCH_BOX(&loom_hip::torch_adapter::bridge_launch_count));
  library.impl("reset_bridge_launch_count", TORCH_BOX(&loom_hip::torch_adapter::reset_bridge_launch_count));
}
