// Shared helpers of the loom-hip PyTorch Stable-ABI adapter.
//
// The adapter is the MI355X counterpart of the reference's
// python/csrc/{common.h, attention.cpp, rope_kv.cpp, telemetry.cpp,
// torch_ops.cpp}: the same `loom_kernels` operator schema, the same tensor
// contract checks and messages, the current HIP stream taken from torch, and
// split-K workspaces allocated from the torch caching allocator (so calls are
// graph-capturable). All launches go through the checked bridge of
// include/loom_hip_bridge.h. Only the Stable ABI is used, so one build loads
// into any torch release from the target version on.
#pragma once

#define TORCH_TARGET_VERSION (((0ULL + 2) << 56) | ((0ULL + 10) << 48))

#include <torch/csrc/inductor/aoti_torch/c/shim.h>
#include <torch/csrc/stable/accelerator.h>
#include <torch/csrc/stable/library.h>
#include <torch/csrc/stable/ops.h>
#include <torch/csrc/stable/tensor.h>
#include <torch/headeronly/core/ScalarType.h>
#include <torch/headeronly/macros/Macros.h>

#include <cmath>
#include <cstdint>
#include <initializer_list>
#include <limits>

#include "loom_hip_bridge.h"

namespace loom_hip::torch_adapter {

using Tensor = torch::stable::Tensor;
using ScalarType = torch::headeronly::ScalarType;

// Makes the tensor's device current for the scope of a launch.
class DeviceScope final {
 public:
  explicit DeviceScope(const torch::stable::Device& device) : guard_(device.index()) {}

 private:
  torch::stable::accelerator::DeviceGuard guard_;
};

// torch's current stream on a device (a hipStream_t on ROCm builds).
inline void* current_stream(int32_t device_index) {
  void* stream = nullptr;
  TORCH_ERROR_CODE_CHECK(aoti_torch_get_current_cuda_stream(device_index, &stream));
  return stream;
}

inline uint64_t tensor_nbytes(const Tensor& t) {
  STD_TORCH_CHECK(t.numel() >= 0, "negative tensor element count");
  const auto n = static_cast<uint64_t>(t.numel());
  const auto e = static_cast<uint64_t>(t.element_size());
  STD_TORCH_CHECK(e == 0 || n <= std::numeric_limits<uint64_t>::max() / e, "tensor byte size exceeds uint64");
  return n * e;
}

inline uint32_t bridge_dtype(const Tensor& t) {
  switch (t.scalar_type()) {
    case ScalarType::Float: return LOOM_HIP_BRIDGE_F32;
    case ScalarType::Half: return LOOM_HIP_BRIDGE_F16;
    case ScalarType::BFloat16: return LOOM_HIP_BRIDGE_BF16;
    default: break;
  }
  STD_TORCH_CHECK(false, "unsupported Loom bridge dtype");
  return 0;
}

// Elements from the first to one past the last addressed element:
// 1 + sum (size - 1) * stride over positive sizes and strides.
inline uint64_t storage_span_elements(const Tensor& t) {
  STD_TORCH_CHECK(t.numel() > 0, "Loom bridge tensors must contain at least one element");
  uint64_t span = 1;
  for (int64_t d = 0; d < t.dim(); ++d) {
    STD_TORCH_CHECK(t.size(d) > 0 && t.stride(d) > 0, "Loom bridge requires positive tensor sizes and strides");
    const auto extent = static_cast<uint64_t>(t.size(d) - 1);
    const auto stride = static_cast<uint64_t>(t.stride(d));
    STD_TORCH_CHECK(extent == 0 || stride <= (std::numeric_limits<uint64_t>::max() - span) / extent,
                    "Loom tensor storage span exceeds the bridge ABI");
    span += extent * stride;
  }
  return span;
}

inline void check_bridge_status(int status, const char* operation) {
  STD_TORCH_CHECK(status == LOOM_HIP_BRIDGE_SUCCESS, "Loom HIP ", operation,
                  " bridge failed: ", loom_hip_bridge_last_error_message(), " (status ", status, ")");
}

// Overlap of the byte ranges [data, data + numel * element_size).
inline bool byte_ranges_overlap(const Tensor& a, const Tensor& b) {
  const auto a0 = reinterpret_cast<uintptr_t>(a.const_data_ptr());
  const auto b0 = reinterpret_cast<uintptr_t>(b.const_data_ptr());
  const auto an = tensor_nbytes(a), bn = tensor_nbytes(b);
  STD_TORCH_CHECK(an <= std::numeric_limits<uintptr_t>::max() - a0 && bn <= std::numeric_limits<uintptr_t>::max() - b0,
                  "tensor byte range exceeds uintptr_t");
  return a0 < b0 + bn && b0 < a0 + an;
}

// [blocks, block_size, heads, dim] with only the block stride allowed gaps.
inline bool has_dense_nhd_inner_strides(const Tensor& t) {
  if (t.dim() != 4) return false;
  const int64_t block = t.size(1) * t.size(2) * t.size(3);
  return t.stride(3) == 1 && t.stride(2) == t.size(3) && t.stride(1) == t.size(2) * t.size(3) &&
         t.stride(0) >= block;
}

}  // namespace loom_hip::torch_adapter
