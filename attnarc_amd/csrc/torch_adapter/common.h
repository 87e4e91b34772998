// Framework glue of the loom-hip PyTorch Stable-ABI adapter.
//
// The adapter does not check tensors itself. It describes every operand as a
// loom_hip_tensor_view and hands the set to the library's view front end
// (include/loom_hip_views.h), which holds each operator's tensor contract as
// a table and submits through the checked bridge. What stays here is what
// only torch can provide: the device guard, torch's current HIP stream, the
// split-K workspace from the caching allocator (so a call under
// torch.cuda.graph allocates from the graph's pool), and turning a refusal
// into a torch error. Only the Stable ABI is used, so one build loads into
// any torch release from the target version on.
#pragma once

#define TORCH_TARGET_VERSION (((0ULL + 2) << 56) | ((0ULL + 10) << 48))

#include <torch/csrc/inductor/aoti_torch/c/shim.h>
#include <torch/csrc/stable/accelerator.h>
#include <torch/csrc/stable/library.h>
#include <torch/csrc/stable/ops.h>
#include <torch/csrc/stable/tensor.h>
#include <torch/headeronly/core/ScalarType.h>
#include <torch/headeronly/macros/Macros.h>

#include <cstdint>

#include "loom_hip_bridge.h"
#include "loom_hip_views.h"

namespace loom_hip::torch_adapter {

using Tensor = torch::stable::Tensor;
using ScalarType = torch::headeronly::ScalarType;

inline uint32_t view_dtype(ScalarType t) {
  switch (t) {
    case ScalarType::Float: return LOOM_HIP_VIEW_F32;
    case ScalarType::Half: return LOOM_HIP_VIEW_F16;
    case ScalarType::BFloat16: return LOOM_HIP_VIEW_BF16;
    case ScalarType::Byte: return LOOM_HIP_VIEW_U8;
    case ScalarType::Float8_e4m3fn: return LOOM_HIP_VIEW_FP8_E4M3FN;
    case ScalarType::Int: return LOOM_HIP_VIEW_I32;
    case ScalarType::Long: return LOOM_HIP_VIEW_I64;
    default: return LOOM_HIP_VIEW_OTHER;
  }
}

// The view of a tensor as the library's contract tables see it. Ranks above
// the view limit are passed as such and fail the contract's rank rule.
inline loom_hip_tensor_view view_of(const Tensor& t) {
  loom_hip_tensor_view v{};
  v.data = t.const_data_ptr();
  v.device_index = t.is_cuda() ? static_cast<int32_t>(t.device().index()) : -1;
  v.dtype = view_dtype(t.scalar_type());
  v.rank = static_cast<uint32_t>(t.dim());
  for (int64_t d = 0; d < t.dim() && d < LOOM_HIP_VIEW_MAX_RANK; ++d) {
    v.sizes[d] = t.size(d);
    v.strides[d] = t.stride(d);
  }
  return v;
}

// Raises the library's refusal as a torch error: the contract's own message,
// or the bridge's with the operation named.
inline void raise_unless_ok(int status, const char* operation) {
  if (status == LOOM_HIP_VIEWS_OK) return;
  const char* message = loom_hip_views_last_error_message();
  STD_TORCH_CHECK(status != LOOM_HIP_VIEWS_CONTRACT, message);
  STD_TORCH_CHECK(false, "Loom HIP ", operation, " bridge failed: ", message);
}

// torch's current stream on the guarded device (a hipStream_t on ROCm).
inline void* current_stream(int32_t device_index) {
  void* stream = nullptr;
  TORCH_ERROR_CODE_CHECK(aoti_torch_get_current_cuda_stream(device_index, &stream));
  return stream;
}

}  // namespace loom_hip::torch_adapter
