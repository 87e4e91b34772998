// loom_kernels::paged_decode_attention on HIP (schema: python/csrc/torch_ops.cpp).
// The tensor contract lives in the library's view front end; this file only
// sizes and allocates the split-K workspace and picks the stream.
#include "common.h"

namespace loom_hip::torch_adapter {

void paged_decode_attention(const Tensor& query, const Tensor& key_cache, const Tensor& value_cache,
                            const Tensor& block_tables, const Tensor& sequence_lengths, Tensor output,
                            int64_t max_sequence_length, double scale) {
  const loom_hip_tensor_view views[6] = {view_of(query),        view_of(key_cache),        view_of(value_cache),
                                         view_of(block_tables), view_of(sequence_lengths), view_of(output)};
  uint64_t elements = 0;
  raise_unless_ok(loom_hip_views_paged_decode_workspace_elements(views, max_sequence_length, scale, &elements),
                  "paged decode workspace query");
  STD_TORCH_CHECK(elements <= static_cast<uint64_t>(INT64_MAX),
                  "Loom paged decode split-K workspace exceeds PyTorch limits");
  const torch::stable::accelerator::DeviceGuard guard(views[0].device_index);
  Tensor workspace;
  float* states = nullptr;
  if (elements != 0) {
    workspace = torch::stable::new_empty(query, {static_cast<int64_t>(elements)}, ScalarType::Float);
    states = workspace.mutable_data_ptr<float>();
  }
  raise_unless_ok(loom_hip_views_paged_decode_attention(views, max_sequence_length, scale, states, elements,
                                                        current_stream(views[0].device_index)),
                  "paged decode attention");
}

}  // namespace loom_hip::torch_adapter

STABLE_TORCH_LIBRARY_IMPL(loom_kernels, CUDA, library) {
  library.impl("paged_decode_attention", TORCH_BOX(&loom_hip::torch_adapter::paged_decode_attention));
}
