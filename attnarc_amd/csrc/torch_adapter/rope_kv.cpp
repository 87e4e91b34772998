// loom_kernels::rope_paged_kv_write_ on HIP (schema: python/csrc/torch_ops.cpp).
// kv_cache is [blocks, 2, block_size, kv_heads, head_size] (K at index 0 of
// dimension 1, V at 1) in the source dtype or uint8 FP8 E4M3 bytes, NHD or
// HND strides. The contract and the packed-cache split live in the library's
// view front end.
#include "common.h"

namespace loom_hip::torch_adapter {

void rope_paged_kv_write(Tensor query, Tensor key, const Tensor& value, const Tensor& positions,
                         const Tensor& cos_sin_cache, Tensor kv_cache, const Tensor& key_scales,
                         const Tensor& value_scales, const Tensor& slot_mapping, bool is_neox) {
  const loom_hip_tensor_view views[9] = {view_of(query),         view_of(key),          view_of(value),
                                         view_of(positions),     view_of(cos_sin_cache), view_of(kv_cache),
                                         view_of(key_scales),    view_of(value_scales), view_of(slot_mapping)};
  raise_unless_ok(loom_hip_views_rope_paged_kv_check(views), "RoPE+paged-KV");
  const torch::stable::accelerator::DeviceGuard guard(views[0].device_index);
  raise_unless_ok(loom_hip_views_rope_paged_kv_write(views, is_neox ? 1U : 0U, current_stream(views[0].device_index)),
                  "RoPE+paged-KV");
}

}  // namespace loom_hip::torch_adapter

STABLE_TORCH_LIBRARY_IMPL(loom_kernels, CUDA, library) {
  library.impl("rope_paged_kv_write_", TORCH_BOX(&loom_hip::torch_adapter::rope_paged_kv_write));
}
