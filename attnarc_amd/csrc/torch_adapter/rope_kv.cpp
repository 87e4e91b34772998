// loom_kernels::rope_paged_kv_write_ on HIP (python/csrc/rope_kv.cpp).
// kv_cache is [blocks, 2, block_size, kv_heads, head_size] (K at 1-index 0,
// V at 1) in the source dtype or uint8 FP8 E4M3 bytes, NHD or HND strides.
#include "common.h"

namespace loom_hip::torch_adapter {

namespace {

// 1 + sum over `dims` of (size - 1) * stride, overflow-checked.
uint64_t kv_span(const Tensor& kv, std::initializer_list<int64_t> dims) {
  uint64_t span = 1;
  for (const int64_t d : dims) {
    const auto extent = static_cast<uint64_t>(kv.size(d) - 1);
    const auto stride = static_cast<uint64_t>(kv.stride(d));
    STD_TORCH_CHECK(extent == 0 || stride <= (std::numeric_limits<uint64_t>::max() - span) / extent,
                    "Loom packed K/V cache span exceeds the bridge ABI");
    span += extent * stride;
  }
  return span;
}

void check_rope_paged_kv_write_contract(const Tensor& query, const Tensor& key, const Tensor& value,
                                        const Tensor& positions, const Tensor& cos_sin_cache, const Tensor& kv_cache,
                                        const Tensor& key_scales, const Tensor& value_scales,
                                        const Tensor& slot_mapping) {
  STD_TORCH_CHECK(query.is_cuda(), "Loom RoPE+paged-KV query must be on a GPU");
  STD_TORCH_CHECK(key.device() == query.device() && value.device() == query.device() &&
                      positions.device() == query.device() && cos_sin_cache.device() == query.device() &&
                      kv_cache.device() == query.device() && key_scales.device() == query.device() &&
                      value_scales.device() == query.device() && slot_mapping.device() == query.device(),
                  "Loom RoPE+paged-KV tensors must be on one GPU device");
  STD_TORCH_CHECK(query.scalar_type() == key.scalar_type() && query.scalar_type() == value.scalar_type() &&
                      query.scalar_type() == cos_sin_cache.scalar_type(),
                  "Loom RoPE+paged-KV Q/K/V and cos/sin cache must share a dtype");
  STD_TORCH_CHECK(query.scalar_type() == ScalarType::Float || query.scalar_type() == ScalarType::Half ||
                      query.scalar_type() == ScalarType::BFloat16,
                  "Loom RoPE+paged-KV supports F32, FP16, and BF16 sources");
  STD_TORCH_CHECK(query.dim() == 3 && key.dim() == 3 && value.dim() == 3, "Loom RoPE+paged-KV Q/K/V must have rank 3");
  STD_TORCH_CHECK(kv_cache.scalar_type() == query.scalar_type() || kv_cache.scalar_type() == ScalarType::Byte,
                  "Loom paged K/V cache must use the source dtype or uint8 FP8 E4M3 storage");
  STD_TORCH_CHECK(key_scales.scalar_type() == ScalarType::Float && value_scales.scalar_type() == ScalarType::Float &&
                      key_scales.is_contiguous() && value_scales.is_contiguous() &&
                      key_scales.numel() == value_scales.numel() &&
                      (key_scales.numel() == 1 || key_scales.numel() == key.size(1)),
                  "Loom paged K/V cache scales must be contiguous float32 tensors with one element or one element "
                  "per KV head");
  STD_TORCH_CHECK(positions.scalar_type() == ScalarType::Long && slot_mapping.scalar_type() == ScalarType::Long,
                  "Loom RoPE+paged-KV positions and slot mapping must be int64");
  STD_TORCH_CHECK(query.size(0) > 0 && query.size(1) > 0 && query.size(2) > 0,
                  "Loom RoPE+paged-KV query must be non-empty");
  STD_TORCH_CHECK(key.size(0) == query.size(0) && value.size(0) == query.size(0),
                  "Loom RoPE+paged-KV Q/K/V token counts must match");
  STD_TORCH_CHECK(key.size(1) > 0 && key.size(1) == value.size(1), "Loom RoPE+paged-KV K/V head counts must match");
  STD_TORCH_CHECK(key.size(2) == query.size(2), "Loom RoPE+paged-KV Q/K head sizes must match");
  STD_TORCH_CHECK(value.size(2) > 0, "Loom RoPE+paged-KV value head size must be positive");
  STD_TORCH_CHECK(query.stride(2) == 1 && key.stride(2) == 1 && value.stride(2) == 1 && query.stride(0) > 0 &&
                      query.stride(1) > 0 && key.stride(0) > 0 && key.stride(1) > 0 && value.stride(0) > 0 &&
                      value.stride(1) > 0 && positions.is_contiguous() && cos_sin_cache.is_contiguous() &&
                      slot_mapping.is_contiguous(),
                  "Loom RoPE+paged-KV sources require unit dim stride and positive token/head strides; metadata "
                  "must be contiguous");
  STD_TORCH_CHECK(positions.dim() == 1 && positions.numel() == query.size(0) && slot_mapping.dim() == 1 &&
                      slot_mapping.numel() <= query.size(0),
                  "Loom RoPE positions must cover every token and slot_mapping must not exceed the padded token "
                  "count");
  STD_TORCH_CHECK(cos_sin_cache.dim() == 2 && cos_sin_cache.size(0) > 0 && cos_sin_cache.size(1) > 0 &&
                      cos_sin_cache.size(1) % 2 == 0 && cos_sin_cache.size(1) <= query.size(2),
                  "Loom RoPE+paged-KV cos/sin cache must be [max_position, even rotary_dim <= head_size]");
  STD_TORCH_CHECK(kv_cache.dim() == 5 && kv_cache.size(1) == 2,
                  "Loom paged K/V cache must have shape [blocks, 2, block_size, kv_heads, head_size]");
  STD_TORCH_CHECK(kv_cache.size(0) > 0 && kv_cache.size(2) > 0 && kv_cache.size(3) == key.size(1) &&
                      kv_cache.size(4) == key.size(2) && value.size(1) == key.size(1) &&
                      value.size(2) == key.size(2),
                  "Loom packed K/V cache and K/V sources must share head count and head size");
  STD_TORCH_CHECK(kv_cache.stride(4) == 1 && kv_cache.stride(0) > 0 && kv_cache.stride(1) > 0 &&
                      kv_cache.stride(2) > 0 && kv_cache.stride(3) > 0,
                  "Loom packed K/V cache requires unit element stride and positive block/KV/page/head strides");
  const uint64_t part = kv_span(kv_cache, {2, 3, 4});
  const auto kv_stride = static_cast<uint64_t>(kv_cache.stride(1));
  const auto block_stride = static_cast<uint64_t>(kv_cache.stride(0));
  STD_TORCH_CHECK(kv_stride >= part && block_stride >= kv_stride && block_stride - kv_stride >= part,
                  "Loom packed K/V cache partitions must not overlap");
}

void launch_rope_paged_kv_write(Tensor query, Tensor key, const Tensor& value, const Tensor& positions,
                                const Tensor& cos_sin_cache, Tensor kv_cache, const Tensor& key_scales,
                                const Tensor& value_scales, const Tensor& slot_mapping, bool is_neox) {
  const int64_t limits[] = {query.size(0), query.size(1),         key.size(1),      query.size(2),  value.size(2),
                            cos_sin_cache.size(1), cos_sin_cache.size(0), kv_cache.size(0), kv_cache.size(2)};
  for (const int64_t v : limits)
    STD_TORCH_CHECK(v > 0 && v <= std::numeric_limits<uint32_t>::max(), "Loom RoPE+paged-KV shape exceeds the HIP ABI");
  const DeviceScope device(query.device());
  void* stream = current_stream(query.device().index());
  const uint32_t encoding =
      kv_cache.scalar_type() == ScalarType::Byte ? LOOM_HIP_BRIDGE_KV_CACHE_FP8_E4M3 : LOOM_HIP_BRIDGE_KV_CACHE_NATIVE;
  const auto elem = static_cast<uint64_t>(kv_cache.element_size());
  const auto v_offset = static_cast<uint64_t>(kv_cache.stride(1));
  STD_TORCH_CHECK(elem == 0 || v_offset <= std::numeric_limits<uint64_t>::max() / elem,
                  "Loom packed K/V cache byte offset exceeds uint64");
  auto* k_cache = static_cast<uint8_t*>(kv_cache.mutable_data_ptr());
  auto* v_cache = k_cache + v_offset * elem;
  const uint64_t view_span = kv_span(kv_cache, {0, 2, 3, 4});
  const auto block = static_cast<uint64_t>(kv_cache.stride(0));
  const auto page = static_cast<uint64_t>(kv_cache.stride(2));
  const auto head = static_cast<uint64_t>(kv_cache.stride(3));

  const int status = loom_hip_bridge_rope_paged_kv_write(
      bridge_dtype(query), encoding, query.mutable_data_ptr(), storage_span_elements(query), key.mutable_data_ptr(),
      storage_span_elements(key), value.const_data_ptr(), storage_span_elements(value),
      positions.const_data_ptr<int64_t>(), static_cast<uint64_t>(positions.numel()), cos_sin_cache.const_data_ptr(),
      static_cast<uint64_t>(cos_sin_cache.numel()), k_cache, view_span, v_cache, view_span,
      key_scales.const_data_ptr<float>(), static_cast<uint64_t>(key_scales.numel()),
      value_scales.const_data_ptr<float>(), static_cast<uint64_t>(value_scales.numel()),
      slot_mapping.const_data_ptr<int64_t>(), static_cast<uint64_t>(slot_mapping.numel()),
      static_cast<uint32_t>(query.size(0)), static_cast<uint32_t>(slot_mapping.numel()),
      static_cast<uint32_t>(query.size(1)), static_cast<uint32_t>(key.size(1)), static_cast<uint32_t>(query.size(2)),
      static_cast<uint32_t>(value.size(2)), static_cast<uint32_t>(cos_sin_cache.size(1)),
      static_cast<uint32_t>(cos_sin_cache.size(0)), static_cast<uint32_t>(kv_cache.size(0)),
      static_cast<uint32_t>(kv_cache.size(2)), static_cast<uint64_t>(query.stride(0)),
      static_cast<uint64_t>(query.stride(1)), static_cast<uint64_t>(key.stride(0)),
      static_cast<uint64_t>(key.stride(1)), static_cast<uint64_t>(value.stride(0)),
      static_cast<uint64_t>(value.stride(1)), block, page, head, block, page, head, is_neox ? 1U : 0U, stream);
  check_bridge_status(status, "RoPE+paged-KV");
}

}  // namespace

void rope_paged_kv_write(Tensor query, Tensor key, const Tensor& value, const Tensor& positions,
                         const Tensor& cos_sin_cache, Tensor kv_cache, const Tensor& key_scales,
                         const Tensor& value_scales, const Tensor& slot_mapping, bool is_neox) {
  check_rope_paged_kv_write_contract(query, key, value, positions, cos_sin_cache, kv_cache, key_scales, value_scales,
                                     slot_mapping);
  launch_rope_paged_kv_write(query, key, value, positions, cos_sin_cache, kv_cache, key_scales, value_scales,
                             slot_mapping, is_neox);
}

}  // namespace loom_hip::torch_adapter

STABLE_TORCH_LIBRARY_IMPL(loom_kernels, CUDA, library) {
  library.impl("rope_paged_kv_write_", TORCH_BOX(&loom_hip::torch_adapter::rope_paged_kv_write));
}
