"""The Stable-ABI torch adapter loads and registers the reference schema (no GPU needed)."""

from __future__ import annotations

import pytest
import torch

from attnarc_amd import torch_ops

# python/csrc/torch_ops.cpp:74-82 (schema strings the reference registers).
REFERENCE_SCHEMAS = {
    "paged_decode_attention": "loom_kernels::paged_decode_attention(Tensor query, Tensor key_cache, Tensor "
    "value_cache, Tensor block_tables, Tensor sequence_lengths, Tensor(a!) output, int max_sequence_length, "
    "float scale) -> ()",
    "rope_paged_kv_write_": "loom_kernels::rope_paged_kv_write_(Tensor(a!) query, Tensor(b!) key, Tensor value, "
    "Tensor positions, Tensor cos_sin_cache, Tensor(c!) kv_cache, Tensor key_scales, Tensor value_scales, "
    "Tensor slot_mapping, bool is_neox) -> ()",
    "bridge_abi_version": "loom_kernels::bridge_abi_version() -> int",
    "bridge_launch_count": "loom_kernels::bridge_launch_count(int operation) -> int",
    "reset_bridge_launch_count": "loom_kernels::reset_bridge_launch_count(int operation) -> ()",
}


@pytest.mark.parametrize("name", sorted(REFERENCE_SCHEMAS))
def test_schema_matches_the_reference(name):
    assert str(getattr(torch.ops.loom_kernels, name).default._schema) == REFERENCE_SCHEMAS[name]


def test_telemetry_ops():
    assert torch_ops.bridge_abi_version() == 2
    for op in torch_ops.Operator:
        torch_ops.reset_launch_count(op)
        assert torch_ops.launch_count(op) == 0
    with pytest.raises(RuntimeError, match="out of range"):
        torch.ops.loom_kernels.bridge_launch_count(11)
    with pytest.raises(TypeError):
        torch_ops.launch_count(9)


def test_cpu_tensors_have_no_kernel():
    q = torch.zeros(1, 2, 4)
    c = torch.zeros(1, 8, 1, 4)
    with pytest.raises(NotImplementedError, match="CPU"):
        torch_ops.paged_decode_attention(q, c, c, torch.zeros(1, 1, dtype=torch.int32),
                                         torch.ones(1, dtype=torch.int32), max_sequence_length=8)
    with pytest.raises(ValueError, match="inference-only"):
        torch_ops.paged_decode_attention_out(q.requires_grad_(), c, c, torch.zeros(1, 1, dtype=torch.int32),
                                             torch.ones(1, dtype=torch.int32), torch.empty(1, 2, 4),
                                             max_sequence_length=8)
