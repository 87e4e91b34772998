"""Host-side checks of the benchmark workload builders (no GPU)."""

import pytest
import torch

from attnarc_amd import workloads


def test_shape_case_parses_every_key():
    case = workloads.shape_case("B=3,Hq=8,Hkv=2,D=64,L=40,bs=16,part=16,seed=9,dtype=f16,kv=native,layout=HND", "cpu")
    assert (case.sequences, case.query_heads, case.kv_heads, case.head_size, case.value_head_size) == (3, 8, 2, 64, 64)
    assert case.lengths == [40, 40, 40] and case.partition_tokens == 16 and case.block_size == 16
    assert case.dtype == torch.float16 and case.layout == "HND" and case.seed == 9
    assert case.key_cache.shape == (case.num_blocks, 2, 16, 64)  # HND: [blocks, heads, page, dim]
    assert case.num_blocks == 3 * 3  # exactly the needed blocks: ceil(40 / 16) per sequence
    # every sequence's table names distinct physical blocks
    used = case.block_tables[:, :3].flatten().tolist()
    assert sorted(used) == list(range(9))


def test_shape_case_defaults_and_fp8():
    case = workloads.shape_case("B=1,Hq=4,Hkv=1,D=128,L=5,kv=fp8", "cpu")
    assert case.dtype == torch.bfloat16 and case.layout == "NHD" and case.partition_tokens == 0
    assert case.cache_encoding == "fp8" and case.key_scales.numel() == 1


@pytest.mark.parametrize("spec,msg", [("B=1,Hq=4,Hkv=1,L=5", "needs D"), ("B=1,Hq=4,Hkv=1,D=8,L=5,X=1", "unknown shape key")])
def test_shape_case_rejects_bad_specs(spec, msg):
    with pytest.raises(ValueError, match=msg):
        workloads.shape_case(spec, "cpu")
