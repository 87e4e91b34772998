"""The no-allocation entry point against the extended entry point (GPU).

loom_hip_paged_decode_attention_extended_no_alloc runs the same kernels as
loom_hip_paged_decode_attention_extended_* with the split-K states in the
library's static per-device array. Its results must equal the extended entry
point's bit for bit (same kernels, same schedule, only the state address
differs). Two calls in a row, the second smaller, show that nothing the first
call left in the shared array leaks into the second.
"""

from __future__ import annotations

import ctypes

import pytest
import torch

from attnarc_amd import workloads
from attnarc_amd.ops import paged_decode_attention_extended

pytestmark = pytest.mark.gpu

DEV = "cuda:0"


def _case(dtype, lengths, seed, **kw):
    base = dict(query_heads=32, kv_heads=8, head_size=128, value_head_size=128, block_size=16,
                pool_factor=1.25, partition_tokens=512)
    base.update(kw)
    return workloads.make_case(name=f"no_alloc_{seed}", dtype=dtype, sequences=len(lengths), lengths=lengths,
                               seed=seed, device=DEV, **base)


def _run(case, no_alloc):
    out = torch.full((case.sequences, case.query_heads, case.value_head_size), float("nan"), device=DEV,
                     dtype=case.dtype)
    lse = torch.full((case.sequences, case.query_heads), float("nan"), device=DEV, dtype=torch.float32)
    paged_decode_attention_extended(
        case.query, case.key_cache, case.value_cache, case.block_tables, case.sequence_lengths,
        max_sequence_length=case.max_sequence_length, scale=case.scale, layout=case.layout,
        key_scales=case.key_scales, value_scales=case.value_scales, partition_tokens=case.partition_tokens,
        output=out, lse=lse, no_alloc=no_alloc)
    return out, lse


def _check_pair(case):
    want_o, want_l = _run(case, no_alloc=False)
    got_o, got_l = _run(case, no_alloc=True)
    torch.cuda.synchronize()
    assert torch.equal(got_o.view(torch.int16) if got_o.dtype != torch.float32 else got_o,
                       want_o.view(torch.int16) if want_o.dtype != torch.float32 else want_o)
    assert torch.equal(got_l, want_l)


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16, torch.float32])
def test_no_alloc_matches_extended_twice_second_smaller(dtype):
    big = _case(dtype, [8192, 777, 4100, 512, 6000, 3000, 129, 8000], seed=71)
    small = _case(dtype, [1500, 33, 700], seed=72)
    _check_pair(big)
    _check_pair(small)


def test_no_alloc_fp8_hnd_and_single_partition():
    fp8 = _case(torch.bfloat16, [4096, 2000, 17, 3333], seed=73, cache_encoding="fp8", layout="HND",
                query_heads=64)
    _check_pair(fp8)
    whole = _case(torch.bfloat16, [300, 64], seed=74, partition_tokens=0)
    _check_pair(whole)


def test_no_alloc_long_mqa_many_partitions():
    mqa = _case(torch.bfloat16, [65536, 40000], seed=75, query_heads=32, kv_heads=1, partition_tokens=1024)
    small = _case(torch.bfloat16, [5000], seed=76, query_heads=32, kv_heads=1, partition_tokens=1024)
    _check_pair(mqa)
    _check_pair(small)


@pytest.mark.parametrize("handle", [1, 2], ids=["legacy", "per-thread"])
def test_no_alloc_on_special_stream_handles(monkeypatch, handle):
    """hipStreamLegacy (1) and hipStreamPerThread (2) name streams of the
    current device: the no-allocation call accepts them like the null stream."""
    from attnarc_amd import ops

    case = _case(torch.bfloat16, [3000, 900, 4096], seed=77)
    want_o, want_l = _run(case, no_alloc=False)
    torch.cuda.synchronize()
    out = torch.full_like(want_o, float("nan"))
    lse = torch.full_like(want_l, float("nan"))
    torch.cuda.synchronize()  # the special stream does not order after torch's stream
    monkeypatch.setattr(ops, "_stream_handle", lambda device: ctypes.c_void_p(handle))
    paged_decode_attention_extended(
        case.query, case.key_cache, case.value_cache, case.block_tables, case.sequence_lengths,
        max_sequence_length=case.max_sequence_length, scale=case.scale, layout=case.layout,
        key_scales=case.key_scales, value_scales=case.value_scales, partition_tokens=case.partition_tokens,
        output=out, lse=lse, no_alloc=True)
    torch.cuda.synchronize()
    assert torch.equal(out.view(torch.int16), want_o.view(torch.int16))
    assert torch.equal(lse, want_l)
