"""Single-partition calls that the library splits internally (run on an MI355X).

A call with no caller workspace whose (sequence, KV head) items cannot fill
the CUs and whose context reaches 2048 tokens runs as a split-K call with its
partial states in a library-held slot (one static array per device, one slot
for each of the first four streams), then merges into the caller's output. These tests check the
results against the oracle, that the split really ran (a merge launch), that
LOOM_HIP_INTERNAL_SPLIT=0 keeps one partition, that calls on more streams than
there are slots stay correct when they overlap, and that a call under stream
capture keeps one partition and replays correctly.
"""

from __future__ import annotations

import os

import numpy as np
import pytest
import torch

from attnarc_amd import _native, ops, workloads
from gpu_util import LSE_TOL, ORACLE_THREADS, assert_parity, oracle_expected

pytestmark = pytest.mark.gpu

DEV = "cuda"


def _case(seed, lengths=(2048, 1500, 1111, 1024), dtype=torch.bfloat16, hq=12, hkv=2, encoding="native",
          layout="NHD"):
    return workloads.make_case(name=f"split{seed}", dtype=dtype, sequences=len(lengths), query_heads=hq,
                               kv_heads=hkv, head_size=128, value_head_size=128, block_size=16,
                               lengths=list(lengths), seed=seed, device=DEV, pool_factor=1.25,
                               cache_encoding=encoding, layout=layout)


def _merges(fn):
    """Runs fn (one decode call) and returns its result and the number of
    merge kernels it launched."""
    ops.kernel_timing_enable(True)
    try:
        result = fn()
        torch.cuda.synchronize()
        _, merges = ops.kernel_timing_read(_native.KERNEL_MERGE)
    finally:
        ops.kernel_timing_enable(False)
    return result, merges


@pytest.fixture
def no_internal_split():
    os.environ["LOOM_HIP_INTERNAL_SPLIT"] = "0"
    try:
        yield
    finally:
        del os.environ["LOOM_HIP_INTERNAL_SPLIT"]


@pytest.mark.parametrize("dtype,encoding,layout", [
    (torch.bfloat16, "native", "NHD"), (torch.float16, "native", "HND"), (torch.bfloat16, "fp8", "HND"),
    (torch.float32, "native", "NHD")])
def test_small_grid_long_context_splits_internally(dtype, encoding, layout):
    case = _case(11, dtype=dtype, encoding=encoding, layout=layout)
    (out, lse), merges = _merges(lambda: workloads.run_case(case, return_lse=True))
    assert merges == 1, "a single-partition call of 8 items and 2048 tokens should split internally"
    assert ops.last_internal_partition_tokens() == 64  # 32 partitions x 8 items
    expected, want_lse = oracle_expected(case)
    assert_parity(out, expected, dtype, f"internal split {dtype} {encoding} {layout}")
    np.testing.assert_allclose(lse.cpu().numpy(), want_lse, **LSE_TOL)


def test_base_entry_point_splits_internally():
    """The reference-shaped base entry point (no workspace argument at all),
    called through the C ABI."""
    case = _case(12)
    out = torch.empty(case.sequences, case.query_heads, case.value_head_size, dtype=torch.bfloat16, device=DEV)
    nb, bs, hkv, d = case.key_cache.shape
    block_stride = bs * hkv * d

    def call():
        status = _native.lib().loom_hip_paged_decode_attention_bf16(
            case.query.data_ptr(), case.key_cache.data_ptr(), case.value_cache.data_ptr(),
            case.block_tables.data_ptr(), case.sequence_lengths.data_ptr(), out.data_ptr(),
            case.sequences, case.query_heads, case.kv_heads, case.head_size, case.value_head_size,
            case.num_blocks, case.block_size, block_stride, block_stride, case.max_blocks_per_sequence,
            case.max_sequence_length, case.scale, torch.cuda.current_stream().cuda_stream)
        assert status == 0, _native.lib().loom_hip_last_error_message()
        return out

    _, merges = _merges(call)
    assert merges == 1 and ops.last_internal_partition_tokens() == 64
    expected, _ = oracle_expected(case)
    assert_parity(out, expected, torch.bfloat16, "base entry, internal split")


def test_environment_switch_keeps_one_partition(no_internal_split):
    case = _case(13)
    (out, lse), merges = _merges(lambda: workloads.run_case(case, return_lse=True))
    assert merges == 0 and ops.last_internal_partition_tokens() == 0
    expected, want_lse = oracle_expected(case)
    assert_parity(out, expected, torch.bfloat16, "one partition")
    np.testing.assert_allclose(lse.cpu().numpy(), want_lse, **LSE_TOL)


def test_index_order_split_with_ragged_partition_tails():
    """The library's own split of a 16-bit D=128 grid of 1024 items runs its
    items in index order and loads each item's first four block IDs with its
    length; a last partition of 48 tokens or fewer takes the ordinary loads.
    Tails of 0-255 tokens (1, 16, 48, 49, ...), one-token sequences and items
    past a sequence's end, against the oracle."""
    lengths = (4096, 2049, 2064, 2096, 2097, 1, 17, 300, 3333, 256, 257, 304, 4095, 1000, 2500, 3900)
    case = _case(21, lengths=lengths, hq=32, hkv=4)
    (out, lse), merges = _merges(lambda: workloads.run_case(case, return_lse=True))
    assert merges == 1
    assert ops.last_internal_partition_tokens() == 256  # 16 partitions x 64 items: 1024 grouped items
    expected, want_lse = oracle_expected(case)
    assert_parity(out, expected, torch.bfloat16, "index-order internal split, ragged tails")
    np.testing.assert_allclose(lse.cpu().numpy(), want_lse, **LSE_TOL)


def test_large_grid_or_short_context_stays_whole():
    short = _case(14, lengths=(2047, 700, 999, 512))  # contexts under 2048 stay whole
    _, merges = _merges(lambda: workloads.run_case(short))
    assert merges == 0 and ops.last_internal_partition_tokens() == 0
    wide = _case(15, lengths=[1024] * 32, hq=64, hkv=8)  # 256 items
    _, merges = _merges(lambda: workloads.run_case(wide))
    assert merges == 0 and ops.last_internal_partition_tokens() == 0


def test_overlapping_calls_on_more_streams_than_slots():
    """Ten streams (the pool has four slots per device, so some streams run
    whole), each call enqueued behind a long kernel on its stream so that the
    calls overlap; every stream runs two calls with different inputs, then
    all results are checked."""
    cases = [_case(100 + i, lengths=(2048, 1900 - 37 * i, 1024 + 50 * i, 1333)) for i in range(10)]
    second = [_case(200 + i, lengths=(1024 + 64 * i, 2048, 1200, 1800)) for i in range(10)]
    streams = [torch.cuda.Stream() for _ in cases]
    big = torch.randn(4096, 4096, device=DEV)
    outs = []
    torch.cuda.synchronize()
    for s, c1, c2 in zip(streams, cases, second):
        with torch.cuda.stream(s):
            for _ in range(4):
                big = big @ big.T * 1e-4  # keep the stream busy while the others enqueue
            outs.append((workloads.run_case(c1, return_lse=True), workloads.run_case(c2, return_lse=True)))
    torch.cuda.synchronize()
    for (r1, r2), c1, c2 in zip(outs, cases, second):
        for (out, lse), case in ((r1, c1), (r2, c2)):
            expected, want_lse = oracle_expected(case)
            assert_parity(out, expected, torch.bfloat16, case.name)
            np.testing.assert_allclose(lse.cpu().numpy(), want_lse, **LSE_TOL)


def test_call_under_stream_capture_keeps_one_partition_and_replays():
    case = _case(16)
    eager = workloads.run_case(case)
    torch.cuda.synchronize()
    out = torch.empty_like(eager)
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        workloads.run_case(case, output=out)  # warm-up outside the graph
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        workloads.run_case(case, output=out)
    assert ops.last_internal_partition_tokens() == 0  # the captured call kept one partition
    expected, _ = oracle_expected(case)
    for i in range(3):
        out.zero_()
        graph.replay()
        torch.cuda.synchronize()
        assert_parity(out, expected, torch.bfloat16, f"graph replay {i}")
        workloads.run_case(case)  # eager work between replays
        torch.cuda.synchronize()


def test_long_mqa_single_partition_splits_internally():
    """Four MQA items (32 query heads on one KV head) of up to 32768 tokens:
    as one partition each, 4 of the 256 CUs would work."""
    case = _case(17, lengths=(32768, 30001, 16384, 20480), hq=32, hkv=1)
    (out, lse), merges = _merges(lambda: workloads.run_case(case, return_lse=True))
    assert merges == 1 and ops.last_internal_partition_tokens() == 256
    expected, want_lse = oracle_expected(case, threads=ORACLE_THREADS)
    assert_parity(out, expected, torch.bfloat16, "long MQA, internal split")
    np.testing.assert_allclose(lse.cpu().numpy(), want_lse, **LSE_TOL)


@pytest.mark.parametrize("head,hq,hkv,encoding", [
    (64, 16, 2, "native"), (96, 8, 2, "native"), (112, 8, 2, "fp8"), (256, 8, 2, "native"), (128, 48, 1, "native"),
    (128, 64, 1, "fp8")])
def test_internal_split_other_kernels(head, hq, hkv, encoding):
    """The split runs on every streaming kernel family: head sizes 64, 96,
    112 and 256, and the wide-group kernel (48 or 64 query heads per KV head)."""
    case = workloads.make_case(name=f"split_d{head}", dtype=torch.bfloat16, sequences=3, query_heads=hq,
                               kv_heads=hkv, head_size=head, value_head_size=head, block_size=16,
                               lengths=[4096, 2500, 2049], seed=head + hq, device=DEV, pool_factor=1.25,
                               cache_encoding=encoding, layout="HND" if encoding == "fp8" else "NHD")
    (out, lse), merges = _merges(lambda: workloads.run_case(case, return_lse=True))
    assert merges == 1 and ops.last_internal_partition_tokens() > 0
    expected, want_lse = oracle_expected(case, threads=ORACLE_THREADS)
    assert_parity(out, expected, torch.bfloat16, f"internal split d{head} {hq}/{hkv} {encoding}")
    np.testing.assert_allclose(lse.cpu().numpy(), want_lse, **LSE_TOL)


def test_internal_split_on_the_general_kernel():
    """D != Dv runs on the general (vector) kernel; the split applies there too."""
    case = workloads.make_case(name="split_vec", dtype=torch.float16, sequences=2, query_heads=8, kv_heads=2,
                               head_size=128, value_head_size=64, block_size=16, lengths=[3000, 2048], seed=21,
                               device=DEV, pool_factor=1.25)
    (out, lse), merges = _merges(lambda: workloads.run_case(case, return_lse=True))
    assert merges == 1 and ops.last_internal_partition_tokens() > 0
    assert ops.last_kernel_family() == "vector"
    expected, want_lse = oracle_expected(case)
    assert_parity(out, expected, torch.float16, "internal split, general kernel")
    np.testing.assert_allclose(lse.cpu().numpy(), want_lse, **LSE_TOL)


def test_plan_query_agrees_with_the_calls():
    """loom_hip_paged_decode_attention_plan answers, without a launch, what the
    call then does: the internal split's size on this stream, the caller's
    partitions for a split call, one partition for a large grid or under
    capture."""
    bf16 = _native.BF16
    case = _case(18)
    run, internal = ops.plan(bf16, case.sequences, case.query_heads, case.kv_heads, 128, 128,
                             case.max_sequence_length)
    workloads.run_case(case)
    torch.cuda.synchronize()
    assert (run, internal) == (ops.last_internal_partition_tokens(), run != 0)
    assert ops.plan(bf16, 4, 12, 2, 128, 128, 2048, partition_tokens=512) == (512, False)
    assert ops.plan(bf16, 32, 64, 8, 128, 128, 1024) == (0, False)  # 256 items fill the GPU
    side = torch.cuda.Stream()
    graph = torch.cuda.CUDAGraph()
    out = torch.empty(case.sequences, case.query_heads, 128, dtype=torch.bfloat16, device=DEV)
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        workloads.run_case(case, output=out)
    torch.cuda.synchronize()
    with torch.cuda.graph(graph):
        assert ops.plan(bf16, case.sequences, case.query_heads, case.kv_heads, 128, 128,
                        case.max_sequence_length) == (0, False)
        workloads.run_case(case, output=out)
    assert ops.last_internal_partition_tokens() == 0
