"""Split-K partial states and the merge kernels (run on an MI355X).

Partial outputs are F32 sums, as the reference keeps them
(paged_decode_attention.cu:683-702), so each output is rounded to its
storage type once. The first test builds a sequence whose two partitions
hold means of opposite sign that a 16-bit partial cannot represent: a merge
of 16-bit partials would be off by a quarter BF16 ulp of 3 (0.004), past the
parity bar, while F32 partials land on the oracle. The others drive every
merge kernel shape: one wave per row with 2, 4 or 8 loads per lane, four and
eight waves per row (the two-stage merge of long contexts), head sizes 64,
128 and 256, F32 queries, and a workspace whose partial rows are not 16-byte
aligned (the general merge kernels).
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

from attnarc_amd import workloads
from gpu_util import LSE_TOL, assert_parity, oracle_expected

pytestmark = pytest.mark.gpu

DEV = "cuda"


def _case(seed, lengths, *, hq=8, hkv=8, head=128, dtype=torch.bfloat16, part=512, encoding="native",
          layout="NHD"):
    return workloads.make_case(name=f"merge{seed}", dtype=dtype, sequences=len(lengths), query_heads=hq,
                               kv_heads=hkv, head_size=head, value_head_size=head, block_size=16,
                               lengths=list(lengths), seed=seed, device=DEV, pool_factor=1.25,
                               partition_tokens=part, cache_encoding=encoding, layout=layout)


def _check(case, what, workspace=None):
    out, lse = workloads.run_case(case, return_lse=True, workspace=workspace)
    torch.cuda.synchronize()
    expected, want_lse = oracle_expected(case)
    assert_parity(out, expected, case.dtype, what)
    np.testing.assert_allclose(lse.cpu().numpy(), want_lse, **LSE_TOL)


def test_partials_of_opposite_sign_keep_full_precision():
    """Q = 0 (uniform attention) over 32 tokens in two 16-token partitions:
    tokens 0-15 of V alternate a and a + ulp(a) (a = 3, BF16), whose mean
    a + ulp/2 has no BF16 form, and tokens 16-31 hold -a. The exact output is
    ulp(a) / 4 = 0.0039 in every dim."""
    case = _case(1, [32], hq=8, hkv=8, part=16)
    case.query.zero_()
    a = 3.0
    ulp = 2.0 ** -6  # BF16 spacing in [2, 4)
    table = case.block_tables[0].tolist()
    for t in range(32):
        v = (a + (ulp if t % 2 else 0.0)) if t < 16 else -a
        case.value_cache[table[t // 16], t % 16].fill_(v)
    out = workloads.run_case(case)
    torch.cuda.synchronize()
    expected, _ = oracle_expected(case)
    assert np.allclose(expected, ulp / 4, atol=1e-4), "the oracle's exact output"
    assert_parity(out, expected, torch.bfloat16, "partials of opposite sign")


@pytest.mark.parametrize("head", [64, 128, 256])
@pytest.mark.parametrize("parts", [2, 3, 8, 16, 31, 64, 100, 129, 300])
def test_merge_shapes(head, parts):
    """`parts` partitions of 16 tokens for the longest sequence; the other
    sequences are shorter (some one partition, one a single token)."""
    part = 16
    lengths = [parts * part, max(1, parts * part - 7), 1, part, (parts // 2) * part + 3]
    case = _case(10 + parts, lengths, hq=8, hkv=2, head=head, part=part)
    _check(case, f"head {head}, {parts} partitions")


@pytest.mark.parametrize("parts", [5, 40, 150])
def test_f32_queries_merge(parts):
    case = _case(20 + parts, [parts * 32, 100, 33], hq=4, hkv=4, dtype=torch.float32, part=32)
    _check(case, f"f32, {parts} partitions")


@pytest.mark.parametrize("parts", [6, 40])
def test_unaligned_workspace_takes_the_general_merge(parts):
    """A workspace view starting one F32 element into its allocation leaves
    the partial rows 4-byte aligned only."""
    case = _case(30 + parts, [parts * 64, 300, 64], hq=8, hkv=2, part=64)
    from attnarc_amd import ops

    need = ops.extended_workspace_elements(case.sequences, case.query_heads, case.value_head_size,
                                           case.max_sequence_length, case.partition_tokens)
    backing = torch.empty(need + 4, dtype=torch.float32, device=DEV)
    _check(case, f"unaligned workspace, {parts} partitions", workspace=backing[1:need + 1])


def test_fp8_hnd_merge():
    case = _case(40, [4096, 1000, 2500, 17], hq=64, hkv=8, encoding="fp8", layout="HND")
    _check(case, "fp8 hnd")


@pytest.mark.parametrize("hq,hkv,dtype", [(8, 8, torch.bfloat16), (32, 8, torch.bfloat16), (4, 4, torch.float32)])
def test_length_past_max_sequence_length_stays_in_its_share(hq, hkv, dtype):
    """A caller that breaks the contract (a sequence longer than
    max_sequence_length) gets that sequence computed over its first
    max_sequence_length tokens, and no item writes a state outside the
    launch's partitions: a canary after the workspace stays untouched and
    the other sequences match the oracle."""
    from attnarc_amd import ops

    case = _case(50 + hq, [300, 1000, 64], hq=hq, hkv=hkv, dtype=dtype, part=128)
    max_len = 512
    need = ops.extended_workspace_elements(case.sequences, case.query_heads, case.value_head_size, max_len, 128)
    backing = torch.full((need + 4096,), 7.0, dtype=torch.float32, device=DEV)
    out, lse = ops.paged_decode_attention_extended(
        case.query, case.key_cache, case.value_cache, case.block_tables, case.sequence_lengths,
        max_sequence_length=max_len, scale=case.scale, layout=case.layout, partition_tokens=128,
        workspace=backing[:need], return_lse=True)
    torch.cuda.synchronize()
    assert bool((backing[need:] == 7.0).all()), "a state landed past the workspace"
    case.lengths = [300, max_len, 64]
    case.sequence_lengths = torch.tensor(case.lengths, dtype=torch.int32, device=DEV)
    expected, want_lse = oracle_expected(case)
    assert_parity(out, expected, dtype, "overlong sequence clamped to max_sequence_length")
    np.testing.assert_allclose(lse.cpu().numpy(), want_lse, **LSE_TOL)


@pytest.mark.parametrize("head,layout,hkv", [(128, "HND", 8), (128, "NHD", 8), (64, "HND", 8), (128, "HND", 6),
                                             (128, "NHD", 3)])
def test_fp8_two_partition_workgroups(head, layout, hkv):
    """FP8 grids of 1024+ items at head size 128 run four-item workgroups of
    two KV heads x two partitions that leave one state per pair (head size
    64: eight-item workgroups, one state per partition): sequences that end
    inside the first partition of a pair, exactly on a pair boundary, one
    token past it, and single-token ones."""
    rng = np.random.default_rng(head)
    lengths = [int(x) for x in rng.integers(1, 4097, 40)]
    lengths[:8] = [1, 511, 512, 513, 1024, 1025, 2048, 4096]
    case = _case(60 + head + hkv, lengths, hq=4 * hkv, hkv=hkv, head=head, encoding="fp8", layout=layout, part=256)
    _check(case, f"fp8 pairs d{head} {layout}")
    from attnarc_amd import ops

    assert ops.last_kernel_name() == "decode_stream_group_kernel"


@pytest.mark.parametrize("max_len", [2500, 1537])
def test_fp8_pairs_with_an_odd_partition_count(max_len):
    """ceil(max_len / 512) = 5 or 4 partitions (3 or 2 pair states): with 5 the
    last pair has no second partition, and sequences of every length class
    around the pair boundaries run in the same launch."""
    rng = np.random.default_rng(max_len)
    lengths = [int(x) for x in rng.integers(1, max_len + 1, 300)]
    lengths[:6] = [max_len, 2048, 2049, 1024, 1025, 1]
    lengths = [min(x, max_len) for x in lengths]
    case = _case(70 + max_len % 97, lengths, hq=16, hkv=4, encoding="fp8", layout="HND", part=512)
    assert case.max_sequence_length == max_len
    _check(case, f"fp8 pairs, max length {max_len}")
    from attnarc_amd import ops

    assert ops.last_kernel_name() == "decode_stream_group_kernel"
