"""The threaded oracle driver used by the full-size GPU parity tests gives
exactly the single-call oracle's result (host only)."""

from __future__ import annotations

import numpy as np
import torch

from attnarc_amd import workloads
from gpu_util import oracle_expected


def test_threaded_oracle_equals_one_call():
    case = workloads.make_case(name="threads", dtype=torch.bfloat16, sequences=7, query_heads=8, kv_heads=2,
                               head_size=64, value_head_size=64, block_size=16,
                               lengths=[5, 100, 300, 17, 64, 200, 99], seed=3, device="cpu", pool_factor=1.25)
    one = oracle_expected(case)
    many = oracle_expected(case, threads=3)
    assert np.array_equal(one[0], many[0])
    assert np.array_equal(one[1], many[1])
    sub = oracle_expected(case, seqs=[6, 1, 3], threads=2)
    assert np.array_equal(sub[0], one[0][[6, 1, 3]])
