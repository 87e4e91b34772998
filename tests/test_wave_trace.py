"""The per-wave timeline summary (attnarc_amd.wave_trace) on synthetic records (host only)."""

from __future__ import annotations

import numpy as np
import torch

from attnarc_amd import wave_trace, workloads


def test_summary_of_synthetic_records():
    case = workloads.make_case(name="trace", dtype=torch.bfloat16, sequences=2, query_heads=8, kv_heads=2,
                               head_size=64, value_head_size=64, block_size=16, lengths=[1024, 700], seed=1,
                               device="cpu", pool_factor=1.25, partition_tokens=512)
    # four waves: three full 512-token partitions and one 188-token partial one
    rec = np.zeros(4, dtype=wave_trace.RECORD)
    rec["t0"] = [1000, 1000, 3000, 3500]          # 100 MHz ticks
    rec["t1"] = [3000, 3500, 5000, 4500]
    rec["xcc"] = [0, 1, 0, 1]
    rec["tokens"] = [512, 512, 512, 188]
    rec["seq"] = [0, 0, 1, 1]
    rec["part"] = [0, 1, 0, 1]
    text = wave_trace.summarize(rec, case)
    assert "first start to last end: 40.0 us" in text
    row_bytes = 2 * 64 * 2
    total = (3 * 512 + 188) * row_bytes
    assert f"KV bytes recorded: {total / 1e9:.4f} GB" in text
    assert "| 0 | 2 |" in text and "| 1 | 2 |" in text  # two items per XCC
    assert "| 0-20 | 2 | 22.5 / 20.0 / 25.0 |" in text
    assert "wave start times, percentiles 10 / 50 / 90 / 100: 0.0 / 10.0 / 23.5 / 25.0 us" in text


def test_split_items_share_their_bytes():
    case = workloads.make_case(name="trace", dtype=torch.bfloat16, sequences=1, query_heads=8, kv_heads=2,
                               head_size=64, value_head_size=64, block_size=16, lengths=[512], seed=1,
                               device="cpu", pool_factor=1.25, partition_tokens=512)
    # one item split over four waves: every wave records the whole item
    rec = np.zeros(4, dtype=wave_trace.RECORD)
    rec["t0"] = 1000
    rec["t1"] = 2000
    rec["tokens"] = 512
    text = wave_trace.summarize(rec, case)
    assert f"KV bytes recorded: {512 * 2 * 64 * 2 / 1e9:.4f} GB" in text


def test_summary_with_quarter_marks_and_load_waits():
    case = workloads.make_case(name="trace", dtype=torch.bfloat16, sequences=1, query_heads=8, kv_heads=2,
                               head_size=64, value_head_size=64, block_size=16, lengths=[1024], seed=1,
                               device="cpu", pool_factor=1.25, partition_tokens=512)
    # two full items; loop start 1 us after the start, then four 2 us quarters
    rec = np.zeros(2, dtype=wave_trace.RECORD_MARKED)
    rec["t0"] = [0, 0]
    rec["t1"] = [900, 900]
    rec["tokens"] = 512
    rec["part"] = [0, 1]
    rec["marks"] = [[100, 300, 500, 700], [100, 300, 500, 700]]
    rec["stall"] = [[10, 20, 30, 40], [10, 20, 30, 40]]
    text = wave_trace.summarize(rec, case)
    assert "## Over time, from the quarter marks" in text
    assert "| 0-20 | 2 | 9.0 / 9.0 / 9.0 | 1.0 | 2.0 / 2.0 / 2.0 / 2.0 | 0.1 / 0.2 / 0.3 / 0.4 |" in text
