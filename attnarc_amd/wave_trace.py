"""Per-wave timeline of one paged-decode call (profiling tool).

Runs one of the benchmark configurations through the profiling build of the
library (``python -m attnarc_amd.build --wave-trace`` writes
``_build/libloom_hip_wave_trace.so``), in which every wave of the streaming
kernels records its start and end time (the 100 MHz ``s_memrealtime`` clock),
its XCC and CU, and its work item. The summary shows how the launch uses the
chip over time:

* per 10 us window: waves running, items started, and the KV rate implied
  by spreading each item's bytes evenly over its lifetime;
* item durations for full partitions by start time (the spread between waves
  that did the same work);
* per XCC: items, bytes and the time of its last item;
* the spread of full-item durations among the items that ran on one CU.

Usage: ``python -m attnarc_amd.wave_trace --config 3 [--shape SPEC] [--out FILE]``.
"""

from __future__ import annotations

import argparse
import ctypes
import os
import sys

import numpy as np

RECORD = np.dtype([("t0", "<u8"), ("t1", "<u8"), ("xcc", "<u4"), ("hw_id", "<u4"), ("seq", "<u4"),
                   ("part", "<u4"), ("kvh", "<u4"), ("tokens", "<u4")])
RECORDS = 1 << 16
# A record with the times at which the wave started its step loop (Q and the
# first steps' K/V arrived) and reached 1/4, 1/2 and 3/4 of its steps.
# ``stall``: per quarter of the steps, the time spent waiting for step loads.
RECORD_MARKED = np.dtype(RECORD.descr + [("marks", "<u8", (4,)), ("stall", "<u8", (4,))])


def collect(config: int, warmup: int = 5, shape: str | None = None, prepare=None) -> tuple[np.ndarray, object]:
    """Records of one call of configuration ``config`` (or of ``shape``, a
    workloads.shape_case spec); ``prepare(case)`` may edit the case first."""
    from . import build as _build

    if not os.path.exists(_build.WAVE_TRACE_LIB_PATH):
        raise FileNotFoundError(f"{_build.WAVE_TRACE_LIB_PATH} is missing: run python -m attnarc_amd.build --wave-trace")
    os.environ["LOOM_HIP_LIBRARY"] = _build.WAVE_TRACE_LIB_PATH
    import torch

    from . import _native, workloads

    case = workloads.shape_case(shape, "cuda:0") if shape else workloads.config(config, "cuda:0")
    if prepare is not None:
        prepare(case)
    lib = _native.lib()
    if os.path.realpath(_native.LIB_PATH) != os.path.realpath(_build.WAVE_TRACE_LIB_PATH):
        raise RuntimeError("the regular library was loaded before wave_trace selected the profiling build")
    read = lib.loom_hip_wave_trace_read
    read.argtypes = [ctypes.c_void_p, ctypes.c_uint64]
    read.restype = ctypes.c_int
    buf = np.zeros(RECORDS, dtype=RECORD)
    for _ in range(warmup):
        workloads.run_case(case)
    torch.cuda.synchronize()
    if read(buf.ctypes.data, buf.nbytes) != 0:  # clears the records of the warm-up calls
        raise RuntimeError("wave trace read failed")
    workloads.run_case(case)
    torch.cuda.synchronize()
    if read(buf.ctypes.data, buf.nbytes) != 0:
        raise RuntimeError("wave trace read failed")
    # A single-partition call on a small grid runs split inside the library:
    # its items are partitions of that size.
    lib.loom_hip_last_internal_partition_tokens.restype = ctypes.c_uint32
    case.traced_partition_tokens = int(lib.loom_hip_last_internal_partition_tokens()) or case.partition_tokens
    marks_read = lib.loom_hip_wave_trace_marks_read
    marks_read.argtypes = [ctypes.c_void_p, ctypes.c_uint64]
    marks_read.restype = ctypes.c_int
    marks = np.zeros((RECORDS, 4), dtype="<u8")
    if marks_read(marks.ctypes.data, marks.nbytes) != 0:
        raise RuntimeError("wave trace marks read failed")
    stall_read = lib.loom_hip_wave_trace_stall_read
    stall_read.argtypes = [ctypes.c_void_p, ctypes.c_uint64]
    stall_read.restype = ctypes.c_int
    stall = np.zeros((RECORDS, 4), dtype="<u8")
    if stall_read(stall.ctypes.data, stall.nbytes) != 0:
        raise RuntimeError("wave trace stall read failed")
    live = buf["tokens"] > 0
    rec = np.zeros(int(live.sum()), dtype=RECORD_MARKED)
    for name in RECORD.names:
        rec[name] = buf[name][live]
    rec["marks"] = marks[live]
    rec["stall"] = stall[live]
    return rec, case


def summarize(rec: np.ndarray, case) -> str:
    t0 = rec["t0"].min()
    start = (rec["t0"] - t0) / 100.0
    end = (rec["t1"] - t0) / 100.0
    dur = end - start
    row_bytes = (case.head_size + case.value_head_size) * case.kv_elem_bytes
    # Waves that split one item (the 4-wave split of small grids) each record
    # the whole item: share its bytes among them.
    key = (rec["seq"].astype(np.uint64) << np.uint64(40)) | (rec["part"].astype(np.uint64) << np.uint64(20)) \
        | rec["kvh"].astype(np.uint64)
    _, inverse, counts = np.unique(key, return_inverse=True, return_counts=True)
    nbytes = rec["tokens"].astype(np.float64) * row_bytes / counts[inverse]
    full = rec["tokens"] == getattr(case, "traced_partition_tokens", case.partition_tokens)
    lines = [f"# Wave timeline: {case.name}", "",
             f"- waves with work: {len(rec)}; first start to last end: {end.max():.1f} us",
             f"- KV bytes recorded: {nbytes.sum() / 1e9:.4f} GB (the call's algorithmic bytes: {case.kv_bytes() / 1e9:.4f} GB)",
             f"- whole-launch rate: {nbytes.sum() / end.max() / 1e3:.0f} GB/s",
             "- wave start times, percentiles 10 / 50 / 90 / 100: "
             + " / ".join(f"{np.percentile(start, q):.1f}" for q in (10, 50, 90, 100)) + " us",
             "- wave end times, percentiles 0 / 10 / 50 / 90: "
             + " / ".join(f"{np.percentile(end, q):.1f}" for q in (0, 10, 50, 90)) + " us", "",
             "## Over time (10 us windows)", "",
             "| window (us) | waves running | items started (full / partial) | KV GB/s, items spread evenly |",
             "|---|---|---|---|"]
    for lo in np.arange(0, end.max(), 10.0):
        hi = lo + 10.0
        overlap = np.clip(np.minimum(end, hi) - np.maximum(start, lo), 0, None)
        rate = (nbytes * overlap / np.maximum(dur, 1e-9)).sum() / 10e-6 / 1e9
        started = (start >= lo) & (start < hi)
        lines.append(f"| {lo:.0f}-{hi:.0f} | {int(((start < hi) & (end > lo)).sum())} | "
                     f"{int((started & full).sum())} / {int((started & ~full).sum())} | {rate:.0f} |")
    if "marks" in rec.dtype.names:
        # Each wave's bytes split evenly over its four quarters of steps: the
        # rate follows each wave's own progress instead of its lifetime.
        marks = (rec["marks"][:, 1:].astype(np.float64) - t0) / 100.0
        loop0 = (rec["marks"][:, 0].astype(np.float64) - t0) / 100.0
        edges = np.column_stack([start, marks, end])
        lines += ["", "## Over time, from the quarter marks (10 us windows)", "",
                  "| window (us) | KV GB/s, each quarter of a wave's steps spread over its own time |", "|---|---|"]
        for lo in np.arange(0, end.max(), 10.0):
            hi = lo + 10.0
            total = 0.0
            for q in range(4):
                a, b = edges[:, q], edges[:, q + 1]
                overlap = np.clip(np.minimum(b, hi) - np.maximum(a, lo), 0, None)
                total += (nbytes / 4 * overlap / np.maximum(b - a, 1e-9)).sum()
            lines.append(f"| {lo:.0f}-{hi:.0f} | {total / 10e-6 / 1e9:.0f} |")
    has_marks = "marks" in rec.dtype.names
    lines += ["", "## Full-partition items by start time", "",
              "| start (us) | items | duration mean / min / max (us) |"
              + (" start to loop, mean us | quarters of the steps, mean us | of which waiting for loads, mean us |"
                 if has_marks else ""),
              "|---|---|---|" + ("---|---|---|" if has_marks else "")]
    for lo in np.arange(0, end.max(), 20.0):
        m = full & (start >= lo) & (start < lo + 20.0)
        if m.any():
            row = (f"| {lo:.0f}-{lo + 20:.0f} | {int(m.sum())} | "
                   f"{dur[m].mean():.1f} / {dur[m].min():.1f} / {dur[m].max():.1f} |")
            if has_marks:
                q = np.diff(np.column_stack([loop0, edges[:, 1:]])[m], axis=1).mean(axis=0)
                row += f" {(loop0[m] - start[m]).mean():.1f} | " + " / ".join(f"{x:.1f}" for x in q) + " |"
                if "stall" in rec.dtype.names:
                    w = (rec["stall"][m].astype(np.float64) / 100.0).mean(axis=0)
                    row += " " + " / ".join(f"{x:.1f}" for x in w) + " |"
                else:
                    row += " - |"
            lines.append(row)
    xcc = rec["xcc"] & 0xF
    lines += ["", "## Per XCC", "", "| XCC | items | GB | last end (us) |", "|---|---|---|---|"]
    for x in np.unique(xcc):
        m = xcc == x
        lines.append(f"| {int(x)} | {int(m.sum())} | {nbytes[m].sum() / 1e9:.4f} | {end[m].max():.1f} |")
    # CU identity: XCC, shader engine, shader array, CU (HW_ID fields of gfx9).
    hw = rec["hw_id"]
    cu = xcc * 1000 + ((hw >> 13) & 7) * 100 + ((hw >> 12) & 1) * 16 + ((hw >> 8) & 0xF)
    per_cu = [dur[full & (cu == c)].std() for c in np.unique(cu) if (full & (cu == c)).sum() > 1]
    if per_cu:
        lines += ["", f"- spread of full-item durations among the items of one CU (mean standard deviation): "
                      f"{np.mean(per_cu):.1f} us"]
    return "\n".join(lines) + "\n"


def main(argv=None) -> int:
    ap = argparse.ArgumentParser(description=__doc__.splitlines()[0])
    ap.add_argument("--config", type=int, default=3)
    ap.add_argument("--shape", default=None, help="a workloads.shape_case spec instead of a configuration")
    ap.add_argument("--out", default=None, help="also write the summary to this file")
    args = ap.parse_args(argv)
    rec, case = collect(args.config, shape=args.shape)
    text = summarize(rec, case)
    print(text)
    if args.out:
        with open(args.out, "w") as f:
            f.write(text)
    return 0


if __name__ == "__main__":
    sys.exit(main())
