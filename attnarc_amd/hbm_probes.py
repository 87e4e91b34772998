"""HBM read probes behind two design choices (measurement tooling).

Not part of the operator or of ``bench.py``: these re-run the probes whose
results settled the K/V load policy and the internal split of small grids.

* ``policies``: 4 GiB read once in contiguous per-workgroup ranges under each
  load policy (plain or non-temporal, register loads or LDS DMA), per grid
  size: the evidence for the decode kernels' non-temporal K/V loads.
* ``slice``: N 512-thread workgroups (one per CU) each streaming a contiguous
  slice: what a grid that covers only N CUs can read.

Usage: ``python -m attnarc_amd.hbm_probes policies|slice`` (one JSON line per
measurement). The kernels are in ``csrc/hbm_probe.hip``
(``_build/libloom_hip_probe.so``).
"""

from __future__ import annotations

import ctypes
import json
import sys

PROBE_POLICIES = {0: "plain 16-byte loads", 1: "non-temporal 16-byte loads", 2: "LDS DMA",
                  3: "LDS DMA, non-temporal"}


def _lib():
    from . import build as _b

    return ctypes.CDLL(_b.PROBE_LIB_PATH)


def policy_probe(policy: int, nbytes: int = 4 << 30, iters: int = 10, per_cu=(2, 4, 8)) -> dict:
    """GB/s of one load policy (``PROBE_POLICIES``) by workgroups per CU."""
    import torch

    fn = _lib().loom_hip_probe_policy_read
    fn.argtypes = [ctypes.c_void_p, ctypes.c_uint64, ctypes.c_void_p, ctypes.c_uint32, ctypes.c_uint32,
                   ctypes.c_void_p]
    props = torch.cuda.get_device_properties(0)
    src = torch.ones(nbytes // 4, dtype=torch.int32, device="cuda")
    sink = torch.empty(props.multi_processor_count * max(per_cu) * 256, dtype=torch.int32, device="cuda")
    stream = ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)
    rates = {}
    for k in per_cu:
        blocks = props.multi_processor_count * k
        assert fn(src.data_ptr(), nbytes, sink.data_ptr(), blocks, policy, stream) == 0
        torch.cuda.synchronize()
        a = torch.cuda.Event(enable_timing=True)
        b = torch.cuda.Event(enable_timing=True)
        a.record()
        for _ in range(iters):
            fn(src.data_ptr(), nbytes, sink.data_ptr(), blocks, policy, stream)
        b.record()
        torch.cuda.synchronize()
        rates[k] = round(nbytes * iters / (a.elapsed_time(b) * 1e-3) / 1e9, 1)
    return rates


def slice_probe(workgroups: int, nbytes: int = 64 << 20, copies: int = 16, iters: int = 20) -> float:
    """GB/s of ``workgroups`` 512-thread workgroups each streaming a slice;
    ``copies`` rotated buffers keep the reads out of the Infinity Cache."""
    import torch

    lib = _lib()
    lib.loom_hip_probe_slice_read.argtypes = [ctypes.c_void_p, ctypes.c_uint64, ctypes.c_void_p, ctypes.c_uint32,
                                              ctypes.c_void_p]
    bufs = [torch.ones(nbytes // 4, dtype=torch.int32, device="cuda") for _ in range(copies)]
    sink = torch.empty(workgroups * 512, dtype=torch.int32, device="cuda")
    stream = ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)
    nb = nbytes - nbytes % (16 * workgroups)
    for i in range(copies):
        assert lib.loom_hip_probe_slice_read(bufs[i].data_ptr(), nb, sink.data_ptr(), workgroups, stream) == 0
    torch.cuda.synchronize()
    a = torch.cuda.Event(enable_timing=True)
    b = torch.cuda.Event(enable_timing=True)
    a.record()
    for i in range(iters):
        assert lib.loom_hip_probe_slice_read(bufs[i % copies].data_ptr(), nb, sink.data_ptr(), workgroups, stream) == 0
    b.record()
    torch.cuda.synchronize()
    return nb * iters / (a.elapsed_time(b) * 1e-3) / 1e9


def main(argv: list[str]) -> int:
    if not argv or argv[0] not in ("policies", "slice"):
        print(__doc__, file=sys.stderr)
        return 2
    if argv[0] == "policies":
        for policy, name in PROBE_POLICIES.items():
            print(json.dumps({"probe": "policies", "policy": name, "bytes": 4 << 30,
                              "GB/s by workgroups per CU": policy_probe(policy)}), flush=True)
    else:
        for wgs in (64, 128, 256, 512):
            print(json.dumps({"probe": "slice", "workgroups": wgs, "threads": 512, "bytes": 64 << 20,
                              "GB/s": round(slice_probe(wgs), 1)}), flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main(sys.argv[1:]))
