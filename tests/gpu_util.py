"""Shared helpers of the GPU parity tests: device tensors -> oracle inputs."""

from __future__ import annotations

import numpy as np
import torch

import oracle

ORACLE_DTYPE = {torch.float32: oracle.F32, torch.float16: oracle.F16, torch.bfloat16: oracle.BF16}

# Parity bars (tolerances of the paged-decode north star).
TOL = {
    torch.float32: dict(atol=1e-5, rtol=0.0),
    torch.float16: dict(atol=2e-3, rtol=1e-2),
    torch.bfloat16: dict(atol=2e-3, rtol=1e-2),
}
LSE_TOL = dict(atol=1e-4, rtol=1e-5)

# Host threads for full-size oracle runs (the GPU box gives a job 16 CPUs).
ORACLE_THREADS = 16


def to_host(t: torch.Tensor) -> np.ndarray:
    """Bit-exact host copy: BF16 as uint16, F16 as float16, FP8 as uint8."""
    t = t.detach().contiguous().cpu()
    if t.dtype == torch.bfloat16:
        return t.view(torch.int16).numpy().view(np.uint16)
    if t.dtype == torch.float16:
        return t.numpy()
    if t.dtype == torch.float32:
        return t.numpy()
    if t.dtype == getattr(torch, "float8_e4m3fn", None) or t.dtype == torch.uint8:
        return t.view(torch.uint8).numpy()
    if t.dtype in (torch.int32, torch.int64):
        return t.numpy()
    raise TypeError(t.dtype)


def as_f64(t: torch.Tensor) -> np.ndarray:
    return t.detach().float().cpu().numpy().astype(np.float64)


def oracle_expected(case, seqs=None, threads=None, _host_caches=None):
    """Oracle output (F64 of the dtype-rounded result) and LSE for a DecodeCase.

    ``seqs`` restricts the oracle to a subset of sequences (the caches are
    shared, so only Q, tables and lengths are sliced). With ``threads`` > 1
    the sequences are split into that many groups run concurrently (ctypes
    releases the GIL); each group is the same single-threaded oracle, so the
    result is identical to one call.
    """
    idx = list(range(case.sequences)) if seqs is None else list(seqs)
    if threads and threads > 1 and len(idx) > 1:
        from concurrent.futures import ThreadPoolExecutor

        # Longest sequences first, dealt round-robin, so the groups take similar time.
        order = sorted(idx, key=lambda i: -case.lengths[i])
        groups = [sorted(order[g::threads]) for g in range(min(threads, len(idx)))]
        with ThreadPoolExecutor(len(groups)) as pool:
            caches = (to_host(case.key_cache), to_host(case.value_cache))
            parts = list(pool.map(lambda g: oracle_expected(case, g, _host_caches=caches), groups))
        out = np.empty((len(idx), case.query_heads, case.value_head_size), dtype=np.float64)
        lse = np.empty((len(idx), case.query_heads), dtype=np.float64)
        pos = {s: k for k, s in enumerate(idx)}
        for g, (o, l) in zip(groups, parts):
            rows = [pos[s] for s in g]
            out[rows] = o
            lse[rows] = l
        return out, lse
    q = case.query[idx]
    tables = case.block_tables[idx]
    lens = case.sequence_lengths[idx]
    lengths = [case.lengths[i] for i in idx]
    dt = ORACLE_DTYPE[case.dtype]
    spec = oracle.spec_new(
        len(idx), case.query_heads, case.kv_heads, case.head_size, case.value_head_size, case.num_blocks,
        case.block_size, case.max_blocks_per_sequence, max(lengths), case.scale, dt,
    )
    kc, vc = _host_caches if _host_caches is not None else (to_host(case.key_cache), to_host(case.value_cache))
    if case.layout == "NHD":
        kl = oracle.CacheLayout.nhd(case.block_size, case.kv_heads, case.head_size)
        vl = oracle.CacheLayout.nhd(case.block_size, case.kv_heads, case.value_head_size)
    else:
        kl = oracle.CacheLayout.hnd(case.block_size, case.kv_heads, case.head_size)
        vl = oracle.CacheLayout.hnd(case.block_size, case.kv_heads, case.value_head_size)
    kwargs = {}
    if case.cache_encoding == "fp8":
        kwargs = dict(
            cache_encoding=oracle.FP8_E4M3,
            key_scales=case.key_scales.cpu().numpy(),
            value_scales=case.value_scales.cpu().numpy(),
            scale_stride=1 if case.key_scales.numel() > 1 else 0,
        )
    out, lse = oracle.ext(spec, to_host(q), kc, vc, to_host(tables), to_host(lens), key_layout=kl,
                          value_layout=vl, **kwargs)
    if dt == oracle.BF16:
        out64 = oracle.bf16_bits_to_f32(out).astype(np.float64)
    else:
        out64 = out.astype(np.float64)
    return out64, lse


def assert_parity(actual: torch.Tensor, expected: np.ndarray, dtype, what=""):
    got = as_f64(actual)
    tol = TOL[dtype]
    bad = ~np.isclose(got, expected, **tol)
    if bad.any():
        i = np.argwhere(bad)[0]
        raise AssertionError(
            f"{what}: {int(bad.sum())} of {bad.size} elements outside atol={tol['atol']} rtol={tol['rtol']}; "
            f"first at {tuple(i)}: got {got[tuple(i)]!r} expected {expected[tuple(i)]!r}; "
            f"max abs err {np.abs(got - expected).max():.3e}"
        )
