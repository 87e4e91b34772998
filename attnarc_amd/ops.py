"""PyTorch-facing paged decode attention over the loom-hip C ABI.

Mirrors the reference's public Python surface
(python/src/loom_kernels/ops/attention.py:1-154): same function names,
argument meaning, default scale ``head_size ** -0.5`` and RuntimeError /
ValueError behaviour. The tensor contract of the reference's adapter
(python/csrc/attention.cpp:5-88) is not restated here: the operands go to the
library as tensor views and its contract tables decide (include/
loom_hip_views.h), the same code the torch Stable-ABI adapter uses.
Differences: no 1024-token context cap, and an extended entry point for FP8
E4M3 caches, HND layouts, log-sum-exp output and fixed split-K partitions.

Torch is only plumbing here: tensors provide device memory and the current
HIP stream; all work runs in ``libloom_hip.so``.
"""

from __future__ import annotations

import ctypes

import torch

from . import _native

# The reference capped context at 1024 (ops/attention.py:11). The HIP kernels
# stream K/V with an online softmax, so the only limit is the uint32 ABI.
PAGED_DECODE_MAX_CONTEXT = 0xFFFF_FFFF

_DTYPE_CODES = {
    torch.float32: _native.F32,
    torch.float16: _native.F16,
    torch.bfloat16: _native.BF16,
}
_FP8_DTYPES = tuple(
    dt for dt in (getattr(torch, "float8_e4m3fn", None), torch.uint8) if dt is not None
)


def _require_inference_tensors(*tensors: torch.Tensor) -> None:
    if any(t is not None and t.requires_grad for t in tensors):
        raise ValueError("Loom Kernels operators are inference-only")


_VIEW_DTYPES = {
    torch.float32: _native.VIEW_F32,
    torch.float16: _native.VIEW_F16,
    torch.bfloat16: _native.VIEW_BF16,
    torch.uint8: _native.VIEW_U8,
    torch.int32: _native.VIEW_I32,
    torch.int64: _native.VIEW_I64,
}
if getattr(torch, "float8_e4m3fn", None) is not None:
    _VIEW_DTYPES[torch.float8_e4m3fn] = _native.VIEW_FP8_E4M3FN


def _views(*tensors: torch.Tensor):
    """The operands as ``loom_hip_tensor_view``s, for the library's contract tables."""
    views = (_native.TensorView * len(tensors))()
    for v, t in zip(views, tensors):
        v.data = t.data_ptr()
        v.device_index = t.device.index if t.is_cuda else -1
        v.dtype = _VIEW_DTYPES.get(t.dtype, _native.VIEW_OTHER)
        v.rank = t.dim()
        for d in range(min(t.dim(), 5)):
            v.sizes[d] = t.shape[d]
            v.strides[d] = t.stride(d)
    return views


_I64 = (-(1 << 63), (1 << 63) - 1)
_U32_MAX = (1 << 32) - 1


def _abi_i64(value: int) -> bool:
    """Whether ``value`` passes to an int64 ABI argument unchanged (ctypes
    would wrap it silently otherwise)."""
    return _I64[0] <= value <= _I64[1]


def _abi_u32(value: int, what: str = "shape") -> int:
    """``value`` for a uint32 ABI argument; anything outside [0, 2^32) is
    refused with the contract's ABI message instead of wrapping."""
    value = int(value)
    if not 0 <= value <= _U32_MAX:
        raise RuntimeError(f"Loom paged decode {what} exceeds the HIP ABI")
    return value


def _raise_unless_ok(status: int, operation: str) -> None:
    """A refused view set raises RuntimeError: the contract's message, or the bridge's."""
    if status == _native.VIEWS_OK:
        return
    message = _native.lib().loom_hip_views_last_error_message().decode()
    if status == _native.VIEWS_CONTRACT:
        raise RuntimeError(message)
    raise _native.LoomHipError(status, f"Loom HIP {operation} bridge failed: {message}")


def supports_paged_decode_attention(
    query: torch.Tensor,
    key_cache: torch.Tensor,
    value_cache: torch.Tensor,
    block_tables: torch.Tensor,
    sequence_lengths: torch.Tensor,
    *,
    max_sequence_length: int,
) -> bool:
    """Whether these tensors are accepted by ``paged_decode_attention``.

    The predicate of python/src/loom_kernels/ops/attention.py:29-96 without
    its 1024-token cap: the library's decode contract applied to the five
    inputs (the output and scale rules need the call itself), plus the two
    facts only Python sees (an ``int`` length, no autograd).
    """
    if isinstance(max_sequence_length, bool) or not isinstance(max_sequence_length, int):
        return False
    if not _abi_i64(max_sequence_length):  # the library's range check never sees a wrapped value
        return False
    if any(t.requires_grad for t in (query, key_cache, value_cache)):
        return False
    views = _views(query, key_cache, value_cache, block_tables, sequence_lengths)
    return _native.lib().loom_hip_views_paged_decode_check(views, 5, max_sequence_length, 1.0) == _native.VIEWS_OK


def _stream_handle(device: torch.device) -> ctypes.c_void_p:
    return ctypes.c_void_p(torch.cuda.current_stream(device).cuda_stream)


def _ptr(t: torch.Tensor | None) -> ctypes.c_void_p | None:
    return None if t is None else ctypes.c_void_p(t.data_ptr())


def paged_decode_attention_out(
    query: torch.Tensor,
    key_cache: torch.Tensor,
    value_cache: torch.Tensor,
    block_tables: torch.Tensor,
    sequence_lengths: torch.Tensor,
    output: torch.Tensor,
    *,
    max_sequence_length: int,
    scale: float | None = None,
) -> torch.Tensor:
    """Execute paged decode attention into caller-owned output storage.

    The library checks the views against its decode contract and sizes the
    split-K workspace; the workspace comes from the torch allocator on the
    current stream, and the call goes through the checked bridge.
    """
    _require_inference_tensors(query, key_cache, value_cache, output)
    if scale is None:
        scale = query.shape[-1] ** -0.5
    lib = _native.lib()
    views = _views(query, key_cache, value_cache, block_tables, sequence_lengths, output)
    max_sequence_length = int(max_sequence_length)
    if not _abi_i64(max_sequence_length):
        raise RuntimeError("Loom paged decode shape exceeds the HIP ABI")
    elements = ctypes.c_uint64()
    _raise_unless_ok(
        lib.loom_hip_views_paged_decode_workspace_elements(views, max_sequence_length, float(scale),
                                                           ctypes.byref(elements)),
        "paged decode workspace query",
    )
    with torch.cuda.device(query.device):
        workspace = None
        if elements.value:
            workspace = torch.empty(int(elements.value), device=query.device, dtype=torch.float32)
        _raise_unless_ok(
            lib.loom_hip_views_paged_decode_attention(views, max_sequence_length, float(scale), _ptr(workspace),
                                                      elements.value, _stream_handle(query.device)),
            "paged decode attention",
        )
    return output


def paged_decode_attention(
    query: torch.Tensor,
    key_cache: torch.Tensor,
    value_cache: torch.Tensor,
    block_tables: torch.Tensor,
    sequence_lengths: torch.Tensor,
    *,
    max_sequence_length: int,
    scale: float | None = None,
) -> torch.Tensor:
    """Execute paged MQA/GQA for one query token per sequence (ops/attention.py:127-154)."""
    if query.dim() != 3 or value_cache.dim() != 4:
        raise ValueError("paged decode query/value cache must have ranks 3 and 4")
    output = torch.empty(
        (query.shape[0], query.shape[1], value_cache.shape[3]),
        device=query.device,
        dtype=query.dtype,
    )
    return paged_decode_attention_out(
        query, key_cache, value_cache, block_tables, sequence_lengths, output,
        max_sequence_length=max_sequence_length, scale=scale,
    )


# ---------------------------------------------------------------------------
# Extended entry point: FP8 E4M3 caches, NHD/HND views, LSE, partitions.
# ---------------------------------------------------------------------------


def cache_strides(cache: torch.Tensor, layout: str) -> tuple[int, int, int, int, int, int]:
    """(num_blocks, block_size, kv_heads, dim, (block, page, head) strides) of a cache view.

    ``NHD`` tensors are [blocks, block_size, kv_heads, dim]; ``HND`` tensors
    are [blocks, kv_heads, block_size, dim]. The dim stride must be 1.
    """
    if cache.dim() != 4 or cache.stride(3) != 1:
        raise RuntimeError("Loom paged decode caches must be rank 4 with a unit dim stride")
    if layout == "NHD":
        nb, bs, hkv, dim = cache.shape
        return int(nb), int(bs), int(hkv), int(dim), (cache.stride(0), cache.stride(1), cache.stride(2))
    if layout == "HND":
        nb, hkv, bs, dim = cache.shape
        return int(nb), int(bs), int(hkv), int(dim), (cache.stride(0), cache.stride(2), cache.stride(1))
    raise ValueError(f"unknown cache layout {layout!r}; expected 'NHD' or 'HND'")


def extended_workspace_elements(
    sequences: int, query_heads: int, value_head_size: int, max_sequence_length: int,
    partition_tokens: int,
) -> int:
    return int(
        _native.lib().loom_hip_paged_decode_attention_extended_workspace_elements(
            sequences, query_heads, value_head_size, max_sequence_length, partition_tokens
        )
    )


def paged_decode_attention_extended(
    query: torch.Tensor,
    key_cache: torch.Tensor,
    value_cache: torch.Tensor,
    block_tables: torch.Tensor,
    sequence_lengths: torch.Tensor,
    *,
    max_sequence_length: int,
    scale: float | None = None,
    layout: str = "NHD",
    key_scales: torch.Tensor | None = None,
    value_scales: torch.Tensor | None = None,
    partition_tokens: int = 0,
    output: torch.Tensor | None = None,
    lse: torch.Tensor | None = None,
    return_lse: bool = False,
    workspace: torch.Tensor | None = None,
    no_alloc: bool = False,
):
    """Paged decode over native or FP8 E4M3 caches in NHD or HND layout.

    FP8 caches (``torch.float8_e4m3fn`` or ``torch.uint8``) take F32 scales of
    one element (per tensor) or ``kv_heads`` elements (per KV head); the
    logical value is ``fp8_to_f32(byte) * scale[kv_head]``. With
    ``partition_tokens > 0`` each sequence is split into partitions of that
    many tokens merged by log-sum-exp; the F32 workspace is allocated here
    unless given. ``no_alloc=True`` calls the no-allocation entry point
    instead: the partial states go to the library's static per-device array
    (``output`` and ``lse`` must then be given when they are wanted, and no
    ``workspace`` is taken). Returns ``output`` or ``(output, lse)``.
    """
    _require_inference_tensors(query, key_cache, value_cache)
    if query.dim() != 3 or not query.is_contiguous():
        raise RuntimeError("Loom paged decode query must be a contiguous rank-3 tensor")
    if query.dtype not in _DTYPE_CODES:
        raise RuntimeError("Loom paged decode supports F32, FP16, and BF16 queries")
    nb, bs, hkv, dk, kstr = cache_strides(key_cache, layout)
    nbv, bsv, hkvv, dv, vstr = cache_strides(value_cache, layout)
    if (nb, bs, hkv) != (nbv, bsv, hkvv):
        raise RuntimeError("Loom paged decode K/V cache prefixes must match")
    if dk != query.shape[2]:
        raise RuntimeError("Loom paged decode Q/K head sizes must match")
    fp8 = key_cache.dtype in _FP8_DTYPES
    if fp8:
        if value_cache.dtype not in _FP8_DTYPES:
            raise RuntimeError("Loom paged decode K/V caches must share an encoding")
        if key_scales is None or value_scales is None:
            raise RuntimeError("Loom paged decode FP8 caches require key and value scales")
        if key_scales.dtype != torch.float32 or value_scales.dtype != torch.float32:
            raise RuntimeError("Loom paged decode FP8 scales must be F32")
        if key_scales.numel() != value_scales.numel() or key_scales.numel() not in (1, hkv):
            raise RuntimeError("Loom paged decode FP8 scales must have 1 or kv_heads elements")
        scale_stride = 0 if key_scales.numel() == 1 else 1
        encoding = _native.KV_CACHE_FP8_E4M3
        key_scales = key_scales.contiguous()
        value_scales = value_scales.contiguous()
    else:
        if key_cache.dtype != query.dtype or value_cache.dtype != query.dtype:
            raise RuntimeError("Loom paged decode data tensors must share a dtype")
        if key_scales is not None or value_scales is not None:
            raise RuntimeError("Loom paged decode native caches take no scales")
        scale_stride = 0
        encoding = _native.KV_CACHE_NATIVE
    if block_tables.dtype != torch.int32 or sequence_lengths.dtype != torch.int32:
        raise RuntimeError("Loom paged decode metadata must use int32")
    if not (block_tables.is_contiguous() and sequence_lengths.is_contiguous()):
        raise RuntimeError("Loom paged decode metadata must be contiguous")
    if scale is None:
        scale = query.shape[-1] ** -0.5
    sequences, query_heads, head_size = (int(x) for x in query.shape)
    max_sequence_length = _abi_u32(max_sequence_length)
    partition_tokens = _abi_u32(partition_tokens, "partition size")
    if output is None:
        output = torch.empty((sequences, query_heads, dv), device=query.device, dtype=query.dtype)
    if lse is None and return_lse:
        lse = torch.empty((sequences, query_heads), device=query.device, dtype=torch.float32)
    code = _DTYPE_CODES[query.dtype]
    if no_alloc:
        if workspace is not None:
            raise RuntimeError("Loom paged decode no-allocation calls take no workspace")
        with torch.cuda.device(query.device):
            status = _native.lib().loom_hip_paged_decode_attention_extended_no_alloc(
                code, _ptr(query), _ptr(key_cache), _ptr(value_cache), _ptr(key_scales), _ptr(value_scales),
                _ptr(block_tables), _ptr(sequence_lengths), _ptr(output), _ptr(lse),
                sequences, query_heads, hkv, head_size, dv, nb, bs, encoding, scale_stride,
                *kstr, *vstr, int(block_tables.shape[1]), max_sequence_length, int(partition_tokens),
                float(scale), _stream_handle(query.device),
            )
        _native.check(status, "Loom paged decode attention (no allocation)")
        return (output, lse) if return_lse else output
    need = extended_workspace_elements(sequences, query_heads, dv, max_sequence_length, partition_tokens)
    if need and workspace is None:
        workspace = torch.empty(need, device=query.device, dtype=torch.float32)
    if not need:
        workspace = None
    code = _DTYPE_CODES[query.dtype]
    suffix = {_native.F32: "f32", _native.F16: "f16", _native.BF16: "bf16"}[code]
    with torch.cuda.device(query.device):
        status = getattr(_native.lib(), f"loom_hip_paged_decode_attention_extended_{suffix}")(
            _ptr(query), _ptr(key_cache), _ptr(value_cache), _ptr(key_scales), _ptr(value_scales),
            _ptr(block_tables), _ptr(sequence_lengths), _ptr(output), _ptr(lse), _ptr(workspace),
            0 if workspace is None else workspace.numel(),
            sequences, query_heads, hkv, head_size, dv, nb, bs, encoding, scale_stride,
            *kstr, *vstr, int(block_tables.shape[1]), max_sequence_length, int(partition_tokens),
            float(scale), _stream_handle(query.device),
        )
    _native.check(status, "Loom paged decode attention")
    return (output, lse) if return_lse else output


# ---------------------------------------------------------------------------
# Fused RoPE + paged K/V cache write.
# ---------------------------------------------------------------------------


def supports_rope_paged_kv_write(
    query: torch.Tensor,
    key: torch.Tensor,
    value: torch.Tensor,
    positions: torch.Tensor,
    cos_sin_cache: torch.Tensor,
    kv_cache: torch.Tensor,
    key_scales: torch.Tensor,
    value_scales: torch.Tensor,
    slot_mapping: torch.Tensor,
) -> bool:
    """Whether the tensors match the native/FP8 RoPE+paged-write ABI.

    The predicate of python/src/loom_kernels/ops/rope_kv.py:11-97: the
    library's RoPE+paged-KV contract, plus no autograd on the sources.
    """
    if any(t.requires_grad for t in (query, key, value, cos_sin_cache)):
        return False
    views = _views(query, key, value, positions, cos_sin_cache, kv_cache, key_scales, value_scales, slot_mapping)
    return _native.lib().loom_hip_views_rope_paged_kv_check(views) == _native.VIEWS_OK


def rope_paged_kv_write_(
    query: torch.Tensor,
    key: torch.Tensor,
    value: torch.Tensor,
    positions: torch.Tensor,
    cos_sin_cache: torch.Tensor,
    kv_cache: torch.Tensor,
    key_scales: torch.Tensor,
    value_scales: torch.Tensor,
    slot_mapping: torch.Tensor,
    is_neox: bool = True,
) -> tuple[torch.Tensor, torch.Tensor, torch.Tensor]:
    """Rotate Q/K in place and write native or scaled FP8 E4M3 paged K/V caches.

    Mirrors python/src/loom_kernels/ops/rope_kv.py:100-134. ``kv_cache`` is
    [blocks, 2, block_size, kv_heads, head_size] (K at index 0, V at 1) in the
    source dtype, or uint8 holding FP8 E4M3FN bytes. Scale tensors are always
    passed; native caches ignore them, FP8 caches index them per tensor (one
    element) or per KV head. ``slot_mapping`` covers the first
    ``slot_mapping.numel()`` tokens; negative slots are padding. The library
    checks the views and submits through the checked bridge. Returns
    ``(query, key, kv_cache)``.
    """
    _require_inference_tensors(query, key, value, cos_sin_cache, kv_cache, key_scales, value_scales)
    views = _views(query, key, value, positions, cos_sin_cache, kv_cache, key_scales, value_scales, slot_mapping)
    lib = _native.lib()
    _raise_unless_ok(lib.loom_hip_views_rope_paged_kv_check(views), "RoPE+paged-KV")
    with torch.cuda.device(query.device):
        _raise_unless_ok(
            lib.loom_hip_views_rope_paged_kv_write(views, 1 if is_neox else 0, _stream_handle(query.device)),
            "RoPE+paged-KV",
        )
    return query, key, kv_cache


def rope_paged_kv_write_strided(
    query: torch.Tensor,
    key: torch.Tensor,
    value: torch.Tensor,
    positions: torch.Tensor,
    cos_sin_cache: torch.Tensor,
    key_cache: torch.Tensor,
    value_cache: torch.Tensor,
    key_scales: torch.Tensor | None,
    value_scales: torch.Tensor | None,
    slot_mapping: torch.Tensor | None,
    *,
    num_blocks: int,
    block_size: int,
    key_cache_strides: tuple[int, int, int],
    value_cache_strides: tuple[int, int, int],
    scale_stride: int = 0,
    is_neox: bool = True,
) -> None:
    """Direct binding of ``loom_hip_rope_paged_kv_write_*`` over explicit strides.

    Caches are separate K and V tensors addressed through (block, page, head)
    element strides, so NHD ([blocks, block_size, heads, dim]), HND
    ([blocks, heads, block_size, dim]) and packed views all fit. A uint8 (or
    float8_e4m3fn) key cache selects FP8 E4M3 encoding with the given scales.
    Native caches ignore the scales (they may be None). The caller is
    responsible for the storage covering every addressed slot.
    """
    if query.dtype not in _DTYPE_CODES:
        raise RuntimeError("Loom RoPE+paged-KV supports F32, FP16, and BF16 sources")
    fp8 = key_cache.dtype in _FP8_DTYPES
    encoding = _native.KV_CACHE_FP8_E4M3 if fp8 else _native.KV_CACHE_NATIVE
    if fp8 and (key_scales is None or value_scales is None):
        raise RuntimeError("Loom RoPE+paged-KV FP8 caches require key and value scales")
    tokens = int(query.shape[0])
    cache_tokens = 0 if slot_mapping is None else int(slot_mapping.numel())
    code = _DTYPE_CODES[query.dtype]
    suffix = {_native.F32: "f32", _native.F16: "f16", _native.BF16: "bf16"}[code]
    with torch.cuda.device(query.device):
        status = getattr(_native.lib(), f"loom_hip_rope_paged_kv_write_{suffix}")(
            _ptr(query), _ptr(key), _ptr(value), _ptr(positions), _ptr(cos_sin_cache),
            _ptr(key_cache), _ptr(value_cache), _ptr(key_scales), _ptr(value_scales),
            _ptr(slot_mapping) if cache_tokens else None,
            tokens, cache_tokens, int(query.shape[1]), int(key.shape[1]), int(query.shape[2]),
            int(value.shape[2]), int(cos_sin_cache.shape[1]), int(cos_sin_cache.shape[0]),
            int(num_blocks), int(block_size), encoding, int(scale_stride),
            query.stride(0), query.stride(1), key.stride(0), key.stride(1), value.stride(0), value.stride(1),
            *key_cache_strides, *value_cache_strides, 1 if is_neox else 0, _stream_handle(query.device),
        )
    _native.check(status, "Loom RoPE+paged-KV")


# ---------------------------------------------------------------------------
# Capability query and telemetry.
# ---------------------------------------------------------------------------


def supports(
    dtype: int, cache_encoding: int, sequences: int, query_heads: int, kv_heads: int,
    head_size: int, value_head_size: int, num_blocks: int, block_size: int,
    max_blocks_per_sequence: int, max_sequence_length: int, scale: float,
) -> tuple[int, str, str]:
    """Backend::supports for PagedDecodeAttention: (status, reason, kernel family)."""
    reason = ctypes.c_char_p()
    family = ctypes.c_char_p()
    status = _native.lib().loom_hip_paged_decode_attention_supports(
        dtype, cache_encoding, sequences, query_heads, kv_heads, head_size, value_head_size,
        num_blocks, block_size, max_blocks_per_sequence, max_sequence_length, scale,
        ctypes.byref(reason), ctypes.byref(family),
    )
    return status, reason.value.decode(), family.value.decode()


def last_kernel_family() -> str:
    """Kernel family the last successful paged-decode call on this thread launched."""
    return _native.lib().loom_hip_last_kernel_family().decode()


def last_internal_partition_tokens() -> int:
    """Partition size of the internal split of the last successful paged-decode
    call on this thread (0: it ran as the caller asked)."""
    return int(_native.lib().loom_hip_last_internal_partition_tokens())


def last_kernel_name() -> str:
    """Decode kernel the last successful paged-decode call on this thread launched."""
    return _native.lib().loom_hip_last_kernel_name().decode()


def plan(dtype: int, sequences: int, query_heads: int, kv_heads: int, head_size: int, value_head_size: int,
         max_sequence_length: int, partition_tokens: int = 0, stream=None) -> tuple[int, bool]:
    """(partition tokens the call would run with, whether that is the
    library's internal split) for a paged-decode call on ``stream`` (a torch
    stream or raw handle; the current stream by default), without a launch."""
    if stream is None:
        stream = torch.cuda.current_stream().cuda_stream
    elif hasattr(stream, "cuda_stream"):
        stream = stream.cuda_stream
    run = ctypes.c_uint32()
    internal = ctypes.c_uint32()
    _native.check(
        _native.lib().loom_hip_paged_decode_attention_plan(
            dtype, sequences, query_heads, kv_heads, head_size, value_head_size, _abi_u32(max_sequence_length),
            _abi_u32(partition_tokens, "partition size"), ctypes.c_void_p(stream), ctypes.byref(run),
            ctypes.byref(internal)),
        "paged decode plan",
    )
    return int(run.value), bool(internal.value)


def launch_count(operation: int = _native.PAGED_DECODE_ATTENTION) -> int:
    count = ctypes.c_uint64()
    _native.check(_native.lib().loom_hip_launch_count(operation, ctypes.byref(count)), "launch count")
    return int(count.value)


def reset_launch_count(operation: int = _native.PAGED_DECODE_ATTENTION) -> None:
    _native.check(_native.lib().loom_hip_reset_launch_count(operation), "reset launch count")


def kernel_timing_enable(enable: bool) -> None:
    _native.check(_native.lib().loom_hip_kernel_timing_enable(1 if enable else 0), "kernel timing")


def kernel_timing_read(kernel: int) -> tuple[float, int]:
    ms = ctypes.c_double()
    n = ctypes.c_uint64()
    _native.check(
        _native.lib().loom_hip_kernel_timing_read(kernel, ctypes.byref(ms), ctypes.byref(n)),
        "kernel timing read",
    )
    return float(ms.value), int(n.value)
