"""PyTorch-facing paged decode attention over the loom-hip C ABI.

Mirrors the reference's public Python surface
(python/src/loom_kernels/ops/attention.py:1-154) and its Stable-ABI adapter
(python/csrc/attention.cpp:5-162): same function names, argument meaning,
default scale ``head_size ** -0.5`` and RuntimeError/ValueError behaviour.
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


def _has_dense_nhd_inner_strides(tensor: torch.Tensor) -> bool:
    """Only the outer cache-block stride may contain gaps (ops/attention.py:14-26)."""
    if tensor.dim() != 4:
        return False
    _, block_size, heads, width = tensor.shape
    block_elements = block_size * heads * width
    return bool(
        tensor.stride(3) == 1
        and tensor.stride(2) == width
        and tensor.stride(1) == heads * width
        and tensor.stride(0) >= block_elements
        and tensor.stride(0) <= 0xFFFF_FFFF_FFFF_FFFF
    )


def _u32(*values: int) -> bool:
    return all(0 < int(v) <= 0xFFFF_FFFF for v in values)


def supports_paged_decode_attention(
    query: torch.Tensor,
    key_cache: torch.Tensor,
    value_cache: torch.Tensor,
    block_tables: torch.Tensor,
    sequence_lengths: torch.Tensor,
    *,
    max_sequence_length: int,
) -> bool:
    """Return whether tensors match the native paged-decode kernel family.

    Same predicate as ops/attention.py:29-96 without the 1024 context cap.
    """
    if (
        query.dim() != 3
        or key_cache.dim() != 4
        or value_cache.dim() != 4
        or block_tables.dim() != 2
        or sequence_lengths.dim() != 1
        or query.numel() == 0
        or key_cache.numel() == 0
        or value_cache.numel() == 0
        or isinstance(max_sequence_length, bool)
        or not isinstance(max_sequence_length, int)
    ):
        return False
    sequences, query_heads, head_size = query.shape
    num_blocks, block_size, kv_heads, key_head_size = key_cache.shape
    return bool(
        query.device.type == "cuda"
        and key_cache.device == query.device
        and value_cache.device == query.device
        and block_tables.device == query.device
        and sequence_lengths.device == query.device
        and query.dtype in _DTYPE_CODES
        and key_cache.dtype == query.dtype
        and value_cache.dtype == query.dtype
        and block_tables.dtype == torch.int32
        and sequence_lengths.dtype == torch.int32
        and query.is_contiguous()
        and _has_dense_nhd_inner_strides(key_cache)
        and _has_dense_nhd_inner_strides(value_cache)
        and block_tables.is_contiguous()
        and sequence_lengths.is_contiguous()
        and not query.requires_grad
        and not key_cache.requires_grad
        and not value_cache.requires_grad
        and head_size == key_head_size
        and value_cache.shape[:3] == (num_blocks, block_size, kv_heads)
        and value_cache.shape[3] > 0
        and query_heads % kv_heads == 0
        and block_tables.shape[0] == sequences
        and block_tables.shape[1] > 0
        and sequence_lengths.shape[0] == sequences
        and 0 < max_sequence_length <= PAGED_DECODE_MAX_CONTEXT
        and max_sequence_length <= block_tables.shape[1] * block_size
        and _u32(
            sequences,
            query_heads,
            kv_heads,
            head_size,
            value_cache.shape[3],
            num_blocks,
            block_size,
            block_tables.shape[1],
        )
        and sequences * query_heads <= 0x7FFF_FFFF
    )


def _stream_handle(device: torch.device) -> ctypes.c_void_p:
    return ctypes.c_void_p(torch.cuda.current_stream(device).cuda_stream)


def _ptr(t: torch.Tensor | None) -> ctypes.c_void_p | None:
    return None if t is None else ctypes.c_void_p(t.data_ptr())


def _overlaps(a: torch.Tensor, b: torch.Tensor) -> bool:
    """Byte-range overlap of the storage spans of two tensors."""
    def span(t):
        if t.numel() == 0:
            return (0, 0)
        lo = t.data_ptr()
        hi = lo + (sum((s - 1) * st for s, st in zip(t.shape, t.stride())) + 1) * t.element_size()
        return (lo, hi)

    a0, a1 = span(a)
    b0, b1 = span(b)
    return a0 < b1 and b0 < a1


def _check_paged_decode_contract(
    query, key_cache, value_cache, block_tables, sequence_lengths, output,
    max_sequence_length, scale,
) -> None:
    """python/csrc/attention.cpp:5-87 without the 1024 cap."""
    def check(cond, msg):
        if not cond:
            raise RuntimeError(msg)

    check(query.is_cuda, "Loom paged decode query must be on a GPU")
    check(
        key_cache.device == query.device
        and value_cache.device == query.device
        and block_tables.device == query.device
        and sequence_lengths.device == query.device
        and output.device == query.device,
        "Loom paged decode tensors must be on one GPU device",
    )
    check(query.dtype in _DTYPE_CODES, "Loom paged decode supports F32, FP16, and BF16 native caches")
    check(
        key_cache.dtype == query.dtype and value_cache.dtype == query.dtype and output.dtype == query.dtype,
        "Loom paged decode data tensors must share a dtype",
    )
    check(
        block_tables.dtype == torch.int32 and sequence_lengths.dtype == torch.int32,
        "Loom paged decode metadata must use int32",
    )
    check(
        query.dim() == 3 and key_cache.dim() == 4 and value_cache.dim() == 4
        and block_tables.dim() == 2 and sequence_lengths.dim() == 1 and output.dim() == 3,
        "Loom paged decode requires rank-3 query/output, rank-4 K/V caches, "
        "rank-2 block tables, and rank-1 sequence lengths",
    )
    check(
        min(query.shape) > 0 and min(key_cache.shape[:3]) > 0 and value_cache.shape[3] > 0,
        "Loom paged decode dimensions must be positive",
    )
    check(key_cache.shape[3] == query.shape[2], "Loom paged decode Q/K head sizes must match")
    check(value_cache.shape[:3] == key_cache.shape[:3], "Loom paged decode K/V cache prefixes must match")
    check(query.shape[1] % key_cache.shape[2] == 0, "Loom paged decode query heads must be divisible by KV heads")
    check(
        block_tables.shape[0] == query.shape[0] and block_tables.shape[1] > 0
        and sequence_lengths.shape[0] == query.shape[0],
        "Loom paged decode metadata batch dimensions must match query",
    )
    check(
        tuple(output.shape) == (query.shape[0], query.shape[1], value_cache.shape[3]),
        "Loom paged decode output must have shape [B, Hq, Dv]",
    )
    check(
        query.is_contiguous() and _has_dense_nhd_inner_strides(key_cache)
        and _has_dense_nhd_inner_strides(value_cache) and block_tables.is_contiguous()
        and sequence_lengths.is_contiguous() and output.is_contiguous(),
        "Loom paged decode requires contiguous query/output/metadata and "
        "dense-inner NHD caches with an optional block stride",
    )
    check(
        0 < max_sequence_length <= block_tables.shape[1] * key_cache.shape[1],
        "Loom paged decode max_sequence_length must be within table capacity",
    )
    check(max_sequence_length <= PAGED_DECODE_MAX_CONTEXT, "Loom paged decode shape exceeds the HIP ABI")
    check(scale == scale and 0.0 < scale < float("inf"), "Loom paged decode scale must be finite and positive")
    check(
        not any(_overlaps(output, t) for t in (query, key_cache, value_cache, block_tables, sequence_lengths)),
        "Loom paged decode output storage must not overlap inputs",
    )
    check(
        _u32(
            query.shape[0], query.shape[1], key_cache.shape[2], query.shape[2],
            value_cache.shape[3], key_cache.shape[0], key_cache.shape[1],
            block_tables.shape[1], max_sequence_length,
        ),
        "Loom paged decode shape exceeds the HIP ABI",
    )
    check(query.shape[0] * query.shape[1] <= 0x7FFF_FFFF, "Loom paged decode grid exceeds the HIP ABI")


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

    Like the reference adapter (attention.cpp:89-149) this asks the library
    whether the shape selects split-K, allocates that F32 workspace from the
    torch allocator when it does, and launches on the current stream.
    """
    _require_inference_tensors(query, key_cache, value_cache, output)
    if scale is None:
        scale = query.shape[-1] ** -0.5
    max_sequence_length = int(max_sequence_length)
    scale = float(scale)
    _check_paged_decode_contract(
        query, key_cache, value_cache, block_tables, sequence_lengths, output,
        max_sequence_length, scale,
    )
    lib = _native.lib()
    code = _DTYPE_CODES[query.dtype]
    suffix = {_native.F32: "f32", _native.F16: "f16", _native.BF16: "bf16"}[code]
    sequences, query_heads, head_size = (int(x) for x in query.shape)
    num_blocks, block_size, kv_heads, _ = (int(x) for x in key_cache.shape)
    value_head_size = int(value_cache.shape[3])
    max_blocks = int(block_tables.shape[1])
    with torch.cuda.device(query.device):
        stream = _stream_handle(query.device)
        workspace_elements = lib.loom_hip_paged_decode_attention_split_k_workspace_elements(
            sequences, query_heads, kv_heads, head_size, value_head_size, max_sequence_length
        )
        common_tail = (
            sequences, query_heads, kv_heads, head_size, value_head_size, num_blocks,
            block_size, key_cache.stride(0), value_cache.stride(0), max_blocks,
            max_sequence_length, scale, stream,
        )
        if workspace_elements:
            workspace = torch.empty(int(workspace_elements), device=query.device, dtype=torch.float32)
            status = getattr(lib, f"loom_hip_paged_decode_attention_split_k_{suffix}")(
                _ptr(query), _ptr(key_cache), _ptr(value_cache), _ptr(block_tables),
                _ptr(sequence_lengths), _ptr(output), _ptr(workspace), workspace_elements,
                *common_tail,
            )
        else:
            status = getattr(lib, f"loom_hip_paged_decode_attention_{suffix}")(
                _ptr(query), _ptr(key_cache), _ptr(value_cache), _ptr(block_tables),
                _ptr(sequence_lengths), _ptr(output), *common_tail,
            )
    _native.check(status, "Loom paged decode attention")
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
    max_sequence_length = int(max_sequence_length)
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

    Same predicate as python/src/loom_kernels/ops/rope_kv.py:11-97.
    """
    try:
        _check_rope_paged_kv_write_contract(
            query, key, value, positions, cos_sin_cache, kv_cache, key_scales, value_scales, slot_mapping
        )
    except RuntimeError:
        return False
    return not any(t.requires_grad for t in (query, key, value, cos_sin_cache))


def _kv_span(kv_cache: torch.Tensor, dims: tuple[int, ...]) -> int:
    return 1 + sum((kv_cache.shape[d] - 1) * kv_cache.stride(d) for d in dims)


def _check_rope_paged_kv_write_contract(
    query, key, value, positions, cos_sin_cache, kv_cache, key_scales, value_scales, slot_mapping,
) -> None:
    """python/csrc/rope_kv.cpp:37-133 and the ABI limits of :141-150."""
    def check(cond, msg):
        if not cond:
            raise RuntimeError(msg)

    check(query.is_cuda, "Loom RoPE+paged-KV query must be on a GPU")
    check(
        all(t.device == query.device for t in (
            key, value, positions, cos_sin_cache, kv_cache, key_scales, value_scales, slot_mapping)),
        "Loom RoPE+paged-KV tensors must be on one GPU device",
    )
    check(
        key.dtype == query.dtype and value.dtype == query.dtype and cos_sin_cache.dtype == query.dtype,
        "Loom RoPE+paged-KV Q/K/V and cos/sin cache must share a dtype",
    )
    check(query.dtype in _DTYPE_CODES, "Loom RoPE+paged-KV supports F32, FP16, and BF16 sources")
    check(query.dim() == 3 and key.dim() == 3 and value.dim() == 3, "Loom RoPE+paged-KV Q/K/V must have rank 3")
    check(
        kv_cache.dtype == query.dtype or kv_cache.dtype == torch.uint8,
        "Loom paged K/V cache must use the source dtype or uint8 FP8 E4M3 storage",
    )
    check(
        key_scales.dtype == torch.float32 and value_scales.dtype == torch.float32
        and key_scales.is_contiguous() and value_scales.is_contiguous()
        and key_scales.numel() == value_scales.numel()
        and key_scales.numel() in (1, key.shape[1]),
        "Loom paged K/V cache scales must be contiguous float32 tensors with one element or one element per KV head",
    )
    check(
        positions.dtype == torch.int64 and slot_mapping.dtype == torch.int64,
        "Loom RoPE+paged-KV positions and slot mapping must be int64",
    )
    check(min(query.shape) > 0, "Loom RoPE+paged-KV query must be non-empty")
    check(
        key.shape[0] == query.shape[0] and value.shape[0] == query.shape[0],
        "Loom RoPE+paged-KV Q/K/V token counts must match",
    )
    check(key.shape[1] > 0 and key.shape[1] == value.shape[1], "Loom RoPE+paged-KV K/V head counts must match")
    check(key.shape[2] == query.shape[2], "Loom RoPE+paged-KV Q/K head sizes must match")
    check(value.shape[2] > 0, "Loom RoPE+paged-KV value head size must be positive")
    check(
        query.stride(2) == 1 and key.stride(2) == 1 and value.stride(2) == 1
        and min(query.stride(0), query.stride(1), key.stride(0), key.stride(1),
                value.stride(0), value.stride(1)) > 0
        and positions.is_contiguous() and cos_sin_cache.is_contiguous() and slot_mapping.is_contiguous(),
        "Loom RoPE+paged-KV sources require unit dim stride and positive token/head strides; "
        "metadata must be contiguous",
    )
    check(
        positions.dim() == 1 and positions.numel() == query.shape[0]
        and slot_mapping.dim() == 1 and slot_mapping.numel() <= query.shape[0],
        "Loom RoPE positions must cover every token and slot_mapping must not exceed the padded token count",
    )
    check(
        cos_sin_cache.dim() == 2 and cos_sin_cache.shape[0] > 0 and cos_sin_cache.shape[1] > 0
        and cos_sin_cache.shape[1] % 2 == 0 and cos_sin_cache.shape[1] <= query.shape[2],
        "Loom RoPE+paged-KV cos/sin cache must be [max_position, even rotary_dim <= head_size]",
    )
    check(
        kv_cache.dim() == 5 and kv_cache.shape[1] == 2,
        "Loom paged K/V cache must have shape [blocks, 2, block_size, kv_heads, head_size]",
    )
    check(
        kv_cache.shape[0] > 0 and kv_cache.shape[2] > 0 and kv_cache.shape[3] == key.shape[1]
        and kv_cache.shape[4] == key.shape[2] and value.shape[1] == key.shape[1]
        and value.shape[2] == key.shape[2],
        "Loom packed K/V cache and K/V sources must share head count and head size",
    )
    check(
        kv_cache.stride(4) == 1 and min(kv_cache.stride()[:4]) > 0,
        "Loom packed K/V cache requires unit element stride and positive block/KV/page/head strides",
    )
    part = _kv_span(kv_cache, (2, 3, 4))
    check(
        kv_cache.stride(1) >= part and kv_cache.stride(0) >= kv_cache.stride(1)
        and kv_cache.stride(0) - kv_cache.stride(1) >= part,
        "Loom packed K/V cache partitions must not overlap",
    )
    check(
        _u32(query.shape[0], query.shape[1], key.shape[1], query.shape[2], value.shape[2],
             cos_sin_cache.shape[1], cos_sin_cache.shape[0], kv_cache.shape[0], kv_cache.shape[2])
        and query.shape[0] <= 0x7FFF_FFFF,
        "Loom RoPE+paged-KV shape exceeds the HIP ABI",
    )


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

    Mirrors python/src/loom_kernels/ops/rope_kv.py:100-134 and the adapter
    python/csrc/rope_kv.cpp:135-220. ``kv_cache`` is
    [blocks, 2, block_size, kv_heads, head_size] (K at index 0, V at 1) in the
    source dtype, or uint8 holding FP8 E4M3FN bytes. Scale tensors are always
    passed; native caches ignore them, FP8 caches index them per tensor (one
    element) or per KV head. ``slot_mapping`` covers the first
    ``slot_mapping.numel()`` tokens; negative slots are padding. Returns
    ``(query, key, kv_cache)``.
    """
    _require_inference_tensors(query, key, value, cos_sin_cache, kv_cache, key_scales, value_scales)
    _check_rope_paged_kv_write_contract(
        query, key, value, positions, cos_sin_cache, kv_cache, key_scales, value_scales, slot_mapping
    )
    value_cache = kv_cache[:, 1]
    block, page, head = kv_cache.stride(0), kv_cache.stride(2), kv_cache.stride(3)
    rope_paged_kv_write_strided(
        query, key, value, positions, cos_sin_cache, kv_cache[:, 0], value_cache,
        key_scales, value_scales, slot_mapping,
        num_blocks=int(kv_cache.shape[0]), block_size=int(kv_cache.shape[2]),
        key_cache_strides=(block, page, head), value_cache_strides=(block, page, head),
        scale_stride=0 if key_scales.numel() == 1 else 1, is_neox=is_neox,
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
