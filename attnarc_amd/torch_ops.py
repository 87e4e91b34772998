"""PyTorch operators through the Stable-ABI adapter and the checked bridge.

Counterpart of the reference's ``loom_kernels.torch_ops`` facade
(python/src/loom_kernels/torch_ops.py, _torch_dispatch.py, ops/attention.py,
ops/rope_kv.py, ops/telemetry.py) for the two operators this library
implements. Loading registers ``torch.ops.loom_kernels.paged_decode_attention``,
``torch.ops.loom_kernels.rope_paged_kv_write_`` and the bridge telemetry ops
from ``attnarc_amd/_build/libloom_hip_torch.so``; every launch runs the
library's tensor-view contract tables -> bridge checks -> HIP kernels, on
torch's current stream, with split-K workspaces from the torch caching
allocator.

``attnarc_amd.ops`` is the ctypes path over the same kernels (and the extended
decode entry point); this module is the one a torch program or torch.compile
graph binds, as it would bind the reference's extension.
"""

from __future__ import annotations

import os
import threading
from enum import IntEnum

import torch

from . import build as _build
from . import ops as _ops

PAGED_DECODE_MAX_CONTEXT = _ops.PAGED_DECODE_MAX_CONTEXT
BRIDGE_ABI_VERSION = 2

_LOCK = threading.Lock()
_LOADED = False


def load_torch_extension() -> None:
    """Load the adapter library once (raises if it was not built)."""
    global _LOADED
    if _LOADED:
        return
    with _LOCK:
        if _LOADED:
            return
        path = _build.ADAPTER_LIB_PATH
        if not os.path.exists(path):
            raise ImportError(
                f"loom-hip torch adapter not found at {path}; run `python -m attnarc_amd.build`"
            )
        torch.ops.load_library(path)
        version = int(torch.ops.loom_kernels.bridge_abi_version())
        if version != BRIDGE_ABI_VERSION:
            raise RuntimeError(
                f"loom-hip bridge ABI version {version} does not match the Python facade ({BRIDGE_ABI_VERSION})"
            )
        _LOADED = True


load_torch_extension()

_paged_decode_attention = torch.ops.loom_kernels.paged_decode_attention.default
_rope_paged_kv_write = torch.ops.loom_kernels.rope_paged_kv_write_.default
_bridge_abi_version = torch.ops.loom_kernels.bridge_abi_version.default
_bridge_launch_count = torch.ops.loom_kernels.bridge_launch_count.default
_reset_bridge_launch_count = torch.ops.loom_kernels.reset_bridge_launch_count.default

supports_paged_decode_attention = _ops.supports_paged_decode_attention
supports_rope_paged_kv_write = _ops.supports_rope_paged_kv_write


class Operator(IntEnum):
    """Bridge operator ids (loom_cuda_bridge.h:28-40, ops/telemetry.py:14-25)."""

    RMS_NORM = 0
    ADD_RMS_NORM = 1
    RMS_NORM_DYNAMIC_FP8 = 2
    SILU_AND_MUL = 3
    SILU_AND_MUL_DYNAMIC_FP8 = 4
    ROPE_PAGED_KV_WRITE = 5
    GREEDY_SAMPLE_LOGPROBS = 6
    SELECTED_TOKEN_LOGPROBS = 7
    MIN_P_FILTER = 8
    PAGED_DECODE_ATTENTION = 9
    GREEDY_SPECULATIVE_VERIFY = 10


def _operator_id(operator: Operator) -> int:
    if not isinstance(operator, Operator):
        raise TypeError("operator must be an attnarc_amd.torch_ops.Operator")
    return int(operator)


def bridge_abi_version() -> int:
    """The loaded bridge's ABI version."""
    return int(_bridge_abi_version())


def launch_count(operator: Operator) -> int:
    """Successful bridge submissions of one operator."""
    return int(_bridge_launch_count(_operator_id(operator)))


def reset_launch_count(operator: Operator) -> None:
    _reset_bridge_launch_count(_operator_id(operator))


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
    """Paged decode into caller-owned output (ops/attention.py:99-123)."""
    _ops._require_inference_tensors(query, key_cache, value_cache, output)
    if scale is None:
        scale = query.shape[-1] ** -0.5
    _paged_decode_attention(query, key_cache, value_cache, block_tables, sequence_lengths, output,
                            int(max_sequence_length), float(scale))
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
    """Paged MQA/GQA decode for one query token per sequence (ops/attention.py:126-154)."""
    if query.dim() != 3 or value_cache.dim() != 4:
        raise ValueError("paged decode query/value cache must have ranks 3 and 4")
    output = torch.empty((query.shape[0], query.shape[1], value_cache.shape[3]), device=query.device,
                         dtype=query.dtype)
    return paged_decode_attention_out(query, key_cache, value_cache, block_tables, sequence_lengths, output,
                                      max_sequence_length=max_sequence_length, scale=scale)


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
    """Rotate Q/K and write native or FP8 E4M3 paged K/V caches (ops/rope_kv.py:100-134)."""
    _ops._require_inference_tensors(query, key, value, cos_sin_cache, kv_cache, key_scales, value_scales)
    _rope_paged_kv_write(query, key, value, positions, cos_sin_cache, kv_cache, key_scales, value_scales,
                         slot_mapping, bool(is_neox))
    return query, key, kv_cache


__all__ = [
    "Operator",
    "PAGED_DECODE_MAX_CONTEXT",
    "bridge_abi_version",
    "launch_count",
    "load_torch_extension",
    "paged_decode_attention",
    "paged_decode_attention_out",
    "reset_launch_count",
    "rope_paged_kv_write_",
    "supports_paged_decode_attention",
    "supports_rope_paged_kv_write",
]
