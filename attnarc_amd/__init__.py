"""loom-hip paged MQA/GQA decode attention for MI355X (gfx950).

The compute path is ``_build/libloom_hip.so`` (HIP kernels + the C ABI of
``include/loom_hip.h``); this package is its PyTorch-facing host layer,
mirroring the reference's ``loom_kernels.ops.attention`` surface.
"""

from .ops import (  # noqa: F401
    PAGED_DECODE_MAX_CONTEXT,
    cache_strides,
    extended_workspace_elements,
    kernel_timing_enable,
    kernel_timing_read,
    launch_count,
    paged_decode_attention,
    paged_decode_attention_extended,
    paged_decode_attention_out,
    reset_launch_count,
    supports,
    supports_paged_decode_attention,
)
from ._native import LoomHipError  # noqa: F401

__all__ = [
    "PAGED_DECODE_MAX_CONTEXT",
    "LoomHipError",
    "cache_strides",
    "extended_workspace_elements",
    "kernel_timing_enable",
    "kernel_timing_read",
    "launch_count",
    "paged_decode_attention",
    "paged_decode_attention_extended",
    "paged_decode_attention_out",
    "reset_launch_count",
    "supports",
    "supports_paged_decode_attention",
]
