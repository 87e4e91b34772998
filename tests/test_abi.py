"""C-ABI tests that run without a GPU.

The library must load, export every function declared in include/loom_hip.h,
and reject invalid arguments on the host before touching a device
(paged_decode_attention.cu:999-1049 semantics, minus the 1024 cap). Fake,
non-dereferenced pointers stand in for device buffers, as the reference's
bridge tests do with fake host addresses.
"""

from __future__ import annotations

import ctypes
import os
import re

import pytest
import torch

from attnarc_amd import _native, ops

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HEADERS = [os.path.join(ROOT, "include", h) for h in ("loom_hip.h", "loom_hip_bridge.h", "loom_hip_views.h")]


def declared_functions():
    text = "\n".join(open(h).read() for h in HEADERS)
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(loom_hip_[a-z0-9_]+)\s*\(", text)))


def test_library_exports_every_declared_symbol():
    lib = _native.lib()
    names = declared_functions()
    assert len(names) >= 20
    for name in names:
        assert hasattr(lib, name), name
        assert name in _native.SIGNATURES, f"{name} has no ctypes signature"
    assert set(_native.SIGNATURES) == set(names)


def test_status_strings_and_identity():
    assert _native.status_string(0) == "success"
    assert _native.status_string(1) == "invalid argument"
    assert _native.status_string(2) == "unsupported"
    assert _native.status_string(3) == "HIP launch error"
    assert _native.status_string(4) == "HIP unavailable"
    assert _native.status_string(99) == "unknown Loom HIP status"
    lib = _native.lib()
    assert lib.loom_hip_backend_name() == b"loom-hip"
    assert lib.loom_hip_abi_version() == 1


# Fake device addresses: distinct, 256-byte aligned, far apart.
FAKE = {name: ctypes.c_void_p(0x7F0000000000 + i * 0x100000000) for i, name in enumerate(
    ["q", "k", "v", "tables", "lens", "out", "ws", "lse", "ks", "vs"])}


def base_args(**kw):
    a = dict(q=FAKE["q"], k=FAKE["k"], v=FAKE["v"], tables=FAKE["tables"], lens=FAKE["lens"], out=FAKE["out"],
             B=4, Hq=8, Hkv=2, D=64, Dv=64, NB=64, bs=16, kbs=16 * 2 * 64, vbs=16 * 2 * 64, maxb=16, maxlen=256,
             scale=0.125)
    a.update(kw)
    return a


def call_base(suffix="f32", **kw):
    a = base_args(**kw)
    fn = getattr(_native.lib(), f"loom_hip_paged_decode_attention_{suffix}")
    return fn(a["q"], a["k"], a["v"], a["tables"], a["lens"], a["out"], a["B"], a["Hq"], a["Hkv"], a["D"], a["Dv"],
              a["NB"], a["bs"], a["kbs"], a["vbs"], a["maxb"], a["maxlen"], a["scale"], None)


@pytest.mark.parametrize("suffix", ["f32", "f16", "bf16"])
@pytest.mark.parametrize("change", [
    dict(q=None), dict(k=None), dict(v=None), dict(tables=None), dict(lens=None), dict(out=None),
    dict(B=0), dict(Hq=0), dict(Hkv=0), dict(D=0), dict(Dv=0), dict(NB=0), dict(bs=0), dict(maxb=0),
    dict(maxlen=0), dict(Hq=6, Hkv=4), dict(scale=0.0), dict(scale=-1.0), dict(scale=float("nan")),
    dict(scale=float("inf")), dict(maxlen=257), dict(kbs=16 * 2 * 64 - 1), dict(vbs=1),
    dict(out=ctypes.c_void_p(FAKE["q"].value + 64)),  # output overlaps the query
    dict(B=0x10000, Hq=0x10000, Hkv=1),  # grid exceeds INT_MAX
])
def test_base_entry_points_reject_invalid_arguments(suffix, change):
    assert call_base(suffix, **change) == _native.INVALID_ARGUMENT
    assert _native.last_error() != ""


# Valid arguments with fake pointers would launch kernels on a GPU host: these
# two tests only run where no HIP device exists.
no_device = pytest.mark.skipif(torch.cuda.is_available(), reason="valid calls with fake pointers need a GPU-less host")


@no_device
def test_long_context_is_not_capped():
    # The reference rejected max_sequence_length > 1024; here it passes host
    # validation and only fails because this host has no HIP device.
    status = call_base("bf16", D=128, Dv=128, kbs=16 * 2 * 128, vbs=16 * 2 * 128, maxb=8192, maxlen=131072)
    assert status == _native.UNAVAILABLE
    assert "no HIP device" in _native.last_error()


def test_split_k_sizing_policy():
    lib = _native.lib()
    ws = lib.loom_hip_paged_decode_attention_split_k_workspace_elements
    # plenty of (sequence, kv head) work or a short context: base path
    assert ws(256, 32, 8, 128, 128, 8192) == 0
    assert ws(32, 32, 8, 128, 128, 8192) == 0  # 256 work items fill the CUs
    assert ws(16, 32, 8, 128, 128, 4096) == 16 * 32 * 8 * 130  # 128 work items: 8 parts of 512
    assert ws(32, 12, 2, 128, 128, 2048) == 32 * 12 * 16 * 130  # C2: 64 work items, 16 parts of 128
    assert ws(8, 32, 8, 128, 128, 511) == 0
    # fewer work items than CUs: 64-token partitions from a 512-token context on
    assert ws(8, 32, 8, 128, 128, 512) == 8 * 32 * 8 * 130
    assert ws(8, 32, 8, 128, 128, 1024) == 8 * 32 * 16 * 130
    # a grid that already covers the CUs stays whole
    assert ws(32, 32, 8, 128, 128, 512) == 0
    assert ws(32, 32, 8, 128, 128, 1024) == 0
    assert ws(0, 32, 8, 128, 128, 4096) == 0
    assert ws(8, 30, 8, 128, 128, 4096) == 0  # heads not divisible
    # long context, small grid: split; size = B*Hq*parts*(Dv+2)
    n = ws(8, 32, 1, 128, 128, 131072)
    assert n > 0 and n % (8 * 32 * 130) == 0
    parts = n // (8 * 32 * 130)
    assert parts >= 2


def test_extended_workspace_sizing():
    ws = _native.lib().loom_hip_paged_decode_attention_extended_workspace_elements
    assert ws(64, 32, 128, 8192, 512) == 64 * 32 * 16 * 130
    assert ws(64, 32, 128, 8192, 0) == 0
    assert ws(64, 32, 128, 512, 512) == 0
    assert ws(64, 32, 128, 513, 512) == 64 * 32 * 2 * 130
    assert ws(8, 32, 128, 131072, 1024) == 8 * 32 * 128 * 130


def ext_args(**kw):
    a = dict(q=FAKE["q"], k=FAKE["k"], v=FAKE["v"], ks=None, vs=None, tables=FAKE["tables"], lens=FAKE["lens"],
             out=FAKE["out"], lse=None, ws=None, wsn=0, B=4, Hq=8, Hkv=2, D=128, Dv=128, NB=64, bs=16, enc=0,
             sstride=0, kb=16 * 2 * 128, kp=2 * 128, kh=128, vb=16 * 2 * 128, vp=2 * 128, vh=128, maxb=16,
             maxlen=256, part=0, scale=0.0883)
    a.update(kw)
    return a


def call_ext(suffix="bf16", **kw):
    a = ext_args(**kw)
    fn = getattr(_native.lib(), f"loom_hip_paged_decode_attention_extended_{suffix}")
    return fn(a["q"], a["k"], a["v"], a["ks"], a["vs"], a["tables"], a["lens"], a["out"], a["lse"], a["ws"],
              a["wsn"], a["B"], a["Hq"], a["Hkv"], a["D"], a["Dv"], a["NB"], a["bs"], a["enc"], a["sstride"],
              a["kb"], a["kp"], a["kh"], a["vb"], a["vp"], a["vh"], a["maxb"], a["maxlen"], a["part"], a["scale"],
              None)


@pytest.mark.parametrize("change", [
    dict(enc=2),  # unknown encoding
    dict(enc=1),  # FP8 without scales
    dict(enc=1, ks=FAKE["ks"], vs=FAKE["vs"], sstride=2),  # bad scale stride
    dict(ks=FAKE["ks"], vs=FAKE["vs"]),  # native cache with scales
    dict(sstride=1),  # native cache with a scale stride
    dict(kp=0), dict(vh=0), dict(kb=0),  # zero strides
    dict(kb=2**62),  # span overflows
    dict(part=64),  # partitioned but no workspace
    dict(part=64, ws=FAKE["ws"], wsn=10),  # workspace too small
    dict(ws=FAKE["ws"], wsn=100),  # single partition with a workspace
    dict(lse=ctypes.c_void_p(FAKE["out"].value + 128)),  # LSE overlaps the output
    dict(lse=ctypes.c_void_p(FAKE["tables"].value)),  # LSE overlaps an input
    dict(part=64, ws=ctypes.c_void_p(FAKE["k"].value + 4096), wsn=4 * 8 * 4 * 130),  # workspace inside K
])
def test_extended_entry_points_reject_invalid_arguments(change):
    assert call_ext(**change) == _native.INVALID_ARGUMENT


@no_device
def test_extended_valid_arguments_reach_the_device_check():
    need = _native.lib().loom_hip_paged_decode_attention_extended_workspace_elements(4, 8, 128, 256, 64)
    for change in [dict(), dict(enc=1, ks=FAKE["ks"], vs=FAKE["vs"], sstride=1), dict(part=64, ws=FAKE["ws"], wsn=need),
                   dict(lse=FAKE["lse"]), dict(kb=16 * 2 * 128, kp=128, kh=16 * 128)]:
        assert call_ext(**change) == _native.UNAVAILABLE, (change, _native.last_error())


def test_capability_query():
    s, reason, fam = ops.supports(2, 0, 64, 32, 8, 128, 128, 21800, 16, 512, 8192, 0.088)
    assert (s, fam) == (0, "mfma-stream")
    s, reason, fam = ops.supports(2, 0, 64, 32, 8, 128, 128, 21800, 8, 1024, 8192, 0.088)
    assert (s, fam) == (0, "mfma")
    s, reason, fam = ops.supports(1, 0, 64, 64, 2, 128, 128, 21800, 16, 512, 8192, 0.088)
    assert (s, fam) == (0, "mfma-stream")  # 32 heads per KV head: two 16-head tiles per wave
    s, reason, fam = ops.supports(1, 0, 64, 64, 2, 128, 128, 21800, 8, 1024, 8192, 0.088)
    assert (s, fam) == (0, "mfma")
    s, reason, fam = ops.supports(0, 0, 4, 8, 8, 64, 64, 64, 16, 16, 256, 0.125)
    assert (s, fam) == (0, "vector")
    s, reason, fam = ops.supports(2, 0, 4, 8, 8, 64, 64, 64, 16, 16, 256, 0.125)
    assert (s, fam) == (0, "mfma-stream")  # head size 64, 16-bit cache: 128-byte rows
    s, reason, fam = ops.supports(2, 1, 4, 8, 8, 64, 64, 64, 16, 16, 256, 0.125)
    assert (s, fam) == (0, "mfma-stream")  # FP8 cache at head size 64: 64-byte rows
    s, reason, fam = ops.supports(2, 0, 4, 8, 8, 96, 96, 64, 16, 16, 256, 0.102)
    assert (s, fam) == (0, "mfma-stream")  # head size 96, 16-bit cache: 192-byte rows
    s, reason, fam = ops.supports(2, 1, 4, 8, 8, 96, 96, 64, 16, 16, 256, 0.102)
    assert (s, fam) == (0, "mfma-stream")  # FP8 cache at head size 96: 96-byte rows
    s, reason, fam = ops.supports(2, 0, 4, 8, 8, 80, 80, 64, 16, 16, 256, 0.11)
    assert (s, fam) == (0, "mfma-stream")  # head size 80, 16-bit cache: 160-byte rows
    s, reason, fam = ops.supports(2, 0, 4, 8, 8, 112, 112, 64, 16, 16, 256, 0.094)
    assert (s, fam) == (0, "mfma-stream")  # head size 112, 16-bit cache: 224-byte rows
    s, reason, fam = ops.supports(2, 1, 4, 8, 8, 80, 80, 64, 16, 16, 256, 0.11)
    assert (s, fam) == (0, "mfma-stream")  # FP8 cache at head size 80: 80-byte rows
    s, reason, fam = ops.supports(2, 0, 4, 8, 8, 72, 72, 64, 16, 16, 256, 0.11)
    assert (s, fam) == (0, "vector")  # head size 72: general kernel
    s, reason, fam = ops.supports(2, 0, 4, 16, 8, 256, 256, 64, 16, 16, 256, 0.0625)
    assert (s, fam) == (0, "mfma-stream")  # head size 256, 16-bit cache: 512-byte rows
    s, reason, fam = ops.supports(2, 1, 4, 16, 8, 256, 256, 64, 16, 16, 256, 0.0625)
    assert (s, fam) == (0, "mfma-stream")  # head size 256, FP8 cache: 256-byte rows
    s, reason, fam = ops.supports(2, 0, 4, 32, 1, 256, 256, 64, 16, 16, 256, 0.0625)
    assert (s, fam) == (0, "vector")  # head size 256 takes one head tile: groups up to 16
    s, reason, fam = ops.supports(2, 1, 128, 64, 8, 128, 128, 32768, 16, 256, 4096, 0.088)
    assert (s, fam) == (0, "mfma-stream")
    s, reason, fam = ops.supports(2, 1, 32, 64, 1, 128, 128, 8192, 16, 256, 4096, 0.088)
    assert (s, fam) == (0, "mfma-stream")  # MQA group of 64: one wave per 32 heads
    s, reason, fam = ops.supports(2, 0, 8, 71, 1, 64, 64, 8192, 16, 256, 4096, 0.125)
    assert (s, fam) == (0, "mfma-stream")  # group of 71 at head size 64: three waves
    s, reason, fam = ops.supports(2, 0, 8, 129, 1, 128, 128, 8192, 16, 256, 4096, 0.088)
    assert (s, fam) == (0, "vector")  # groups above 128 heads: general kernel
    s, reason, fam = ops.supports(2, 0, 8, 64, 1, 128, 128, 8192, 8, 512, 4096, 0.088)
    assert (s, fam) == (0, "vector")  # wide groups need blocks of at least 16 tokens


def test_capability_query_family_boundaries():
    """The streaming families at the edges of each launch shape."""
    def fam(dtype, enc, hq, hkv, d, bs=16):
        s, _, f = ops.supports(dtype, enc, 8, hq, hkv, d, d, 8192, bs, 512 * 16 // bs, 4096, d ** -0.5)
        assert s == 0
        return f
    assert fam(2, 0, 32, 1, 128) == "mfma-stream"   # 32 heads: two tiles in one wave
    assert fam(2, 0, 33, 1, 128) == "mfma-stream"   # 33 heads: the wide-group kernel, 2 waves
    assert fam(1, 1, 128, 1, 128) == "mfma-stream"  # 128 heads, F16, FP8 cache: 4 waves
    assert fam(2, 1, 129, 1, 128) == "vector"       # above 128 heads
    assert fam(2, 0, 96, 1, 64) == "mfma-stream"    # 96 heads at head size 64: 3 waves
    assert fam(2, 0, 64, 1, 96) == "vector"         # wide groups only at head sizes 64 and 128
    assert fam(2, 1, 16, 1, 112) == "mfma-stream"   # FP8 at head size 112
    assert fam(2, 1, 17, 1, 112) == "vector"        # head sizes 80-112 take one head tile
    assert fam(0, 0, 8, 8, 128) == "vector"         # F32 queries: general kernel
    assert fam(2, 0, 16, 1, 80, bs=8) == "vector"   # streaming steps need blocks of 16 or more
    s, reason, fam = ops.supports(2, 0, 8, 32, 1, 128, 128, 65536, 16, 8192, 131072, 0.088)
    assert (s, fam) == (0, "mfma-stream")
    s, reason, _ = ops.supports(7, 0, 4, 8, 8, 64, 64, 64, 16, 16, 256, 0.125)
    assert s == _native.UNSUPPORTED and "F32, FP16 and BF16" in reason
    s, reason, _ = ops.supports(2, 0, 4, 6, 4, 64, 64, 64, 16, 16, 256, 0.125)
    assert s == _native.INVALID_ARGUMENT
    s, reason, _ = ops.supports(2, 0, 4, 8, 8, 64, 64, 64, 16, 16, 257, 0.125)
    assert s == _native.INVALID_ARGUMENT and "capacity" in reason


def test_launch_count_api():
    ops.reset_launch_count()
    assert ops.launch_count() == 0
    with pytest.raises(_native.LoomHipError):
        ops.launch_count(3)


def test_support_predicate_rejects_cpu_tensors():
    """python/tests/test_paged_decode_attention.py:353-367."""
    query = torch.empty((1, 2, 4))
    key_cache = torch.empty((1, 8, 1, 4))
    value_cache = torch.empty_like(key_cache)
    tables = torch.zeros((1, 1), dtype=torch.int32)
    lengths = torch.ones(1, dtype=torch.int32)
    assert not ops.supports_paged_decode_attention(
        query, key_cache, value_cache, tables, lengths, max_sequence_length=8
    )


def test_python_contract_errors_on_cpu_tensors():
    query = torch.zeros((1, 2, 4))
    cache = torch.zeros((1, 8, 1, 4))
    with pytest.raises(RuntimeError, match="GPU"):
        ops.paged_decode_attention(query, cache, cache, torch.zeros((1, 1), dtype=torch.int32),
                                   torch.ones(1, dtype=torch.int32), max_sequence_length=8)
    with pytest.raises(ValueError, match="ranks 3 and 4"):
        ops.paged_decode_attention(query[0], cache, cache, torch.zeros((1, 1), dtype=torch.int32),
                                   torch.ones(1, dtype=torch.int32), max_sequence_length=8)
    with pytest.raises(ValueError, match="inference-only"):
        ops.paged_decode_attention(query.requires_grad_(), cache, cache, torch.zeros((1, 1), dtype=torch.int32),
                                   torch.ones(1, dtype=torch.int32), max_sequence_length=8)


def call_no_alloc(dtype=_native.BF16, **kw):
    a = ext_args(**kw)
    return _native.lib().loom_hip_paged_decode_attention_extended_no_alloc(
        dtype, a["q"], a["k"], a["v"], a["ks"], a["vs"], a["tables"], a["lens"], a["out"], a["lse"],
        a["B"], a["Hq"], a["Hkv"], a["D"], a["Dv"], a["NB"], a["bs"], a["enc"], a["sstride"],
        a["kb"], a["kp"], a["kh"], a["vb"], a["vp"], a["vh"], a["maxb"], a["maxlen"], a["part"], a["scale"], None)


def test_no_alloc_rejects_states_beyond_the_static_workspace():
    # 128 x 64 heads x 256 partitions x 130 > 16 Mi elements: rejected on the host, before any device use.
    need = 128 * 64 * 256 * 130
    assert need > _native.STATIC_WORKSPACE_ELEMENTS
    status = call_no_alloc(B=128, Hq=64, Hkv=8, NB=1 << 20, maxb=8192, maxlen=131072, part=512)
    assert status == _native.UNSUPPORTED
    assert "static workspace" in _native.last_error()


@pytest.mark.parametrize("change", [dict(q=None), dict(out=None), dict(Hq=6, Hkv=4), dict(scale=0.0), dict(maxlen=257)])
def test_no_alloc_validates_like_the_extended_entry_point(change):
    assert call_no_alloc(**change) == _native.INVALID_ARGUMENT


def test_no_alloc_rejects_unknown_dtype():
    assert call_no_alloc(dtype=7) == _native.INVALID_ARGUMENT
    assert "dtype" in _native.last_error()


@no_device
def test_no_alloc_valid_call_needs_a_device():
    assert call_no_alloc(maxlen=256, part=64) == _native.UNAVAILABLE


def test_plan_query_on_the_host():
    """The plan of a split call needs no device; invalid shapes and null
    outputs are rejected; with no device a single-partition call plans one
    partition (the internal split needs a device and a stream slot)."""
    lib = _native.lib()
    run, internal = ctypes.c_uint32(7), ctypes.c_uint32(7)
    args = [_native.BF16, 4, 32, 8, 128, 128, 4096]
    assert lib.loom_hip_paged_decode_attention_plan(*args, 512, None, ctypes.byref(run), ctypes.byref(internal)) == 0
    assert (run.value, internal.value) == (512, 0)
    assert lib.loom_hip_paged_decode_attention_plan(*args, 0, None, None, ctypes.byref(internal)) == 1
    bad = [_native.BF16, 4, 30, 8, 128, 128, 4096]  # 30 query heads over 8 KV heads
    assert lib.loom_hip_paged_decode_attention_plan(*bad, 0, None, ctypes.byref(run), ctypes.byref(internal)) == 1
    if not torch.cuda.is_available():
        assert lib.loom_hip_paged_decode_attention_plan(*args, 0, None, ctypes.byref(run), ctypes.byref(internal)) == 0
        assert (run.value, internal.value) == (0, 0)
