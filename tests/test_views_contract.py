"""The library's tensor-view contracts (include/loom_hip_views.h), on the host.

Both framework bindings (the torch Stable-ABI adapter and attnarc_amd.ops)
hand their operands to these checks, so every rule of the reference adapters'
contracts (python/csrc/attention.cpp:5-88, python/csrc/rope_kv.cpp:37-150) is
exercised here once, with fake device addresses that are never dereferenced:
each case breaks one rule of a valid view set and expects that rule's message.
"""

from __future__ import annotations

import ctypes

import pytest

from attnarc_amd import _native

F32, F16, BF16, U8, FP8, I32, I64, OTHER = (
    _native.VIEW_F32, _native.VIEW_F16, _native.VIEW_BF16, _native.VIEW_U8, _native.VIEW_FP8_E4M3FN,
    _native.VIEW_I32, _native.VIEW_I64, _native.VIEW_OTHER)
ELEM = {F32: 4, F16: 2, BF16: 2, U8: 1, FP8: 1, I32: 4, I64: 8, OTHER: 1}


def contiguous(sizes):
    strides, acc = [], 1
    for s in reversed(sizes):
        strides.append(acc)
        acc *= s
    return list(reversed(strides))


class V:
    """A fake tensor: base address, dtype, sizes, strides, device."""

    _next = 0x7E0000000000

    def __init__(self, dtype, sizes, strides=None, device=0, addr=None):
        self.dtype, self.sizes = dtype, list(sizes)
        self.strides = list(strides) if strides is not None else contiguous(sizes)
        self.device = device
        if addr is None:
            V._next += 1 << 32
            addr = V._next
        self.addr = addr


def pack(views):
    arr = (_native.TensorView * len(views))()
    for a, v in zip(arr, views):
        a.data, a.device_index, a.dtype, a.rank = v.addr, v.device, v.dtype, len(v.sizes)
        for d in range(min(len(v.sizes), 5)):
            a.sizes[d], a.strides[d] = v.sizes[d], v.strides[d]
    return arr


def message():
    return _native.lib().loom_hip_views_last_error_message().decode()


# ---------------------------------------------------------------------------
# Paged decode: B=3, Hq=8, Hkv=2, D=64, Dv=32, 10 blocks of 16, 4 table slots.
# ---------------------------------------------------------------------------


def decode_views(dt=F16):
    return dict(
        q=V(dt, [3, 8, 64]), k=V(dt, [10, 16, 2, 64]), v=V(dt, [10, 16, 2, 32]),
        tables=V(I32, [3, 4]), lens=V(I32, [3]), out=V(dt, [3, 8, 32]))


ORDER = ["q", "k", "v", "tables", "lens", "out"]


def decode_check(views, max_len=64, scale=0.125, count=6):
    arr = pack([views[n] for n in ORDER[:count]])
    return _native.lib().loom_hip_views_paged_decode_check(arr, count, max_len, scale)


@pytest.mark.parametrize("dt", [F32, F16, BF16])
def test_decode_valid_views_pass(dt):
    assert decode_check(decode_views(dt)) == _native.VIEWS_OK
    # a padded block stride (vLLM interleaved K/V) is allowed
    v = decode_views(dt)
    v["k"].strides[0] = 2 * 16 * 2 * 64
    assert decode_check(v) == _native.VIEWS_OK


def mutate(**changes):
    def apply(views):
        for key, fn in changes.items():
            fn(views[key])
    return apply


def setattr_(field, value):
    return lambda v: setattr(v, field, value)


def set_size(d, n):
    def f(v):
        v.sizes[d] = n
        v.strides = contiguous(v.sizes)
    return f


DECODE_CASES = [
    (dict(q=setattr_("device", -1)), {}, "query must be on a GPU"),
    (dict(lens=setattr_("device", 1)), {}, "must be on one GPU device"),
    (dict(q=setattr_("dtype", I64)), {}, "supports F32, FP16, and BF16"),
    (dict(v=setattr_("dtype", BF16)), {}, "data tensors must share a dtype"),
    (dict(out=setattr_("dtype", F32)), {}, "data tensors must share a dtype"),
    (dict(tables=setattr_("dtype", I64)), {}, "metadata must use int32"),
    (dict(lens=setattr_("dtype", U8)), {}, "metadata must use int32"),
    (dict(q=lambda v: (v.sizes.append(1), v.strides.append(1))), {}, "rank-3 query/output"),
    (dict(k=set_size(1, 0)), {}, "dimensions must be positive"),
    (dict(k=set_size(3, 32)), {}, "Q/K head sizes must match"),
    (dict(v=set_size(0, 9)), {}, "K/V cache prefixes must match"),
    (dict(tables=set_size(0, 2)), {}, "metadata batch dimensions must match query"),
    (dict(lens=set_size(0, 4)), {}, "metadata batch dimensions must match query"),
    (dict(out=set_size(2, 64)), {}, "output must have shape [B, Hq, Dv]"),
    (dict(q=setattr_("strides", [8 * 64, 1, 8])), {}, "dense-inner NHD caches"),
    (dict(k=setattr_("strides", [16 * 2 * 64, 64, 2 * 64, 1])), {}, "dense-inner NHD caches"),
    (dict(k=setattr_("strides", [100, 2 * 64, 64, 1])), {}, "dense-inner NHD caches"),
    (dict(out=setattr_("strides", [8 * 32, 1, 8])), {}, "dense-inner NHD caches"),
    (dict(tables=setattr_("strides", [1, 3])), {}, "dense-inner NHD caches"),
    ({}, dict(max_len=65), "within table capacity"),
    ({}, dict(max_len=0), "within table capacity"),
    ({}, dict(scale=0.0), "finite and positive"),
    ({}, dict(scale=float("nan")), "finite and positive"),
    ({}, dict(scale=float("inf")), "finite and positive"),
]


@pytest.mark.parametrize("changes,scalars,expect", DECODE_CASES)
def test_decode_rules(changes, scalars, expect):
    views = decode_views()
    mutate(**changes)(views)
    assert decode_check(views, **scalars) == _native.VIEWS_CONTRACT
    assert expect in message()


def test_decode_divisibility_and_abi_limits():
    v = decode_views()
    v["q"] = V(F16, [3, 6, 64])
    v["out"] = V(F16, [3, 6, 32])
    v["k"] = V(F16, [10, 16, 4, 64])
    v["v"] = V(F16, [10, 16, 4, 32])
    assert decode_check(v) == _native.VIEWS_CONTRACT and "divisible by KV heads" in message()
    big = decode_views()
    big["q"].sizes[0] = big["tables"].sizes[0] = big["lens"].sizes[0] = big["out"].sizes[0] = 1 << 29
    big["out"].addr = 1 << 62  # clear of every input's span
    assert decode_check(big) == _native.VIEWS_CONTRACT and "grid exceeds the HIP ABI" in message()
    huge = decode_views()
    huge["k"].sizes[0] = huge["v"].sizes[0] = 1 << 33
    huge["out"].addr = 1 << 62
    assert decode_check(huge) == _native.VIEWS_CONTRACT and "shape exceeds the HIP ABI" in message()


@pytest.mark.parametrize("victim", ["q", "k", "v", "tables", "lens"])
def test_decode_output_must_not_overlap_an_input(victim):
    views = decode_views()
    views["out"].addr = views[victim].addr + 2
    assert decode_check(views) == _native.VIEWS_CONTRACT
    assert "output storage must not overlap inputs" in message()
    views["out"].addr = views[victim].addr + 10 * 16 * 2 * 64 * 8  # past every input's span
    assert decode_check(views) == _native.VIEWS_OK


def test_decode_predicate_mode_ignores_output_and_scale():
    views = decode_views()
    views["out"].dtype = F32
    assert decode_check(views, count=5, scale=float("nan")) == _native.VIEWS_OK
    assert decode_check(views, count=6) == _native.VIEWS_CONTRACT
    assert decode_check(views, count=4) == _native.VIEWS_CONTRACT


def test_decode_workspace_sizing_goes_through_the_bridge():
    lib = _native.lib()
    n = ctypes.c_uint64(99)
    views = decode_views(BF16)
    # 3 x 2 items, 64 tokens: the base path, no workspace
    assert lib.loom_hip_views_paged_decode_workspace_elements(pack([views[k] for k in ORDER]), 64, 0.125,
                                                              ctypes.byref(n)) == 0
    assert n.value == 0
    bad = decode_views(BF16)
    bad["tables"].dtype = I64
    assert lib.loom_hip_views_paged_decode_workspace_elements(pack([bad[k] for k in ORDER]), 64, 0.125,
                                                              ctypes.byref(n)) == _native.VIEWS_CONTRACT


# ---------------------------------------------------------------------------
# RoPE + paged-KV write: T=5, Hq=4, Hkv=2, D=32, rotary 16, 100 positions,
# 6 blocks of 8 in a packed [blocks, 2, 8, 2, 32] cache.
# ---------------------------------------------------------------------------

ROPE_ORDER = ["q", "k", "v", "pos", "cs", "kv", "ks", "vs", "slots"]


def rope_views(dt=BF16, cache=None):
    return dict(
        q=V(dt, [5, 4, 32]), k=V(dt, [5, 2, 32]), v=V(dt, [5, 2, 32]), pos=V(I64, [5]), cs=V(dt, [100, 16]),
        kv=V(dt if cache is None else cache, [6, 2, 8, 2, 32]), ks=V(F32, [2]), vs=V(F32, [2]),
        slots=V(I64, [5]))


def rope_check(views):
    return _native.lib().loom_hip_views_rope_paged_kv_check(pack([views[n] for n in ROPE_ORDER]))


@pytest.mark.parametrize("dt", [F32, F16, BF16])
@pytest.mark.parametrize("cache", [None, U8, FP8])
def test_rope_valid_views_pass(dt, cache):
    assert rope_check(rope_views(dt, cache)) == _native.VIEWS_OK
    # HND strides of the same packed cache, per-tensor scales, a short slot mapping
    v = rope_views(dt, cache)
    v["kv"].strides = [2 * 8 * 2 * 32, 8 * 2 * 32, 32, 8 * 32, 1]
    v["ks"] = V(F32, [1])
    v["vs"] = V(F32, [1])
    v["slots"] = V(I64, [3])
    assert rope_check(v) == _native.VIEWS_OK


ROPE_CASES = [
    (dict(q=setattr_("device", -1)), "query must be on a GPU"),
    (dict(slots=setattr_("device", 3)), "must be on one GPU device"),
    (dict(q=setattr_("dtype", I32)), "supports F32, FP16, and BF16 sources"),
    (dict(k=setattr_("dtype", F16)), "Q/K/V and cos/sin cache must share a dtype"),
    (dict(cs=setattr_("dtype", F32)), "Q/K/V and cos/sin cache must share a dtype"),
    (dict(kv=setattr_("dtype", F16)), "source dtype or uint8 FP8 E4M3 storage"),
    (dict(ks=setattr_("dtype", F16)), "one element or one element per KV head"),
    (dict(pos=setattr_("dtype", I32)), "positions and slot mapping must be int64"),
    (dict(slots=setattr_("dtype", I32)), "positions and slot mapping must be int64"),
    (dict(v=lambda v: (v.sizes.pop(), v.strides.pop())), "Q/K/V must have rank 3"),
    (dict(kv=lambda v: (v.sizes.pop(), v.strides.pop())), "[blocks, 2, block_size, kv_heads, head_size]"),
    (dict(q=set_size(1, 0)), "query must be non-empty"),
    (dict(k=set_size(0, 4)), "Q/K/V token counts must match"),
    (dict(v=set_size(0, 6)), "Q/K/V token counts must match"),
    (dict(k=set_size(2, 16)), "Q/K head sizes must match"),
    (dict(v=set_size(1, 1)), "K/V head counts must match"),
    (dict(v=set_size(2, 16)), "share head count and head size"),
    (dict(kv=set_size(3, 4)), "share head count and head size"),
    (dict(kv=set_size(1, 3)), "[blocks, 2, block_size, kv_heads, head_size]"),
    (dict(pos=set_size(0, 4)), "positions must cover every token"),
    (dict(slots=set_size(0, 6)), "slot_mapping must not exceed the padded token count"),
    (dict(cs=set_size(1, 15)), "even rotary_dim <= head_size"),
    (dict(cs=set_size(1, 34)), "even rotary_dim <= head_size"),
    (dict(ks=set_size(0, 3)), "one element or one element per KV head"),
    (dict(vs=set_size(0, 1)), "one element or one element per KV head"),
    (dict(ks=setattr_("strides", [2])), "one element or one element per KV head"),
    (dict(q=setattr_("strides", [128, 32, 2])), "unit dim stride"),
    (dict(pos=setattr_("strides", [2])), "metadata must be contiguous"),
    (dict(cs=setattr_("strides", [1, 100])), "metadata must be contiguous"),
    (dict(kv=setattr_("strides", [1024, 512, 64, 32, 2])), "unit element stride and positive"),
    (dict(kv=setattr_("strides", [1024, 256, 64, 32, 1])), "partitions must not overlap"),
    (dict(kv=setattr_("strides", [700, 512, 64, 32, 1])), "partitions must not overlap"),
]


@pytest.mark.parametrize("changes,expect", ROPE_CASES)
def test_rope_rules(changes, expect):
    views = rope_views()
    mutate(**changes)(views)
    assert rope_check(views) == _native.VIEWS_CONTRACT
    assert expect in message()


def test_other_dtypes_and_oversized_ranks_are_refused():
    views = decode_views()
    views["q"].dtype = OTHER
    assert decode_check(views) == _native.VIEWS_CONTRACT
    views = decode_views()
    views["q"].sizes += [1, 1, 1]
    views["q"].strides += [1, 1, 1]
    assert decode_check(views) == _native.VIEWS_CONTRACT and "rank-3" in message()
