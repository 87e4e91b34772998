"""Host-side tests of the checked bridge (include/loom_hip_bridge.h).

Every check runs before the device is touched, so fake, never-dereferenced
addresses stand in for device buffers, as the reference's bridge tests do
(crates/loom-cuda-bridge/src/cuda/tests.rs:3-12). Cases follow the checks of
attention_bridge.rs:71-200 and rope_kv_bridge.rs:17-372 and their messages.
"""

from __future__ import annotations

import ctypes

import pytest
import torch

from attnarc_amd import _native

BASE = 0x7D0000000000
GiB = 1 << 30


def addr(i, off=0):
    return ctypes.c_void_p(BASE + i * 4 * GiB + off)


def last():
    return _native.lib().loom_hip_bridge_last_error_message().decode()


# ---------------------------------------------------------------------------
# Telemetry and identity
# ---------------------------------------------------------------------------


def test_abi_version_and_telemetry():
    lib = _native.lib()
    assert lib.loom_hip_bridge_abi_version() == 2
    c = ctypes.c_uint64(7)
    for op in range(11):
        assert lib.loom_hip_bridge_reset_launch_count(op) == 0
        assert lib.loom_hip_bridge_launch_count(op, ctypes.byref(c)) == 0 and c.value == 0
    assert lib.loom_hip_bridge_launch_count(11, ctypes.byref(c)) == _native.BRIDGE_INVALID_ARGUMENT
    assert "unknown bridge operator code 11" in last()
    assert lib.loom_hip_bridge_launch_count(9, None) == _native.BRIDGE_INVALID_ARGUMENT
    assert "null or misaligned" in last()
    assert lib.loom_hip_bridge_reset_launch_count(12) == _native.BRIDGE_INVALID_ARGUMENT


# ---------------------------------------------------------------------------
# Paged decode
# ---------------------------------------------------------------------------


def dec_args(**kw):
    a = dict(dtype=2, B=4, Hq=8, Hkv=2, D=64, Dv=64, NB=64, bs=16, kbs=2048, vbs=2048, maxb=16, maxlen=256,
             scale=0.125, ws=None, wsn=None)
    a.update(kw)
    el = {"F32": 4}.get(a["dtype"], 2)
    a.setdefault("qn", a["B"] * a["Hq"] * a["D"])
    a.setdefault("kn", (a["NB"] - 1) * a["kbs"] + a["bs"] * a["Hkv"] * a["D"])
    a.setdefault("vn", (a["NB"] - 1) * a["vbs"] + a["bs"] * a["Hkv"] * a["Dv"])
    a.setdefault("tn", a["B"] * a["maxb"])
    a.setdefault("ln", a["B"])
    a.setdefault("on", a["B"] * a["Hq"] * a["Dv"])
    for i, n in enumerate(["q", "k", "v", "t", "l", "o"]):
        a.setdefault(n, addr(i))
    return a


def workspace_for(a):
    n = ctypes.c_uint64()
    st = _native.lib().loom_hip_bridge_paged_decode_workspace_elements(
        a["dtype"], a["B"], a["Hq"], a["Hkv"], a["D"], a["Dv"], a["NB"], a["bs"], a["maxb"], a["maxlen"], a["scale"],
        ctypes.byref(n))
    return st, n.value


def call_dec(**kw):
    a = dec_args(**kw)
    if a["wsn"] is None:
        st, n = workspace_for(a)
        a["wsn"] = n if st == 0 else 0
        if a["ws"] is None and a["wsn"]:
            a["ws"] = addr(7)
    return _native.lib().loom_hip_bridge_paged_decode_attention(
        a["dtype"], a["q"], a["qn"], a["k"], a["kn"], a["v"], a["vn"], a["t"], a["tn"], a["l"], a["ln"], a["o"],
        a["on"], a["ws"], a["wsn"], a["B"], a["Hq"], a["Hkv"], a["D"], a["Dv"], a["NB"], a["bs"], a["kbs"], a["vbs"],
        a["maxb"], a["maxlen"], a["scale"], None)


@pytest.mark.parametrize("change,message", [
    (dict(dtype=3), "unknown bridge dtype code 3"),
    (dict(B=0), "tensor dimensions must be non-zero"),
    (dict(Hq=6, Hkv=4), "query head count 6 must be divisible by KV head count 4"),
    (dict(scale=0.0), "attention scale must be finite and positive, got 0"),
    (dict(scale=-1.5), "attention scale must be finite and positive, got -1.5"),
    (dict(scale=float("nan")), "attention scale must be finite and positive, got NaN"),
    (dict(scale=float("inf")), "attention scale must be finite and positive, got inf"),
    (dict(scale=-1e-7), "attention scale must be finite and positive, got -0.0000001"),
    (dict(scale=-3e20), "attention scale must be finite and positive, got -300000000000000000000"),
    (dict(maxlen=257), "maximum sequence length 257 exceeds block-table capacity 256"),
    (dict(kbs=2047), "paged key block stride is smaller than one dense NHD block"),
    (dict(vbs=1), "paged value block stride is smaller than one dense NHD block"),
    (dict(q=None), "paged decode query pointer is null"),
    (dict(qn=0), "paged decode query region is empty"),
    (dict(k=addr(1, 1)), "paged decode key cache pointer is not aligned to 2 bytes"),
    (dict(t=addr(3, 2)), "paged decode block tables pointer is not aligned to 4 bytes"),
    (dict(o=addr(0, 64)), "paged decode regions output and query must not overlap"),
    (dict(o=addr(4)), "paged decode regions output and sequence lengths must not overlap"),
    (dict(qn=4 * 8 * 64 + 1), "paged decode query has 2049 elements, expected 2048"),
    (dict(kn=10), "paged decode key cache has 10 elements, expected"),
    (dict(tn=63), "paged decode block tables has 63 elements, expected 64"),
    (dict(on=1), "paged decode output has 1 elements, expected 2048"),
])
def test_decode_rejections(change, message):
    assert call_dec(**change) == _native.BRIDGE_INVALID_ARGUMENT
    assert last().startswith("invalid operator contract: ")
    assert message in last(), last()


def test_decode_workspace_must_match_the_sizing_call():
    # Few sequences and a long context: the library splits (non-zero workspace).
    a = dict(B=1, Hq=8, Hkv=1, D=128, Dv=128, NB=4096, bs=16, kbs=2048, vbs=2048, maxb=4096, maxlen=65536)
    st, n = workspace_for(dec_args(**a))
    assert st == 0 and n > 0
    assert call_dec(**a, ws=None, wsn=n) == _native.BRIDGE_INVALID_ARGUMENT
    assert "split-K paged decode requires a workspace pointer" in last()
    assert call_dec(**a, ws=addr(7), wsn=n - 1) == _native.BRIDGE_INVALID_ARGUMENT
    assert f"workspace has {n - 1} F32 elements, expected {n}" in last()
    assert call_dec(**a, ws=addr(0, 256), wsn=n) == _native.BRIDGE_INVALID_ARGUMENT
    assert "regions workspace and query must not overlap" in last()
    # A shape that needs no workspace rejects one.
    st, n0 = workspace_for(dec_args())
    assert st == 0 and n0 == 0
    assert call_dec(ws=addr(7), wsn=0) == _native.BRIDGE_INVALID_ARGUMENT
    assert "base paged decode requires a null workspace pointer" in last()


def test_workspace_sizing_rejects_bad_output_pointer_and_contract():
    lib = _native.lib()
    assert lib.loom_hip_bridge_paged_decode_workspace_elements(2, 4, 8, 2, 64, 64, 64, 16, 16, 256, 0.1,
                                                               None) == _native.BRIDGE_INVALID_ARGUMENT
    assert "workspace-size output pointer is null or misaligned" in last()
    n = ctypes.c_uint64()
    assert lib.loom_hip_bridge_paged_decode_workspace_elements(2, 4, 6, 4, 64, 64, 64, 16, 16, 256, 0.1,
                                                               ctypes.byref(n)) == _native.BRIDGE_INVALID_ARGUMENT


no_device = pytest.mark.skipif(torch.cuda.is_available(), reason="valid calls with fake pointers need a GPU-less host")


@no_device
def test_valid_decode_reaches_the_device_and_maps_unavailable():
    lib = _native.lib()
    lib.loom_hip_bridge_reset_launch_count(9)
    assert call_dec() == _native.BRIDGE_UNAVAILABLE
    assert "no HIP device" in last()
    c = ctypes.c_uint64()
    lib.loom_hip_bridge_launch_count(9, ctypes.byref(c))
    assert c.value == 0  # failures are not counted


# ---------------------------------------------------------------------------
# RoPE + paged-KV write
# ---------------------------------------------------------------------------


def rope_args(**kw):
    a = dict(dtype=2, enc=0, T=8, CT=8, Hq=8, Hkv=2, D=64, Dv=64, rd=64, maxpos=128, NB=4, bs=16,
             qt=512, qh=64, kt=128, kh=64, vt=128, vh=64, kcb=2048, kcp=128, kch=64, vcb=2048, vcp=128, vch=64,
             neox=1, ksn=1, vsn=1)
    a.update(kw)
    a.setdefault("qn", (a["T"] - 1) * a["qt"] + (a["Hq"] - 1) * a["qh"] + a["D"])
    a.setdefault("kn", (a["T"] - 1) * a["kt"] + (a["Hkv"] - 1) * a["kh"] + a["D"])
    a.setdefault("vn", (a["T"] - 1) * a["vt"] + (a["Hkv"] - 1) * a["vh"] + a["Dv"])
    a.setdefault("pn", a["T"])
    a.setdefault("cn", a["maxpos"] * a["rd"])
    a.setdefault("kcn", (a["NB"] - 1) * a["kcb"] + (a["bs"] - 1) * a["kcp"] + (a["Hkv"] - 1) * a["kch"] + a["D"])
    a.setdefault("vcn", (a["NB"] - 1) * a["vcb"] + (a["bs"] - 1) * a["vcp"] + (a["Hkv"] - 1) * a["vch"] + a["Dv"])
    a.setdefault("sn", a["CT"])
    for i, n in enumerate(["q", "k", "v", "p", "c", "kc", "vc", "ks", "vs", "s"]):
        a.setdefault(n, addr(i))
    return a


def call_rope(**kw):
    a = rope_args(**kw)
    return _native.lib().loom_hip_bridge_rope_paged_kv_write(
        a["dtype"], a["enc"], a["q"], a["qn"], a["k"], a["kn"], a["v"], a["vn"], a["p"], a["pn"], a["c"], a["cn"],
        a["kc"], a["kcn"], a["vc"], a["vcn"], a["ks"], a["ksn"], a["vs"], a["vsn"], a["s"], a["sn"], a["T"], a["CT"],
        a["Hq"], a["Hkv"], a["D"], a["Dv"], a["rd"], a["maxpos"], a["NB"], a["bs"], a["qt"], a["qh"], a["kt"],
        a["kh"], a["vt"], a["vh"], a["kcb"], a["kcp"], a["kch"], a["vcb"], a["vcp"], a["vch"], a["neox"], None)


@pytest.mark.parametrize("change,message", [
    (dict(dtype=9), "unknown bridge dtype code 9"),
    (dict(neox=2), "RoPE style flag must be 0 or 1"),
    (dict(Hq=0), "tensor dimensions must be non-zero"),
    (dict(rd=63), "got rotary_dim=63, head_size=64"),
    (dict(rd=66), "got rotary_dim=66, head_size=64"),
    (dict(ksn=2), "scale tensors must have the same length"),
    (dict(ksn=3, vsn=3), "one value or one value per KV head"),
    (dict(enc=2), "unsupported paged K/V cache encoding"),
    (dict(NB=0), "tensor dimensions must be non-zero"),
    (dict(CT=0, sn=1), "cache token count must be in [1, tokens]"),
    (dict(CT=9), "cache token count must be in [1, tokens]"),
    (dict(qh=32), "RoPE query layout overlaps itself"),
    (dict(kcp=64), "paged key cache layout overlaps itself"),
    (dict(q=None), "RoPE query pointer is null"),
    (dict(p=addr(3, 4)), "RoPE positions pointer is not aligned to 8 bytes"),
    (dict(s=addr(9, 4)), "paged slot mapping pointer is not aligned to 8 bytes"),
    (dict(k=addr(0, 128), kt=256, kh=96), "overlap without a dense packed layout"),
    (dict(k=addr(0, 128)), "packed regions query and key must share an outer stride"),
    (dict(kc=addr(0, 0)), "regions query and key cache must not overlap"),
    (dict(vc=addr(2, 64)), "regions value cache and value must not overlap"),
    (dict(qn=1), "RoPE query has 1 elements, expected"),
    (dict(cn=5), "RoPE cos/sin cache has 5 elements, expected 8192"),
    (dict(sn=7), "paged slot mapping has 7 elements, expected 8"),
    (dict(kcn=8), "paged key cache has 8 elements, expected"),
])
def test_rope_rejections(change, message):
    assert call_rope(**change) == _native.BRIDGE_INVALID_ARGUMENT
    assert message in last(), last()


def test_packed_qkv_views_pass_the_alias_checks():
    # Q, K, V as column slices of one [T, (Hq + 2 Hkv) * D] row (rope_kv_bridge.rs:197-248).
    row = (8 + 2 * 2) * 64
    q = addr(0)
    k = addr(0, 8 * 64 * 2)
    v = addr(0, (8 + 2) * 64 * 2)
    kw = dict(q=q, k=k, v=v, qt=row, kt=row, vt=row)
    st = call_rope(**kw)
    assert st in (_native.BRIDGE_UNAVAILABLE, _native.BRIDGE_SUCCESS) or "no HIP device" in last(), last()
    # Shifting K by one element into Q's span is caught.
    kw["k"] = addr(0, 8 * 64 * 2 - 2)
    assert call_rope(**kw) == _native.BRIDGE_INVALID_ARGUMENT
    assert "logical elements in packed regions query and key overlap" in last()
    # Different outer strides cannot share bytes.
    kw2 = dict(q=q, k=addr(0, 8 * 64 * 2), v=addr(2), qt=row, kt=row + 64)
    assert call_rope(**kw2) == _native.BRIDGE_INVALID_ARGUMENT
    assert "must share an outer stride" in last()


def test_packed_kv_cache_passes_the_alias_checks():
    # vLLM [NB, 2, bs, Hkv, D]: K and V interleave per block with one block stride.
    part = 16 * 2 * 64
    kw = dict(kc=addr(5), vc=addr(5, part * 2), kcb=2 * part, vcb=2 * part)
    kw["kcn"] = (4 - 1) * 2 * part + part
    kw["vcn"] = kw["kcn"]
    st = call_rope(**kw)
    assert st != _native.BRIDGE_INVALID_ARGUMENT, last()
    kw["vc"] = addr(5, part * 2 - 2)
    assert call_rope(**kw) == _native.BRIDGE_INVALID_ARGUMENT


@no_device
@pytest.mark.parametrize("change", [dict(), dict(enc=1, ksn=2, vsn=2), dict(CT=3, sn=3), dict(neox=0, rd=16),
                                    dict(kcp=64, kch=1024)])
def test_valid_rope_reaches_the_device(change):
    assert call_rope(**change) == _native.BRIDGE_UNAVAILABLE, last()
