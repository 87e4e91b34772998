"""C-ABI tests of loom_hip_rope_paged_kv_write_* that run without a GPU.

Host validation must reject what the reference launcher rejects
(crates/loom-cuda-sys/cuda/src/rope_paged_kv.cu:231-250) before any device
call, and valid arguments must get as far as the device check. Fake,
non-dereferenced pointers stand in for device buffers.
"""

from __future__ import annotations

import ctypes

import pytest
import torch

from attnarc_amd import _native, ops

FAKE = {name: ctypes.c_void_p(0x7E0000000000 + i * 0x100000000) for i, name in enumerate(
    ["q", "k", "v", "pos", "cs", "kc", "vc", "ks", "vs", "slots"])}


def call(suffix="bf16", **kw):
    a = dict(q=FAKE["q"], k=FAKE["k"], v=FAKE["v"], pos=FAKE["pos"], cs=FAKE["cs"], kc=FAKE["kc"], vc=FAKE["vc"],
             ks=None, vs=None, slots=FAKE["slots"], T=8, CT=8, Hq=8, Hkv=2, D=64, Dv=64, rd=64, maxpos=128,
             NB=4, bs=16, enc=0, sstride=0, qt=512, qh=64, kt=128, kh=64, vt=128, vh=64,
             kcb=2048, kcp=128, kch=64, vcb=2048, vcp=128, vch=64, neox=1)
    a.update(kw)
    fn = getattr(_native.lib(), f"loom_hip_rope_paged_kv_write_{suffix}")
    return fn(a["q"], a["k"], a["v"], a["pos"], a["cs"], a["kc"], a["vc"], a["ks"], a["vs"], a["slots"],
              a["T"], a["CT"], a["Hq"], a["Hkv"], a["D"], a["Dv"], a["rd"], a["maxpos"], a["NB"], a["bs"],
              a["enc"], a["sstride"], a["qt"], a["qh"], a["kt"], a["kh"], a["vt"], a["vh"],
              a["kcb"], a["kcp"], a["kch"], a["vcb"], a["vcp"], a["vch"], a["neox"], None)


@pytest.mark.parametrize("suffix", ["f32", "f16", "bf16"])
@pytest.mark.parametrize("change", [
    dict(q=None), dict(k=None), dict(v=None), dict(pos=None), dict(cs=None), dict(kc=None), dict(vc=None),
    dict(enc=1), dict(enc=1, ks=FAKE["ks"]), dict(enc=2),
    dict(T=0), dict(slots=None), dict(CT=9),
    dict(Hq=0), dict(Hkv=0), dict(D=0), dict(Dv=0), dict(maxpos=0), dict(NB=0), dict(bs=0),
    dict(rd=0), dict(rd=63), dict(rd=66),
    dict(qt=0), dict(qh=0), dict(kt=0), dict(kh=0), dict(vt=0), dict(vh=0),
    dict(kcb=0), dict(kcp=0), dict(kch=0), dict(vcb=0), dict(vcp=0), dict(vch=0),
    dict(neox=2), dict(sstride=2), dict(T=0x80000000, CT=0),
])
def test_rope_entry_points_reject_invalid_arguments(suffix, change):
    assert call(suffix, **change) == _native.INVALID_ARGUMENT
    assert _native.last_error() != ""


no_device = pytest.mark.skipif(torch.cuda.is_available(), reason="valid calls with fake pointers need a GPU-less host")


@no_device
@pytest.mark.parametrize("change", [
    dict(), dict(slots=None, CT=0), dict(CT=3), dict(rd=16, neox=0), dict(Dv=32),
    dict(enc=1, ks=FAKE["ks"], vs=FAKE["vs"], sstride=1), dict(kcp=64 * 2, kch=64 * 16),
])
def test_rope_valid_arguments_reach_the_device_check(change):
    assert call("f16", **change) == _native.UNAVAILABLE, (change, _native.last_error())
    assert "no HIP device" in _native.last_error()


def test_rope_launch_counter_is_addressable():
    ops.reset_launch_count(_native.ROPE_PAGED_KV_WRITE)
    assert ops.launch_count(_native.ROPE_PAGED_KV_WRITE) == 0


def test_rope_python_contract_requires_gpu_tensors():
    q = torch.zeros((2, 2, 8))
    k = torch.zeros((2, 1, 8))
    cs = torch.zeros((4, 8))
    kv = torch.zeros((1, 2, 4, 1, 8))
    s = torch.ones(1)
    args = (q, k, k.clone(), torch.zeros(2, dtype=torch.int64), cs, kv, s, s, torch.zeros(2, dtype=torch.int64))
    assert not ops.supports_rope_paged_kv_write(*args)
    with pytest.raises(RuntimeError, match="GPU"):
        ops.rope_paged_kv_write_(*args)
    with pytest.raises(ValueError, match="inference-only"):
        ops.rope_paged_kv_write_(q.requires_grad_(), *args[1:])
