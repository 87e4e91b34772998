"""Integer arguments of the Python operators that ctypes would wrap (host).

ctypes converts a Python int to c_int64 or c_uint32 modulo 2^64 or 2^32
without complaint, so a max_sequence_length of 2^64 + 2048 would reach the
library as 2048. The operators refuse such values before any library call:
the predicate answers False and the calls raise the contract's ABI message
(python/csrc/attention.cpp:82, "shape exceeds the ... ABI").
"""

from __future__ import annotations

import pytest
import torch

from attnarc_amd import _native, ops


def _tensors():
    q = torch.zeros(2, 4, 64, dtype=torch.float16)
    k = torch.zeros(8, 16, 2, 64, dtype=torch.float16)
    v = torch.zeros(8, 16, 2, 64, dtype=torch.float16)
    tables = torch.zeros(2, 4, dtype=torch.int32)
    lens = torch.ones(2, dtype=torch.int32)
    return q, k, v, tables, lens


@pytest.fixture
def no_library(monkeypatch):
    def refuse():
        raise AssertionError("the library was called with a value ctypes would wrap")

    monkeypatch.setattr(_native, "lib", refuse)


@pytest.mark.parametrize("value", [2 ** 64 + 2048, 2 ** 63, -(2 ** 63) - 1])
def test_predicate_refuses_wrapping_lengths(no_library, value):
    assert ops.supports_paged_decode_attention(*_tensors(), max_sequence_length=value) is False


@pytest.mark.parametrize("value", [2 ** 64 + 2048, 2 ** 63])
def test_out_call_raises_for_wrapping_lengths(value, monkeypatch):
    # _out takes the library handle first; the range check precedes every call on it
    monkeypatch.setattr(_native, "lib", lambda: object())
    q, k, v, tables, lens = _tensors()
    out = torch.empty(2, 4, 64, dtype=torch.float16)
    with pytest.raises(RuntimeError, match="shape exceeds the HIP ABI"):
        ops.paged_decode_attention_out(q, k, v, tables, lens, out, max_sequence_length=value)


@pytest.mark.parametrize("kw,what", [
    (dict(max_sequence_length=2 ** 32 + 64), "shape"),
    (dict(max_sequence_length=-1), "shape"),
    (dict(max_sequence_length=64, partition_tokens=2 ** 32 + 16), "partition size"),
])
def test_extended_call_raises_for_u32_overflow(no_library, kw, what):
    q, k, v, tables, lens = _tensors()
    with pytest.raises(RuntimeError, match=f"{what} exceeds the HIP ABI"):
        ops.paged_decode_attention_extended(q, k, v, tables, lens, **kw)


def test_u32_helper_bounds():
    assert ops._abi_u32(0) == 0 and ops._abi_u32(2 ** 32 - 1) == 2 ** 32 - 1
    with pytest.raises(RuntimeError):
        ops._abi_u32(2 ** 32)
