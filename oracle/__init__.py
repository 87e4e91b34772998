"""ctypes front end of the CPU oracle (test infrastructure only).

Only ``tests/``, ``__graft_entry__.smoke()`` and the ``cpu_baseline`` leg of
``bench.py`` may import this package. It is the checker the HIP path is
compared against and is never called by the product library.

The C++ restatements live in ``paged_decode_oracle.cpp`` (paged decode) and
``rope_kv_oracle.cpp`` (RoPE + paged K/V write); each function there cites
the Rust reference (``crates/loom-kernels/src/attention.rs``, ``rope_kv.rs``
and friends) it follows. Arrays are numpy: F32 as ``float32``, F16 as
``float16``, BF16 as raw ``uint16`` bit patterns, FP8 E4M3FN as ``uint8``.
"""

from __future__ import annotations

import ctypes
import os
import subprocess
from dataclasses import dataclass

import numpy as np

_HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(_HERE, "_build", "libloom_oracle.so")

F32, F16, BF16, FP8 = 0, 1, 2, 3
NATIVE, FP8_E4M3 = 0, 1

# ContractError kinds (contract.rs:80-164, attention variants).
ZERO_DIMENSION = 1
ELEMENT_COUNT_OVERFLOW = 2
INVALID_SCALE = 3
HEAD_COUNT_NOT_DIVISIBLE = 4
SEQUENCE_LENGTH_OUT_OF_BOUNDS = 5
MAX_SEQUENCE_LENGTH_OUT_OF_BOUNDS = 6
BLOCK_ID_OUT_OF_BOUNDS = 7
LENGTH_MISMATCH = 8
UNSUPPORTED_DTYPE = 9
INVALID_ROTARY_DIMENSION = 10
POSITION_OUT_OF_BOUNDS = 11
SLOT_OUT_OF_BOUNDS = 12
DUPLICATE_SLOT = 13

NEOX, INTERLEAVED = 0, 1
PER_TENSOR, PER_HEAD = 0, 1


class OracleSpec(ctypes.Structure):
    _fields_ = [
        ("sequences", ctypes.c_uint64),
        ("query_heads", ctypes.c_uint64),
        ("kv_heads", ctypes.c_uint64),
        ("head_size", ctypes.c_uint64),
        ("value_head_size", ctypes.c_uint64),
        ("num_blocks", ctypes.c_uint64),
        ("block_size", ctypes.c_uint64),
        ("max_blocks_per_sequence", ctypes.c_uint64),
        ("max_sequence_length", ctypes.c_uint64),
        ("scale", ctypes.c_float),
        ("dtype", ctypes.c_int32),
    ]


class OracleError(ctypes.Structure):
    _fields_ = [
        ("kind", ctypes.c_int32),
        ("a", ctypes.c_uint64),
        ("b", ctypes.c_uint64),
        ("c", ctypes.c_uint64),
        ("value", ctypes.c_int64),
        ("fvalue", ctypes.c_float),
        ("buffer", ctypes.c_char * 32),
        ("message", ctypes.c_char * 256),
    ]


class OracleRotarySpec(ctypes.Structure):
    _fields_ = [
        ("tokens", ctypes.c_uint64),
        ("query_heads", ctypes.c_uint64),
        ("key_heads", ctypes.c_uint64),
        ("head_size", ctypes.c_uint64),
        ("rotary_dim", ctypes.c_uint64),
        ("max_position", ctypes.c_uint64),
        ("dtype", ctypes.c_int32),
        ("style", ctypes.c_int32),
    ]


class OracleRopeWriteSpec(ctypes.Structure):
    _fields_ = [
        ("rotary", OracleRotarySpec),
        ("value_head_size", ctypes.c_uint64),
        ("num_blocks", ctypes.c_uint64),
        ("block_size", ctypes.c_uint64),
        ("encoding", ctypes.c_int32),
        ("granularity", ctypes.c_int32),
    ]


@dataclass
class ContractError(Exception):
    kind: int
    a: int
    b: int
    c: int
    value: int
    fvalue: float
    buffer: str
    message: str

    def __str__(self) -> str:  # pragma: no cover - trivial
        return self.message


_lib = None


def build() -> str:
    """Compile the oracle with its committed Makefile (g++)."""
    subprocess.run(["make", "-s", "-C", _HERE], check=True)
    return LIB_PATH


def lib() -> ctypes.CDLL:
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            build()
        l = ctypes.CDLL(LIB_PATH)
        P = ctypes.c_void_p
        U64 = ctypes.c_uint64
        l.oracle_spec_new.argtypes = [U64] * 9 + [
            ctypes.c_float,
            ctypes.c_int32,
            ctypes.POINTER(OracleSpec),
            ctypes.POINTER(OracleError),
        ]
        l.oracle_spec_new.restype = ctypes.c_int32
        l.oracle_paged_decode_attention_reference.argtypes = [
            P, U64, P, U64, P, U64, P, U64, P, U64, P, U64,
            ctypes.POINTER(OracleSpec), ctypes.c_int32, ctypes.POINTER(OracleError),
        ]
        l.oracle_paged_decode_attention_reference.restype = ctypes.c_int32
        l.oracle_paged_decode_attention_ext.argtypes = [
            P, P, P, ctypes.c_int32, P, P, ctypes.c_uint32, P, P, P, P,
            ctypes.POINTER(OracleSpec), U64, U64, U64, U64, U64, U64,
            ctypes.POINTER(OracleError),
        ]
        l.oracle_paged_decode_attention_ext.restype = ctypes.c_int32
        l.oracle_partition_states.argtypes = [
            P, P, P, ctypes.c_int32, P, P, ctypes.c_uint32, P, P,
            ctypes.POINTER(OracleSpec), U64, U64, U64, U64, U64, U64, U64, U64,
            P, P, P, ctypes.POINTER(OracleError),
        ]
        l.oracle_partition_states.restype = ctypes.c_int32
        l.oracle_merge_states.argtypes = [P, P, P, U64, U64, U64, P, P]
        l.oracle_merge_states.restype = None
        l.oracle_fp8_e4m3fn_to_f32.argtypes = [ctypes.c_uint8]
        l.oracle_fp8_e4m3fn_to_f32.restype = ctypes.c_float
        l.oracle_fp8_e4m3fn_from_f32.argtypes = [ctypes.c_float]
        l.oracle_fp8_e4m3fn_from_f32.restype = ctypes.c_uint8
        l.oracle_f32_to_bf16.argtypes = [ctypes.c_float]
        l.oracle_f32_to_bf16.restype = ctypes.c_uint16
        l.oracle_bf16_to_f32.argtypes = [ctypes.c_uint16]
        l.oracle_bf16_to_f32.restype = ctypes.c_float
        l.oracle_f32_to_f16.argtypes = [ctypes.c_float]
        l.oracle_f32_to_f16.restype = ctypes.c_uint16
        l.oracle_f16_to_f32.argtypes = [ctypes.c_uint16]
        l.oracle_f16_to_f32.restype = ctypes.c_float
        for name in ("oracle_fp8_encode_array", "oracle_bf16_encode_array", "oracle_f16_encode_array"):
            getattr(l, name).argtypes = [P, P, U64]
            getattr(l, name).restype = None
        I32 = ctypes.c_int32
        l.oracle_rotary_spec_new.argtypes = [U64] * 6 + [I32, I32, ctypes.POINTER(OracleRotarySpec),
                                                          ctypes.POINTER(OracleError)]
        l.oracle_rotary_spec_new.restype = I32
        l.oracle_rope_write_spec_new.argtypes = [ctypes.POINTER(OracleRotarySpec), U64, U64, U64, I32, I32,
                                                 ctypes.POINTER(OracleRopeWriteSpec), ctypes.POINTER(OracleError)]
        l.oracle_rope_write_spec_new.restype = I32
        l.oracle_rope_scale_elements.argtypes = [ctypes.POINTER(OracleRopeWriteSpec)]
        l.oracle_rope_scale_elements.restype = U64
        l.oracle_rotary_embedding.argtypes = [P, U64, P, U64, P, U64, P, U64, ctypes.POINTER(OracleRotarySpec), I32,
                                              ctypes.POINTER(OracleError)]
        l.oracle_rotary_embedding.restype = I32
        l.oracle_rope_paged_kv_write.argtypes = [P, U64] * 10 + [ctypes.POINTER(OracleRopeWriteSpec), I32,
                                                                 ctypes.POINTER(OracleError)]
        l.oracle_rope_paged_kv_write.restype = I32
        _lib = l
    return _lib


def _ptr(a: np.ndarray | None):
    if a is None:
        return None
    assert a.flags["C_CONTIGUOUS"], "oracle arrays must be C-contiguous"
    return ctypes.c_void_p(a.ctypes.data)


def _raise(err: OracleError) -> None:
    raise ContractError(
        kind=err.kind,
        a=err.a,
        b=err.b,
        c=err.c,
        value=err.value,
        fvalue=err.fvalue,
        buffer=err.buffer.decode(),
        message=err.message.decode(),
    )


def spec_new(
    sequences, query_heads, kv_heads, head_size, value_head_size, num_blocks,
    block_size, max_blocks_per_sequence, max_sequence_length, scale, dtype,
) -> OracleSpec:
    """PagedDecodeAttentionSpec::new (attention.rs:34-98); raises ContractError."""
    spec = OracleSpec()
    err = OracleError()
    rc = lib().oracle_spec_new(
        sequences, query_heads, kv_heads, head_size, value_head_size, num_blocks,
        block_size, max_blocks_per_sequence, max_sequence_length, scale, dtype,
        ctypes.byref(spec), ctypes.byref(err),
    )
    if rc != 0:
        _raise(err)
    return spec


def reference(dtype, query, key_cache, value_cache, block_tables, sequence_lengths, output, spec):
    """paged_decode_attention_{f32,f16,bf16}_reference (attention.rs:169-357).

    ``output`` is written in place and left untouched on error.
    """
    tables = np.ascontiguousarray(block_tables, dtype=np.int64)
    lens = np.ascontiguousarray(sequence_lengths, dtype=np.int64)
    err = OracleError()
    rc = lib().oracle_paged_decode_attention_reference(
        _ptr(query), query.size, _ptr(key_cache), key_cache.size,
        _ptr(value_cache), value_cache.size, _ptr(tables), tables.size,
        _ptr(lens), lens.size, _ptr(output), output.size,
        ctypes.byref(spec), dtype, ctypes.byref(err),
    )
    if rc != 0:
        _raise(err)
    return output


@dataclass
class CacheLayout:
    """Element strides of a logical [num_blocks, block_size, kv_heads, dim] cache."""

    block: int
    page: int
    head: int

    @staticmethod
    def nhd(block_size: int, kv_heads: int, dim: int) -> "CacheLayout":
        return CacheLayout(block_size * kv_heads * dim, kv_heads * dim, dim)

    @staticmethod
    def hnd(block_size: int, kv_heads: int, dim: int) -> "CacheLayout":
        return CacheLayout(block_size * kv_heads * dim, dim, block_size * dim)


def ext(
    spec, query, key_cache, value_cache, block_tables, sequence_lengths, *,
    key_layout: CacheLayout, value_layout: CacheLayout, cache_encoding=NATIVE,
    key_scales=None, value_scales=None, scale_stride=0, want_lse=True,
):
    """Extension oracle: FP8 KV, explicit strides and LSE. Returns (out, lse)."""
    out_dtype = {F32: np.float32, F16: np.float16, BF16: np.uint16}[spec.dtype]
    out = np.zeros((spec.sequences, spec.query_heads, spec.value_head_size), dtype=out_dtype)
    lse = np.zeros((spec.sequences, spec.query_heads), dtype=np.float64) if want_lse else None
    tables = np.ascontiguousarray(block_tables, dtype=np.int64)
    lens = np.ascontiguousarray(sequence_lengths, dtype=np.int64)
    ks = None if key_scales is None else np.ascontiguousarray(key_scales, dtype=np.float32)
    vs = None if value_scales is None else np.ascontiguousarray(value_scales, dtype=np.float32)
    err = OracleError()
    rc = lib().oracle_paged_decode_attention_ext(
        _ptr(query), _ptr(key_cache), _ptr(value_cache), cache_encoding,
        _ptr(ks), _ptr(vs), scale_stride, _ptr(tables), _ptr(lens), _ptr(out), _ptr(lse),
        ctypes.byref(spec), key_layout.block, key_layout.page, key_layout.head,
        value_layout.block, value_layout.page, value_layout.head, ctypes.byref(err),
    )
    if rc != 0:
        _raise(err)
    return out, lse


def partition_states(
    spec, query, key_cache, value_cache, block_tables, sequence_lengths, *,
    key_layout: CacheLayout, value_layout: CacheLayout, partition_tokens: int,
    cache_encoding=NATIVE, key_scales=None, value_scales=None, scale_stride=0,
):
    """Per-partition (m, l, o) states in F64; shapes [B, Hq, P], [B, Hq, P], [B, Hq, P, Dv]."""
    max_parts = -(-int(spec.max_sequence_length) // partition_tokens)
    rows = spec.sequences * spec.query_heads
    m = np.zeros((rows, max_parts), dtype=np.float64)
    l = np.zeros((rows, max_parts), dtype=np.float64)
    o = np.zeros((rows, max_parts, spec.value_head_size), dtype=np.float64)
    tables = np.ascontiguousarray(block_tables, dtype=np.int64)
    lens = np.ascontiguousarray(sequence_lengths, dtype=np.int64)
    ks = None if key_scales is None else np.ascontiguousarray(key_scales, dtype=np.float32)
    vs = None if value_scales is None else np.ascontiguousarray(value_scales, dtype=np.float32)
    err = OracleError()
    rc = lib().oracle_partition_states(
        _ptr(query), _ptr(key_cache), _ptr(value_cache), cache_encoding,
        _ptr(ks), _ptr(vs), scale_stride, _ptr(tables), _ptr(lens), ctypes.byref(spec),
        key_layout.block, key_layout.page, key_layout.head,
        value_layout.block, value_layout.page, value_layout.head,
        partition_tokens, max_parts, _ptr(m), _ptr(l), _ptr(o), ctypes.byref(err),
    )
    if rc != 0:
        _raise(err)
    shape = (spec.sequences, spec.query_heads, max_parts)
    return m.reshape(shape), l.reshape(shape), o.reshape(shape + (spec.value_head_size,))


def merge_states(m, l, o):
    """Stable LSE merge (paged_decode_attention.cu:780-852) in F64. Returns (out, lse)."""
    m = np.ascontiguousarray(m, dtype=np.float64)
    l = np.ascontiguousarray(l, dtype=np.float64)
    o = np.ascontiguousarray(o, dtype=np.float64)
    lead = m.shape[:-1]
    parts = m.shape[-1]
    dv = o.shape[-1]
    rows = int(np.prod(lead))
    out = np.zeros(lead + (dv,), dtype=np.float64)
    lse = np.zeros(lead, dtype=np.float64)
    lib().oracle_merge_states(_ptr(m), _ptr(l), _ptr(o), rows, parts, dv, _ptr(out), _ptr(lse))
    return out, lse


def fp8_to_f32(bits: int) -> float:
    return lib().oracle_fp8_e4m3fn_to_f32(bits)


def fp8_from_f32(value: float) -> int:
    return lib().oracle_fp8_e4m3fn_from_f32(value)


def encode_fp8(values: np.ndarray) -> np.ndarray:
    src = np.ascontiguousarray(values, dtype=np.float32)
    dst = np.empty(src.shape, dtype=np.uint8)
    lib().oracle_fp8_encode_array(_ptr(src), _ptr(dst), src.size)
    return dst


def encode_bf16(values: np.ndarray) -> np.ndarray:
    src = np.ascontiguousarray(values, dtype=np.float32)
    dst = np.empty(src.shape, dtype=np.uint16)
    lib().oracle_bf16_encode_array(_ptr(src), _ptr(dst), src.size)
    return dst


def encode_f16(values: np.ndarray) -> np.ndarray:
    src = np.ascontiguousarray(values, dtype=np.float32)
    dst = np.empty(src.shape, dtype=np.uint16)
    lib().oracle_f16_encode_array(_ptr(src), _ptr(dst), src.size)
    return dst


def bf16_bits_to_f32(bits: np.ndarray) -> np.ndarray:
    return (np.asarray(bits, dtype=np.uint16).astype(np.uint32) << 16).view(np.float32)


# ---------------------------------------------------------------------------
# RoPE + paged K/V write (rope_kv_oracle.cpp)
# ---------------------------------------------------------------------------


def rotary_spec_new(tokens, query_heads, key_heads, head_size, rotary_dim, max_position, dtype, style=NEOX):
    """RotaryEmbeddingSpec::new (rope_kv.rs:66-113); raises ContractError."""
    spec = OracleRotarySpec()
    err = OracleError()
    rc = lib().oracle_rotary_spec_new(tokens, query_heads, key_heads, head_size, rotary_dim, max_position, dtype,
                                      style, ctypes.byref(spec), ctypes.byref(err))
    if rc != 0:
        _raise(err)
    return spec


def rope_write_spec_new(rotary, value_head_size, num_blocks, block_size, encoding=NATIVE, granularity=PER_TENSOR):
    """RopePagedKvWriteSpec::new (rope_kv.rs:176-211); raises ContractError."""
    spec = OracleRopeWriteSpec()
    err = OracleError()
    rc = lib().oracle_rope_write_spec_new(ctypes.byref(rotary), value_head_size, num_blocks, block_size, encoding,
                                          granularity, ctypes.byref(spec), ctypes.byref(err))
    if rc != 0:
        _raise(err)
    return spec


def rope_scale_elements(spec) -> int:
    """RopePagedKvWriteSpec::scale_elements (rope_kv.rs:232-234)."""
    return int(lib().oracle_rope_scale_elements(ctypes.byref(spec)))


def rotary_embedding(query, key, positions, cos_sin_cache, spec, dtype=None):
    """rotary_embedding_*_reference (rope_kv.rs:499-511): rotates copies of
    ``query`` and ``key`` and returns them; raises ContractError."""
    q = np.ascontiguousarray(query).copy()
    k = np.ascontiguousarray(key).copy()
    pos = np.ascontiguousarray(positions, dtype=np.int64)
    cs = np.ascontiguousarray(cos_sin_cache)
    err = OracleError()
    rc = lib().oracle_rotary_embedding(_ptr(q), q.size, _ptr(k), k.size, _ptr(pos), pos.size, _ptr(cs), cs.size,
                                       ctypes.byref(spec), spec.dtype if dtype is None else dtype, ctypes.byref(err))
    if rc != 0:
        _raise(err)
    return q, k


def rope_paged_kv_write(query, key, value, positions, cos_sin_cache, key_cache, value_cache, slot_mapping, spec,
                        key_scales=None, value_scales=None, dtype=None):
    """rope_paged_kv_write_*_reference and the FP8 variant (rope_kv.rs:513-631)
    on contiguous NHD caches. Works on copies and returns (query, key,
    key_cache, value_cache); raises ContractError (nothing changed)."""
    q = np.ascontiguousarray(query).copy()
    k = np.ascontiguousarray(key).copy()
    v = np.ascontiguousarray(value)
    pos = np.ascontiguousarray(positions, dtype=np.int64)
    cs = np.ascontiguousarray(cos_sin_cache)
    kc = np.ascontiguousarray(key_cache).copy()
    vc = np.ascontiguousarray(value_cache).copy()
    slots = np.ascontiguousarray(slot_mapping, dtype=np.int64)
    ks = np.ascontiguousarray(key_scales if key_scales is not None else np.zeros(0), dtype=np.float32)
    vs = np.ascontiguousarray(value_scales if value_scales is not None else np.zeros(0), dtype=np.float32)
    err = OracleError()
    rc = lib().oracle_rope_paged_kv_write(
        _ptr(q), q.size, _ptr(k), k.size, _ptr(v), v.size, _ptr(pos), pos.size, _ptr(cs), cs.size,
        _ptr(kc), kc.size, _ptr(vc), vc.size, _ptr(slots), slots.size, _ptr(ks), ks.size, _ptr(vs), vs.size,
        ctypes.byref(spec), spec.rotary.dtype if dtype is None else dtype, ctypes.byref(err))
    if rc != 0:
        _raise(err)
    return q, k, kc, vc
