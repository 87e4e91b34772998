"""GPU parity of the fused RoPE + paged-KV write against the CPU oracle.

Integer/byte bar: rotated Q and K, and every byte of both caches (including
untouched sentinel slots), must equal oracle/rope_kv_oracle.cpp bit for bit.
Cases follow python/tests/test_rope_paged_kv.py: F32/F16/BF16 sources,
NeoX and interleaved pairing, partial rotary, NHD and HND packed caches,
native and FP8 E4M3 caches with per-tensor and per-head scales, padding slots,
a short slot mapping, packed QKV views, the current external stream, graph
replay, launch telemetry and rejection before launch. A write -> decode round
trip checks that the writer and the decode kernels agree on the cache layout.
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

import oracle
from attnarc_amd import _native, ops
from gpu_util import ORACLE_DTYPE, assert_parity, to_host

pytestmark = pytest.mark.gpu

DEV = "cuda"
DTYPES = [torch.float32, torch.float16, torch.bfloat16]


def cos_sin_cache(max_position, rotary_dim, dtype):
    """The reference tests' cache (test_rope_paged_kv.py:15-29), built on the host."""
    inv = 1.0 / (10000 ** (torch.arange(0, rotary_dim, 2, dtype=torch.float32) / rotary_dim))
    freqs = torch.outer(torch.arange(max_position, dtype=torch.float32), inv)
    return torch.cat((freqs.cos(), freqs.sin()), dim=-1).to(dtype).to(DEV)


def packed_cache(num_blocks, block_size, kv_heads, head_size, dtype, layout):
    """[blocks, 2, block_size, kv_heads, head_size] view, NHD or HND strides."""
    shape = (num_blocks, 2, block_size, kv_heads, head_size)
    if layout == "NHD":
        kv = torch.empty(shape, device=DEV, dtype=dtype)
    else:
        part = block_size * kv_heads * head_size
        kv = torch.empty_strided(shape, (2 * part, part, head_size, block_size * head_size, 1), device=DEV,
                                 dtype=dtype)
    kv.fill_(0xA5 if dtype == torch.uint8 else -7.0)
    return kv


def oracle_write(q, k, v, positions, cs, kv, slots, is_neox, key_scales=None, value_scales=None):
    """Oracle result for a call on these (pre-call) device tensors.

    Returns host arrays (q, k, key cache NHD, value cache NHD). ``slots`` may
    be shorter than the token count; missing entries are padding (-1).
    """
    T, Hq, D = q.shape
    Hkv, Dv = k.shape[1], v.shape[2]
    NB, bs = kv.shape[0], kv.shape[2]
    fp8 = kv.dtype == torch.uint8
    dt = ORACLE_DTYPE[q.dtype]
    style = oracle.NEOX if is_neox else oracle.INTERLEAVED
    rot = oracle.rotary_spec_new(T, Hq, Hkv, D, cs.shape[1], cs.shape[0], dt, style)
    gran = oracle.PER_HEAD if (key_scales is not None and key_scales.numel() > 1) else oracle.PER_TENSOR
    spec = oracle.rope_write_spec_new(rot, Dv, NB, bs, oracle.FP8_E4M3 if fp8 else oracle.NATIVE, gran)
    full = np.full(T, -1, dtype=np.int64)
    full[: slots.numel()] = slots.cpu().numpy()
    kw = {}
    if fp8:
        kw = dict(key_scales=key_scales.reshape(-1).cpu().numpy(), value_scales=value_scales.reshape(-1).cpu().numpy())
    return oracle.rope_paged_kv_write(
        to_host(q), to_host(k), to_host(v), positions.cpu().numpy(), to_host(cs), to_host(kv[:, 0]).reshape(-1),
        to_host(kv[:, 1]).reshape(-1), full, spec, **kw)


def bits(a: np.ndarray) -> np.ndarray:
    return np.ascontiguousarray(a).reshape(-1).view(np.uint8)


def assert_bits(actual: torch.Tensor, expected: np.ndarray, what: str):
    got = bits(to_host(actual))
    exp = bits(expected)
    assert got.shape == exp.shape, what
    bad = np.flatnonzero(got != exp)
    assert bad.size == 0, f"{what}: {bad.size} differing bytes, first at byte {bad[0]}"


def random_slots(tokens, capacity, gen, pad_every=4):
    slots = torch.randperm(capacity, generator=gen)[:tokens].to(torch.int64)
    slots[::pad_every] = -1
    return slots


def check_case(dtype, layout, encoding, is_neox, T, Hq, Hkv, D, rd, maxpos, NB, bs, seed, cache_tokens=None,
               big_heads=False, misalign=False):
    gen = torch.Generator().manual_seed(seed)
    q = torch.randn((T, Hq, D), generator=gen).to(dtype).to(DEV)
    if misalign:
        # A query view one element off 16-byte alignment takes the general (per-element) kernel.
        buf = torch.empty(q.numel() + 1, device=DEV, dtype=dtype)
        buf[1:].copy_(q.reshape(-1))
        q = buf[1:].view(T, Hq, D)
    k = torch.randn((T, Hkv, D), generator=gen)
    if big_heads:
        k[:, 0] *= 300.0  # saturates FP8 with scale < 1
    k = k.to(dtype).to(DEV)
    v = torch.randn((T, Hkv, D), generator=gen).to(dtype).to(DEV)
    positions = torch.randint(0, maxpos, (T,), generator=gen).to(DEV)
    cs = cos_sin_cache(maxpos, rd, dtype)
    slots = random_slots(T, NB * bs, gen)
    if cache_tokens is not None:
        slots = slots[:cache_tokens]
    slots = slots.to(DEV)
    cache_dtype = torch.uint8 if encoding != "native" else dtype
    kv = packed_cache(NB, bs, Hkv, D, cache_dtype, layout)
    if encoding == "per-head":
        ks = (torch.rand(Hkv, generator=gen) * 0.5 + 0.05).to(DEV)
        vs = (torch.rand(Hkv, generator=gen) * 0.5 + 0.05).to(DEV)
    else:
        ks = torch.tensor([0.37], device=DEV)
        vs = torch.tensor([1.0], device=DEV)
    expected = oracle_write(q, k, v, positions, cs, kv, slots, is_neox,
                            ks if encoding != "native" else None, vs if encoding != "native" else None)
    ret = ops.rope_paged_kv_write_(q, k, v, positions, cs, kv, ks, vs, slots, is_neox)
    torch.cuda.synchronize()
    assert ret[0] is q and ret[1] is k and ret[2] is kv
    assert_bits(q, expected[0], "query")
    assert_bits(k, expected[1], "key")
    assert_bits(kv[:, 0], expected[2], "key cache")
    assert_bits(kv[:, 1], expected[3], "value cache")


@pytest.mark.parametrize("dtype", DTYPES)
@pytest.mark.parametrize("is_neox", [True, False])
@pytest.mark.parametrize("layout", ["NHD", "HND"])
@pytest.mark.parametrize("encoding", ["native", "per-tensor", "per-head"])
def test_small_cases_match_oracle(dtype, is_neox, layout, encoding):
    # Shape of test_rope_paged_kv.py:67-99: partial rotary (8 of 16 dims).
    check_case(dtype, layout, encoding, is_neox, T=5, Hq=4, Hkv=2, D=16, rd=8, maxpos=32, NB=3, bs=8, seed=73,
               big_heads=True)


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
@pytest.mark.parametrize("layout", ["NHD", "HND"])
@pytest.mark.parametrize("encoding", ["native", "per-head"])
def test_llama_shape_matches_oracle(dtype, layout, encoding):
    # Llama-3-8B decode step: 32 query heads, 8 KV heads, full 128-dim rotary.
    check_case(dtype, layout, encoding, True, T=64, Hq=32, Hkv=8, D=128, rd=128, maxpos=8192, NB=64, bs=16,
               seed=11)


@pytest.mark.parametrize("is_neox", [True, False])
@pytest.mark.parametrize("encoding", ["native", "per-head"])
def test_unaligned_views_match_oracle(is_neox, encoding):
    check_case(torch.bfloat16, "NHD", encoding, is_neox, T=32, Hq=32, Hkv=8, D=128, rd=128, maxpos=4096, NB=16,
               bs=16, seed=12, misalign=True)


@pytest.mark.parametrize("dtype", DTYPES)
@pytest.mark.parametrize("is_neox", [True, False])
@pytest.mark.parametrize("encoding", ["native", "per-tensor"])
def test_vector_path_partial_rotary_and_tail(dtype, is_neox, encoding):
    # rotary 64 of 192 dims: vector rotary items, tail chunks and value chunks all active.
    check_case(dtype, "HND", encoding, is_neox, T=40, Hq=6, Hkv=2, D=192, rd=64, maxpos=300, NB=24, bs=8, seed=9,
               cache_tokens=33, big_heads=True)


@pytest.mark.parametrize("dtype", DTYPES)
def test_wide_heads_partial_rotary_and_short_slot_mapping(dtype):
    # head_size 256 > one wave, rotary 64: tail loops and value loops run 4 lanes deep.
    check_case(dtype, "HND", "per-tensor", False, T=9, Hq=3, Hkv=3, D=256, rd=64, maxpos=100, NB=4, bs=4, seed=5,
               cache_tokens=6)


def test_value_head_size_differs_through_the_strided_entry_point():
    gen = torch.Generator().manual_seed(8)
    T, Hq, Hkv, D, Dv, rd, NB, bs = 7, 4, 2, 64, 40, 32, 3, 4
    q = torch.randn((T, Hq, D), generator=gen).to(torch.bfloat16).to(DEV)
    k = torch.randn((T, Hkv, D), generator=gen).to(torch.bfloat16).to(DEV)
    v = torch.randn((T, Hkv, Dv), generator=gen).to(torch.bfloat16).to(DEV)
    pos = torch.randint(0, 50, (T,), generator=gen).to(DEV)
    cs = cos_sin_cache(50, rd, torch.bfloat16)
    slots = random_slots(T, NB * bs, gen).to(DEV)
    kc = torch.full((NB, bs, Hkv, D), -3.0, device=DEV, dtype=torch.bfloat16)
    vc = torch.full((NB, bs, Hkv, Dv), -3.0, device=DEV, dtype=torch.bfloat16)
    rot = oracle.rotary_spec_new(T, Hq, Hkv, D, rd, 50, oracle.BF16, oracle.NEOX)
    spec = oracle.rope_write_spec_new(rot, Dv, NB, bs)
    exp = oracle.rope_paged_kv_write(to_host(q), to_host(k), to_host(v), pos.cpu().numpy(), to_host(cs),
                                     to_host(kc).reshape(-1), to_host(vc).reshape(-1), slots.cpu().numpy(), spec)
    ops.rope_paged_kv_write_strided(q, k, v, pos, cs, kc, vc, None, None, slots, num_blocks=NB, block_size=bs,
                                    key_cache_strides=(kc.stride(0), kc.stride(1), kc.stride(2)),
                                    value_cache_strides=(vc.stride(0), vc.stride(1), vc.stride(2)))
    torch.cuda.synchronize()
    for got, e, what in zip((q, k, kc, vc), exp, ("query", "key", "key cache", "value cache")):
        assert_bits(got, e, what)


def test_out_of_range_positions_leave_the_token_untouched():
    gen = torch.Generator().manual_seed(21)
    T, Hq, Hkv, D, maxpos = 6, 2, 2, 32, 16
    q = torch.randn((T, Hq, D), generator=gen).to(DEV)
    k = torch.randn((T, Hkv, D), generator=gen).to(DEV)
    v = torch.randn((T, Hkv, D), generator=gen).to(DEV)
    pos = torch.tensor([3, -1, 15, 16, 0, 7], device=DEV)
    slots = torch.tensor([0, 1, 2, 3, 4, 5], device=DEV)
    cs = cos_sin_cache(maxpos, D, torch.float32)
    kv = packed_cache(2, 4, Hkv, D, torch.float32, "NHD")
    ones = torch.ones(1, device=DEV)
    bad = [1, 3]
    # Expected: the oracle on the valid tokens; the invalid ones keep Q/K and write nothing.
    safe_pos = pos.clone()
    safe_pos[bad] = 0
    safe_slots = slots.clone()
    safe_slots[bad] = -1
    exp = oracle_write(q, k, v, safe_pos, cs, kv, safe_slots, True)
    eq, ek = exp[0].reshape(T, Hq, D), exp[1].reshape(T, Hkv, D)
    eq[bad] = q.cpu().numpy()[bad]
    ek[bad] = k.cpu().numpy()[bad]
    ops.rope_paged_kv_write_(q, k, v, pos, cs, kv, ones, ones, slots, True)
    torch.cuda.synchronize()
    assert_bits(q, eq, "query")
    assert_bits(k, ek, "key")
    assert_bits(kv[:, 0], exp[2], "key cache")
    assert_bits(kv[:, 1], exp[3], "value cache")


@pytest.mark.parametrize("cache", ["native", "fp8"])
def test_packed_qkv_and_short_slot_mapping(cache):
    # test_rope_paged_kv.py:401-488: Q/K/V are column slices of one packed row.
    gen = torch.Generator().manual_seed(97)
    T, Hq, Hkv, D = 5, 4, 2, 16
    packed = torch.randn((T, (Hq + 2 * Hkv) * D), generator=gen).to(torch.bfloat16).to(DEV)
    q, k, v = packed.split((Hq * D, Hkv * D, Hkv * D), dim=-1)
    q, k, v = q.view(T, Hq, D), k.view(T, Hkv, D), v.view(T, Hkv, D)
    assert not q.is_contiguous() and q.stride(0) == k.stride(0) == v.stride(0)
    pos = torch.arange(T, device=DEV)
    slots = torch.tensor([0, 7, 9], device=DEV)
    cs = cos_sin_cache(16, D, torch.bfloat16)
    kv = packed_cache(2, 8, Hkv, D, torch.uint8 if cache == "fp8" else torch.bfloat16, "NHD")
    scale = torch.ones((), device=DEV)
    exp = oracle_write(q, k, v, pos, cs, kv, slots, True, scale if cache == "fp8" else None,
                       scale if cache == "fp8" else None)
    ops.rope_paged_kv_write_(q, k, v, pos, cs, kv, scale, scale, slots, True)
    torch.cuda.synchronize()
    assert_bits(q, exp[0], "query")
    assert_bits(k, exp[1], "key")
    assert_bits(v, to_host(v), "value")
    assert_bits(kv[:, 0], exp[2], "key cache")
    assert_bits(kv[:, 1], exp[3], "value cache")


@pytest.mark.parametrize("scale", [1.0, 0.37, 3.0e-3, 1.7e-38])
@pytest.mark.parametrize("rotary_dim", [2, 8])  # 2: general kernel; 8: 16-byte vector kernel
def test_fp8_encoding_sweep_is_exact(scale, rotary_dim):
    """Every FP8 rounding boundary, saturation, NaN/inf, signed zero and F32
    subnormals pass through the device encoder (F32 V rows: no source rounding)."""
    codes = np.arange(0x7F, dtype=np.uint8)
    vals = np.array([oracle.fp8_to_f32(int(c)) for c in codes], dtype=np.float64)
    mids = ((vals[:-1] + vals[1:]) / 2).astype(np.float32)
    near = np.concatenate([mids, np.nextafter(mids, np.float32(0)), np.nextafter(mids, np.float32(1e9))])
    special = np.array([0.0, 448, 449, 464, 464.0001, 480, 1e30, np.inf, np.nan, 1e-45, 1e-40, 2.0 ** -10,
                        2.0 ** -9, 2.0 ** -9 * 1.5, 2.0 ** -6, 2.0 ** -6 * 0.99], dtype=np.float32)
    sweep = np.concatenate([near, special, vals.astype(np.float32)])
    sweep = np.concatenate([sweep, -sweep]).astype(np.float32) * np.float32(scale)
    D = 64
    pad = (-sweep.size) % D
    sweep = np.concatenate([sweep, np.zeros(pad, np.float32)])
    T = sweep.size // D
    v = torch.from_numpy(sweep.reshape(T, 1, D)).to(DEV)
    q = torch.zeros((T, 1, D), device=DEV)
    k = torch.zeros((T, 1, D), device=DEV)
    pos = torch.zeros(T, dtype=torch.int64, device=DEV)
    cs = cos_sin_cache(1, rotary_dim, torch.float32)
    kv = packed_cache(T, 1, 1, D, torch.uint8, "NHD")
    slots = torch.arange(T, device=DEV)
    st = torch.tensor([scale], dtype=torch.float32, device=DEV)
    exp = oracle_write(q, k, v, pos, cs, kv, slots, True, st, st)
    ops.rope_paged_kv_write_(q, k, v, pos, cs, kv, st, st, slots, True)
    torch.cuda.synchronize()
    assert_bits(kv[:, 1], exp[3], "value cache")
    # Cross-check the bytes against the encoder itself on the divided values.
    assert_bits(kv[:, 1], oracle.encode_fp8(sweep / np.float32(scale)), "encoder")


def test_uses_the_current_external_stream():
    # test_rope_paged_kv.py:490-527
    gen = torch.Generator().manual_seed(4)
    q = torch.randn((2, 2, 8), generator=gen).half().to(DEV)
    k = torch.randn((2, 1, 8), generator=gen).half().to(DEV)
    v = torch.randn((2, 1, 8), generator=gen).half().to(DEV)
    pos = torch.tensor([1, 2], device=DEV)
    slots = torch.tensor([0, 5], device=DEV)
    cs = cos_sin_cache(8, 8, torch.float16)
    kv = packed_cache(1, 8, 1, 8, torch.float16, "NHD")
    scale = torch.ones((), device=DEV)
    stream = torch.cuda.Stream()
    with torch.cuda.stream(stream):
        ops.rope_paged_kv_write_(q, k, v, pos, cs, kv, scale, scale, slots, True)
    stream.synchronize()
    assert torch.isfinite(q).all() and torch.isfinite(k).all()
    assert torch.equal(kv[0, 0, 0], k[0]) and torch.equal(kv[0, 0, 5], k[1])
    assert torch.equal(kv[0, 1, 0], v[0]) and torch.equal(kv[0, 1, 5], v[1])


def small_fp8_case(seed):
    gen = torch.Generator().manual_seed(seed)
    q = torch.randn((3, 4, 16), generator=gen).bfloat16().to(DEV)
    k = torch.randn((3, 2, 16), generator=gen).bfloat16().to(DEV)
    v = torch.randn((3, 2, 16), generator=gen).bfloat16().to(DEV)
    pos = torch.tensor([0, 5, 9], device=DEV)
    cs = cos_sin_cache(16, 16, torch.bfloat16)
    kv = packed_cache(2, 8, 2, 16, torch.uint8, "HND")
    ks = torch.tensor([0.5, 0.25], device=DEV)
    vs = torch.tensor([0.75, 2.0], device=DEV)
    slots = torch.tensor([3, 12, -1], device=DEV)
    return [q, k, v, pos, cs, kv, ks, vs, slots, True]


def test_launch_counter_and_rejection_before_launch():
    # test_rope_paged_kv.py:293-332
    args = small_fp8_case(1)
    ops.reset_launch_count(_native.ROPE_PAGED_KV_WRITE)
    ops.rope_paged_kv_write_(*args)
    torch.cuda.synchronize()
    assert ops.launch_count(_native.ROPE_PAGED_KV_WRITE) == 1
    bad_scales = torch.ones(3, device=DEV)
    with pytest.raises(RuntimeError, match="one element or one element per KV head"):
        ops.rope_paged_kv_write_(*args[:6], bad_scales, bad_scales, *args[8:])
    storage = torch.empty(128, device=DEV, dtype=torch.uint8)
    overlapping = torch.as_strided(storage, (1, 2, 8, 2, 16), (128, 1, 8, 8, 1))
    with pytest.raises(RuntimeError, match="partitions must not overlap"):
        ops.rope_paged_kv_write_(*args[:5], overlapping, *args[6:])
    assert ops.launch_count(_native.ROPE_PAGED_KV_WRITE) == 1


def test_graph_replays_match_eager():
    # test_rope_paged_kv.py:379-399, with several replays and eager work between them.
    expected = small_fp8_case(103)
    ops.rope_paged_kv_write_(*expected)
    actual = small_fp8_case(103)
    q0, k0 = actual[0].clone(), actual[1].clone()
    stream = torch.cuda.Stream()
    stream.wait_stream(torch.cuda.current_stream())
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph, stream=stream):
        ops.rope_paged_kv_write_(*actual)
    torch.cuda.synchronize()
    for _ in range(3):
        actual[0].copy_(q0)
        actual[1].copy_(k0)
        actual[5].fill_(0xA5)
        torch.cuda.synchronize()
        graph.replay()
        torch.cuda.synchronize()
        assert torch.equal(actual[0], expected[0])
        assert torch.equal(actual[1], expected[1])
        assert torch.equal(actual[5], expected[5])


@pytest.mark.parametrize("encoding", ["native", "fp8"])
def test_write_then_decode_round_trip(encoding):
    """Tokens written by the RoPE write are read back by paged decode: the
    decode output over the GPU-written HND cache matches the oracle's decode
    over the oracle-written cache (the caches themselves are bit-equal)."""
    gen = torch.Generator().manual_seed(31)
    lens = [37, 64, 5, 100]
    B, Hq, Hkv, D, bs = len(lens), 32, 8, 128, 16
    maxb = max((n + bs - 1) // bs for n in lens)
    NB = B * maxb + 3
    tables = torch.randperm(NB, generator=gen)[: B * maxb].reshape(B, maxb).to(torch.int32)
    pos = torch.cat([torch.arange(n) for n in lens])
    seq = torch.cat([torch.full((n,), b) for b, n in enumerate(lens)])
    slots = tables[seq, pos // bs].to(torch.int64) * bs + pos % bs
    T = int(pos.numel())
    dtype = torch.bfloat16
    q = torch.randn((T, Hq, D), generator=gen).to(dtype).to(DEV)
    k = torch.randn((T, Hkv, D), generator=gen).to(dtype).to(DEV)
    v = torch.randn((T, Hkv, D), generator=gen).to(dtype).to(DEV)
    cs = cos_sin_cache(128, D, dtype)
    fp8 = encoding == "fp8"
    kv = packed_cache(NB, bs, Hkv, D, torch.uint8 if fp8 else dtype, "HND")
    ks = (torch.rand(Hkv, generator=gen) * 0.02 + 0.01).to(DEV)
    vs = (torch.rand(Hkv, generator=gen) * 0.02 + 0.01).to(DEV)
    pos_d, slots_d = pos.to(DEV), slots.to(DEV)
    exp = oracle_write(q, k, v, pos_d, cs, kv, slots_d, True, ks if fp8 else None, vs if fp8 else None)
    ops.rope_paged_kv_write_(q, k, v, pos_d, cs, kv, ks, vs, slots_d, True)
    torch.cuda.synchronize()
    assert_bits(kv[:, 0], exp[2], "key cache")
    assert_bits(kv[:, 1], exp[3], "value cache")

    dq = torch.randn((B, Hq, D), generator=gen).to(dtype).to(DEV)
    lengths = torch.tensor(lens, dtype=torch.int32)
    key_cache = kv[:, 0].permute(0, 2, 1, 3)  # [blocks, heads, block_size, dim] view of the HND storage
    value_cache = kv[:, 1].permute(0, 2, 1, 3)
    out = ops.paged_decode_attention_extended(
        dq, key_cache, value_cache, tables.to(DEV), lengths.to(DEV), max_sequence_length=max(lens),
        layout="HND", key_scales=ks if fp8 else None, value_scales=vs if fp8 else None, partition_tokens=32)
    torch.cuda.synchronize()
    spec = oracle.spec_new(B, Hq, Hkv, D, D, NB, bs, maxb, max(lens), D ** -0.5, oracle.BF16)
    kw = dict(cache_encoding=oracle.FP8_E4M3, key_scales=ks.cpu().numpy(), value_scales=vs.cpu().numpy(),
              scale_stride=1) if fp8 else {}
    ref, _ = oracle.ext(spec, to_host(dq), exp[2], exp[3], tables.numpy(), lengths.numpy(),
                        key_layout=oracle.CacheLayout.nhd(bs, Hkv, D), value_layout=oracle.CacheLayout.nhd(bs, Hkv, D),
                        **kw)
    assert_parity(out, oracle.bf16_bits_to_f32(ref).astype(np.float64).reshape(B, Hq, D), dtype, "round trip")


@pytest.mark.parametrize("rotary_dim", [2, 8])
def test_fp8_random_magnitudes_and_scales_are_exact(rotary_dim):
    """One million log-uniform F32 values over the whole E4M3 range (and past
    both ends) with random per-head scales: the device's division and
    conversion must give the oracle's bytes for every one."""
    rng = np.random.default_rng(2024)
    T, H, D = 4096, 4, 64
    mag = np.exp2(rng.uniform(-16, 12, size=(T, H, D))) * rng.choice([-1.0, 1.0], size=(T, H, D))
    v = torch.from_numpy(mag.astype(np.float32)).to(DEV)
    q = torch.zeros((T, 1, D), device=DEV)
    k = torch.from_numpy((mag[::-1].copy() * 0.75).astype(np.float32)).to(DEV)
    pos = torch.zeros(T, dtype=torch.int64, device=DEV)
    cs = cos_sin_cache(1, rotary_dim, torch.float32)
    kv = packed_cache(T // 4, 4, H, D, torch.uint8, "HND")
    slots = torch.from_numpy(rng.permutation(T)).to(DEV)
    ks = torch.from_numpy(np.exp2(rng.uniform(-8, 8, H)).astype(np.float32)).to(DEV)
    vs = torch.from_numpy(np.exp2(rng.uniform(-8, 8, H)).astype(np.float32)).to(DEV)
    exp = oracle_write(q, k, v, pos, cs, kv, slots, True, ks, vs)
    ops.rope_paged_kv_write_(q, k, v, pos, cs, kv, ks, vs, slots, True)
    torch.cuda.synchronize()
    assert_bits(kv[:, 0], exp[2], "key cache")
    assert_bits(kv[:, 1], exp[3], "value cache")
