"""Pins the CPU oracle (oracle/paged_decode_oracle.cpp) before it is trusted.

Checks, each chosen so that a plausible restatement mistake fails one:
  * the reference's own known-answer tests (golden fixture),
  * FP8 E4M3FN decode of all 256 codes against torch's float8_e4m3fn cast and
    encode (RNE + finite saturation) against the reference KAT table and
    torch's cast on clamped inputs,
  * BF16/F16 rounding (the `half` crate boundary) against torch's casts,
  * an independent numpy dense softmax on random paged inputs (tests/brute.py),
  * invariants: block permutation, identical heads, K = 0 gives mean(V),
    split-into-partitions + LSE merge equals the unsplit result, NHD == HND.
"""

from __future__ import annotations

import json
import math
import os

import numpy as np
import pytest
import torch

import oracle
from brute import paged_attention

GOLDEN = os.path.join(os.path.dirname(__file__), "golden", "paged_decode_golden.json")
DT = {"f32": oracle.F32, "f16": oracle.F16, "bf16": oracle.BF16}


@pytest.fixture(scope="module")
def golden():
    with open(GOLDEN) as f:
        return json.load(f)


def encode(values, dtype):
    values = np.asarray(values, dtype=np.float32)
    if dtype == oracle.F32:
        return values.copy()
    if dtype == oracle.BF16:
        return oracle.encode_bf16(values)
    return oracle.encode_f16(values).view(np.float16)


def decode(values, dtype):
    if dtype == oracle.F32:
        return np.asarray(values, dtype=np.float64)
    if dtype == oracle.BF16:
        return oracle.bf16_bits_to_f32(values).astype(np.float64)
    return np.asarray(values, dtype=np.float16).astype(np.float64)


def spec_from(v):
    *dims, scale, dt = v
    return oracle.spec_new(*dims, scale, DT[dt])


def affine_values(n, mod, center, step):
    idx = np.arange(n, dtype=np.float32)
    if mod is not None:
        idx = idx % np.float32(mod)
    return ((idx - np.float32(center)) * np.float32(step)).astype(np.float32)


# ---------------------------------------------------------------------------
# Reference known-answer tests
# ---------------------------------------------------------------------------


def test_reference_attention_kats(golden):
    for case in golden["attention_kat"]:
        spec = spec_from(case["spec"])
        dt = spec.dtype
        q = encode(case["query"], dt)
        k = encode(case["key_cache"], dt)
        v = encode(case["value_cache"], dt)
        out = encode([-1.0] * len(case["expected"]), dt)
        oracle.reference(dt, q, k, v, np.array(case["block_tables"]), np.array(case["sequence_lengths"]), out, spec)
        np.testing.assert_allclose(decode(out, dt), case["expected"], rtol=0, atol=case["tolerance"], err_msg=case["name"])


def test_reference_attention_error_kats(golden):
    errs = golden["attention_errors"]
    for case in errs["spec_errors"]:
        with pytest.raises(oracle.ContractError) as info:
            spec_from(case["spec"])
        e = info.value
        if case["kind"] == "HeadCountNotDivisible":
            assert e.kind == oracle.HEAD_COUNT_NOT_DIVISIBLE
            assert (e.a, e.b) == (case["fields"]["query_heads"], case["fields"]["kv_heads"])
            assert str(e) == "query head count 3 must be divisible by KV head count 2"
        else:
            assert e.kind == oracle.INVALID_SCALE and e.fvalue == case["fields"]["scale"]
            assert str(e) == "attention scale must be finite and positive, got 0"
    spec = spec_from(errs["buffer_spec"])
    q = np.array(errs["query"], np.float32)
    k = np.array(errs["key_cache"], np.float32)
    v = np.array(errs["value_cache"], np.float32)
    for case in errs["cases"]:
        out = np.full(2, errs["sentinel"], np.float32)
        with pytest.raises(oracle.ContractError) as info:
            oracle.reference(oracle.F32, q, k, v, np.array(case["block_tables"]), np.array(case["sequence_lengths"]), out, spec)
        e = info.value
        f = case["fields"]
        if case["kind"] == "SequenceLengthOutOfBounds":
            assert e.kind == oracle.SEQUENCE_LENGTH_OUT_OF_BOUNDS
            assert (e.a, e.value, e.b) == (f["sequence"], f["length"], f["capacity"])
            assert str(e) == "sequence length 5 for sequence 1 is outside [1, 4]"
        else:
            assert e.kind == oracle.BLOCK_ID_OUT_OF_BOUNDS
            assert (e.a, e.b, e.value, e.c) == (f["sequence"], f["logical_block"], f["block_id"], f["num_blocks"])
            assert str(e) == "physical block ID 2 for sequence 0, logical block 1 is outside [0, 2)"
        assert (out == errs["sentinel"]).all(), "output must stay untouched on error"


def test_spec_validation_variants():
    with pytest.raises(oracle.ContractError) as info:
        oracle.spec_new(0, 1, 1, 1, 1, 1, 1, 1, 1, 1.0, oracle.F32)
    assert info.value.kind == oracle.ZERO_DIMENSION
    with pytest.raises(oracle.ContractError) as info:
        oracle.spec_new(1, 1, 1, 1, 1, 1, 16, 1, 17, 1.0, oracle.F32)
    assert info.value.kind == oracle.MAX_SEQUENCE_LENGTH_OUT_OF_BOUNDS
    assert str(info.value) == "maximum sequence length 17 exceeds block-table capacity 16"
    with pytest.raises(oracle.ContractError) as info:
        oracle.spec_new(1, 1, 1, 1, 1, 1, 1, 1, 1, float("nan"), oracle.F32)
    assert info.value.kind == oracle.INVALID_SCALE
    with pytest.raises(oracle.ContractError) as info:
        oracle.spec_new(2**40, 2**40, 1, 1, 1, 1, 1, 1, 1, 1.0, oracle.F32)
    assert info.value.kind == oracle.ELEMENT_COUNT_OVERFLOW
    spec = oracle.spec_new(1, 1, 1, 2, 2, 1, 2, 1, 2, 1.0, oracle.F32)
    out = np.zeros(2, np.float32)
    with pytest.raises(oracle.ContractError) as info:
        oracle.reference(oracle.F32, np.zeros(3, np.float32), np.zeros(4, np.float32), np.zeros(4, np.float32),
                         np.array([0]), np.array([1]), out, spec)
    assert info.value.kind == oracle.LENGTH_MISMATCH
    assert str(info.value) == "query length mismatch: expected 2, got 3"
    with pytest.raises(oracle.ContractError) as info:
        oracle.reference(oracle.BF16, np.zeros(2, np.float32), np.zeros(4, np.float32), np.zeros(4, np.float32),
                         np.array([0]), np.array([1]), out, spec)
    assert info.value.kind == oracle.UNSUPPORTED_DTYPE
    assert str(info.value) == "CPU reference does not support dtype F32"


def test_affine_cases_against_independent_dense_result(golden):
    for case in golden["affine_cases"]:
        B, Hq, Hkv, D, Dv, NB, bs, maxb, maxlen, scale = case["spec"]
        spec = oracle.spec_new(B, Hq, Hkv, D, Dv, NB, bs, maxb, maxlen, scale, oracle.F32)
        q = affine_values(B * Hq * D, *case["query_affine"])
        k = affine_values(NB * bs * Hkv * D, *case["key_affine"])
        v = affine_values(NB * bs * Hkv * Dv, *case["value_affine"])
        out = np.zeros(B * Hq * Dv, np.float32)
        oracle.reference(oracle.F32, q, k, v, np.array(case["block_tables"]), np.array(case["sequence_lengths"]), out, spec)
        np.testing.assert_allclose(out, case["expected"], rtol=0, atol=2e-6, err_msg=case["name"])
        o2, lse = oracle.ext(spec, q, k, v, np.array(case["block_tables"]), np.array(case["sequence_lengths"]),
                             key_layout=oracle.CacheLayout.nhd(bs, Hkv, D),
                             value_layout=oracle.CacheLayout.nhd(bs, Hkv, Dv))
        np.testing.assert_array_equal(o2.ravel(), out)
        np.testing.assert_allclose(lse.ravel(), case["expected_lse"], rtol=0, atol=1e-12)


# ---------------------------------------------------------------------------
# Element conversions
# ---------------------------------------------------------------------------


def test_fp8_kat(golden):
    kat = golden["fp8_kat"]
    for value, bits in kat["encode"]:
        assert oracle.fp8_from_f32(value) == bits, value
    assert oracle.fp8_from_f32(float("nan")) == kat["encode_nan"]
    for bits, value in kat["decode"]:
        assert oracle.fp8_to_f32(bits) == value


def test_fp8_decode_all_codes_match_torch_float8_e4m3fn():
    codes = np.arange(256, dtype=np.uint8)
    ours = np.array([oracle.fp8_to_f32(int(c)) for c in codes], dtype=np.float32)
    theirs = torch.from_numpy(codes).view(torch.float8_e4m3fn).to(torch.float32).numpy()
    nan = np.isnan(theirs)
    assert list(np.nonzero(nan)[0]) == [0x7F, 0xFF]
    assert np.isnan(ours[nan]).all()
    np.testing.assert_array_equal(ours[~nan].view(np.uint32), theirs[~nan].view(np.uint32))


def test_fp8_encode_matches_torch_cast_with_saturation():
    rng = np.random.default_rng(7)
    x = np.concatenate([
        rng.normal(0, 1, 20000) / rng.uniform(0.01, 0.1, 20000),
        rng.normal(0, 1e-3, 5000),
        # every midpoint between adjacent finite codes (RNE ties) and their neighbours
        np.array([(oracle.fp8_to_f32(c) + oracle.fp8_to_f32(c + 1)) / 2 for c in range(0, 0x7E)]),
        np.array([-(oracle.fp8_to_f32(c) + oracle.fp8_to_f32(c + 1)) / 2 for c in range(0, 0x7E)]),
        [448.0, 464.0, 480.0, 1e6, -1e6, 0.0, -0.0],
    ]).astype(np.float32)
    ours = oracle.encode_fp8(x)
    theirs = torch.from_numpy(np.clip(x, -448.0, 448.0)).to(torch.float8_e4m3fn).view(torch.uint8).numpy()
    np.testing.assert_array_equal(ours, theirs)


def _rounding_inputs():
    rng = np.random.default_rng(11)
    bits = rng.integers(0, 2**32, 200000, dtype=np.uint64).astype(np.uint32)
    # exact ties for BF16 (low half 0x8000) and for F16 (13 low bits 0x1000)
    ties = (bits & np.uint32(0xFFFF0000)) | np.uint32(0x8000)
    f16ties = (bits & np.uint32(0xFFFFE000)) | np.uint32(0x1000)
    x = np.concatenate([bits, ties, f16ties]).view(np.float32)
    return x[np.isfinite(x)]


def test_bf16_rounding_matches_torch():
    x = _rounding_inputs()
    ours = oracle.encode_bf16(x)
    theirs = torch.from_numpy(x).to(torch.bfloat16).view(torch.int16).numpy().view(np.uint16)
    np.testing.assert_array_equal(ours, theirs)
    back = oracle.bf16_bits_to_f32(ours)
    np.testing.assert_array_equal(back, torch.from_numpy(ours.view(np.int16)).view(torch.bfloat16).float().numpy())


def test_f16_rounding_matches_torch():
    x = _rounding_inputs()
    ours = oracle.encode_f16(x)
    with np.errstate(over="ignore"):
        theirs = x.astype(np.float16).view(np.uint16)
    np.testing.assert_array_equal(ours, theirs)


# ---------------------------------------------------------------------------
# Random paged inputs against the dense restatement
# ---------------------------------------------------------------------------

# (sequences, query_heads, kv_heads, head_size, value_head_size, block_size, lengths):
# the shape list of python/tests/test_paged_decode_attention.py:114-136 (sizes
# that stay fast on the CPU) plus long/ragged and block-size-1 cases.
SHAPES = [
    (3, 8, 1, 32, 24, 16, [1, 17, 31]),
    (4, 8, 2, 64, 64, 16, [16, 33, 64, 7]),
    (3, 12, 4, 80, 48, 32, [63, 129, 255]),
    (2, 8, 2, 128, 96, 32, [257, 511]),
    (2, 8, 2, 33, 17, 8, [17, 23]),
    (2, 14, 2, 64, 64, 16, [17, 32]),
    (4, 32, 8, 128, 128, 16, [512, 501, 489, 477]),
    (1, 8, 8, 128, 128, 16, [257]),
    (2, 4, 1, 16, 16, 1, [5, 9]),
]


def random_case(rng, shape, dtype):
    B, Hq, Hkv, D, Dv, bs, lengths = shape
    maxb = -(-max(lengths) // bs)
    NB = B * maxb + 7
    perm = rng.permutation(NB)[: B * maxb].reshape(B, maxb)
    tables = np.full((B, maxb), -1, np.int64)
    for s, length in enumerate(lengths):
        n = -(-length // bs)
        tables[s, :n] = perm[s, :n]
    q = encode(rng.normal(size=(B, Hq, D)), dtype)
    k = encode(rng.normal(size=(NB, bs, Hkv, D)), dtype)
    v = encode(rng.normal(size=(NB, bs, Hkv, Dv)), dtype)
    spec = oracle.spec_new(B, Hq, Hkv, D, Dv, NB, bs, maxb, max(lengths), D ** -0.5, dtype)
    return spec, q, k, v, tables, np.array(lengths)


@pytest.mark.parametrize("dtype", [oracle.F32, oracle.F16, oracle.BF16])
@pytest.mark.parametrize("shape", SHAPES)
def test_oracle_matches_dense_restatement(shape, dtype):
    rng = np.random.default_rng(307 + dtype)
    spec, q, k, v, tables, lens = random_case(rng, shape, dtype)
    out = encode(np.zeros((spec.sequences, spec.query_heads, spec.value_head_size)), dtype)
    oracle.reference(dtype, q, k, v, tables, lens, out, spec)
    want, want_lse = paged_attention(decode(q, dtype), decode(k, dtype), decode(v, dtype), tables, lens,
                                     np.float32(spec.scale), spec.block_size)
    got = decode(out, dtype)
    # the oracle rounds its F64 result once to the storage dtype
    # (F16 subnormals below 2^-14 have an absolute spacing of 2^-24)
    ulp = {oracle.F32: 2.0**-23, oracle.F16: 2.0**-10, oracle.BF16: 2.0**-7}[dtype]
    floor = {oracle.F32: 1e-12, oracle.F16: 2.0**-25, oracle.BF16: 1e-12}[dtype]
    np.testing.assert_allclose(got, want, rtol=ulp, atol=floor)
    out2, lse = oracle.ext(spec, q, k, v, tables, lens, key_layout=oracle.CacheLayout.nhd(spec.block_size, spec.kv_heads, spec.head_size),
                           value_layout=oracle.CacheLayout.nhd(spec.block_size, spec.kv_heads, spec.value_head_size))
    np.testing.assert_array_equal(out2, out.reshape(out2.shape))
    np.testing.assert_allclose(lse, want_lse, rtol=1e-12, atol=1e-12)


def test_invariants_permutation_identical_heads_and_uniform_scores():
    rng = np.random.default_rng(5)
    spec, q, k, v, tables, lens = random_case(rng, (3, 8, 2, 64, 48, 16, [40, 64, 17]), oracle.F32)
    out = np.zeros((3, 8, 48), np.float32)
    oracle.reference(oracle.F32, q, k, v, tables, lens, out, spec)
    # permute physical blocks and the table consistently: output unchanged
    NB = spec.num_blocks
    perm = rng.permutation(NB)
    k2 = np.empty_like(k.reshape(NB, -1))
    v2 = np.empty_like(v.reshape(NB, -1))
    k2[perm] = k.reshape(NB, -1)
    v2[perm] = v.reshape(NB, -1)
    t2 = np.where(tables >= 0, perm[np.maximum(tables, 0)], -1)
    out2 = np.zeros_like(out)
    oracle.reference(oracle.F32, q, k2.ravel(), v2.ravel(), t2, lens, out2, spec)
    np.testing.assert_array_equal(out, out2)
    # identical query heads within a group give identical rows
    q3 = q.copy().reshape(3, 8, 64)
    q3[:, 1] = q3[:, 0]
    out3 = np.zeros_like(out)
    oracle.reference(oracle.F32, q3.ravel(), k, v, tables, lens, out3, spec)
    np.testing.assert_array_equal(out3[:, 0], out3[:, 1])
    # K = 0: uniform weights, output = mean of the active V rows
    out4 = np.zeros_like(out)
    oracle.reference(oracle.F32, q, np.zeros_like(k), v, tables, lens, out4, spec)
    vv = v.reshape(NB, 16, 2, 48)
    for s in range(3):
        n = int(lens[s])
        pos = np.arange(n)
        rows = vv[tables[s, pos // 16], pos % 16]  # [n, 2, 48]
        mean = rows.astype(np.float64).mean(axis=0)
        for h in range(8):
            np.testing.assert_allclose(out4[s, h], mean[h // 4], rtol=1e-6, atol=1e-7)


@pytest.mark.parametrize("partition_tokens", [1, 7, 16, 64, 1000])
def test_partition_states_merge_to_unsplit_result(partition_tokens):
    rng = np.random.default_rng(partition_tokens)
    spec, q, k, v, tables, lens = random_case(rng, (4, 8, 2, 32, 24, 16, [1, 100, 257, 64]), oracle.F32)
    kl = oracle.CacheLayout.nhd(16, 2, 32)
    vl = oracle.CacheLayout.nhd(16, 2, 24)
    out, lse = oracle.ext(spec, q, k, v, tables, lens, key_layout=kl, value_layout=vl)
    m, l, o = oracle.partition_states(spec, q, k, v, tables, lens, key_layout=kl, value_layout=vl,
                                      partition_tokens=partition_tokens)
    # partitions beyond a sequence are empty states (-inf, 0, 0)
    for s, n in enumerate(lens):
        first_empty = -(-int(n) // partition_tokens)
        assert np.isneginf(m[s, :, first_empty:]).all()
        assert (l[s, :, first_empty:] == 0).all()
    merged, mlse = oracle.merge_states(m, l, o)
    np.testing.assert_allclose(merged, out.astype(np.float64), rtol=2e-7, atol=1e-7)
    np.testing.assert_allclose(mlse, lse, rtol=1e-13, atol=1e-12)


def test_fp8_and_hnd_against_dense_restatement():
    rng = np.random.default_rng(9)
    B, Hq, Hkv, D, bs, lens = 3, 8, 2, 64, 16, np.array([33, 5, 70])
    maxb = 5
    NB = 16
    tables = rng.permutation(NB)[: B * maxb].reshape(B, maxb).astype(np.int64)
    ks = rng.uniform(0.01, 0.1, Hkv).astype(np.float32)
    vs = rng.uniform(0.01, 0.1, Hkv).astype(np.float32)
    kx = rng.normal(size=(NB, bs, Hkv, D)) / ks[None, None, :, None]
    vx = rng.normal(size=(NB, bs, Hkv, D)) / vs[None, None, :, None]
    kb = oracle.encode_fp8(np.clip(kx, -448, 448))
    vb = oracle.encode_fp8(np.clip(vx, -448, 448))
    q = oracle.encode_bf16(rng.normal(size=(B, Hq, D)))
    spec = oracle.spec_new(B, Hq, Hkv, D, D, NB, bs, maxb, 70, D ** -0.5, oracle.BF16)
    dec = np.array([oracle.fp8_to_f32(c) for c in range(256)], np.float32)
    kf = dec[kb] * ks[None, None, :, None]
    vf = dec[vb] * vs[None, None, :, None]
    want, want_lse = paged_attention(decode(q, oracle.BF16), kf, vf, tables, lens, np.float32(spec.scale), bs)
    nhd = oracle.CacheLayout.nhd(bs, Hkv, D)
    out, lse = oracle.ext(spec, q, kb, vb, tables, lens, key_layout=nhd, value_layout=nhd,
                          cache_encoding=oracle.FP8_E4M3, key_scales=ks, value_scales=vs, scale_stride=1)
    np.testing.assert_allclose(decode(out, oracle.BF16), want, rtol=2.0**-7, atol=1e-12)
    np.testing.assert_allclose(lse, want_lse, rtol=1e-6, atol=1e-6)
    # the same logical cache stored HND ([NB, Hkv, bs, D]) gives identical bytes out
    hnd = oracle.CacheLayout.hnd(bs, Hkv, D)
    kh = np.ascontiguousarray(kb.transpose(0, 2, 1, 3))
    vh = np.ascontiguousarray(vb.transpose(0, 2, 1, 3))
    out_h, lse_h = oracle.ext(spec, q, kh, vh, tables, lens, key_layout=hnd, value_layout=hnd,
                              cache_encoding=oracle.FP8_E4M3, key_scales=ks, value_scales=vs, scale_stride=1)
    np.testing.assert_array_equal(out_h, out)
    np.testing.assert_array_equal(lse_h, lse)
    # per-tensor scale (scale_stride 0) reads element 0 for every head
    out_t, _ = oracle.ext(spec, q, kb, vb, tables, lens, key_layout=nhd, value_layout=nhd,
                          cache_encoding=oracle.FP8_E4M3, key_scales=ks[:1], value_scales=vs[:1], scale_stride=0)
    kf0 = dec[kb] * ks[0]
    vf0 = dec[vb] * vs[0]
    want0, _ = paged_attention(decode(q, oracle.BF16), kf0, vf0, tables, lens, np.float32(spec.scale), bs)
    np.testing.assert_allclose(decode(out_t, oracle.BF16), want0, rtol=2.0**-7, atol=1e-12)
    # invalid scales are rejected before any write
    bad = ks.copy()
    bad[1] = 0.0
    with pytest.raises(oracle.ContractError) as info:
        oracle.ext(spec, q, kb, vb, tables, lens, key_layout=nhd, value_layout=nhd,
                   cache_encoding=oracle.FP8_E4M3, key_scales=bad, value_scales=vs, scale_stride=1)
    assert info.value.kind == oracle.INVALID_SCALE


def test_single_token_returns_value_row_exactly():
    """attention_tests.rs:32-56 generalised: one token -> out == V (any dtype)."""
    rng = np.random.default_rng(3)
    for dtype in (oracle.F32, oracle.F16, oracle.BF16):
        spec, q, k, v, tables, _ = random_case(rng, (2, 4, 2, 16, 12, 4, [1, 1]), dtype)
        out = encode(np.zeros((2, 4, 12)), dtype)
        oracle.reference(dtype, q, k, v, tables, np.array([1, 1]), out, spec)
        vv = decode(v, dtype).reshape(-1, 4, 2, 12)
        got = decode(out, dtype).reshape(2, 4, 12)
        for s in range(2):
            for h in range(4):
                np.testing.assert_array_equal(got[s, h], vv[tables[s, 0], 0, h // 2])
