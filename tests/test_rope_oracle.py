"""Pins the RoPE + paged-KV write oracle (oracle/rope_kv_oracle.cpp).

Checks, each chosen so that a plausible restatement mistake fails one:
  * the reference's known-answer tests (crates/loom-kernels/src/tests/
    rope_kv_tests.rs:3-226): contract errors, NeoX/interleaved pairing with a
    partial rotary tail, padding slots, duplicate slots, out-of-range
    positions, per-head FP8 scales, invalid scales, no mutation on error;
  * an independent restatement of the rotation as complex multiplication in
    float64 (x_first + i x_second) * exp(i theta), which catches a swapped
    sign, a swapped pair index or cos/sin halves read the wrong way round;
  * invariants: position with cos = 1, sin = 0 is the identity; the 2-D norm
    of every pair is preserved; the unrotated tail is copied unchanged;
  * the FP8 cache bytes equal the (separately pinned) FP8 encoder applied to
    the stored value divided by the head's scale.
"""

from __future__ import annotations

import numpy as np
import pytest

import oracle

F32 = oracle.F32


def rot(tokens, hq, hk, d, rd, maxpos, dtype=F32, style=oracle.NEOX):
    return oracle.rotary_spec_new(tokens, hq, hk, d, rd, maxpos, dtype, style)


def f32(*v):
    return np.array(v, dtype=np.float32)


# ---------------------------------------------------------------------------
# Reference known-answer tests
# ---------------------------------------------------------------------------


def test_rotary_contract_rejects_invalid_partial_dimensions():
    # rope_kv_tests.rs:3-20
    for rd in (3, 10):
        with pytest.raises(oracle.ContractError) as e:
            rot(1, 2, 1, 8, rd, 16, oracle.F16)
        assert e.value.kind == oracle.INVALID_ROTARY_DIMENSION
        assert (e.value.a, e.value.b) == (rd, 8)


def test_rotary_supports_both_pairing_styles_and_partial_rope():
    # rope_kv_tests.rs:22-55
    cs = f32(1, 1, 0, 0, 0, 0, 1, 1)
    pos = np.array([1], dtype=np.int64)
    q0, k0 = f32(1, 2, 3, 4, 5, 6), f32(7, 8, 9, 10, 11, 12)
    q, k = oracle.rotary_embedding(q0, k0, pos, cs, rot(1, 1, 1, 6, 4, 2, style=oracle.NEOX))
    assert q.tolist() == [-3, -4, 1, 2, 5, 6]
    assert k.tolist() == [-9, -10, 7, 8, 11, 12]
    q, k = oracle.rotary_embedding(q0, k0, pos, cs, rot(1, 1, 1, 6, 4, 2, style=oracle.INTERLEAVED))
    assert q.tolist() == [-2, 1, -4, 3, 5, 6]
    assert k.tolist() == [-8, 7, -10, 9, 11, 12]


def test_fused_write_rotates_padding_but_skips_its_cache_slot():
    # rope_kv_tests.rs:56-90
    spec = oracle.rope_write_spec_new(rot(2, 1, 1, 4, 4, 2), 2, 2, 2)
    assert oracle.rope_scale_elements(spec) == 0
    q, k, kc, vc = oracle.rope_paged_kv_write(
        f32(1, 2, 3, 4, 5, 6, 7, 8), f32(9, 10, 11, 12, 13, 14, 15, 16), f32(17, 18, 19, 20),
        np.array([0, 1]), f32(1, 1, 0, 0, 0, 0, 1, 1), np.full(16, -99, np.float32),
        np.full(8, -99, np.float32), np.array([3, -1]), spec)
    assert q.tolist() == [1, 2, 3, 4, -7, -8, 5, 6]
    assert k[4:].tolist() == [-15, -16, 13, 14]
    assert (kc[:12] == -99).all() and kc[12:].tolist() == [9, 10, 11, 12]
    assert (vc[:6] == -99).all() and vc[6:].tolist() == [17, 18]


def test_fused_write_rejects_bad_metadata_before_mutation():
    # rope_kv_tests.rs:92-140
    spec = oracle.rope_write_spec_new(rot(2, 1, 1, 4, 4, 2), 4, 1, 2)
    original = np.ones(8, np.float32)
    cache = f32(1, 1, 0, 0, 1, 1, 0, 0)
    with pytest.raises(oracle.ContractError) as e:
        oracle.rope_paged_kv_write(original, original, np.full(8, 2, np.float32), np.array([0, 1]), cache,
                                   np.zeros(8, np.float32), np.zeros(8, np.float32), np.array([1, 1]), spec)
    assert e.value.kind == oracle.DUPLICATE_SLOT
    assert (e.value.a, e.value.b, e.value.c) == (0, 1, 1)
    with pytest.raises(oracle.ContractError) as e:
        oracle.rotary_embedding(original, original, np.array([0, 2]), cache, rot(2, 1, 1, 4, 4, 2))
    assert e.value.kind == oracle.POSITION_OUT_OF_BOUNDS
    assert (e.value.a, e.value.value, e.value.b) == (1, 2, 2)
    assert (original == 1).all()


def test_fused_write_quantizes_fp8_with_per_head_scales():
    # rope_kv_tests.rs:141-189
    spec = oracle.rope_write_spec_new(rot(1, 1, 2, 4, 4, 1), 2, 1, 2, oracle.FP8_E4M3, oracle.PER_HEAD)
    assert oracle.rope_scale_elements(spec) == 2
    _, _, kc, vc = oracle.rope_paged_kv_write(
        f32(1, 2, 3, 4), f32(1, 2, 3, 4, 10, 20, 30, 40), f32(2, 4, 8, 12), np.array([0]), f32(1, 1, 0, 0),
        np.full(16, 0xAA, np.uint8), np.full(8, 0xAA, np.uint8), np.array([1]), spec,
        key_scales=f32(1, 10), value_scales=f32(2, 4), dtype=F32)
    assert (kc[:8] == 0xAA).all()
    assert kc[8:].tolist() == oracle.encode_fp8(f32(1, 2, 3, 4, 1, 2, 3, 4)).tolist()
    assert (vc[:4] == 0xAA).all()
    assert vc[4:].tolist() == oracle.encode_fp8(f32(1, 2, 2, 3)).tolist()


def test_fp8_write_rejects_invalid_scales_before_mutation():
    # rope_kv_tests.rs:190-226
    spec = oracle.rope_write_spec_new(rot(1, 1, 1, 4, 4, 1), 4, 1, 1, oracle.FP8_E4M3, oracle.PER_TENSOR)
    original = f32(1, 2, 3, 4)
    with pytest.raises(oracle.ContractError) as e:
        oracle.rope_paged_kv_write(original, original, original, np.array([0]), f32(0, 0, 1, 1),
                                   np.zeros(4, np.uint8), np.zeros(4, np.uint8), np.array([0]), spec,
                                   key_scales=f32(0), value_scales=f32(1), dtype=F32)
    assert e.value.kind == oracle.INVALID_SCALE
    assert e.value.fvalue == 0.0
    assert original.tolist() == [1, 2, 3, 4]


def test_slot_out_of_bounds_is_rejected():
    # validate_slot_mapping (rope_kv.rs:700-724): bounds are checked per token.
    spec = oracle.rope_write_spec_new(rot(2, 1, 1, 4, 4, 2), 4, 1, 2)
    with pytest.raises(oracle.ContractError) as e:
        oracle.rope_paged_kv_write(np.ones(8, np.float32), np.ones(8, np.float32), np.ones(8, np.float32),
                                   np.array([0, 1]), f32(1, 1, 0, 0, 1, 1, 0, 0), np.zeros(8, np.float32),
                                   np.zeros(8, np.float32), np.array([0, 2]), spec)
    assert e.value.kind == oracle.SLOT_OUT_OF_BOUNDS


# ---------------------------------------------------------------------------
# Independent restatements and invariants
# ---------------------------------------------------------------------------


def _cos_sin(maxpos, rd, rng):
    theta = rng.uniform(-np.pi, np.pi, size=(maxpos, rd // 2))
    return np.concatenate([np.cos(theta), np.sin(theta)], axis=1).astype(np.float32), theta


@pytest.mark.parametrize("style", [oracle.NEOX, oracle.INTERLEAVED])
@pytest.mark.parametrize("rd", [16, 6])
def test_rotation_matches_complex_multiplication(style, rd):
    rng = np.random.default_rng(11 + rd + style)
    tokens, hq, hk, d, maxpos = 7, 3, 2, 16, 9
    cs, _ = _cos_sin(maxpos, rd, rng)
    q0 = rng.standard_normal((tokens, hq, d)).astype(np.float32)
    k0 = rng.standard_normal((tokens, hk, d)).astype(np.float32)
    pos = rng.integers(0, maxpos, tokens)
    q, k = oracle.rotary_embedding(q0, k0, pos, cs, rot(tokens, hq, hk, d, rd, maxpos, style=style))
    half = rd // 2
    idx = np.arange(half)
    i1, i2 = (idx, idx + half) if style == oracle.NEOX else (2 * idx, 2 * idx + 1)
    c = cs[pos, :half].astype(np.float64)[:, None, :]
    s = cs[pos, half:].astype(np.float64)[:, None, :]
    for src, got in ((q0, q), (k0, k)):
        z = (src[..., i1].astype(np.float64) + 1j * src[..., i2].astype(np.float64)) * (c + 1j * s)
        np.testing.assert_allclose(got[..., i1], z.real, atol=1e-5)
        np.testing.assert_allclose(got[..., i2], z.imag, atol=1e-5)
        np.testing.assert_array_equal(got[..., rd:], src[..., rd:])
        # pairwise 2-D norm is preserved
        n0 = np.hypot(src[..., i1].astype(np.float64), src[..., i2])
        n1 = np.hypot(got[..., i1].astype(np.float64), got[..., i2])
        np.testing.assert_allclose(n1, n0, rtol=1e-5, atol=1e-6)


@pytest.mark.parametrize("dtype", [oracle.F16, oracle.BF16])
def test_identity_position_is_exact_in_16_bit(dtype):
    rng = np.random.default_rng(5)
    d = rd = 8
    cs = np.zeros((2, rd), np.float32)
    cs[0, : rd // 2] = 1.0
    enc = oracle.encode_f16 if dtype == oracle.F16 else oracle.encode_bf16
    q0 = enc(rng.standard_normal((1, 2, d)))
    k0 = enc(rng.standard_normal((1, 1, d)))
    q, k = oracle.rotary_embedding(q0, k0, np.array([0]), enc(cs), rot(1, 2, 1, d, rd, 2, dtype=dtype))
    np.testing.assert_array_equal(q, q0)
    np.testing.assert_array_equal(k, k0)


def test_fp8_cache_bytes_are_encoded_stored_values_over_scale():
    rng = np.random.default_rng(3)
    tokens, hq, hk, d, rd, nb, bs = 6, 2, 2, 8, 4, 2, 4
    cs, _ = _cos_sin(8, rd, rng)
    q0 = rng.standard_normal((tokens, hq, d)).astype(np.float32) * 40
    k0 = rng.standard_normal((tokens, hk, d)).astype(np.float32) * 40
    v0 = rng.standard_normal((tokens, hk, d)).astype(np.float32) * 40
    pos = rng.integers(0, 8, tokens)
    slots = np.array([5, -1, 0, 7, 2, 3])
    ks, vs = f32(0.5, 3.0), f32(0.25, 7.0)
    spec = oracle.rope_write_spec_new(rot(tokens, hq, hk, d, rd, 8), d, nb, bs, oracle.FP8_E4M3, oracle.PER_HEAD)
    _, k, kc, vc = oracle.rope_paged_kv_write(q0, k0, v0, pos, cs, np.zeros(nb * bs * hk * d, np.uint8),
                                              np.zeros(nb * bs * hk * d, np.uint8), slots, spec,
                                              key_scales=ks, value_scales=vs, dtype=F32)
    kc = kc.reshape(nb * bs, hk, d)
    vc = vc.reshape(nb * bs, hk, d)
    k = k.reshape(tokens, hk, d)
    for t, slot in enumerate(slots):
        if slot < 0:
            continue
        for h in range(hk):
            np.testing.assert_array_equal(kc[slot, h], oracle.encode_fp8(k[t, h] / ks[h]))
            np.testing.assert_array_equal(vc[slot, h], oracle.encode_fp8(v0[t, h] / vs[h]))
