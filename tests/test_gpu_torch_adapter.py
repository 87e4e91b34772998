"""GPU tests of the Stable-ABI torch adapter and the checked bridge under it.

They follow python/tests/test_paged_decode_attention.py and
python/tests/test_rope_paged_kv.py, calling ``torch.ops.loom_kernels.*``
(adapter contract -> bridge checks -> HIP kernels). Decode parity uses the
tolerances of tests/gpu_util.py against the CPU oracle; the RoPE write is
bit-exact against it.
"""

from __future__ import annotations

import ctypes

import numpy as np
import pytest
import torch

import oracle
from attnarc_amd import _native, ops, torch_ops, workloads
from gpu_util import assert_parity, oracle_expected, to_host
from test_gpu_rope import assert_bits, cos_sin_cache, oracle_write, packed_cache, small_fp8_case

pytestmark = pytest.mark.gpu

DEV = "cuda"
DTYPES = [torch.float32, torch.float16, torch.bfloat16]
Op = torch_ops.Operator

# A subset of python/tests/test_paged_decode_attention.py:114-136 plus long contexts.
SHAPES = [
    (3, 8, 1, 32, 24, 16, [1, 17, 31]),
    (3, 12, 4, 80, 48, 32, [63, 129, 255]),
    (16, 32, 8, 32, 24, 16, list(range(17, 33))),
    (2, 8, 2, 33, 17, 8, [17, 23]),
    (4, 32, 8, 128, 128, 16, [512, 501, 489, 477]),
    (2, 16, 2, 128, 128, 16, [3000, 1]),
    (1, 32, 8, 128, 128, 16, [20000]),  # one long sequence: split-K with a torch-allocated workspace
]


def case_from(shape, dtype, seed):
    B, Hq, Hkv, D, Dv, bs, lengths = shape
    return workloads.make_case(name="adapter", dtype=dtype, sequences=B, query_heads=Hq, kv_heads=Hkv, head_size=D,
                               value_head_size=Dv, block_size=bs, lengths=lengths, seed=seed, device=DEV)


def run(case, output=None):
    if output is None:
        return torch_ops.paged_decode_attention(case.query, case.key_cache, case.value_cache, case.block_tables,
                                                case.sequence_lengths, max_sequence_length=case.max_sequence_length,
                                                scale=case.scale)
    return torch_ops.paged_decode_attention_out(case.query, case.key_cache, case.value_cache, case.block_tables,
                                                case.sequence_lengths, output,
                                                max_sequence_length=case.max_sequence_length, scale=case.scale)


@pytest.mark.parametrize("dtype", DTYPES)
@pytest.mark.parametrize("shape", SHAPES)
def test_adapter_decode_matches_oracle(dtype, shape):
    case = case_from(shape, dtype, seed=71)
    torch_ops.reset_launch_count(Op.PAGED_DECODE_ATTENTION)
    actual = run(case)
    torch.cuda.synchronize()
    assert torch_ops.launch_count(Op.PAGED_DECODE_ATTENTION) == 1
    expected, _ = oracle_expected(case)
    assert_parity(actual, expected, dtype, f"adapter {shape} {dtype}")
    # Same kernels as the ctypes path: identical bits.
    direct = ops.paged_decode_attention(case.query, case.key_cache, case.value_cache, case.block_tables,
                                        case.sequence_lengths, max_sequence_length=case.max_sequence_length,
                                        scale=case.scale)
    torch.cuda.synchronize()
    assert torch.equal(actual, direct)


def test_adapter_decode_interleaved_kv_and_current_stream():
    torch.manual_seed(5)
    B, Hq, Hkv, D, bs = 4, 16, 4, 128, 16
    lengths = [33, 900, 5, 257]
    maxb = -(-max(lengths) // bs)
    NB = B * maxb + 3
    kv = torch.randn((NB, 2, bs, Hkv, D), device=DEV).bfloat16()
    key_cache, value_cache = kv.unbind(1)
    q = torch.randn((B, Hq, D), device=DEV).bfloat16()
    tables = torch.randperm(NB, device=DEV)[: B * maxb].reshape(B, maxb).int().contiguous()
    lens = torch.tensor(lengths, device=DEV, dtype=torch.int32)
    out = torch.empty((B, Hq, D), device=DEV, dtype=torch.bfloat16)
    stream = torch.cuda.Stream()
    stream.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(stream):
        torch_ops.paged_decode_attention_out(q, key_cache, value_cache, tables, lens, out,
                                             max_sequence_length=max(lengths))
    stream.synchronize()
    ref = ops.paged_decode_attention(q, key_cache, value_cache, tables, lens, max_sequence_length=max(lengths))
    torch.cuda.synchronize()
    assert torch.equal(out, ref)


def test_adapter_decode_contract_errors_do_not_launch():
    case = case_from((2, 4, 1, 32, 32, 16, [5, 19]), torch.float16, seed=9)
    torch_ops.reset_launch_count(Op.PAGED_DECODE_ATTENTION)
    with pytest.raises(RuntimeError, match="table capacity"):
        torch_ops.paged_decode_attention(case.query, case.key_cache, case.value_cache, case.block_tables,
                                         case.sequence_lengths, max_sequence_length=10_000)
    with pytest.raises(RuntimeError, match="int32"):
        torch_ops.paged_decode_attention(case.query, case.key_cache, case.value_cache, case.block_tables.long(),
                                         case.sequence_lengths, max_sequence_length=19)
    with pytest.raises(RuntimeError, match="must not overlap inputs"):
        torch_ops.paged_decode_attention_out(case.query, case.key_cache, case.value_cache, case.block_tables,
                                             case.sequence_lengths, case.query, max_sequence_length=19)
    with pytest.raises(RuntimeError, match="finite and positive"):
        torch_ops.paged_decode_attention(case.query, case.key_cache, case.value_cache, case.block_tables,
                                         case.sequence_lengths, max_sequence_length=19, scale=float("nan"))
    assert torch_ops.launch_count(Op.PAGED_DECODE_ATTENTION) == 0


def test_adapter_decode_graph_replays_match_eager():
    """Split-K workspace from the torch allocator inside capture; several
    replays with eager work between them, each checked against eager."""
    case = case_from((1, 32, 8, 128, 128, 16, [20000]), torch.bfloat16, seed=13)
    eager = run(case)
    out = torch.empty_like(eager)
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        run(case, out)
    torch.cuda.current_stream().wait_stream(s)
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        run(case, out)
    for _ in range(3):
        out.fill_(float("nan"))
        torch.cuda.synchronize()
        g.replay()
        torch.cuda.synchronize()
        assert torch.equal(out, eager)


def test_opcheck_schema_and_fake_tensor():
    case = case_from((2, 8, 2, 64, 64, 16, [40, 7]), torch.bfloat16, seed=3)
    out = torch.empty((2, 8, 64), device=DEV, dtype=torch.bfloat16)
    torch.library.opcheck(
        torch.ops.loom_kernels.paged_decode_attention.default,
        (case.query, case.key_cache, case.value_cache, case.block_tables, case.sequence_lengths, out,
         case.max_sequence_length, case.scale),
        test_utils=("test_schema", "test_faketensor"),
    )
    args = small_fp8_case(1)
    torch.library.opcheck(torch.ops.loom_kernels.rope_paged_kv_write_.default, tuple(args),
                          test_utils=("test_schema", "test_faketensor"))


# ---------------------------------------------------------------------------
# RoPE + paged-KV write through the adapter
# ---------------------------------------------------------------------------


@pytest.mark.parametrize("dtype", DTYPES)
@pytest.mark.parametrize("layout", ["NHD", "HND"])
@pytest.mark.parametrize("encoding", ["native", "fp8"])
def test_adapter_rope_matches_oracle(dtype, layout, encoding):
    gen = torch.Generator().manual_seed(17)
    T, Hq, Hkv, D, rd, maxpos, NB, bs = 24, 8, 2, 64, 64, 100, 8, 8
    q = torch.randn((T, Hq, D), generator=gen).to(dtype).to(DEV)
    k = torch.randn((T, Hkv, D), generator=gen).to(dtype).to(DEV)
    v = torch.randn((T, Hkv, D), generator=gen).to(dtype).to(DEV)
    pos = torch.randint(0, maxpos, (T,), generator=gen).to(DEV)
    cs = cos_sin_cache(maxpos, rd, dtype)
    slots = torch.randperm(NB * bs, generator=gen)[:20].to(DEV)
    slots[3] = -1
    fp8 = encoding == "fp8"
    kv = packed_cache(NB, bs, Hkv, D, torch.uint8 if fp8 else dtype, layout)
    ks = torch.tensor([0.2, 0.05], device=DEV)
    vs = torch.tensor([0.1, 0.3], device=DEV)
    exp = oracle_write(q, k, v, pos, cs, kv, slots, True, ks if fp8 else None, vs if fp8 else None)
    torch_ops.reset_launch_count(Op.ROPE_PAGED_KV_WRITE)
    torch_ops.rope_paged_kv_write_(q, k, v, pos, cs, kv, ks, vs, slots, True)
    torch.cuda.synchronize()
    assert torch_ops.launch_count(Op.ROPE_PAGED_KV_WRITE) == 1
    assert_bits(q, exp[0], "query")
    assert_bits(k, exp[1], "key")
    assert_bits(kv[:, 0], exp[2], "key cache")
    assert_bits(kv[:, 1], exp[3], "value cache")


def test_adapter_rope_packed_qkv_and_rejections():
    gen = torch.Generator().manual_seed(97)
    T, Hq, Hkv, D = 5, 4, 2, 16
    packed = torch.randn((T, (Hq + 2 * Hkv) * D), generator=gen).to(torch.bfloat16).to(DEV)
    q, k, v = (x.view(T, -1, D) for x in packed.split((Hq * D, Hkv * D, Hkv * D), dim=-1))
    pos = torch.arange(T, device=DEV)
    slots = torch.tensor([0, 7, 9], device=DEV)
    cs = cos_sin_cache(16, D, torch.bfloat16)
    kv = packed_cache(2, 8, Hkv, D, torch.uint8, "NHD")
    scale = torch.ones((), device=DEV)
    exp = oracle_write(q, k, v, pos, cs, kv, slots, True, scale, scale)
    torch_ops.rope_paged_kv_write_(q, k, v, pos, cs, kv, scale, scale, slots, True)
    torch.cuda.synchronize()
    assert_bits(q, exp[0], "query")
    assert_bits(k, exp[1], "key")
    assert_bits(kv, np.concatenate([exp[2].reshape(2, 1, 8, Hkv, D), exp[3].reshape(2, 1, 8, Hkv, D)], axis=1),
                "kv cache")
    torch_ops.reset_launch_count(Op.ROPE_PAGED_KV_WRITE)
    with pytest.raises(RuntimeError, match="one element or one element per KV head"):
        bad = torch.ones(3, device=DEV)
        torch_ops.rope_paged_kv_write_(q, k, v, pos, cs, kv, bad, bad, slots, True)
    storage = torch.empty(128, device=DEV, dtype=torch.uint8)
    overlapping = torch.as_strided(storage, (1, 2, 8, 2, 16), (128, 1, 8, 8, 1))
    with pytest.raises(RuntimeError, match="partitions must not overlap"):
        torch_ops.rope_paged_kv_write_(q, k, v, pos, cs, overlapping, scale, scale, slots, True)
    # The bridge's own alias check: K shifted onto Q's last element (same packed row).
    shifted = packed.view(-1)[Hq * D - 1:].as_strided((T, Hkv, D), (packed.stride(0), D, 1))
    with pytest.raises(RuntimeError, match="bridge failed: invalid operator contract"):
        torch_ops.rope_paged_kv_write_(q, shifted, v, pos, cs, kv, scale, scale, slots, True)
    assert torch_ops.launch_count(Op.ROPE_PAGED_KV_WRITE) == 0


def test_bridge_direct_calls_match_the_unchecked_entry_points():
    """The bridge through ctypes: same bytes as the unchecked call, counted once."""
    lib = _native.lib()
    case = case_from((4, 32, 8, 128, 128, 16, [512, 501, 489, 477]), torch.bfloat16, seed=21)
    out = torch.empty((4, 32, 128), device=DEV, dtype=torch.bfloat16)
    n = ctypes.c_uint64()
    assert lib.loom_hip_bridge_paged_decode_workspace_elements(
        2, 4, 32, 8, 128, 128, case.num_blocks, 16, case.max_blocks_per_sequence, case.max_sequence_length,
        case.scale, ctypes.byref(n)) == 0
    ws = torch.empty(max(n.value, 1), device=DEV, dtype=torch.float32) if n.value else None
    lib.loom_hip_bridge_reset_launch_count(9)
    span = lambda t: 1 + sum((s - 1) * st for s, st in zip(t.shape, t.stride()))  # noqa: E731
    st = lib.loom_hip_bridge_paged_decode_attention(
        2, ctypes.c_void_p(case.query.data_ptr()), case.query.numel(), ctypes.c_void_p(case.key_cache.data_ptr()),
        span(case.key_cache), ctypes.c_void_p(case.value_cache.data_ptr()), span(case.value_cache),
        ctypes.c_void_p(case.block_tables.data_ptr()), case.block_tables.numel(),
        ctypes.c_void_p(case.sequence_lengths.data_ptr()), case.sequence_lengths.numel(),
        ctypes.c_void_p(out.data_ptr()), out.numel(), None if ws is None else ctypes.c_void_p(ws.data_ptr()),
        n.value, 4, 32, 8, 128, 128, case.num_blocks, 16, case.key_cache.stride(0), case.value_cache.stride(0),
        case.max_blocks_per_sequence, case.max_sequence_length, case.scale,
        ctypes.c_void_p(torch.cuda.current_stream().cuda_stream))
    assert st == 0, lib.loom_hip_bridge_last_error_message()
    torch.cuda.synchronize()
    c = ctypes.c_uint64()
    lib.loom_hip_bridge_launch_count(9, ctypes.byref(c))
    assert c.value == 1
    ref = ops.paged_decode_attention(case.query, case.key_cache, case.value_cache, case.block_tables,
                                     case.sequence_lengths, max_sequence_length=case.max_sequence_length,
                                     scale=case.scale)
    torch.cuda.synchronize()
    assert torch.equal(out, ref)
