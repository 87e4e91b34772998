"""GPU parity of the HIP path against the CPU oracle (run on an MI355X).

Every test calls the C ABI (through attnarc_amd.ops) on seeded inputs and
compares with the oracle on the same bytes: abs 2e-3 / rel 1e-2 for BF16,
FP16 and FP8-KV, abs 1e-5 for F32; LSE abs 1e-4. Test design follows
python/tests/test_paged_decode_attention.py (shape list, interleaved cache
stride, current stream, telemetry, contract errors) and adds the extended
contract (FP8 E4M3 K/V, HND, LSE, fixed partitions) and the five benchmark
configurations (full size where the oracle finishes in seconds, a seeded
subset of sequences otherwise, plus size-independent properties).
"""

from __future__ import annotations

import math

import numpy as np
import pytest
import torch

import oracle
from attnarc_amd import ops, workloads
from gpu_util import LSE_TOL, ORACLE_THREADS, assert_parity, as_f64, oracle_expected

pytestmark = pytest.mark.gpu

DEV = "cuda"
DTYPES = [torch.float32, torch.float16, torch.bfloat16]

# python/tests/test_paged_decode_attention.py:114-136
CASES = [
    (3, 8, 1, 32, 24, 16, [1, 17, 31]),
    (4, 8, 2, 64, 64, 16, [16, 33, 64, 7]),
    (3, 12, 4, 80, 48, 32, [63, 129, 255]),
    (2, 8, 2, 128, 96, 32, [257, 511]),
    (16, 32, 8, 32, 24, 16, list(range(17, 33))),
    (2, 8, 2, 33, 17, 8, [17, 23]),
    (2, 14, 2, 64, 64, 16, [17, 32]),
    (64, 14, 2, 64, 64, 16, list(range(17, 33)) * 4),
    (1, 32, 8, 128, 128, 16, [128]),
    (4, 32, 8, 128, 128, 16, [512, 501, 489, 477]),
    (8, 32, 8, 128, 128, 32, list(range(491, 499))),
    (2, 14, 2, 128, 128, 16, [129, 256]),
    (1, 8, 8, 128, 128, 16, [257]),
    # beyond the reference's 1024 cap, block size 1, and a 32-head MQA group
    (2, 16, 2, 128, 128, 16, [3000, 1]),
    (2, 4, 1, 128, 128, 1, [70, 33]),
    (2, 32, 1, 128, 128, 16, [1500, 77]),
    # general kernel: two 256-dim value tiles; a head size past the query's LDS stage
    (2, 8, 2, 64, 320, 16, [100, 300]),
    (2, 4, 2, 640, 64, 16, [70, 150]),
]


def case_from(shape, dtype, seed, **kw):
    B, Hq, Hkv, D, Dv, bs, lengths = shape
    return workloads.make_case(
        name="shape", dtype=dtype, sequences=B, query_heads=Hq, kv_heads=Hkv, head_size=D,
        value_head_size=Dv, block_size=bs, lengths=lengths, seed=seed, device=DEV, **kw,
    )


@pytest.mark.parametrize("dtype", DTYPES)
@pytest.mark.parametrize("shape", CASES)
def test_paged_decode_matches_oracle(dtype, shape):
    case = case_from(shape, dtype, seed=307)
    actual = ops.paged_decode_attention(
        case.query, case.key_cache, case.value_cache, case.block_tables, case.sequence_lengths,
        max_sequence_length=case.max_sequence_length, scale=case.scale,
    )
    torch.cuda.synchronize()
    expected, _ = oracle_expected(case)
    assert_parity(actual, expected, dtype, f"{shape} {dtype}")


@pytest.mark.parametrize("dtype", DTYPES)
def test_paged_decode_accepts_vllm_interleaved_kv_stride(dtype):
    """test_paged_decode_attention.py:180-218: K/V views of one [NB, 2, bs, Hkv, D] cache."""
    torch.manual_seed(353)
    B, Hq, Hkv, D, bs = 16, 32, 8, 128, 16
    lengths = list(range(17, 33)) * 1
    lengths[3] = 1200
    maxb = -(-max(lengths) // bs)
    NB = B * maxb + 7
    kv = torch.randn((NB, 2, bs, Hkv, D), device=DEV).to(dtype)
    key_cache, value_cache = kv.unbind(1)
    assert not key_cache.is_contiguous() and key_cache.stride(0) == 2 * key_cache[0].numel()
    query = torch.randn((B, Hq, D), device=DEV).to(dtype)
    perm = torch.randperm(NB, device=DEV)[: B * maxb].reshape(B, maxb).to(torch.int32).contiguous()
    lens = torch.tensor(lengths, device=DEV, dtype=torch.int32)
    assert ops.supports_paged_decode_attention(query, key_cache, value_cache, perm, lens,
                                               max_sequence_length=max(lengths))
    actual = ops.paged_decode_attention(query, key_cache, value_cache, perm, lens,
                                        max_sequence_length=max(lengths), scale=D ** -0.5)
    torch.cuda.synchronize()
    # oracle on the same bytes: the interleaved layout is block stride 2*bs*Hkv*D
    dt = {torch.float32: oracle.F32, torch.float16: oracle.F16, torch.bfloat16: oracle.BF16}[dtype]
    from gpu_util import to_host

    spec = oracle.spec_new(B, Hq, Hkv, D, D, NB, bs, maxb, max(lengths), D ** -0.5, dt)
    flat = to_host(kv).reshape(-1)
    k_lay = oracle.CacheLayout(2 * bs * Hkv * D, Hkv * D, D)
    v_flat = np.ascontiguousarray(flat[bs * Hkv * D:])
    out, _ = oracle.ext(spec, to_host(query), flat, v_flat, to_host(perm), to_host(lens), key_layout=k_lay,
                        value_layout=k_lay)
    expected = oracle.bf16_bits_to_f32(out).astype(np.float64) if dt == oracle.BF16 else out.astype(np.float64)
    assert_parity(actual, expected, dtype, "interleaved")


def test_paged_decode_uses_current_stream_and_caller_output():
    case = case_from((3, 8, 2, 64, 48, 16, [9, 23, 47]), torch.bfloat16, seed=401)
    output = torch.empty((3, 8, 48), device=DEV, dtype=torch.bfloat16)
    stream = torch.cuda.Stream()
    with torch.cuda.stream(stream):
        stream.wait_stream(torch.cuda.default_stream())
        returned = ops.paged_decode_attention_out(
            case.query, case.key_cache, case.value_cache, case.block_tables, case.sequence_lengths, output,
            max_sequence_length=case.max_sequence_length, scale=case.scale,
        )
    stream.synchronize()
    assert returned is output
    expected, _ = oracle_expected(case)
    assert_parity(output, expected, torch.bfloat16, "stream")


def test_paged_decode_contract_and_launch_telemetry():
    case = case_from((2, 4, 1, 32, 32, 16, [5, 19]), torch.float16, seed=607)
    ops.reset_launch_count()
    ops.paged_decode_attention(case.query, case.key_cache, case.value_cache, case.block_tables,
                               case.sequence_lengths, max_sequence_length=19)
    torch.cuda.synchronize()
    assert ops.launch_count() == 1
    with pytest.raises(RuntimeError, match="table capacity"):
        ops.paged_decode_attention(case.query, case.key_cache, case.value_cache, case.block_tables,
                                   case.sequence_lengths, max_sequence_length=10_000)
    with pytest.raises(RuntimeError, match="int32"):
        ops.paged_decode_attention(case.query, case.key_cache, case.value_cache, case.block_tables.long(),
                                   case.sequence_lengths, max_sequence_length=19)
    assert ops.launch_count() == 1


@pytest.mark.parametrize("dtype", DTYPES)
def test_split_k_entry_points_match_oracle(dtype):
    """The reference-compatible split-K ABI: the sizing function selects it for
    a long context on a small grid and the op allocates the workspace."""
    shape = (2, 8, 2, 128, 128, 16, [6000, 2500])
    case = case_from(shape, dtype, seed=11)
    from attnarc_amd import _native

    ws = _native.lib().loom_hip_paged_decode_attention_split_k_workspace_elements(2, 8, 2, 128, 128, 6000)
    assert ws > 0
    actual = ops.paged_decode_attention(case.query, case.key_cache, case.value_cache, case.block_tables,
                                        case.sequence_lengths, max_sequence_length=6000, scale=case.scale)
    torch.cuda.synchronize()
    expected, _ = oracle_expected(case)
    assert_parity(actual, expected, dtype, "split-k")


# ---------------------------------------------------------------------------
# Extended contract: FP8 E4M3 caches, HND, LSE, partitions
# ---------------------------------------------------------------------------

EXT = [
    # (dtype, encoding, layout, per_head, partition_tokens, shape)
    (torch.bfloat16, "fp8", "HND", True, 512, (4, 64, 8, 128, 128, 16, [4096, 1, 700, 2049])),
    (torch.bfloat16, "fp8", "NHD", False, 0, (3, 16, 2, 128, 128, 16, [33, 1000, 64])),
    (torch.float16, "fp8", "HND", True, 100, (3, 8, 2, 128, 128, 32, [300, 7, 1001])),
    (torch.bfloat16, "native", "HND", False, 64, (3, 12, 2, 128, 128, 16, [513, 64, 65])),
    (torch.float16, "native", "NHD", False, 31, (2, 32, 1, 128, 128, 16, [500, 40])),
    (torch.float32, "fp8", "HND", True, 48, (2, 8, 2, 64, 64, 16, [100, 200])),
    (torch.float32, "native", "NHD", False, 0, (2, 6, 3, 40, 24, 8, [50, 3])),
    (torch.bfloat16, "fp8", "NHD", True, 0, (2, 32, 4, 96, 80, 16, [77, 300])),
]


@pytest.mark.parametrize("dtype,encoding,layout,per_head,partition_tokens,shape", EXT)
def test_extended_matches_oracle(dtype, encoding, layout, per_head, partition_tokens, shape):
    case = case_from(shape, dtype, seed=911, cache_encoding=encoding, layout=layout,
                     partition_tokens=partition_tokens, per_head_scales=per_head)
    out, lse = workloads.run_case(case, return_lse=True)
    torch.cuda.synchronize()
    expected, want_lse = oracle_expected(case)
    assert_parity(out, expected, dtype, f"ext {shape}")
    np.testing.assert_allclose(lse.cpu().numpy(), want_lse, **LSE_TOL)


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
def test_fp8_decode_is_exact_for_every_finite_code(dtype):
    """Single-token sequences return V exactly (attention_tests.rs:32-56), so the
    output is the in-kernel FP8 decode of each byte: all 254 finite codes,
    both signs, against the OCP E4M3FN closed form (quantization.rs:13-29)."""
    B, Hkv, D, bs = 2, 2, 128, 16
    codes = np.array([c for c in range(256) if c & 0x7F != 0x7F], dtype=np.uint8)
    vbytes = np.zeros((B, bs, Hkv, D), dtype=np.uint8)
    flat = vbytes.reshape(-1)
    for i in range(B * Hkv):
        s, h = divmod(i, Hkv)
        vbytes[s, 0, h, :] = codes[(np.arange(D) + i * D) % len(codes)]
    fp8 = torch.float8_e4m3fn
    value_cache = torch.from_numpy(vbytes).to(DEV).view(fp8)
    key_cache = torch.zeros((B, bs, Hkv, D), dtype=fp8, device=DEV)
    query = torch.randn((B, 4, D), device=DEV).to(dtype)
    tables = torch.arange(B, dtype=torch.int32, device=DEV).reshape(B, 1)
    lens = torch.ones(B, dtype=torch.int32, device=DEV)
    ones = torch.ones(1, dtype=torch.float32, device=DEV)
    out = ops.paged_decode_attention_extended(query, key_cache, value_cache, tables, lens, max_sequence_length=1,
                                              key_scales=ones, value_scales=ones)
    torch.cuda.synchronize()
    dec = np.array([oracle.fp8_to_f32(c) for c in range(256)], np.float32)
    got = out.float().cpu().numpy()
    for s in range(B):
        for hq in range(4):
            want = dec[vbytes[s, 0, hq // 2]]
            np.testing.assert_array_equal(got[s, hq], want)
    assert flat.size > 0


def test_mfma_and_vector_kernels_agree():
    """The same BF16 data through the matrix-core kernel and, with a block
    stride that breaks 16-byte alignment, through the general kernel."""
    shape = (4, 32, 8, 128, 128, 16, [700, 1, 33, 2048])
    case = case_from(shape, torch.bfloat16, seed=5)
    s, _, fam = ops.supports(2, 0, 4, 32, 8, 128, 128, case.num_blocks, 16, case.max_blocks_per_sequence, 2048,
                             case.scale)
    assert fam == "mfma-stream"
    fast = workloads.run_case(case)
    # Re-home the caches with a block stride of one block + 4 elements.
    NB = case.num_blocks
    blk = 16 * 8 * 128
    store_k = torch.empty(NB * (blk + 4), dtype=torch.bfloat16, device=DEV)
    store_v = torch.empty_like(store_k)
    kview = store_k.as_strided((NB, 16, 8, 128), (blk + 4, 8 * 128, 128, 1))
    vview = store_v.as_strided((NB, 16, 8, 128), (blk + 4, 8 * 128, 128, 1))
    kview.copy_(case.key_cache)
    vview.copy_(case.value_cache)
    slow = ops.paged_decode_attention_extended(case.query, kview, vview, case.block_tables, case.sequence_lengths,
                                               max_sequence_length=2048, scale=case.scale)
    torch.cuda.synchronize()
    expected, _ = oracle_expected(case)
    assert_parity(fast, expected, torch.bfloat16, "mfma")
    assert_parity(slow, expected, torch.bfloat16, "vector")


# ---------------------------------------------------------------------------
# Benchmark configurations
# ---------------------------------------------------------------------------


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
@pytest.mark.parametrize("encoding", ["native", "fp8"])
@pytest.mark.parametrize("block_size,partition_tokens,family", [
    (16, 512, "mfma-stream"),   # 16-token steps, one wave per partition
    (64, 0, "mfma-stream"),     # single partition split over 4 waves, 4 steps per block
    (16, 520, "mfma"),          # partition not a multiple of 16: 32-token kernel
    (8, 256, "mfma"),           # block smaller than a 16-token step: 32-token kernel
])
def test_matrix_core_kernels_match_oracle(dtype, encoding, block_size, partition_tokens, family):
    """The two matrix-core kernels on the same data, each against the oracle,
    with ragged lengths (1, a partial last step, several blocks)."""
    shape = (4, 32, 8, 128, 128, block_size, [700, 1, 33, 2050])
    case = case_from(shape, dtype, seed=23, cache_encoding=encoding, layout="NHD",
                     partition_tokens=partition_tokens)
    out, lse = workloads.run_case(case, return_lse=True)
    assert ops.last_kernel_family() == family
    torch.cuda.synchronize()
    expected, want_lse = oracle_expected(case)
    assert_parity(out, expected, dtype, f"{family} bs{block_size} part{partition_tokens} {encoding}")
    np.testing.assert_allclose(lse.cpu().numpy(), want_lse, **LSE_TOL)


@pytest.mark.parametrize("partition_tokens,misaligned", [(512, "output"), (0, "output"), (512, "workspace")])
def test_unaligned_output_or_workspace_takes_the_vector_kernel(partition_tokens, misaligned):
    """The matrix-core kernels store four 16-bit elements at a time (8 bytes):
    an output view or a workspace that is only element-aligned runs on the
    general kernel, with the same results."""
    shape = (4, 32, 8, 128, 128, 16, [700, 1, 33, 2050])
    case = case_from(shape, torch.bfloat16, seed=29, partition_tokens=partition_tokens)
    expected, want_lse = oracle_expected(case)
    aligned = workloads.run_case(case)
    assert ops.last_kernel_family() == "mfma-stream"
    out = None
    workspace = None
    if misaligned == "output":
        store = torch.empty(aligned.numel() + 1, device=DEV, dtype=torch.bfloat16)
        out = store[1:].view(aligned.shape)  # 2-byte aligned
    else:
        need = ops.extended_workspace_elements(case.sequences, case.query_heads, case.value_head_size,
                                               case.max_sequence_length, partition_tokens)
        workspace = torch.empty(need + 1, device=DEV, dtype=torch.float32)[1:]  # 4-byte aligned
    got, lse = workloads.run_case(case, output=out, workspace=workspace, return_lse=True)
    assert ops.last_kernel_family() == "vector"
    torch.cuda.synchronize()
    assert_parity(got, expected, torch.bfloat16, f"unaligned {misaligned}")
    np.testing.assert_allclose(lse.cpu().numpy(), want_lse, **LSE_TOL)


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
@pytest.mark.parametrize("encoding", ["native", "fp8"])
@pytest.mark.parametrize("shape", [
    (3, 32, 1, 128, 128, 16, [1100, 1, 530]),   # MQA group of 32: two full 16-head waves
    (3, 48, 2, 128, 128, 16, [17, 700, 1030]),  # group of 24: the second wave has 8 live heads
])
@pytest.mark.parametrize("partition_tokens", [512, 0])
def test_stream_kernel_two_head_tiles(dtype, encoding, shape, partition_tokens):
    """Groups of 17-32 query heads per KV head on the streaming kernel: two
    waves of one 16-head tile each on one shared ring of K/V stages, so the
    K and V rows are read once for both tiles."""
    B, Hq, Hkv, D, Dv, bs, lengths = shape
    case = case_from(shape, dtype, seed=61, cache_encoding=encoding, partition_tokens=partition_tokens)
    _, _, fam = ops.supports(2, 0, B, Hq, Hkv, D, Dv, case.num_blocks, bs, case.max_blocks_per_sequence,
                             case.max_sequence_length, case.scale)
    assert fam == "mfma-stream"
    out, lse = workloads.run_case(case, return_lse=True)
    torch.cuda.synchronize()
    expected, want_lse = oracle_expected(case)
    assert_parity(out, expected, dtype, f"tiles {shape} part{partition_tokens} {encoding}")
    np.testing.assert_allclose(lse.cpu().numpy(), want_lse, **LSE_TOL)


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
@pytest.mark.parametrize("encoding", ["native", "fp8"])
@pytest.mark.parametrize("layout", ["NHD", "HND"])
@pytest.mark.parametrize("shape,partition_tokens", [
    ((3, 64, 1, 128, 128, 16, [1100, 1, 530]), 512),       # MQA group of 64: four 16-head waves (FP8: two 32-head)
    ((2, 96, 2, 128, 128, 16, [700, 2049]), 256),          # group of 48: three 16-head waves
    ((2, 128, 1, 128, 128, 32, [33, 900]), 0),             # group of 128: eight 16-head waves (FP8: four 32-head), one partition
    ((3, 71, 1, 64, 64, 16, [513, 17, 1600]), 512),        # group of 71 at head size 64: three waves, the last 7 heads live
    ((2, 80, 2, 64, 64, 16, [640, 90]), 64),               # group of 40, 64-token partitions: the third wave 8 heads live
    ((2, 33, 1, 128, 128, 16, [300, 1500]), 256),          # group of 33: the third wave one head live
    ((2, 100, 1, 64, 64, 16, [1000, 70]), 128),            # group of 100: seven 16-head waves, the seventh 4 heads live
    ((2, 113, 1, 128, 128, 16, [700, 1500]), 256),         # group of 113: eight 16-head waves, the eighth 1 head live
])
def test_stream_kernel_wide_groups(dtype, encoding, layout, shape, partition_tokens):
    """Groups of 33-128 query heads per KV head: one workgroup per item, each
    wave computing 16 or 32 heads of the group from the same K/V rows."""
    B, Hq, Hkv, D, Dv, bs, lengths = shape
    case = case_from(shape, dtype, seed=81, layout=layout, partition_tokens=partition_tokens,
                     cache_encoding=encoding)
    enc = 1 if encoding == "fp8" else 0
    qdt = 2 if dtype == torch.bfloat16 else 1
    _, _, fam = ops.supports(qdt, enc, B, Hq, Hkv, D, Dv, case.num_blocks, bs, case.max_blocks_per_sequence,
                             case.max_sequence_length, case.scale)
    assert fam == "mfma-stream"
    out, lse = workloads.run_case(case, return_lse=True)
    torch.cuda.synchronize()
    expected, want_lse = oracle_expected(case)
    assert_parity(out, expected, dtype, f"wide group {shape[:6]} part{partition_tokens} {encoding} {layout}")
    np.testing.assert_allclose(lse.cpu().numpy(), want_lse, **LSE_TOL)


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
@pytest.mark.parametrize("encoding", ["native", "fp8"])
@pytest.mark.parametrize("layout", ["NHD", "HND"])
@pytest.mark.parametrize("shape,partition_tokens", [
    ((4, 32, 8, 64, 64, 16, [700, 1, 33, 2050]), 512),   # split over 4 waves, partial last steps
    ((4, 32, 8, 64, 64, 32, [700, 1, 33, 2050]), 64),    # 64-token partitions, 32-token blocks
    ((3, 16, 2, 64, 64, 16, [90, 17, 300]), 0),          # single partition, 8 heads per KV head
    ((3, 32, 1, 64, 64, 16, [1100, 1, 530]), 512),       # MQA group of 32: two head tiles per wave
    ((256, 16, 8, 64, 64, 16, [300 - (i % 37) for i in range(256)]), 128),  # >= 4096 items: grouped launch
])
def test_stream_kernel_head_size_64(dtype, encoding, layout, shape, partition_tokens):
    """Head size 64 on the streaming kernel: 16-bit cache (128-byte rows) or
    FP8 cache (64-byte rows converted in LDS)."""
    B, Hq, Hkv, D, Dv, bs, lengths = shape
    case = case_from(shape, dtype, seed=71, layout=layout, partition_tokens=partition_tokens,
                     cache_encoding=encoding)
    enc = 1 if encoding == "fp8" else 0
    _, _, fam = ops.supports(2, enc, B, Hq, Hkv, D, Dv, case.num_blocks, bs, case.max_blocks_per_sequence,
                             case.max_sequence_length, case.scale)
    assert fam == "mfma-stream"
    out, lse = workloads.run_case(case, return_lse=True)
    torch.cuda.synchronize()
    expected, want_lse = oracle_expected(case)
    assert_parity(out, expected, dtype, f"d64 {shape[:6]} part{partition_tokens} {encoding} {layout}")
    np.testing.assert_allclose(lse.cpu().numpy(), want_lse, **LSE_TOL)


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
@pytest.mark.parametrize("encoding", ["native", "fp8"])
@pytest.mark.parametrize("layout", ["NHD", "HND"])
@pytest.mark.parametrize("shape,partition_tokens", [
    ((4, 16, 8, 256, 256, 16, [700, 1, 33, 1500]), 512),   # split over 4 waves, partial last steps
    ((3, 8, 4, 256, 256, 32, [90, 17, 300]), 64),           # one wave per item, 32-token blocks
    ((2, 32, 2, 256, 256, 16, [400, 129]), 0),              # single partition, 16 heads per KV head
    ((128, 8, 4, 256, 256, 16, [200 - (i % 29) for i in range(128)]), 32),  # >= 4096 items: grouped launch
])
def test_stream_kernel_head_size_256(dtype, encoding, layout, shape, partition_tokens):
    """Head size 256 on the streaming kernel: 16-bit cache (512-byte rows) or
    FP8 cache (256-byte rows converted in LDS)."""
    B, Hq, Hkv, D, Dv, bs, lengths = shape
    case = case_from(shape, dtype, seed=73, layout=layout, partition_tokens=partition_tokens,
                     cache_encoding=encoding)
    enc = 1 if encoding == "fp8" else 0
    _, _, fam = ops.supports(2, enc, B, Hq, Hkv, D, Dv, case.num_blocks, bs, case.max_blocks_per_sequence,
                             case.max_sequence_length, case.scale)
    assert fam == "mfma-stream"
    out, lse = workloads.run_case(case, return_lse=True)
    torch.cuda.synchronize()
    expected, want_lse = oracle_expected(case)
    assert_parity(out, expected, dtype, f"d256 {shape[:6]} part{partition_tokens} {encoding} {layout}")
    np.testing.assert_allclose(lse.cpu().numpy(), want_lse, **LSE_TOL)


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
@pytest.mark.parametrize("head_size,encoding,layout", [(128, "native", "NHD"), (128, "fp8", "HND"), (64, "native", "NHD")])
def test_stream_kernel_grouped_mid_grid(dtype, head_size, encoding, layout):
    """1024-4095 work items with partitions of 8+ steps: four adjacent-head
    items per workgroup (16 sequences x 8 KV heads x 8 partitions)."""
    lengths = [2048 - 61 * i for i in range(16)]
    shape = (16, 32, 8, head_size, head_size, 16, lengths)
    case = case_from(shape, dtype, seed=79, cache_encoding=encoding, layout=layout, partition_tokens=256)
    out, lse = workloads.run_case(case, return_lse=True)
    torch.cuda.synchronize()
    subset = [0, 7, 15]
    expected, want_lse = oracle_expected(case, subset)
    assert_parity(out[subset], expected, dtype, f"grouped mid grid d{head_size} {encoding} {layout}")
    np.testing.assert_allclose(lse[subset].cpu().numpy(), want_lse, **LSE_TOL)


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
@pytest.mark.parametrize("layout", ["NHD", "HND"])
@pytest.mark.parametrize("head", [80, 96, 112])
@pytest.mark.parametrize("encoding", ["native", "fp8"])
@pytest.mark.parametrize("shape,partition_tokens", [
    ((4, 32, 32, [700, 1, 33, 1500]), 512),     # MHA (Phi-2 / Phi-3 shapes), split over 4 waves
    ((3, 16, 4, [90, 17, 300]), 64),            # one wave per item, 32-token blocks below
    ((2, 16, 2, [400, 129]), 0),                # single partition, 8 heads per KV head
    ((64, 32, 32, [150 - (i % 23) for i in range(64)]), 64),  # >= 4096 items: grouped launch
])
def test_stream_kernel_rotated_head_sizes(dtype, layout, head, encoding, shape, partition_tokens):
    """Head sizes 80, 96 and 112 on the streaming kernel: 16-bit caches (rows
    of 10, 12 or 14 chunks, rotated at head size 96) or FP8 caches (rows of 5,
    6 or 7 chunks, converted into the 16-bit V layout); the QK operand chunks
    past the head size are zero."""
    B, Hq, Hkv, lengths = shape
    bs = 32 if partition_tokens == 64 and B == 3 else 16
    full = (B, Hq, Hkv, head, head, bs, lengths)
    case = case_from(full, dtype, seed=83 + head, layout=layout, partition_tokens=partition_tokens,
                     cache_encoding=encoding)
    enc = 1 if encoding == "fp8" else 0
    _, _, fam = ops.supports(2, enc, B, Hq, Hkv, head, head, case.num_blocks, bs, case.max_blocks_per_sequence,
                             case.max_sequence_length, case.scale)
    assert fam == "mfma-stream"
    out, lse = workloads.run_case(case, return_lse=True)
    torch.cuda.synchronize()
    expected, want_lse = oracle_expected(case)
    assert_parity(out, expected, dtype, f"d{head} {full[:6]} part{partition_tokens} {encoding} {layout}")
    np.testing.assert_allclose(lse.cpu().numpy(), want_lse, **LSE_TOL)


def test_config1_f32_plumbing_full():
    case = workloads.config(1, DEV)
    out, lse = workloads.run_case(case, return_lse=True)
    base = ops.paged_decode_attention(case.query, case.key_cache, case.value_cache, case.block_tables,
                                      case.sequence_lengths, max_sequence_length=case.max_sequence_length)
    torch.cuda.synchronize()
    expected, want_lse = oracle_expected(case)
    assert_parity(out, expected, torch.float32, "c1")
    assert_parity(base, expected, torch.float32, "c1 base")
    np.testing.assert_allclose(lse.cpu().numpy(), want_lse, **LSE_TOL)


def test_config2_single_partition_full():
    case = workloads.config(2, DEV)
    out, lse = workloads.run_case(case, return_lse=True)
    torch.cuda.synchronize()
    expected, want_lse = oracle_expected(case)
    assert_parity(out, expected, torch.bfloat16, "c2")
    np.testing.assert_allclose(lse.cpu().numpy(), want_lse, **LSE_TOL)


@pytest.mark.parametrize("index", [3, 4, 5])
def test_config_full_against_oracle_and_split_invariance(index):
    """Every sequence of C3, C4 and C5 against the oracle (threaded over
    sequences), then split-K invariance over other partition sizes."""
    case = workloads.config(index, DEV)
    out, lse = workloads.run_case(case, return_lse=True)
    torch.cuda.synchronize()
    expected, want_lse = oracle_expected(case, threads=ORACLE_THREADS)
    assert_parity(out, expected, case.dtype, f"c{index} full")
    np.testing.assert_allclose(lse.cpu().numpy(), want_lse, **LSE_TOL)
    # Size-independent property over every sequence: one partition per
    # sequence and a different partition size give the same result.
    for other in (0, 3 * case.partition_tokens // 2 + 16):
        case.partition_tokens = other
        out2, lse2 = workloads.run_case(case, return_lse=True)
        torch.cuda.synchronize()
        diff = (out2.float() - out.float()).abs()
        bound = 2e-3 + 1e-2 * out.float().abs()
        assert bool((diff <= bound).all()), f"partition {other}: max diff {diff.max().item()}"
        assert torch.allclose(lse2, lse, atol=1e-4, rtol=1e-5)
    assert math.isfinite(float(out.float().abs().max()))


@pytest.mark.parametrize("encoding", ["native", "fp8"])
@pytest.mark.parametrize("shape,partition_tokens,kernel", [
    ((48, 24, 6, 128, 128, 16, [700 + 9 * i for i in range(48)]), 128, "decode_stream_group_kernel"),
    ((3, 12, 6, 128, 128, 16, [300, 1000, 50]), 256, "decode_stream_kernel"),
    ((5, 24, 12, 64, 64, 16, [513, 1, 1024, 77, 900]), 128, "decode_stream_kernel"),
    ((2, 288, 6, 128, 128, 16, [600, 1300]), 256, "decode_stream_heads_kernel"),
])
def test_kv_head_counts_that_are_not_powers_of_two(encoding, shape, partition_tokens, kernel):
    """6 and 12 KV heads on the scheduled streaming kernels. Odd (sequence,
    partition) pairs swap the halves of the KV heads only when their count is
    a power of two: XOR with half of 6 would send head 4 to 7 and never
    compute heads 4 and 5."""
    case = case_from(shape, torch.bfloat16, seed=91, partition_tokens=partition_tokens, cache_encoding=encoding)
    out, lse = workloads.run_case(case, return_lse=True)
    torch.cuda.synchronize()
    assert ops.last_kernel_name() == kernel
    expected, want_lse = oracle_expected(case)
    assert_parity(out, expected, torch.bfloat16, f"{shape[:3]} {encoding}")
    np.testing.assert_allclose(lse.cpu().numpy(), want_lse, **LSE_TOL)
