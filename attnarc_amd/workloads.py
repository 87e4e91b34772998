"""Seeded synthetic paged-decode inputs for the named benchmark shapes.

Every case is fully determined by its seed: sequence lengths and block tables
come from ``numpy.random.default_rng(seed)``; Q/K/V come from a torch
generator seeded with ``seed`` on the target device, drawn as N(0, 1) F32 and
rounded once (round-to-nearest-even) to the storage dtype. FP8 caches are
``fp8_e4m3fn(clamp(x / scale[kv_head], -448, 448))``, the static-scale
encoding of docs/design/fp8-kv-cache.md:42-48 with finite saturation.

Unused block-table slots hold -1 (the sentinel the reference oracle accepts
in inactive slots, crates/loom-kernels/src/tests/attention_tests.rs:82).
"""

from __future__ import annotations

import math
from dataclasses import dataclass, field

import numpy as np
import torch

FP8_MAX = 448.0


@dataclass
class DecodeCase:
    name: str
    dtype: torch.dtype  # query / output dtype
    cache_encoding: str  # "native" or "fp8"
    layout: str  # "NHD" or "HND"
    sequences: int
    query_heads: int
    kv_heads: int
    head_size: int
    value_head_size: int
    block_size: int
    num_blocks: int
    max_blocks_per_sequence: int
    lengths: list
    partition_tokens: int
    scale: float
    seed: int
    query: torch.Tensor = None
    key_cache: torch.Tensor = None
    value_cache: torch.Tensor = None
    key_scales: torch.Tensor = None
    value_scales: torch.Tensor = None
    block_tables: torch.Tensor = None
    sequence_lengths: torch.Tensor = None
    extra: dict = field(default_factory=dict)

    @property
    def max_sequence_length(self) -> int:
        return int(max(self.lengths))

    @property
    def kv_elem_bytes(self) -> int:
        if self.cache_encoding == "fp8":
            return 1
        return torch.empty((), dtype=self.dtype).element_size()

    def kv_bytes(self) -> int:
        """Algorithmic KV bytes of one call: sum(len) * Hkv * (D + Dv) * elem."""
        return int(sum(self.lengths)) * self.kv_heads * (self.head_size + self.value_head_size) * self.kv_elem_bytes

    def flops(self) -> int:
        return 2 * int(sum(self.lengths)) * self.query_heads * (self.head_size + self.value_head_size)

    def describe(self) -> dict:
        return {
            "workload": self.name,
            "dtype": str(self.dtype).replace("torch.", ""),
            "kv_cache": "fp8_e4m3fn" if self.cache_encoding == "fp8" else "native",
            "layout": self.layout,
            "batch": self.sequences,
            "query_heads": self.query_heads,
            "kv_heads": self.kv_heads,
            "head_dim": self.head_size,
            "block_size": self.block_size,
            "num_blocks": self.num_blocks,
            "context_min": int(min(self.lengths)),
            "context_max": int(max(self.lengths)),
            "context_sum": int(sum(self.lengths)),
            "partition_tokens": self.partition_tokens,
            "seed": self.seed,
        }


def _tables_from_pool(rng, lengths, block_size, pool_blocks, max_blocks):
    """Assign shuffled physical blocks from a pool to each sequence in order."""
    perm = rng.permutation(pool_blocks)
    tables = np.full((len(lengths), max_blocks), -1, dtype=np.int32)
    cursor = 0
    for s, length in enumerate(lengths):
        n = -(-int(length) // block_size)
        tables[s, :n] = perm[cursor : cursor + n]
        cursor += n
    return tables


def _randn(shape, gen, device, dtype, chunk_elems=1 << 26):
    """N(0,1) F32 rounded to ``dtype``, generated in chunks to bound memory."""
    out = torch.empty(shape, device=device, dtype=dtype)
    flat = out.view(-1)
    n = flat.numel()
    for start in range(0, n, chunk_elems):
        stop = min(n, start + chunk_elems)
        flat[start:stop] = torch.randn(stop - start, generator=gen, device=device, dtype=torch.float32).to(dtype)
    return out


def _fp8_cache(shape, head_dim_axis, scales, gen, device, chunk_blocks=4096):
    """fp8_e4m3fn(clamp(N(0,1) / scale[kv_head])) with the kv-head axis given."""
    fp8 = getattr(torch, "float8_e4m3fn")
    out = torch.empty(shape, device=device, dtype=fp8)
    view_shape = [1, 1, 1, 1]
    view_shape[head_dim_axis] = -1
    inv = (1.0 / scales).view(view_shape)
    for start in range(0, shape[0], chunk_blocks):
        stop = min(shape[0], start + chunk_blocks)
        x = torch.randn((stop - start,) + tuple(shape[1:]), generator=gen, device=device, dtype=torch.float32)
        out[start:stop] = (x * inv).clamp_(-FP8_MAX, FP8_MAX).to(fp8)
    return out


def make_case(
    *,
    name: str,
    dtype: torch.dtype,
    sequences: int,
    query_heads: int,
    kv_heads: int,
    head_size: int,
    value_head_size: int,
    block_size: int,
    lengths,
    seed: int,
    device,
    cache_encoding: str = "native",
    layout: str = "NHD",
    pool_factor: float | None = None,
    num_blocks: int | None = None,
    partition_tokens: int = 0,
    scale: float | None = None,
    scale_range=(0.01, 0.1),
    per_head_scales: bool = True,
) -> DecodeCase:
    rng = np.random.default_rng(seed)
    lengths = [int(x) for x in lengths]
    max_len = max(lengths)
    max_blocks = -(-max_len // block_size)
    needed = sum(-(-l // block_size) for l in lengths)
    if num_blocks is None:
        num_blocks = math.ceil(needed * pool_factor) if pool_factor else sequences * max_blocks
    num_blocks = max(num_blocks, needed)
    tables = _tables_from_pool(rng, lengths, block_size, num_blocks, max_blocks)
    if scale is None:
        scale = head_size ** -0.5
    gen = torch.Generator(device=device)
    gen.manual_seed(seed)
    query = _randn((sequences, query_heads, head_size), gen, device, dtype)
    if layout == "NHD":
        kshape = (num_blocks, block_size, kv_heads, head_size)
        vshape = (num_blocks, block_size, kv_heads, value_head_size)
        head_axis = 2
    elif layout == "HND":
        kshape = (num_blocks, kv_heads, block_size, head_size)
        vshape = (num_blocks, kv_heads, block_size, value_head_size)
        head_axis = 1
    else:
        raise ValueError(layout)
    key_scales = value_scales = None
    if cache_encoding == "fp8":
        n_scales = kv_heads if per_head_scales else 1
        lo, hi = scale_range
        key_scales = torch.tensor(rng.uniform(lo, hi, n_scales), dtype=torch.float32, device=device)
        value_scales = torch.tensor(rng.uniform(lo, hi, n_scales), dtype=torch.float32, device=device)
        ks = key_scales if per_head_scales else key_scales.expand(kv_heads)
        vs = value_scales if per_head_scales else value_scales.expand(kv_heads)
        key_cache = _fp8_cache(kshape, head_axis, ks, gen, device)
        value_cache = _fp8_cache(vshape, head_axis, vs, gen, device)
    else:
        key_cache = _randn(kshape, gen, device, dtype)
        value_cache = _randn(vshape, gen, device, dtype)
    return DecodeCase(
        name=name,
        dtype=dtype,
        cache_encoding=cache_encoding,
        layout=layout,
        sequences=sequences,
        query_heads=query_heads,
        kv_heads=kv_heads,
        head_size=head_size,
        value_head_size=value_head_size,
        block_size=block_size,
        num_blocks=num_blocks,
        max_blocks_per_sequence=max_blocks,
        lengths=lengths,
        partition_tokens=partition_tokens,
        scale=float(scale),
        seed=seed,
        query=query,
        key_cache=key_cache,
        value_cache=value_cache,
        key_scales=key_scales,
        value_scales=value_scales,
        block_tables=torch.from_numpy(tables).to(device),
        sequence_lengths=torch.tensor(lengths, dtype=torch.int32, device=device),
    )


def config(index: int, device, seed: int | None = None, layout: str | None = None) -> DecodeCase:
    """The five benchmark configurations of the paged-decode north star (1-based).

    ``layout`` overrides the configuration's cache layout (NHD/HND) for
    layout comparisons; the default is the configuration's own.
    """
    case = _config(index, device, seed, layout)
    return case


def _config(index: int, device, seed, layout) -> DecodeCase:
    seed = 1000 + index if seed is None else seed
    rng = np.random.default_rng(seed ^ 0x5EED)
    if index == 1:
        # F32 MHA plumbing case: B4, H8/8, D64, len U[1,256], bs16, a seeded
        # permutation of 64 physical blocks (16 per sequence), no split-K.
        lengths = rng.integers(1, 257, size=4)
        return make_case(
            name="c1_f32_mha_plumbing", dtype=torch.float32, sequences=4, query_heads=8, kv_heads=8,
            head_size=64, value_head_size=64, block_size=16, lengths=lengths, seed=seed, device=device,
            num_blocks=64, layout=layout or "NHD",
        )
    if index == 2:
        # Qwen2.5-1.5B GQA: B32, H12/2, D128, len 2048, bs16, single partition.
        return make_case(
            name="c2_qwen2.5_1.5b_gqa_bf16", dtype=torch.bfloat16, sequences=32, query_heads=12,
            kv_heads=2, head_size=128, value_head_size=128, block_size=16, lengths=[2048] * 32,
            seed=seed, device=device, layout=layout or "NHD",
        )
    if index == 3:
        # Llama-3-8B GQA: B64, H32/8, D128, len U[512,8192], bs16, pool 1.25x, split-K 512.
        lengths = rng.integers(512, 8193, size=64)
        return make_case(
            name="c3_llama3_8b_gqa_bf16", dtype=torch.bfloat16, sequences=64, query_heads=32,
            kv_heads=8, head_size=128, value_head_size=128, block_size=16, lengths=lengths,
            seed=seed, device=device, pool_factor=1.25, partition_tokens=512, layout=layout or "NHD",
        )
    if index == 4:
        # FP8-KV at Llama-3-70B head geometry: B128, H64/8, D128, len 4096, bs16, HND,
        # per-head scales U[0.01,0.1], BF16 Q/out, split-K 512.
        return make_case(
            name="c4_llama3_70b_fp8kv_hnd", dtype=torch.bfloat16, sequences=128, query_heads=64,
            kv_heads=8, head_size=128, value_head_size=128, block_size=16, lengths=[4096] * 128,
            seed=seed, device=device, cache_encoding="fp8", layout=layout or "HND", partition_tokens=512,
        )
    if index == 5:
        # Long-context MQA: B8, H32/1, D128, len U[65536,131072], bs16, split-K 1024.
        lengths = rng.integers(65536, 131073, size=8)
        return make_case(
            name="c5_long_mqa_bf16", dtype=torch.bfloat16, sequences=8, query_heads=32, kv_heads=1,
            head_size=128, value_head_size=128, block_size=16, lengths=lengths, seed=seed,
            device=device, partition_tokens=1024, layout=layout or "NHD",
        )
    raise ValueError(f"unknown config {index}")


_SHAPE_KEYS = {"B": int, "Hq": int, "Hkv": int, "D": int, "Dv": int, "L": int, "bs": int, "part": int,
               "seed": int, "dtype": str, "kv": str, "layout": str}
_DTYPES = {"bf16": torch.bfloat16, "f16": torch.float16, "f32": torch.float32}


def shape_case(spec: str, device) -> DecodeCase:
    """A decode workload outside the five configurations, from
    ``"B=64,Hq=16,Hkv=8,D=256,L=2048,part=512"``: every sequence at length L,
    a seeded shuffled pool of exactly the needed blocks. Keys: B, Hq, Hkv, D,
    Dv (default D), L, bs (16), part (split-K tokens, 0 = one partition),
    seed (7), dtype (bf16|f16|f32), kv (native|fp8), layout (NHD|HND)."""
    vals = {"bs": 16, "part": 0, "seed": 7, "dtype": "bf16", "kv": "native", "layout": "NHD"}
    for item in spec.split(","):
        key, _, raw = item.partition("=")
        key = key.strip()
        if key not in _SHAPE_KEYS:
            raise ValueError(f"unknown shape key {key!r} (keys: {', '.join(_SHAPE_KEYS)})")
        vals[key] = _SHAPE_KEYS[key](raw.strip())
    for key in ("B", "Hq", "Hkv", "D", "L"):
        if key not in vals:
            raise ValueError(f"shape needs {key}")
    d, dv = vals["D"], vals.get("Dv", vals["D"])
    name = (f"shape_{vals['dtype']}_{vals['kv']}_{vals['layout'].lower()}_b{vals['B']}_h{vals['Hq']}x{vals['Hkv']}"
            f"_d{d}_l{vals['L']}_p{vals['part']}")
    return make_case(
        name=name, dtype=_DTYPES[vals["dtype"]], sequences=vals["B"], query_heads=vals["Hq"],
        kv_heads=vals["Hkv"], head_size=d, value_head_size=dv, block_size=vals["bs"],
        lengths=[vals["L"]] * vals["B"], seed=vals["seed"], device=device, cache_encoding=vals["kv"],
        layout=vals["layout"], partition_tokens=vals["part"],
    )


def run_case(case: DecodeCase, *, output=None, lse=None, workspace=None, return_lse=False):
    """One call of the hot path for a case (extended entry point)."""
    from .ops import paged_decode_attention_extended

    return paged_decode_attention_extended(
        case.query, case.key_cache, case.value_cache, case.block_tables, case.sequence_lengths,
        max_sequence_length=case.max_sequence_length, scale=case.scale, layout=case.layout,
        key_scales=case.key_scales, value_scales=case.value_scales,
        partition_tokens=case.partition_tokens, output=output, lse=lse, workspace=workspace,
        return_lse=return_lse,
    )


# ---------------------------------------------------------------------------
# RoPE + paged K/V write workloads
# ---------------------------------------------------------------------------


@dataclass
class RopeWriteCase:
    """Inputs of one fused RoPE + paged-KV write call (``ops.rope_paged_kv_write_``)."""

    name: str
    dtype: torch.dtype
    cache_encoding: str  # "native" or "fp8"
    layout: str  # "NHD" or "HND"
    query: torch.Tensor  # [T, Hq, D]
    key: torch.Tensor  # [T, Hkv, D]
    value: torch.Tensor  # [T, Hkv, D]
    positions: torch.Tensor  # [T] int64
    cos_sin_cache: torch.Tensor  # [max_position, rotary_dim]
    kv_cache: torch.Tensor  # [blocks, 2, block_size, Hkv, D] (NHD or HND strides)
    key_scales: torch.Tensor
    value_scales: torch.Tensor
    slot_mapping: torch.Tensor  # [T] int64
    is_neox: bool = True

    @property
    def tokens(self) -> int:
        return int(self.query.shape[0])

    def algorithmic_bytes(self) -> int:
        """HBM bytes one call must move: Q and K read and written back, V,
        positions, slots and the cos/sin row read, K and V cache rows written."""
        t, hq, d = self.query.shape
        hkv = self.key.shape[1]
        e = self.query.element_size()
        ce = self.kv_cache.element_size()
        rd = self.cos_sin_cache.shape[1]
        return t * (2 * (hq + hkv) * d * e + hkv * d * e + 16 + rd * e + 2 * hkv * d * ce)

    def args(self):
        return (self.query, self.key, self.value, self.positions, self.cos_sin_cache, self.kv_cache,
                self.key_scales, self.value_scales, self.slot_mapping, self.is_neox)

    def describe(self) -> dict:
        return {
            "workload": self.name,
            "tokens": self.tokens,
            "query_heads": int(self.query.shape[1]),
            "kv_heads": int(self.key.shape[1]),
            "head_size": int(self.query.shape[2]),
            "rotary_dim": int(self.cos_sin_cache.shape[1]),
            "dtype": str(self.dtype).replace("torch.", ""),
            "cache_encoding": self.cache_encoding,
            "layout": self.layout,
            "block_size": int(self.kv_cache.shape[2]),
            "num_blocks": int(self.kv_cache.shape[0]),
        }


def rope_write_case(tokens: int, device, *, query_heads=32, kv_heads=8, head_size=128, rotary_dim=128,
                    max_position=8192, block_size=16, dtype=torch.bfloat16, cache_encoding="fp8", layout="HND",
                    seed: int = 7, name: str | None = None) -> RopeWriteCase:
    """Llama-3-8B-shaped write: ``tokens`` new tokens into a pool of 4x that many slots."""
    gen = torch.Generator(device=device).manual_seed(seed)
    q = _randn((tokens, query_heads, head_size), gen, device, dtype)
    k = _randn((tokens, kv_heads, head_size), gen, device, dtype)
    v = _randn((tokens, kv_heads, head_size), gen, device, dtype)
    positions = torch.randint(0, max_position, (tokens,), generator=gen, device=device)
    inv = 1.0 / (10000 ** (torch.arange(0, rotary_dim, 2, dtype=torch.float32, device=device) / rotary_dim))
    freqs = torch.outer(torch.arange(max_position, dtype=torch.float32, device=device), inv)
    cs = torch.cat((freqs.cos(), freqs.sin()), dim=-1).to(dtype)
    num_blocks = max(1, -(-4 * tokens // block_size))
    slots = torch.randperm(num_blocks * block_size, generator=gen, device=device)[:tokens].to(torch.int64)
    cache_dtype = torch.uint8 if cache_encoding == "fp8" else dtype
    shape = (num_blocks, 2, block_size, kv_heads, head_size)
    part = block_size * kv_heads * head_size
    if layout == "NHD":
        kv = torch.zeros(shape, device=device, dtype=cache_dtype)
    else:
        kv = torch.zeros(num_blocks * 2 * part, device=device, dtype=cache_dtype).as_strided(
            shape, (2 * part, part, head_size, block_size * head_size, 1))
    ks = torch.full((kv_heads,), 0.05, device=device)
    vs = torch.full((kv_heads,), 0.05, device=device)
    return RopeWriteCase(
        name=name or f"rope-kv-write T{tokens} Hq{query_heads}/Hkv{kv_heads} D{head_size} "
                     f"{str(dtype).replace('torch.', '')}->{cache_encoding} {layout}",
        dtype=dtype, cache_encoding=cache_encoding, layout=layout, query=q, key=k, value=v, positions=positions,
        cos_sin_cache=cs, kv_cache=kv, key_scales=ks, value_scales=vs, slot_mapping=slots)
