"""Independent dense restatement used to pin the oracle (numpy, F64).

Gathers each sequence's K/V rows through the block table and applies a
library softmax. It shares no code with oracle/paged_decode_oracle.cpp and
follows the PyTorch test oracle's math (python/tests/
test_paged_decode_attention.py:20-52): softmax(scale * q.K^T) V per head.
"""

from __future__ import annotations

import numpy as np
from scipy.special import logsumexp


def gather_rows(cache, tables, seq, length, kv_head, block_size, strides=None):
    """Logical rows [length, dim] of one (sequence, kv head) of a cache.

    ``cache`` is either a dense NHD array [NB, bs, Hkv, dim] or, with
    ``strides=(block, page, head)``, a flat array addressed by element strides.
    """
    pos = np.arange(length)
    blocks = tables[seq, pos // block_size].astype(np.int64)
    pages = pos % block_size
    if strides is None:
        return cache[blocks, pages, kv_head, :]
    b, p, h = strides
    dim = cache.shape[-1] if cache.ndim > 1 else None
    raise NotImplementedError(dim)


def dense_attention(q, k_rows, v_rows, scale):
    """q [G, D], k_rows [T, D], v_rows [T, Dv] -> (out [G, Dv], lse [G]) in F64."""
    scores = (q.astype(np.float64) @ k_rows.astype(np.float64).T) * np.float64(scale)
    lse = logsumexp(scores, axis=1)
    w = np.exp(scores - lse[:, None])
    return w @ v_rows.astype(np.float64), lse


def paged_attention(query, key_cache, value_cache, tables, lengths, scale, block_size):
    """Dense NHD caches given as float arrays; returns (out F64, lse F64)."""
    B, Hq, D = query.shape
    Hkv = key_cache.shape[2]
    G = Hq // Hkv
    Dv = value_cache.shape[3]
    out = np.zeros((B, Hq, Dv))
    lse = np.zeros((B, Hq))
    for s in range(B):
        for kvh in range(Hkv):
            k = gather_rows(key_cache, tables, s, int(lengths[s]), kvh, block_size)
            v = gather_rows(value_cache, tables, s, int(lengths[s]), kvh, block_size)
            o, l = dense_attention(query[s, kvh * G:(kvh + 1) * G], k, v, scale)
            out[s, kvh * G:(kvh + 1) * G] = o
            lse[s, kvh * G:(kvh + 1) * G] = l
    return out, lse
