"""Helpers for the GPU parity tests: seeded pools in the reference slab
layout, uploads, and the error metrics of the parity report."""
from __future__ import annotations

import numpy as np

from paged_util import POISON


def seeded_pool(orc, w, seed: int, poison: bool = True):
    """fp32 K/V slabs [pool, Hkv, bs, d] for workload `w`: every slot a
    sequence holds before its append (positions < L - T) gets N(0, std) from
    the oracle's mt19937_64/Box-Muller stream; everything else is poison, so a
    kernel that reads an unused slot or block shows it."""
    shape = (w.pool_blocks, w.kv_heads, w.block_size, w.head_dim)
    fill = POISON if poison else np.float32(0)
    k = np.full(shape, fill, np.float32)
    v = np.full(shape, fill, np.float32)
    n_rows = w.kv_heads * w.head_dim
    s = seed
    for t, T, L in zip(w.tables, w.query_lens, w.context_lens):
        P = int(L) - int(T)
        if P == 0:
            continue
        kk = orc.fill_normal(P * n_rows, 0.0, w.qkv_std, s).reshape(w.kv_heads, P, w.head_dim)
        vv = orc.fill_normal(P * n_rows, 0.0, w.qkv_std, s + 1).reshape(w.kv_heads, P, w.head_dim)
        s += 2
        for pos in range(P):
            blk = int(t[pos // w.block_size])
            # A shared prefix block ends up holding the last writer's rows;
            # both sharers then read that same physical content.
            k[blk, :, pos % w.block_size, :] = kk[:, pos, :]
            v[blk, :, pos % w.block_size, :] = vv[:, pos, :]
    return k, v


def new_rows(orc, w, seed: int):
    """The step's new K/V rows [sum T, Hkv, d] and queries [sum T, H, d]."""
    R = w.rows
    kn = orc.fill_normal(R * w.kv_heads * w.head_dim, 0.0, w.qkv_std, seed).reshape(
        R, w.kv_heads, w.head_dim)
    vn = orc.fill_normal(R * w.kv_heads * w.head_dim, 0.0, w.qkv_std, seed + 1).reshape(
        R, w.kv_heads, w.head_dim)
    q = orc.fill_normal(R * w.heads * w.head_dim, 0.0, w.qkv_std, seed + 2).reshape(
        R, w.heads, w.head_dim)
    return kn, vn, q


def rel_norm(a, b) -> float:
    """max over (row, head) vectors of max|a-b| / max|b|."""
    a = np.asarray(a, np.float64).reshape(-1, a.shape[-1])
    b = np.asarray(b, np.float64).reshape(-1, b.shape[-1])
    den = np.maximum(np.abs(b).max(axis=1), 1e-30)
    return float((np.abs(a - b).max(axis=1) / den).max()) if a.size else 0.0


def max_abs(a, b) -> float:
    return float(np.abs(np.asarray(a, np.float64) - np.asarray(b, np.float64)).max()) if np.size(a) else 0.0
