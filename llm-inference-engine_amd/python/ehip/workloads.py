"""Synthetic ragged steps for the benchmark configurations (C1-C5).

A step is described the way the engine's scheduler and batch assembly hand it
to the attention path (src/engine/batch.cpp:37-84): per sequence the number of
new query rows T_b, the post-append context L_b, its block table and the slots
of the appended tokens (slot = table[pos // bs] * bs + pos % bs,
src/kvcache/block_table.cpp:60-66). Draws come from numpy's seeded PCG64 in a
fixed order (lengths, pool permutation, sharing), so a seed names one step.
"""
from __future__ import annotations

import math
from dataclasses import dataclass, field

import numpy as np

from . import KV_BF16, KV_F32, KV_INT8


@dataclass
class Workload:
    name: str
    heads: int
    kv_heads: int
    head_dim: int
    block_size: int
    kv_dtype: int
    layers: int
    query_lens: np.ndarray          # [B] int32
    context_lens: np.ndarray        # [B] int64, post-append
    tables: list                    # per sequence int32 block ids (>= ceil(L/bs))
    slot_mapping: np.ndarray        # [sum T] int64
    pool_blocks: int
    refcount: np.ndarray            # [pool_blocks] int32 (0 = free)
    qkv_std: float = 1.0
    notes: dict = field(default_factory=dict)

    @property
    def num_seqs(self) -> int:
        return len(self.context_lens)

    @property
    def rows(self) -> int:
        return int(self.query_lens.sum())

    @property
    def scale(self) -> float:
        # OptimizedModel::RunStack: 1/sqrt(d) in double, then narrowed
        # (src/model/optimized_model.cpp:473-474).
        return float(np.float32(1.0 / math.sqrt(self.head_dim)))

    @property
    def kv_bytes(self) -> int:
        return {KV_BF16: 2, KV_INT8: 1}.get(self.kv_dtype, 4)

    def decode_rows(self) -> np.ndarray:
        return np.flatnonzero(self.query_lens == 1)

    def bytes_per_layer(self, with_append: bool) -> dict:
        """Algorithmic HBM bytes of one layer (decode accounting: each unique
        physical K/V row once, Q read, O written, tables/offsets/lengths read,
        optionally the append's fp32 read + slab write)."""
        bs, s = self.block_size, self.kv_bytes
        L = self.context_lens.astype(np.int64)
        row = self.kv_heads * self.head_dim * s * 2           # K and V of one token
        shared_extra = int(np.maximum(self.refcount - 1, 0).sum())
        unique_kv = row * (int(L.sum()) - bs * shared_extra)
        logical_kv = row * int(L.sum())
        B, H, d = self.num_seqs, self.heads, self.head_dim
        R = self.rows
        q_o = 4 * R * H * d * 2
        bt = 4 * int(np.sum((L + bs - 1) // bs)) + 4 * (B + 1) + 4 * B
        append = R * self.kv_heads * d * 2 * (4 + s) if with_append else 0
        if self.kv_dtype == KV_INT8:
            # the K and V scales of every unique (block, kv head) tile
            unique_kv += 8 * self.kv_heads * (int(np.sum((L + bs - 1) // bs)) - shared_extra)
        return {"unique_kv": unique_kv, "logical_kv": logical_kv, "q_o": q_o, "tables": bt,
                "append": append, "total": unique_kv + q_o + bt + append}

    def prefill_flops_per_layer(self) -> int:
        """4*H*d*(T*P + T(T+1)/2) per chunk (QK^T + PV, causal)."""
        tot = 0
        for T, L in zip(self.query_lens, self.context_lens):
            if T > 1:
                P = int(L) - int(T)
                tot += 4 * self.heads * self.head_dim * (int(T) * P + int(T) * (int(T) + 1) // 2)
        return tot


def _tables_from_pool(need: np.ndarray, pool: int, rng: np.random.Generator):
    perm = rng.permutation(pool).astype(np.int32)
    tables, off = [], 0
    for n in need:
        tables.append(perm[off:off + int(n)].copy())
        off += int(n)
    return tables, perm[off:]


def _append_slots(tables, query_lens, context_lens, bs):
    slots = []
    for t, T, L in zip(tables, query_lens, context_lens):
        for pos in range(int(L) - int(T), int(L)):
            slots.append(int(t[pos // bs]) * bs + pos % bs)
    return np.asarray(slots, np.int64)


def _finish(name, H, Hkv, d, bs, dtype, layers, qlens, clens, tables, pool, std, notes=None):
    rc = np.zeros(pool, np.int32)
    for t in tables:
        np.add.at(rc, t, 1)
    return Workload(name, H, Hkv, d, bs, dtype, layers, np.asarray(qlens, np.int32),
                    np.asarray(clens, np.int64), tables,
                    _append_slots(tables, qlens, clens, bs), pool, rc, std, notes or {})


def c1(seed: int = 1) -> Workload:
    """Qwen2-0.5B single sequence: 14q/2kv, d=64, fp32, 512 cached tokens in
    32 blocks of a 64-block pool (seeded permutation) + 1 appended -> L=513."""
    rng = np.random.default_rng(seed)
    perm = rng.permutation(64).astype(np.int32)
    table = perm[:33].copy()  # the 33rd block is allocated for the appended token
    return _finish("C1", 14, 2, 64, 16, KV_F32, 1, [1], [513], [table], 64, 1.0)


def c2(seed: int = 2, layers: int = 24) -> Workload:
    """Qwen2-0.5B ragged decode: B=32, prior context U[64,2048], +1 appended,
    fp32 pool sized 1.25x the need, 24 layers."""
    rng = np.random.default_rng(seed)
    prev = rng.integers(64, 2048 + 1, 32)
    L = prev + 1
    need = (L + 15) // 16
    pool = int(math.ceil(1.25 * need.sum()))
    tables, _ = _tables_from_pool(need, pool, rng)
    return _finish("C2", 14, 2, 64, 16, KV_F32, layers, np.ones(32, np.int32), L, tables, pool,
                   1.0)


def c3(seed: int = 3, layers: int = 32) -> Workload:
    """Llama-3-8B mixed step: 4 causal prefill chunks T~U[256,1024] (P=0) + 60
    decodes with prior context U[128,4096]; 32q/8kv, d=128, bf16 KV."""
    rng = np.random.default_rng(seed)
    T = rng.integers(256, 1024 + 1, 4)
    prev = rng.integers(128, 4096 + 1, 60)
    qlens = np.concatenate([T, np.ones(60, np.int64)])
    L = np.concatenate([T, prev + 1])
    need = (L + 15) // 16
    pool = int(math.ceil(1.25 * need.sum()))
    tables, _ = _tables_from_pool(need, pool, rng)
    return _finish("C3", 32, 8, 128, 16, KV_BF16, layers, qlens, L, tables, pool, 0.5)


def c4(seed: int = 4, layers: int = 32, num_seqs: int = 256, share_frac: float = 0.10) -> Workload:
    """Llama-3-8B large decode: B=256, prior context log-uniform [256,8192],
    bf16 KV; pairs of sequences share their first full blocks (forked
    prefixes) until ~share_frac of the in-use physical blocks have refcount 2."""
    rng = np.random.default_rng(seed)
    u = rng.random(num_seqs)
    prev = np.rint(np.exp(np.log(256) + u * (np.log(8192) - np.log(256)))).astype(np.int64)
    L = prev + 1
    bs = 16
    need = (L + bs - 1) // bs
    full = prev // bs                      # full blocks before the append position
    # Decide sharing first: the younger (odd) member of each pair maps its
    # first k logical blocks onto the elder's physical blocks.
    share = np.zeros(num_seqs, np.int64)
    # shared / (need - shared) = share_frac of the in-use physical blocks
    target = share_frac * int(need.sum()) / (1.0 + share_frac)
    shared = 0
    for a in range(0, num_seqs - 1, 2):
        if shared >= target:
            break
        k = int(min(full[a], full[a + 1], math.ceil(target - shared)))
        share[a + 1] = k
        shared += k
    own = need - share
    pool = int(math.ceil(1.1 * own.sum()))
    tables_own, _ = _tables_from_pool(own, pool, rng)
    tables = []
    for b in range(num_seqs):
        if share[b] > 0:
            tables.append(np.concatenate([tables[b - 1][:share[b]], tables_own[b]]).astype(np.int32))
        else:
            tables.append(tables_own[b])
    w = _finish("C4", 32, 8, 128, bs, KV_BF16, layers, np.ones(num_seqs, np.int32), L, tables,
                pool, 0.5, {"shared_blocks": int(shared)})
    return w


def c5(seed: int = 5, layers: int = 80) -> Workload:
    """Llama-3-70B long context: 8 sequences at 32768 + 24 at U[1024,8192]
    (post-append), 64q/8kv, d=128, bf16 KV, 80 layers."""
    rng = np.random.default_rng(seed)
    prev = np.concatenate([np.full(8, 32767), rng.integers(1024, 8192 + 1, 24) - 1])
    L = prev + 1
    need = (L + 15) // 16
    pool = int(math.ceil(1.1 * need.sum()))
    tables, _ = _tables_from_pool(need, pool, rng)
    return _finish("C5", 64, 8, 128, 16, KV_BF16, layers, np.ones(32, np.int32), L, tables, pool,
                   0.5)


CONFIGS = {"C1": c1, "C2": c2, "C3": c3, "C4": c4, "C5": c5}
