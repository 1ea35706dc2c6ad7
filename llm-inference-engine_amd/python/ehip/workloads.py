"""Synthetic ragged steps for the benchmark configurations (C1-C5).

A step is described the way the engine's scheduler and batch assembly hand it
to the attention path (src/engine/batch.cpp:37-84): per sequence the number of
new query rows T_b, the post-append context L_b, its block table and the slots
of the appended tokens (slot = table[pos // bs] * bs + pos % bs,
src/kvcache/block_table.cpp:60-66).

Every draw comes from std::mt19937_64 (the reference's seeded engine,
src/tensor/ops.cpp:205-224; here ``ehip_rng_u64``), one seed per config:

* the structure stream ``mt19937_64(seed)`` is consumed in a fixed order:
  1. context lengths (the cached tokens before the step's append; a decode
     row then attends context + 1 keys),
  2. the pool permutation: Fisher-Yates over the pool's block ids, i from
     n-1 down to 1 swapping i with j = floor(u * (i + 1)), u = (x >> 11) *
     2^-53 (std::shuffle's algorithm is implementation-defined, so it is not
     used); tables take consecutive runs of the permuted ids,
  3. the sharing pairs (C4 only): a Fisher-Yates permutation of the sequence
     indices, read as consecutive pairs;
* the values come from the reference's ``fill_normal`` (``ehip_host_fill_normal``,
  src/tensor/ops.cpp:451-477), one fresh engine per tensor, seeded
  ``value_seed(seed, layer, what)``: what = 4 Q, 5 K pool, 6 V pool, 7 new K
  rows, 8 new V rows (the remaining draws 4-7 of the order above).

Integer draws: U[a, b] = a + floor(u * (b - a + 1)); log-uniform [a, b] =
round(exp(ln a + u * (ln b - ln a))). Pools hold ceil(1.25 * blocks needed)
block ids (C1: the 64-block pool the config names).
"""
from __future__ import annotations

import ctypes as C
import math
from dataclasses import dataclass, field

import numpy as np

from . import KV_BF16, KV_F32, KV_FP8, KV_INT8, lib

POOL_SLACK = 1.25
VALUE_Q, VALUE_K, VALUE_V, VALUE_NEW_K, VALUE_NEW_V = 4, 5, 6, 7, 8


def value_seed(seed: int, layer: int, what: int) -> int:
    """Seed of one value tensor of one layer (one fresh engine per tensor, as
    the reference's fill_normal builds one per call)."""
    return (int(seed) << 32) | (int(layer) << 8) | int(what)


class Stream:
    """Sequential reader of mt19937_64(seed) outputs."""

    def __init__(self, seed: int):
        self.seed = int(seed)
        self.pos = 0
        self.buf = np.empty(0, np.uint64)
        self.i = 0

    def _refill(self, n: int):
        n = max(n, 4096)
        buf = np.empty(n, np.uint64)
        rc = lib().ehip_rng_u64(self.seed, self.pos, buf.ctypes.data, n)
        if rc != 0:
            raise RuntimeError(f"ehip_rng_u64 failed ({rc})")
        self.pos += n
        self.buf, self.i = buf, 0

    def raw(self, n: int) -> np.ndarray:
        out = np.empty(n, np.uint64)
        k = 0
        while k < n:
            if self.i == self.buf.size:
                self._refill(n - k)
            m = min(n - k, self.buf.size - self.i)
            out[k:k + m] = self.buf[self.i:self.i + m]
            self.i += m
            k += m
        return out

    def units(self, n: int) -> np.ndarray:
        """n uniforms (x >> 11) * 2^-53 in [0, 1), exact in double."""
        return (self.raw(n) >> np.uint64(11)).astype(np.float64) * (2.0 ** -53)

    def uniform_int(self, a: int, b: int, n: int) -> np.ndarray:
        return (a + np.floor(self.units(n) * (b - a + 1))).astype(np.int64)

    def log_uniform_int(self, a: int, b: int, n: int) -> np.ndarray:
        u = self.units(n)
        return np.rint(np.exp(np.log(a) + u * (np.log(b) - np.log(a)))).astype(np.int64)

    def permutation(self, n: int) -> np.ndarray:
        """Fisher-Yates: for i = n-1 .. 1 swap p[i] with p[floor(u * (i + 1))]."""
        p = np.arange(n, dtype=np.int64)
        if n < 2:
            return p
        u = self.units(n - 1)
        idx = np.arange(n - 1, 0, -1)
        js = np.floor(u * (idx + 1)).astype(np.int64)
        for i, j in zip(idx.tolist(), js.tolist()):
            p[i], p[j] = p[j], p[i]
        return p


def fill_normal(n: int, mean: float, std: float, seed: int) -> np.ndarray:
    """The reference's fill_normal over n fp32 elements (host, threaded)."""
    out = np.empty(int(n), np.float32)
    rc = lib().ehip_host_fill_normal(out.ctypes.data, int(n), C.c_double(mean), C.c_double(std),
                                     C.c_uint64(seed))
    if rc != 0:
        raise RuntimeError(f"ehip_host_fill_normal failed ({rc})")
    return out


def to_bf16_bits(x: np.ndarray) -> np.ndarray:
    """Fp32ToBf16Bits over an fp32 array (host, threaded)."""
    x = np.ascontiguousarray(x, np.float32)
    out = np.empty(x.shape, np.uint16)
    rc = lib().ehip_host_fp32_to_bf16(x.ctypes.data, out.ctypes.data, x.size)
    if rc != 0:
        raise RuntimeError(f"ehip_host_fp32_to_bf16 failed ({rc})")
    return out


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
    seed: int = 0
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
        return {KV_BF16: 2, KV_INT8: 1, KV_FP8: 1}.get(self.kv_dtype, 4)

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
        if self.kv_dtype in (KV_INT8, KV_FP8):
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

    # ------------------------------------------------------------ values
    def q(self, layer: int = 0) -> np.ndarray:
        n = self.rows * self.heads * self.head_dim
        return fill_normal(n, 0.0, self.qkv_std, value_seed(self.seed, layer, VALUE_Q)).reshape(
            self.rows, self.heads, self.head_dim)

    def pool(self, layer: int = 0):
        """fp32 K and V slabs [pool_blocks, Hkv, bs, d], every element drawn."""
        shape = (self.pool_blocks, self.kv_heads, self.block_size, self.head_dim)
        n = int(np.prod(shape))
        k = fill_normal(n, 0.0, self.qkv_std, value_seed(self.seed, layer, VALUE_K))
        v = fill_normal(n, 0.0, self.qkv_std, value_seed(self.seed, layer, VALUE_V))
        return k.reshape(shape), v.reshape(shape)

    def new_kv(self, layer: int = 0):
        """The step's new K and V rows [sum T, Hkv, d] (fp32, pre-append)."""
        n = self.rows * self.kv_heads * self.head_dim
        shape = (self.rows, self.kv_heads, self.head_dim)
        return (fill_normal(n, 0.0, self.qkv_std,
                            value_seed(self.seed, layer, VALUE_NEW_K)).reshape(shape),
                fill_normal(n, 0.0, self.qkv_std,
                            value_seed(self.seed, layer, VALUE_NEW_V)).reshape(shape))


def _tables_from_pool(need: np.ndarray, pool: int, rng):
    """Consecutive runs of a permutation of [0, pool) as the tables. rng is a
    Stream (the structure stream) or a numpy Generator (tests' own cases)."""
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


def _finish(name, H, Hkv, d, bs, dtype, layers, qlens, clens, tables, pool, std, notes=None,
            seed=0):
    rc = np.zeros(pool, np.int32)
    for t in tables:
        np.add.at(rc, t, 1)
    return Workload(name, H, Hkv, d, bs, dtype, layers, np.asarray(qlens, np.int32),
                    np.asarray(clens, np.int64), tables,
                    _append_slots(tables, qlens, clens, bs), pool, rc, std, seed, notes or {})


def _pool_size(blocks: int) -> int:
    return int(math.ceil(POOL_SLACK * blocks))


def c1(seed: int = 1) -> Workload:
    """Qwen2-0.5B single sequence: 14q/2kv, d=64, fp32, 512 cached tokens in
    32 blocks of a 64-block pool (Fisher-Yates permutation) + 1 appended ->
    L=513 (the 33rd block holds the appended token)."""
    st = Stream(seed)
    perm = st.permutation(64).astype(np.int32)
    table = perm[:33].copy()
    return _finish("C1", 14, 2, 64, 16, KV_F32, 1, [1], [513], [table], 64, 1.0, seed=seed)


def c2(seed: int = 2, layers: int = 24) -> Workload:
    """Qwen2-0.5B ragged decode: B=32, context U[64,2048], +1 appended, fp32
    pool sized 1.25x the need, 24 layers."""
    st = Stream(seed)
    L = st.uniform_int(64, 2048, 32) + 1
    need = (L + 15) // 16
    tables, _ = _tables_from_pool(need, _pool_size(int(need.sum())), st)
    return _finish("C2", 14, 2, 64, 16, KV_F32, layers, np.ones(32, np.int32), L, tables,
                   _pool_size(int(need.sum())), 1.0, seed=seed)


def c3(seed: int = 3, layers: int = 32) -> Workload:
    """Llama-3-8B mixed step: 4 causal prefill chunks T~U[256,1024] (P=0) + 60
    decodes with context U[128,4096]; 32q/8kv, d=128, bf16 KV."""
    st = Stream(seed)
    T = st.uniform_int(256, 1024, 4)
    ctx = st.uniform_int(128, 4096, 60)
    qlens = np.concatenate([T, np.ones(60, np.int64)])
    L = np.concatenate([T, ctx + 1])
    need = (L + 15) // 16
    pool = _pool_size(int(need.sum()))
    tables, _ = _tables_from_pool(need, pool, st)
    return _finish("C3", 32, 8, 128, 16, KV_BF16, layers, qlens, L, tables, pool, 0.5, seed=seed)


def c4_sum_context_stats(num_seqs: int = 256) -> tuple[float, float]:
    """Mean and standard deviation of C4's sum of post-append lengths: each
    L = round(exp(U(ln 256, ln 8192))) + 1, so E[e^U] = (b - a) / ln(b/a) and
    E[e^2U] = (b^2 - a^2) / (2 ln(b/a)) for the continuous draw."""
    a, b = 256.0, 8192.0
    r = math.log(b / a)
    m1 = (b - a) / r
    m2 = (b * b - a * a) / (2 * r)
    return num_seqs * (m1 + 1.0), math.sqrt(num_seqs * (m2 - m1 * m1))


def c4(seed: int = 4, layers: int = 32, num_seqs: int = 256, share_frac: float = 0.10) -> Workload:
    """Llama-3-8B large decode: B=256, context log-uniform [256,8192], bf16 KV;
    sequences are paired at random and the younger (higher index) of a pair
    maps its first k logical blocks onto the elder's physical blocks (forked
    prefixes, refcount 2) until about share_frac of the in-use physical blocks
    are shared."""
    bs = 16
    st = Stream(seed)
    ctx = st.log_uniform_int(256, 8192, num_seqs)              # 1. lengths
    L = ctx + 1
    need = (L + bs - 1) // bs
    pool = _pool_size(int(need.sum()))
    perm = st.permutation(pool).astype(np.int32)              # 2. pool permutation
    pairing = st.permutation(num_seqs)                        # 3. sharing pairs
    full = ctx // bs                       # full blocks before the append position
    share = np.zeros(num_seqs, np.int64)
    elder = np.full(num_seqs, -1, np.int64)
    # shared = share_frac * physical, physical = sum(need) - shared
    target = share_frac * int(need.sum()) / (1.0 + share_frac)
    shared = 0
    for i in range(0, num_seqs - 1, 2):
        if shared >= target:
            break
        a, b = sorted((int(pairing[i]), int(pairing[i + 1])))
        k = int(min(full[a], full[b], math.ceil(target - shared)))
        share[b], elder[b] = k, a
        shared += k
    tables, off = [None] * num_seqs, 0
    for b in range(num_seqs):
        own = int(need[b] - share[b])
        mine = perm[off:off + own]
        off += own
        if share[b] > 0:
            tables[b] = np.concatenate([tables[elder[b]][:share[b]], mine]).astype(np.int32)
        else:
            tables[b] = mine.copy()
    return _finish("C4", 32, 8, 128, bs, KV_BF16, layers, np.ones(num_seqs, np.int32), L, tables,
                   pool, 0.5, {"shared_blocks": int(shared)}, seed=seed)


def c5(seed: int = 5, layers: int = 80) -> Workload:
    """Llama-3-70B long context: 8 sequences at context 32768 + 24 at
    U[1024,8192], each +1 appended; 64q/8kv, d=128, bf16 KV, 80 layers."""
    st = Stream(seed)
    ctx = np.concatenate([np.full(8, 32768, np.int64), st.uniform_int(1024, 8192, 24)])
    L = ctx + 1
    need = (L + 15) // 16
    pool = _pool_size(int(need.sum()))
    tables, _ = _tables_from_pool(need, pool, st)
    return _finish("C5", 64, 8, 128, 16, KV_BF16, layers, np.ones(32, np.int32), L, tables, pool,
                   0.5, seed=seed)


CONFIGS = {"C1": c1, "C2": c2, "C3": c3, "C4": c4, "C5": c5}
