"""Test-side builders for paged layouts (numpy), independent of any scatter
kernel: the logical [Hkv, L, d] cache is written into [NB, Hkv, bs, d] slabs
through a permuted block table, and every slot the kernels must not read
(unused blocks, tail slots past L) is poisoned with 1e30 — the same layout the
reference's paged-decode tests build
(tests/unit/paged_decode_attention_kernel_test.cpp:98-155)."""
from __future__ import annotations

import numpy as np

POISON = np.float32(1e30)


def scale_for(d: int) -> float:
    # OptimizedModel::RunStack computes 1/sqrt(d) in double, then narrows
    # (src/model/optimized_model.cpp:473-474).
    return float(np.float32(1.0 / np.sqrt(np.float64(d))))


def normal(rng: np.random.Generator, shape, std=1.0) -> np.ndarray:
    return (rng.standard_normal(shape) * std).astype(np.float32)


def paged_layout(k: np.ndarray, v: np.ndarray, bs: int, extra_blocks: int = 1,
                 reverse: bool = True, rng: np.random.Generator | None = None):
    """k, v: [Hkv, L, d] -> (k_slab, v_slab [NB,Hkv,bs,d], table int32)."""
    hkv, L, d = k.shape
    need = (L + bs - 1) // bs
    nb = need + extra_blocks
    k_slab = np.full((nb, hkv, bs, d), POISON, np.float32)
    v_slab = np.full((nb, hkv, bs, d), POISON, np.float32)
    if rng is not None:
        table = rng.permutation(nb)[:need].astype(np.int32)
    elif reverse:
        table = (nb - 1 - np.arange(need)).astype(np.int32)
    else:
        table = np.arange(need, dtype=np.int32)
    for s in range(L):
        phys = table[s // bs]
        k_slab[phys, :, s % bs, :] = k[:, s, :]
        v_slab[phys, :, s % bs, :] = v[:, s, :]
    return k_slab, v_slab, table


def shared_pool_layout(ks, vs, bs: int, rng: np.random.Generator, slack: float = 1.25):
    """Several sequences' caches in one shared pool with shuffled block ids.
    ks[b], vs[b]: [Hkv, L_b, d]. Returns (k_slab, v_slab, tables)."""
    hkv, _, d = ks[0].shape
    needs = [(k.shape[1] + bs - 1) // bs for k in ks]
    nb = max(int(np.ceil(sum(needs) * slack)), sum(needs) + 1)
    perm = rng.permutation(nb).astype(np.int32)
    k_slab = np.full((nb, hkv, bs, d), POISON, np.float32)
    v_slab = np.full((nb, hkv, bs, d), POISON, np.float32)
    tables, off = [], 0
    for k, v, n in zip(ks, vs, needs):
        t = perm[off:off + n].copy()
        off += n
        L = k.shape[1]
        for s in range(L):
            k_slab[t[s // bs], :, s % bs, :] = k[:, s, :]
            v_slab[t[s // bs], :, s % bs, :] = v[:, s, :]
        tables.append(t)
    return k_slab, v_slab, tables


def brute_force_f64(q, k, v, heads, kv_heads, scale, past=None):
    """fp64 softmax attention: q [T,H,d], k/v [Hkv,L,d], causal with P = L - T."""
    T = q.shape[0]
    L = k.shape[1]
    P = L - T if past is None else past
    g = heads // kv_heads
    out = np.zeros(q.shape, np.float64)
    for t in range(T):
        for h in range(heads):
            hk = h // g
            kk = k[hk, :P + t + 1].astype(np.float64)
            s = kk @ q[t, h].astype(np.float64) * np.float64(scale)
            s -= s.max()
            p = np.exp(s)
            p /= p.sum()
            out[t, h] = p @ v[hk, :P + t + 1].astype(np.float64)
    return out


def max_rel(a, b) -> float:
    """max|a-b| / max(|b|, 1e-6 * max|b|) — the parity report's relative error."""
    a = np.asarray(a, np.float64)
    b = np.asarray(b, np.float64)
    floor = 1e-6 * np.abs(b).max() if b.size else 0.0
    den = np.maximum(np.abs(b), floor)
    den = np.where(den == 0, 1.0, den)
    return float((np.abs(a - b) / den).max()) if a.size else 0.0


def allclose_ref(a, b, rtol, atol) -> bool:
    """The reference criterion |a-b| <= atol + rtol*|b| (src/tensor/ops.h:207)."""
    a = np.asarray(a, np.float64)
    b = np.asarray(b, np.float64)
    return bool(np.all(np.abs(a - b) <= atol + rtol * np.abs(b)))
