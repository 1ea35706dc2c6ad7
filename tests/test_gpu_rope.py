"""GPU parity of the fused RoPE + KV append (ehip_step_rope_kv_append).

The reference rotates q and k with kernels::RopeApplyF32
(src/model/optimized_model.cpp:284-291) and then appends k and v
(PagedKvCache::append, src/kvcache/paged_cache.cpp:62-123). The oracle does
the same on the CPU: orc.rope_apply with the AVX2 row kernel's form (isa 1,
pinned bit for bit against the reference build in test_oracle.py), then
orc.kv_scatter. The bar is bit-exact: q, every slab word (fp32, or bf16 after
round-to-nearest-even), and the untouched source rows.
"""
import numpy as np
import pytest

from gpu_util import new_rows, rel_norm, seeded_pool

pytestmark = pytest.mark.gpu


def ragged_workload(ehip_mod, H, Hkv, d, bs, kv_dtype, seed):
    """Decode rows and causal chunks (fresh and continuation) of one step over
    a shuffled pool."""
    from ehip import workloads
    rng = np.random.default_rng(seed)
    qlens = [1, 37, 1, 5, 130, 1]
    prior = [700, 0, 3, 64, 33, 2047]
    L = [p + t for p, t in zip(prior, qlens)]
    need = [(x + bs - 1) // bs for x in L]
    pool = int(sum(need) * 1.3) + 2
    tables, _ = workloads._tables_from_pool(np.array(need), pool, rng)
    return workloads._finish("rope", H, Hkv, d, bs, kv_dtype, 1, qlens, L, tables, pool, 1.0)


def positions_of(w):
    return np.concatenate([np.arange(int(L) - int(T), int(L)) for T, L in
                           zip(w.query_lens, w.context_lens)]).astype(np.int32)


@pytest.mark.parametrize("bf16", [False, True])
@pytest.mark.parametrize("H,Hkv,d,bs", [(14, 2, 64, 16), (32, 8, 128, 16), (6, 3, 72, 32),
                                        (4, 2, 10, 8)])
def test_step_rope_kv_append_bit_exact(gctx, ehip_mod, orc, bf16, H, Hkv, d, bs):
    """d = 64 and 128: whole 8-pair groups; 72: groups plus the 4-pair tail
    (vector path); 10: the one-pair-per-thread path."""
    kv_dtype = ehip_mod.KV_BF16 if bf16 else ehip_mod.KV_F32
    w = ragged_workload(ehip_mod, H, Hkv, d, bs, kv_dtype, seed=d + H)
    g = ehip_mod.geometry(H, Hkv, d, bs, kv_dtype, w.pool_blocks, w.scale)
    st = ehip_mod.StepArrays(w.query_lens, w.context_lens, w.tables, w.slot_mapping)
    assert gctx.step_upload(g, st) == 0, gctx.last_error()

    kpool, vpool = seeded_pool(orc, w, 71)
    kn, vn, q = new_rows(orc, w, 72)
    n_pos = int(w.context_lens.max()) + 5
    cos, sin = orc.rope_tables(d, n_pos)
    if bf16:
        kb, vb = orc.to_bf16_bits(kpool), orc.to_bf16_bits(vpool)
        dk, dv = gctx.to_device(kb), gctx.to_device(vb)
    else:
        dk, dv = gctx.to_device(kpool), gctx.to_device(vpool)
    dq, dkn, dvn = gctx.to_device(q), gctx.to_device(kn), gctx.to_device(vn)
    dcos, dsin = gctx.to_device(cos), gctx.to_device(sin)
    assert gctx.step_rope_kv_append(dq, dkn, dvn, dcos, dsin, n_pos, dk, dv) == 0, \
        gctx.last_error()
    gctx.sync()  # raises on a device range flag

    pos = positions_of(w)
    q_ref = orc.rope_apply(q, pos, cos, sin, isa=1)
    k_rot = orc.rope_apply(kn, pos, cos, sin, isa=1)
    assert np.array_equal(dq.download(np.float32, q.shape).view(np.uint32),
                          q_ref.view(np.uint32))
    assert np.array_equal(dkn.download(np.float32, kn.shape).view(np.uint32),
                          kn.view(np.uint32)), "source K rows must stay unrotated"
    if bf16:
        orc.kv_scatter(k_rot, vn, w.slot_mapping, Hkv, d, bs, kb, vb)
        assert np.array_equal(dk.download(np.uint16, kb.shape), kb)
        assert np.array_equal(dv.download(np.uint16, vb.shape), vb)
    else:
        orc.kv_scatter(k_rot, vn, w.slot_mapping, Hkv, d, bs, kpool, vpool)
        assert np.array_equal(dk.download(np.float32, kpool.shape).view(np.uint32),
                              kpool.view(np.uint32))
        assert np.array_equal(dv.download(np.float32, vpool.shape).view(np.uint32),
                              vpool.view(np.uint32))
    for b in (dk, dv, dq, dkn, dvn, dcos, dsin):
        b.free()


@pytest.mark.parametrize("bf16", [False, True])
def test_step_rope_kv_append_then_attention(gctx, ehip_mod, orc, bf16):
    """The layer order of the reference (RoPE, append, attention) on one step:
    attention over the rotated cache against the oracle's varlen reference
    over the same (bf16-rounded, for a bf16 pool) cache."""
    H, Hkv, d, bs = 32, 8, 128, 16
    kv_dtype = ehip_mod.KV_BF16 if bf16 else ehip_mod.KV_F32
    w = ragged_workload(ehip_mod, H, Hkv, d, bs, kv_dtype, seed=5)
    g = ehip_mod.geometry(H, Hkv, d, bs, kv_dtype, w.pool_blocks, w.scale)
    st = ehip_mod.StepArrays(w.query_lens, w.context_lens, w.tables, w.slot_mapping)
    assert gctx.step_upload(g, st) == 0, gctx.last_error()
    kpool, vpool = seeded_pool(orc, w, 81)
    kn, vn, q = new_rows(orc, w, 82)
    n_pos = int(w.context_lens.max())
    cos, sin = orc.rope_tables(d, n_pos)
    if bf16:
        kb, vb = orc.to_bf16_bits(kpool), orc.to_bf16_bits(vpool)
        dk, dv = gctx.to_device(kb), gctx.to_device(vb)
    else:
        dk, dv = gctx.to_device(kpool), gctx.to_device(vpool)
    dq, dkn, dvn = gctx.to_device(q), gctx.to_device(kn), gctx.to_device(vn)
    dcos, dsin = gctx.to_device(cos), gctx.to_device(sin)
    out = gctx.alloc(q.nbytes)
    assert gctx.step_rope_kv_append(dq, dkn, dvn, dcos, dsin, n_pos, dk, dv) == 0
    assert gctx.step_attention(dq, dk, dv, out) == 0, gctx.last_error()
    gctx.sync()
    got = out.download(np.float32, q.shape)

    pos = positions_of(w)
    q_ref = orc.rope_apply(q, pos, cos, sin, isa=1)
    k_rot = orc.rope_apply(kn, pos, cos, sin, isa=1)
    if bf16:
        orc.kv_scatter(k_rot, vn, w.slot_mapping, Hkv, d, bs, kb, vb)
        kpool, vpool = orc.bf16_bits_to_f32(kb), orc.bf16_bits_to_f32(vb)
    else:
        orc.kv_scatter(k_rot, vn, w.slot_mapping, Hkv, d, bs, kpool, vpool)
    cu = np.concatenate([[0], np.cumsum(w.query_lens)]).astype(np.int32)
    kseq = [orc.paged_to_contig(kpool, t, int(L), Hkv, d, bs) for t, L in
            zip(w.tables, w.context_lens)]
    vseq = [orc.paged_to_contig(vpool, t, int(L), Hkv, d, bs) for t, L in
            zip(w.tables, w.context_lens)]
    ref = orc.prefill_varlen(q_ref, cu, kseq, vseq, H, Hkv, d, w.scale, isa=1)
    # Decode rows and fp32-pool chunks run in fp32 (1e-4 relative); chunk
    # rows over a bf16 pool run on the MFMA prefill kernel, which also rounds
    # Q and the probabilities to bf16 (1e-2 relative).
    dec = np.repeat(w.query_lens, w.query_lens) == 1
    assert rel_norm(got[dec], ref[dec]) <= 1e-4
    assert rel_norm(got[~dec], ref[~dec]) <= (1e-2 if bf16 else 1e-4)
    for b in (dk, dv, dq, dkn, dvn, dcos, dsin, out):
        b.free()


def test_step_rope_kv_append_rejects_positions_past_the_tables(gctx, ehip_mod, orc):
    """A position at or past table_positions is an argument error (host-side,
    nothing launched), as the reference rejects positions past
    max_position_embeddings (src/model/optimized_model.cpp:529-535)."""
    H, Hkv, d, bs = 4, 2, 64, 16
    w = ragged_workload(ehip_mod, H, Hkv, d, bs, ehip_mod.KV_F32, seed=9)
    g = ehip_mod.geometry(H, Hkv, d, bs, ehip_mod.KV_F32, w.pool_blocks, w.scale)
    st = ehip_mod.StepArrays(w.query_lens, w.context_lens, w.tables, w.slot_mapping)
    assert gctx.step_upload(g, st) == 0
    n_pos = int(w.context_lens.max()) - 1
    kn, vn, q = new_rows(orc, w, 3)
    cos, sin = orc.rope_tables(d, n_pos)
    kpool, vpool = seeded_pool(orc, w, 4)
    bufs = [gctx.to_device(x) for x in (q, kn, vn, cos, sin, kpool, vpool)]
    assert gctx.step_rope_kv_append(*bufs[:5], n_pos, *bufs[5:]) == ehip_mod.INVALID_ARGUMENT
    assert "RoPE tables" in gctx.last_error()
    before = bufs[0].download(np.float32, q.shape)
    assert np.array_equal(before.view(np.uint32), q.view(np.uint32))
    for b in bufs:
        b.free()
