"""GPU parity at the benchmark configurations' full sizes: one layer of the
benched C3, C4 and C5 steps exactly as drawn (the configs' seeded structure
and the reference fill_normal values of layer 0), C5's 4096-token
re-prefill chunk on sampled rows, and a long-context chunk whose prefill
blocks hit the cap on key splits.

Bars: the append bit-exact (whole slabs); decode rows within 1e-4 relative
(per output vector) and inside the reference allclose (rtol 1e-4, atol 1e-5)
against the reference run on the same bf16-rounded K/V; prefill-chunk rows
(bf16 Q and P on the matrix cores) within 1e-2 relative of it; every row
within 2e-2 absolute of the reference on the original fp32 K/V.
"""
import numpy as np
import pytest

from gpu_util import max_abs, rel_norm
from paged_util import allclose_ref

pytestmark = pytest.mark.gpu

FP32_REL = 1e-4
PREFILL_REL = 1e-2
BF16_ABS = 2e-2


def log(msg):
    print(f"[fullsize] {msg}", flush=True)


def run_layer(gctx, ehip_mod, w, q, k32, v32, kn, vn, fused=False):
    """Upload the bf16 slabs and the step's rows, append + attend one layer on
    the GPU; return the output and the post-append slabs. fused: through
    ehip_step_append_attention (the benched call: for an all-decode step one
    launch of the persistent decode kernel with the append folded in, its
    wavefronts taking items by ticket once the plan has more items than
    resident wavefronts), else the append launch, then the attention call."""
    from ehip import workloads
    g = ehip_mod.geometry(w.heads, w.kv_heads, w.head_dim, w.block_size, w.kv_dtype,
                          w.pool_blocks, w.scale)
    st = ehip_mod.StepArrays(w.query_lens, w.context_lens, w.tables, w.slot_mapping)
    assert gctx.step_upload(g, st) == 0, gctx.last_error()
    rows, items, partials = gctx.step_info()
    log(f"{'fused' if fused else 'two launches'}: rows={rows} work items={items} "
        f"partials={partials}")
    dk = gctx.to_device(workloads.to_bf16_bits(k32))
    dv = gctx.to_device(workloads.to_bf16_bits(v32))
    dq, dkn, dvn = gctx.to_device(q), gctx.to_device(kn), gctx.to_device(vn)
    out = gctx.alloc(q.nbytes)
    if fused:
        assert gctx.step_append_attention(dkn, dvn, dq, dk, dv, out) == 0, gctx.last_error()
    else:
        assert gctx.step_kv_append(dkn, dvn, dk, dv) == 0, gctx.last_error()
        assert gctx.step_attention(dq, dk, dv, out) == 0, gctx.last_error()
    gctx.sync()
    got = out.download(np.float32, q.shape)
    shape = k32.shape
    kd, vd = dk.download(np.uint16, shape), dv.download(np.uint16, shape)
    for b in (dk, dv, dq, dkn, dvn, out):
        b.free()
    return got, kd, vd


def references(orc, w, q, k32, v32, kn, vn, kd, vd):
    """The oracle's append on the bf16-rounded pool (checked bit for bit
    against the GPU slabs), then the reference attention on the rounded and on
    the fp32 post-append caches."""
    Hkv, d, bs = w.kv_heads, w.head_dim, w.block_size
    kb, vb = orc.to_bf16_bits(k32), orc.to_bf16_bits(v32)
    orc.kv_scatter(kn, vn, w.slot_mapping, Hkv, d, bs, kb, vb)
    assert np.array_equal(kb, kd), "K slab differs from the oracle's append"
    assert np.array_equal(vb, vd), "V slab differs from the oracle's append"
    del kb, vb
    kr, vr = orc.bf16_bits_to_f32(kd), orc.bf16_bits_to_f32(vd)
    ref_r = attention(orc, w, q, kr, vr)
    del kr, vr
    orc.kv_scatter(kn, vn, w.slot_mapping, Hkv, d, bs, k32, v32)
    ref32 = attention(orc, w, q, k32, v32)
    return ref_r, ref32


def attention(orc, w, q, k, v):
    H, Hkv, d, bs = w.heads, w.kv_heads, w.head_dim, w.block_size
    lens = [int(x) for x in w.context_lens]
    if (w.query_lens == 1).all():
        return orc.paged_decode_batched(q, k, v, w.tables, lens, H, Hkv, d, bs, w.scale,
                                        isa=orc.ISA_AVX2)
    cu = np.concatenate([[0], np.cumsum(w.query_lens)]).astype(np.int32)
    kseq = [orc.paged_to_contig(k, t, L, Hkv, d, bs) for t, L in zip(w.tables, lens)]
    vseq = [orc.paged_to_contig(v, t, L, Hkv, d, bs) for t, L in zip(w.tables, lens)]
    return orc.prefill_varlen(q, cu, kseq, vseq, H, Hkv, d, w.scale, isa=orc.ISA_AVX2)


def check(w, got, ref_r, ref32):
    rows = np.repeat(w.query_lens, w.query_lens)
    dec = rows == 1
    if dec.any():
        r = rel_norm(got[dec], ref_r[dec])
        log(f"decode rows: rel {r:.3e}")
        assert r <= FP32_REL, r
        assert allclose_ref(got[dec], ref_r[dec], 1e-4, 1e-5)
    if (~dec).any():
        r = rel_norm(got[~dec], ref_r[~dec])
        log(f"chunk rows: rel {r:.3e}")
        assert r <= PREFILL_REL, r
    a = max_abs(got, ref32)
    log(f"all rows vs fp32: max_abs {a:.3e}")
    assert a <= BF16_ABS, a


@pytest.mark.parametrize("config", ["C4", "C5", "C3"])
def test_benched_layer_at_full_size(gctx, ehip_mod, orc, config):
    """Layer 0 of the config's benched step as drawn: C4 (256 sequences,
    sum L ~ 609k, pair-shared prefixes), C5 (8 x 32769 + 24 rows, 64q/8kv),
    C3 (4 causal chunks + 60 decodes), each through the two-launch path and
    through the fused call the bench times. C4 (5,640 work items) and C5
    (2,960) have more items than the 2,048 resident decode wavefronts, so the
    fused kernel runs with its item queue active; C3's mixed step takes the
    two launches either way. Both runs leave the same slabs (the oracle's
    append, bit for bit); each run's outputs meet the bars."""
    from ehip import workloads
    w = workloads.CONFIGS[config]()
    log(f"{config}: B={w.num_seqs} rows={w.rows} sumL={int(w.context_lens.sum())} "
        f"pool={w.pool_blocks}")
    k32, v32 = w.pool(0)
    q = w.q(0)
    kn, vn = w.new_kv(0)
    got, kd, vd = run_layer(gctx, ehip_mod, w, q, k32, v32, kn, vn)
    got_f, kd_f, vd_f = run_layer(gctx, ehip_mod, w, q, k32, v32, kn, vn, fused=True)
    assert np.array_equal(kd_f, kd) and np.array_equal(vd_f, vd), \
        "the fused append left different slabs"
    del kd_f, vd_f
    ref_r, ref32 = references(orc, w, q, k32, v32, kn, vn, kd, vd)
    log("two launches:")
    check(w, got, ref_r, ref32)
    log("fused:")
    check(w, got_f, ref_r, ref32)


@pytest.mark.parametrize("heads", [64, 32])
def test_c5_reprefill_chunk_sampled_rows(gctx, ehip_mod, orc, heads):
    """C5's preempt-and-recompute event: an evicted sequence re-prefilled as
    one 4096-row causal chunk (P = 0) with its K/V appended in the same step.
    Row t of the chunk equals a single-row decode over keys [0, t] of the
    post-append cache: checked on the first and last rows and every 64th.
    Both launches have at least 4 prefill workgroups per CU (2048 for g = 8,
    1024 for g = 4 on 256 CUs), so they run the three-workgroups-per-CU
    instances of the prefill kernel."""
    from ehip import workloads
    c5 = workloads.c5()
    T, bs = 4096, c5.block_size
    table = np.asarray(c5.tables[0][:T // bs], np.int32)
    w = workloads._finish("C5-reprefill", heads, c5.kv_heads, c5.head_dim, bs, c5.kv_dtype,
                          1, [T], [T], [table], c5.pool_blocks, c5.qkv_std, seed=c5.seed)
    H, Hkv, d = w.heads, w.kv_heads, w.head_dim
    k32, v32 = c5.pool(0)
    q = workloads.fill_normal(T * H * d, 0.0, w.qkv_std, 91).reshape(T, H, d)
    kn = workloads.fill_normal(T * Hkv * d, 0.0, w.qkv_std, 92).reshape(T, Hkv, d)
    vn = workloads.fill_normal(T * Hkv * d, 0.0, w.qkv_std, 93).reshape(T, Hkv, d)
    got, kd, vd = run_layer(gctx, ehip_mod, w, q, k32, v32, kn, vn)
    kb, vb = orc.to_bf16_bits(k32), orc.to_bf16_bits(v32)
    orc.kv_scatter(kn, vn, w.slot_mapping, Hkv, d, bs, kb, vb)
    assert np.array_equal(kb, kd) and np.array_equal(vb, vd)
    del kb, vb
    kr, vr = orc.bf16_bits_to_f32(kd), orc.bf16_bits_to_f32(vd)
    orc.kv_scatter(kn, vn, w.slot_mapping, Hkv, d, bs, k32, v32)
    rows = sorted(set([0, T - 1] + list(range(63, T, 64))))
    worst_r, worst_a = 0.0, 0.0
    for t in rows:
        ref_r = orc.paged_decode(q[t], kr, vr, table, t + 1, H, Hkv, d, bs, w.scale,
                                 isa=orc.ISA_AVX2)
        ref32 = orc.paged_decode(q[t], k32, v32, table, t + 1, H, Hkv, d, bs, w.scale,
                                 isa=orc.ISA_AVX2)
        worst_r = max(worst_r, rel_norm(got[t], ref_r))
        worst_a = max(worst_a, max_abs(got[t], ref32))
    log(f"re-prefill {len(rows)} sampled rows: rel {worst_r:.3e}, max_abs vs fp32 {worst_a:.3e}")
    assert worst_r <= PREFILL_REL, worst_r
    assert worst_a <= BF16_ABS, worst_a


@pytest.mark.parametrize("H,Hkv,P", [(8, 2, 20000), (16, 2, 40000)])
def test_long_context_chunk_at_split_cap(gctx, ehip_mod, orc, H, Hkv, P):
    """A 16-row chunk after a long cached prefix with few kv heads: the
    prefill blocks are cut at the 64-split cap into fewer, longer pieces
    (626 tiles into 63 pieces at P = 20000), so every split slot the merge
    reads must have been written. Two decode rows ride along."""
    from ehip import workloads
    rng = np.random.default_rng(P + H)
    T, bs, d = 16, 16, 128
    qlens = [T, 1, 1]
    L = [P + T, 700, 3001]
    need = [(x + bs - 1) // bs for x in L]
    pool = int(sum(need) * 1.25) + 2
    tables, _ = workloads._tables_from_pool(np.array(need), pool, rng)
    w = workloads._finish("long-chunk", H, Hkv, d, bs, ehip_mod.KV_BF16, 1, qlens, L, tables,
                          pool, 0.5, seed=P)
    n = pool * Hkv * bs * d
    k32 = workloads.fill_normal(n, 0.0, 0.5, 1).reshape(pool, Hkv, bs, d)
    v32 = workloads.fill_normal(n, 0.0, 0.5, 2).reshape(pool, Hkv, bs, d)
    q = workloads.fill_normal(w.rows * H * d, 0.0, 0.5, 3).reshape(w.rows, H, d)
    kn = workloads.fill_normal(w.rows * Hkv * d, 0.0, 0.5, 4).reshape(w.rows, Hkv, d)
    vn = workloads.fill_normal(w.rows * Hkv * d, 0.0, 0.5, 5).reshape(w.rows, Hkv, d)
    got, kd, vd = run_layer(gctx, ehip_mod, w, q, k32, v32, kn, vn)
    assert gctx.step_info()[2] > 0  # key splits in the plan
    ref_r, ref32 = references(orc, w, q, k32, v32, kn, vn, kd, vd)
    check(w, got, ref_r, ref32)
