"""ehip_step_append_attention: the step's KV append and attention in one
launch for all-decode steps on the matrix-core decode kernel (bf16 slabs, and
fp32 slabs with head_dim 64; the item that ends at a row's last key stores the
row's new K/V and uses them directly), and the two-launch order for every
other step. Either way the slabs must equal the oracle's append bit for bit
and the outputs meet the decode bar against the reference on the same cache
(bf16-rounded for bf16 slabs; 1e-4 relative per output vector, the reference
allclose); fused and separate launches agree to within that bar."""
import numpy as np
import pytest

from gpu_util import max_abs, new_rows, rel_norm, seeded_pool
from paged_util import allclose_ref

pytestmark = pytest.mark.gpu


def _workload(ehip_mod, H, Hkv, d, bs, lens, seed, dtype=None, qlens=None):
    from ehip import workloads
    rng = np.random.default_rng(seed)
    lens = np.asarray(lens, np.int64)
    qlens = np.ones(len(lens), np.int32) if qlens is None else np.asarray(qlens, np.int32)
    need = (lens + bs - 1) // bs
    pool = int(np.ceil(1.25 * need.sum())) + 2
    tables, _ = workloads._tables_from_pool(need, pool, rng)
    return workloads._finish("fused", H, Hkv, d, bs, dtype if dtype is not None else ehip_mod.KV_BF16,
                             1, qlens, lens, tables, pool, 0.5)


def _run(gctx, ehip_mod, orc, w, fused, seed=13):
    H, Hkv, d, bs = w.heads, w.kv_heads, w.head_dim, w.block_size
    bf16 = w.kv_dtype == ehip_mod.KV_BF16
    g = ehip_mod.geometry(H, Hkv, d, bs, w.kv_dtype, w.pool_blocks, w.scale)
    st = ehip_mod.StepArrays(w.query_lens, w.context_lens, w.tables, w.slot_mapping)
    assert gctx.step_upload(g, st) == 0, gctx.last_error()
    kp, vp = seeded_pool(orc, w, seed)
    kn, vn, q = new_rows(orc, w, seed + 100)
    k0 = orc.to_bf16_bits(kp) if bf16 else kp
    v0 = orc.to_bf16_bits(vp) if bf16 else vp
    dk, dv = gctx.to_device(k0), gctx.to_device(v0)
    dq, dkn, dvn = gctx.to_device(q), gctx.to_device(kn), gctx.to_device(vn)
    out = gctx.alloc(q.nbytes)
    if fused:
        assert gctx.step_append_attention(dkn, dvn, dq, dk, dv, out) == 0, gctx.last_error()
    else:
        assert gctx.step_kv_append(dkn, dvn, dk, dv) == 0
        assert gctx.step_attention(dq, dk, dv, out) == 0
    gctx.sync()
    got = out.download(np.float32, q.shape)
    kd, vd = dk.download(k0.dtype, k0.shape), dv.download(v0.dtype, v0.shape)
    # Oracle: the append bit for bit, then the reference on that cache.
    orc.kv_scatter(kn, vn, w.slot_mapping, Hkv, d, bs, k0, v0)
    assert np.array_equal(kd.view(np.uint8), k0.view(np.uint8))
    assert np.array_equal(vd.view(np.uint8), v0.view(np.uint8))
    kr = orc.bf16_bits_to_f32(kd) if bf16 else kd
    vr = orc.bf16_bits_to_f32(vd) if bf16 else vd
    cu = np.concatenate([[0], np.cumsum(w.query_lens)]).astype(np.int32)
    kseq = [orc.paged_to_contig(kr, t, int(L), Hkv, d, bs) for t, L in zip(w.tables, w.context_lens)]
    vseq = [orc.paged_to_contig(vr, t, int(L), Hkv, d, bs) for t, L in zip(w.tables, w.context_lens)]
    ref = orc.prefill_varlen(q, cu, kseq, vseq, H, Hkv, d, w.scale, isa=orc.ISA_AVX2)
    for b in (dk, dv, dq, dkn, dvn, out):
        b.free()
    return got, ref


def _check(got, ref):
    assert rel_norm(got, ref) <= 1e-4, rel_norm(got, ref)
    assert allclose_ref(got, ref, 1e-4, 1e-5)


@pytest.mark.parametrize("H,Hkv,d,bs,kv", [(32, 8, 128, 16, "bf16"), (64, 8, 128, 16, "bf16"),
                                           (14, 2, 64, 16, "bf16"), (8, 8, 128, 32, "bf16"),
                                           (16, 2, 64, 64, "bf16"), (8, 1, 128, 16, "bf16"),
                                           (14, 2, 64, 16, "f32"), (8, 2, 64, 32, "f32"),
                                           (8, 8, 64, 16, "f32")])
def test_fused_append_decode_step(gctx, ehip_mod, orc, H, Hkv, d, bs, kv):
    """Ragged decode rows, including rows of one key (only the new token),
    rows whose last key range holds just the new key, and long split rows."""
    lens = [1, 2, 17, 33, 129, 1025, 1026, 2049, 4000, 64, 65, 8193]
    dtype = ehip_mod.KV_F32 if kv == "f32" else ehip_mod.KV_BF16
    w = _workload(ehip_mod, H, Hkv, d, bs, lens, seed=H + d + bs, dtype=dtype)
    fused, ref = _run(gctx, ehip_mod, orc, w, fused=True)
    _check(fused, ref)
    separate, _ = _run(gctx, ehip_mod, orc, w, fused=False)
    assert rel_norm(fused, separate) <= 1e-5


@pytest.mark.parametrize("fused", [True, False])
@pytest.mark.parametrize("H,Hkv,d,bs", [(14, 2, 64, 16), (8, 8, 64, 16), (8, 2, 64, 32),
                                        (16, 2, 64, 64), (8, 1, 64, 16)])
def test_fp32_items_over_four_wavefronts(gctx, ehip_mod, orc, tctx, H, Hkv, d, bs, fused):
    """Small fp32 steps (256 or more items, every one in one round of
    4-wavefront workgroups) spread each item's tiles over the workgroup's four
    wavefronts, which combine their softmax states in LDS. Rows of one key,
    items shorter than four tiles (wavefronts with no tiles), a last range
    holding only the new key, long split rows; fused append and two launches:
    slabs bit-exact and outputs to the decode bar against the oracle, and
    within the fp32 bar of one wavefront per item (EHIP_DECODE_SPLIT4=0)."""
    base = [1, 2, 17, 33, 63, 64, 65, 97, 129, 300, 1025, 2049]
    # Rows repeated until the plan has 256..480 items: the 4-wavefront
    # launch takes steps of at least 256 items that fit one round (2 such
    # workgroups per CU).
    for reps in range(1, 16):
        w = _workload(ehip_mod, H, Hkv, d, bs, base * reps, seed=H + d + bs + 7,
                      dtype=ehip_mod.KV_F32)
        items = ehip_mod.plan_counts(
            ehip_mod.geometry(H, Hkv, d, bs, w.kv_dtype, w.pool_blocks, w.scale),
            ehip_mod.StepArrays(w.query_lens, w.context_lens, w.tables, w.slot_mapping))[2]
        if items >= 256:
            break
    assert 256 <= items <= 480, items
    got, ref = _run(gctx, ehip_mod, orc, w, fused=fused)
    _check(got, ref)
    one, _ = _run(tctx(EHIP_DECODE_SPLIT4="0"), ehip_mod, orc, w, fused=fused)
    _check(one, ref)
    assert rel_norm(got, one) <= 1e-5


@pytest.mark.parametrize("slots", [None, "5", "64"])
def test_fused_append_with_joint_items(gctx, ehip_mod, orc, tctx, slots):
    """The C4 shape with pair-shared prefixes (joint items never cover a row's
    last key: only the rows' own items append), on a grid covering every item
    and on 5 or 64 persistent wavefronts that take the items, joint and
    appending ones alike, by ticket: bit-identical to the full grid."""
    from ehip import workloads
    w = workloads.c4(num_seqs=24, share_frac=0.3)
    rc, rows, items, partials, split, joint, shared = ehip_mod.plan_counts(
        ehip_mod.geometry(w.heads, w.kv_heads, w.head_dim, w.block_size, w.kv_dtype,
                          w.pool_blocks, w.scale),
        ehip_mod.StepArrays(w.query_lens, w.context_lens, w.tables, w.slot_mapping), joint=True)
    assert rc == 0 and joint > 0
    fused, ref = _run(gctx, ehip_mod, orc, w, fused=True, seed=41)
    _check(fused, ref)
    if slots is not None:
        assert int(slots) < items
        queued, _ = _run(tctx(EHIP_DECODE_SLOTS=slots), ehip_mod, orc, w, fused=True, seed=41)
        assert np.array_equal(queued.view(np.uint32), fused.view(np.uint32))


@pytest.mark.parametrize("slots", ["7", "64"])
@pytest.mark.parametrize("H,Hkv,d,bs,kv", [(32, 8, 128, 16, "bf16"), (64, 8, 128, 16, "bf16"),
                                           (16, 2, 64, 64, "bf16"), (14, 2, 64, 16, "f32")])
def test_fused_append_items_taken_by_ticket(gctx, ehip_mod, orc, tctx, H, Hkv, d, bs, kv, slots):
    """The fused launch with the decode grid capped below the plan's items, so
    its persistent wavefronts take items (the appending ones among them) from
    their sub-queues by ticket, as at the benched sizes (C4: 5,640 items, C5:
    2,960, on 2,048 resident wavefronts). Slabs bit-exact against the oracle's
    append, outputs to the decode bar, and bit-identical to the launch whose
    grid covers every item (an item computes the same sums whichever
    wavefront takes it)."""
    lens = [1, 2, 17, 33, 129, 1025, 1026, 2049, 4000, 64, 65, 8193]
    dtype = ehip_mod.KV_F32 if kv == "f32" else ehip_mod.KV_BF16
    w = _workload(ehip_mod, H, Hkv, d, bs, lens, seed=H + d + bs + 1, dtype=dtype)
    full, ref = _run(gctx, ehip_mod, orc, w, fused=True)
    ctx = tctx(EHIP_DECODE_SLOTS=slots)
    queued, ref_q = _run(ctx, ehip_mod, orc, w, fused=True)
    _, items, _ = ctx.step_info()
    assert int(slots) < items, items
    _check(queued, ref_q)
    assert np.array_equal(queued.view(np.uint32), full.view(np.uint32))


@pytest.mark.parametrize("queues", ["8", "32"])
@pytest.mark.parametrize("spread", ["1", "0"])
@pytest.mark.parametrize("H,Hkv,d,bs", [(32, 8, 128, 16), (64, 8, 128, 16)])
def test_fused_append_sub_queues_across_xcds(gctx, ehip_mod, orc, tctx, H, Hkv, d, bs, spread,
                                             queues):
    """A capped grid of 300 wavefronts (at least 8 per sub-queue) over 8 (the
    default) or 32 sub-queues: with the spread mapping each sub-queue is drawn
    by wavefronts b with b / 8 = q (mod the count), one from every XCD, instead
    of b = q (mod the count). Every item is still served exactly once: the
    same slabs and bit-identical outputs to the launch whose grid covers every
    item."""
    lens = [1, 2, 17, 33, 129, 1025, 1026, 2049, 4000, 64, 65, 8193]
    w = _workload(ehip_mod, H, Hkv, d, bs, lens, seed=H + d + bs + 2)
    full, ref = _run(gctx, ehip_mod, orc, w, fused=True)
    ctx = tctx(EHIP_DECODE_SLOTS="300", EHIP_DECODE_QSPREAD=spread, EHIP_DECODE_QUEUES=queues)
    queued, ref_q = _run(ctx, ehip_mod, orc, w, fused=True)
    _, items, _ = ctx.step_info()
    assert 300 < items, items
    _check(queued, ref_q)
    assert np.array_equal(queued.view(np.uint32), full.view(np.uint32))


@pytest.mark.parametrize("case", ["fp32", "chunk", "valu"])
def test_append_attention_falls_back_to_two_launches(gctx, ehip_mod, orc, case, tctx):
    """fp32 slabs of head_dim 128 (the fp32 matrix-core kernel covers 64), a
    step with a prefill chunk, and the VALU decode kernel take the append
    launch then the attention launch, with the same results."""
    if case == "fp32":
        w = _workload(ehip_mod, 16, 2, 128, 16, [513, 17, 1], seed=5, dtype=ehip_mod.KV_F32)
    elif case == "chunk":
        w = _workload(ehip_mod, 32, 8, 128, 16, [300, 40, 1000], seed=6, qlens=[1, 20, 1])
    else:
        gctx = tctx(EHIP_DECODE_KERNEL="valu")
        w = _workload(ehip_mod, 32, 8, 128, 16, [300, 40, 1000], seed=7)
    got, ref = _run(gctx, ehip_mod, orc, w, fused=True)
    rows = np.repeat(w.query_lens, w.query_lens) == 1
    _check(got[rows], ref[rows])
    if (~rows).any():  # chunk rows: bf16 Q and P on the matrix cores
        assert rel_norm(got[~rows], ref[~rows]) <= 1e-2
