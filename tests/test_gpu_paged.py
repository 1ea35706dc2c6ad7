"""GPU parity: the HIP path (through the C ABI) against the CPU oracle.

Bars (from the path's contract): indexing and append bit-exact; fp32 outputs
within 1e-4 relative error of the scalar reference attention (per output
vector, max|a-b| / max|b|) and inside the reference's own allclose
(rtol 1e-4, atol 1e-5, src/tensor/ops.h:207); bf16-KV outputs within 2e-2
absolute of the fp32 reference, and within 1e-4 relative of the reference run
on the same bf16-rounded K/V.
"""
import os

import numpy as np
import pytest

from gpu_util import max_abs, new_rows, rel_norm, seeded_pool
from paged_util import POISON, allclose_ref, brute_force_f64, normal, paged_layout, scale_for

pytestmark = pytest.mark.gpu

FP32_REL = 1e-4
BF16_ABS = 2e-2


def check_fp32(out, ref):
    assert rel_norm(out, ref) <= FP32_REL, rel_norm(out, ref)
    assert allclose_ref(out, ref, 1e-4, 1e-5)


# ------------------------------------------------------------------ append
@pytest.mark.parametrize("bf16", [False, True])
@pytest.mark.parametrize("d,hkv,bs", [(64, 2, 16), (128, 8, 16), (16, 2, 8), (18, 3, 32),
                                      (24, 1, 64)])
def test_kv_scatter_bit_exact(gctx, orc, bf16, d, hkv, bs):
    rng = np.random.default_rng(d * 7 + hkv + bs)
    nb, T = 40, 97
    slots = rng.permutation(nb * bs)[:T].astype(np.int64)  # boundary-straddling, non-monotone
    src_k = normal(rng, (T, hkv, d), 3.0)
    src_v = normal(rng, (T, hkv, d), 3.0)
    dt = np.uint16 if bf16 else np.float32
    k_ref = np.zeros((nb, hkv, bs, d), dt)
    v_ref = np.zeros((nb, hkv, bs, d), dt)
    orc.kv_scatter(src_k, src_v, slots, hkv, d, bs, k_ref, v_ref)
    dk, dv = gctx.alloc(k_ref.nbytes), gctx.alloc(v_ref.nbytes)
    rc = gctx.kv_scatter(gctx.to_device(src_k), gctx.to_device(src_v), gctx.to_device(slots),
                         T, hkv, d, bs, nb, dk, dv, bf16)
    assert rc == 0, gctx.last_error()
    gctx.sync()
    assert np.array_equal(dk.download(dt, k_ref.shape).view(np.uint8), k_ref.view(np.uint8))
    assert np.array_equal(dv.download(dt, v_ref.shape).view(np.uint8), v_ref.view(np.uint8))


def test_kv_scatter_bf16_special_values(gctx, orc):
    # RNE ties, carry into inf, NaN payload quieting, denormals, signed zero.
    bits = np.array([0x3F808000, 0x3F818000, 0x7F7FFFFF, 0x7F800001, 0xFFC00000, 0x7F810000,
                     0x00000001, 0x80000000, 0x7F800000, 0xFF800000, 0x007FFFFF, 0x3F7FFFFF,
                     0x40490FDB, 0xC0490FDB, 0x00008000, 0x00018000], np.uint32)
    src = bits.view(np.float32).reshape(1, 1, 16)
    slots = np.array([5], np.int64)
    ref_k = np.zeros((2, 1, 8, 16), np.uint16)
    ref_v = np.zeros((2, 1, 8, 16), np.uint16)
    orc.kv_scatter(src, src, slots, 1, 16, 8, ref_k, ref_v)
    dk, dv = gctx.alloc(ref_k.nbytes), gctx.alloc(ref_v.nbytes)
    s = gctx.to_device(src)
    assert gctx.kv_scatter(s, s, gctx.to_device(slots), 1, 1, 16, 8, 2, dk, dv, True) == 0
    gctx.sync()
    assert np.array_equal(dk.download(np.uint16, ref_k.shape), ref_k)


def test_kv_scatter_rejects_out_of_range_slot(gctx, ehip_mod):
    # The kernel bounds every slot before writing; the range error surfaces at sync.
    src = np.ones((2, 1, 16), np.float32)
    slots = np.array([3, 2 * 8], np.int64)  # the second slot is one past a 2-block slab
    dk, dv = gctx.alloc(2 * 8 * 16 * 4), gctx.alloc(2 * 8 * 16 * 4)
    s = gctx.to_device(src)
    assert gctx.kv_scatter(s, s, gctx.to_device(slots), 2, 1, 16, 8, 2, dk, dv, False) == 0
    with pytest.raises(ehip_mod.EhipError) as e:
        gctx.sync()
    assert e.value.code == ehip_mod.INVALID_ARGUMENT
    gctx.sync()  # the flag was cleared
    got = dk.download(np.float32, (2, 1, 8, 16))
    assert np.all(got[0, 0, 3] == 1) and np.count_nonzero(got) == 16


def test_kv_gather_round_trip(gctx, orc):
    rng = np.random.default_rng(11)
    hkv, d, bs, L = 2, 24, 8, 61
    k = normal(rng, (hkv, L, d))
    v = normal(rng, (hkv, L, d))
    ks, vs, table = paged_layout(k, v, bs, extra_blocks=3, rng=rng)
    ok, ov = gctx.alloc(k.nbytes), gctx.alloc(v.nbytes)
    rc = gctx.kv_gather(gctx.to_device(ks), gctx.to_device(vs), gctx.to_device(table), bs, L,
                        hkv, d, ks.shape[0], ok, ov)
    assert rc == 0
    gctx.sync()
    assert np.array_equal(ok.download(np.float32, k.shape), k)
    assert np.array_equal(ov.download(np.float32, v.shape), v)
    rk, rv = orc.kv_gather(ks, vs, table, bs, L, hkv, d)
    assert np.array_equal(rk, k) and np.array_equal(rv, v)


# ------------------------------------------------------------------ decode
def run_single(gctx, q, ks, vs, table, L, H, Hkv, d, bs, scale):
    out = gctx.alloc(q.nbytes)
    rc = gctx.paged_decode(gctx.to_device(q), gctx.to_device(ks), gctx.to_device(vs),
                           gctx.to_device(table), len(table), L, H, Hkv, d, bs, Hkv * bs * d,
                           ks.shape[0], scale, out)
    assert rc == 0, gctx.last_error()
    gctx.sync()
    return out.download(np.float32, q.shape)


def test_c1_single_sequence_decode(gctx, orc, ehip_mod):
    """C1: Qwen2-0.5B shape, 512 cached + 1 appended token in a permuted
    33-of-64 block table; append on the GPU, then attend."""
    from ehip import workloads
    w = workloads.c1()
    kpool, vpool = seeded_pool(orc, w, 101)
    kn, vn, q = new_rows(orc, w, 201)
    d, H, Hkv, bs = w.head_dim, w.heads, w.kv_heads, w.block_size
    dk, dv = gctx.to_device(kpool), gctx.to_device(vpool)
    rc = gctx.kv_scatter(gctx.to_device(kn), gctx.to_device(vn), gctx.to_device(w.slot_mapping),
                         1, Hkv, d, bs, w.pool_blocks, dk, dv, False)
    assert rc == 0
    orc.kv_scatter(kn, vn, w.slot_mapping, Hkv, d, bs, kpool, vpool)
    gctx.sync()
    assert np.array_equal(dk.download(np.float32, kpool.shape).view(np.uint32),
                          kpool.view(np.uint32))
    out = gctx.alloc(q.nbytes)
    rc = gctx.paged_decode(gctx.to_device(q), dk, dv, gctx.to_device(w.tables[0]), 33, 513, H,
                           Hkv, d, bs, Hkv * bs * d, w.pool_blocks, w.scale, out)
    assert rc == 0, gctx.last_error()
    gctx.sync()
    got = out.download(np.float32, (H, d))
    ref = orc.paged_decode(q[0], kpool, vpool, w.tables[0], 513, H, Hkv, d, bs, w.scale)
    check_fp32(got, ref)
    kc = orc.paged_to_contig(kpool, w.tables[0], 513, Hkv, d, bs)
    vc = orc.paged_to_contig(vpool, w.tables[0], 513, Hkv, d, bs)
    bf = brute_force_f64(q, kc, vc, H, Hkv, w.scale)[0]
    assert rel_norm(got, bf) <= FP32_REL


@pytest.mark.parametrize("H,Hkv", [(4, 4), (4, 2), (8, 1), (24, 2), (14, 2), (32, 8), (64, 8)])
@pytest.mark.parametrize("d", [18, 24, 64, 128])
def test_decode_gqa_and_head_dim_sweep(gctx, orc, H, Hkv, d):
    rng = np.random.default_rng(H * 1000 + Hkv * 10 + d)
    L, bs = 300, 16
    q = normal(rng, (H, d), 2.0)
    k = normal(rng, (Hkv, L, d), 2.0)
    v = normal(rng, (Hkv, L, d), 2.0)
    ks, vs, table = paged_layout(k, v, bs, extra_blocks=2)
    scale = scale_for(d)
    got = run_single(gctx, q, ks, vs, table, L, H, Hkv, d, bs, scale)
    ref = orc.paged_decode(q, ks, vs, table, L, H, Hkv, d, bs, scale)
    check_fp32(got, ref)


@pytest.mark.parametrize("bs", [8, 16, 32, 64])
@pytest.mark.parametrize("L", [1, 7, 8, 9, 15, 16, 17, 63, 64, 65, 127, 128, 129, 511, 2048, 4096])
def test_decode_length_and_block_size_sweep(gctx, orc, bs, L):
    rng = np.random.default_rng(L * 131 + bs)
    H, Hkv, d = 8, 2, 64
    q = normal(rng, (H, d))
    k = normal(rng, (Hkv, L, d))
    v = normal(rng, (Hkv, L, d))
    ks, vs, table = paged_layout(k, v, bs, extra_blocks=1)  # reverse-permuted, poisoned
    got = run_single(gctx, q, ks, vs, table, L, H, Hkv, d, bs, scale_for(d))
    ref = orc.paged_decode(q, ks, vs, table, L, H, Hkv, d, bs, scale_for(d))
    check_fp32(got, ref)


def test_decode_single_key_and_equal_keys_closed_forms(gctx):
    # L = 1: out[h] = v[h // g, 0] exactly; equal keys: out = mean of V rows.
    rng = np.random.default_rng(5)
    H, Hkv, d, bs = 8, 2, 64, 16
    q = normal(rng, (H, d))
    k = normal(rng, (Hkv, 1, d))
    v = normal(rng, (Hkv, 1, d))
    ks, vs, table = paged_layout(k, v, bs)
    got = run_single(gctx, q, ks, vs, table, 1, H, Hkv, d, bs, 0.125)
    assert np.array_equal(got, v[np.arange(H) // 4, 0])
    L = 100
    k = np.repeat(normal(rng, (Hkv, 1, d)), L, axis=1)
    v = normal(rng, (Hkv, L, d))
    ks, vs, table = paged_layout(k, v, bs)
    got = run_single(gctx, q, ks, vs, table, L, H, Hkv, d, bs, 0.125)
    mean = v.astype(np.float64).mean(axis=1)[np.arange(H) // 4]
    assert rel_norm(got, mean) <= 1e-5


@pytest.mark.parametrize("L", [512, 2048])
def test_decode_large_magnitude_rescale(gctx, orc, L):
    # The reference's LargeMagnitudeRescale case: std 2 => logit std ~4, so
    # the running-max rescale is exercised (paged_decode_attention_kernel_test.cpp:227-249).
    rng = np.random.default_rng(4000 + L)
    H, Hkv, d, bs = 4, 2, 64, 16
    q, k, v = (normal(rng, s, 2.0) for s in ((H, d), (Hkv, L, d), (Hkv, L, d)))
    ks, vs, table = paged_layout(k, v, bs, extra_blocks=2)
    got = run_single(gctx, q, ks, vs, table, L, H, Hkv, d, bs, scale_for(d))
    ref = orc.paged_decode(q, ks, vs, table, L, H, Hkv, d, bs, scale_for(d))
    check_fp32(got, ref)
    oracle = orc.cpu_attention(q[None], k, v, H, Hkv, d, scale_for(d))[0]
    assert allclose_ref(got, oracle, 1e-4, 1e-5)


def test_decode_very_peaked_softmax_vs_fp64(gctx, orc):
    # std 6 (logits ~ +-40): beyond what fp32 summation-order differences
    # keep inside the elementwise allclose (the reference's own scalar and
    # AVX2 kernels disagree there too), so this case is held to the fp64
    # brute force per output vector.
    rng = np.random.default_rng(9)
    H, Hkv, d, bs, L = 32, 8, 128, 16, 1500
    q = normal(rng, (H, d), 6.0)
    k = normal(rng, (Hkv, L, d), 6.0)
    v = normal(rng, (Hkv, L, d), 2.0)
    ks, vs, table = paged_layout(k, v, bs, rng=rng, extra_blocks=7)
    got = run_single(gctx, q, ks, vs, table, L, H, Hkv, d, bs, scale_for(d))
    bf = brute_force_f64(q[None], k, v, H, Hkv, scale_for(d))[0]
    assert rel_norm(got, bf) <= FP32_REL


@pytest.mark.parametrize("name", ["l0_prefill_empty", "l1_prefill_empty", "l0_prefill_continue",
                                  "l1_prefill_continue", "l0_decode"])
def test_decode_matches_hf_goldens(gctx, golden, name):
    # Last query row of each HF case is the decode of its final token
    # (tests/unit/paged_decode_attention_kernel_test.cpp:388-444, bs = 8).
    q, k, v, ctx = (golden[f"{name}.{s}"] for s in ("q_rot", "k_all", "v_all", "ctx"))
    ks, vs, table = paged_layout(k, v, 8, extra_blocks=1)
    got = run_single(gctx, q[-1], ks, vs, table, k.shape[1], 4, 2, 16, 8, 0.25)
    assert allclose_ref(got, ctx[-1], 1e-4, 1e-4)


def test_decode_rejects_bad_block_size_and_zero_batch(gctx, ehip_mod):
    q = np.zeros((4, 16), np.float32)
    dq = gctx.to_device(q)
    slab = gctx.alloc(4 * 2 * 12 * 16 * 4)
    tab = gctx.to_device(np.arange(4, dtype=np.int32))
    out = gctx.alloc(q.nbytes)
    rc = gctx.paged_decode(dq, slab, slab, tab, 4, 20, 4, 2, 16, 12, 2 * 12 * 16, 4, 0.25, out)
    assert rc == ehip_mod.INVALID_ARGUMENT
    assert "block_size" in gctx.last_error()
    # B == 0 is a no-op (paged_attention.h: "B == 0 is a no-op").
    rc = gctx.paged_decode_batched(None, None, None, [], [], 4, 2, 16, 16, 0, 4, 0.25, None)
    assert rc == 0


def test_decode_table_id_out_of_range_is_reported(gctx, ehip_mod):
    # Device-resident table: the kernel bounds every id it dereferences and
    # the host learns of the bad id at sync.
    H, Hkv, d, bs, L = 4, 2, 64, 16, 40
    q = np.ones((H, d), np.float32)
    slab = gctx.alloc(4 * Hkv * bs * d * 4)
    tab = gctx.to_device(np.array([0, 1, 99], np.int32))
    out = gctx.alloc(q.nbytes)
    assert gctx.paged_decode(gctx.to_device(q), slab, slab, tab, 3, L, H, Hkv, d, bs,
                             Hkv * bs * d, 4, 0.125, out) == 0
    with pytest.raises(ehip_mod.EhipError) as e:
        gctx.sync()
    assert e.value.code == ehip_mod.INVALID_ARGUMENT
    # Host tables are validated before anything is enqueued.
    rc = gctx.paged_decode_batched(gctx.to_device(q), slab, slab, [np.array([0, 1, 99], np.int32)],
                                   [L], H, Hkv, d, bs, 0, 4, 0.125, out)
    assert rc == ehip_mod.INVALID_ARGUMENT


# ------------------------------------------------------------------ batched
def batched_case(orc, rng, lengths, H, Hkv, d, bs):
    ks_l = [normal(rng, (Hkv, L, d)) for L in lengths]
    vs_l = [normal(rng, (Hkv, L, d)) for L in lengths]
    from paged_util import shared_pool_layout
    k_slab, v_slab, tables = shared_pool_layout(ks_l, vs_l, bs, rng)
    q = normal(rng, (len(lengths), H, d))
    return q, k_slab, v_slab, tables


@pytest.mark.parametrize("bs", [8, 16, 32, 64])
def test_batched_decode_heterogeneous_lengths(gctx, orc, bs):
    rng = np.random.default_rng(bs)
    lengths = [1, bs, 2 * bs + 1, 63, 128, 300, 1000]
    H, Hkv, d = 14, 2, 64
    q, ks, vs, tables = batched_case(orc, rng, lengths, H, Hkv, d, bs)
    out = gctx.alloc(q.nbytes)
    rc = gctx.paged_decode_batched(gctx.to_device(q), gctx.to_device(ks), gctx.to_device(vs),
                                   tables, lengths, H, Hkv, d, bs, 0, ks.shape[0],
                                   scale_for(d), out)
    assert rc == 0, gctx.last_error()
    gctx.sync()
    got = out.download(np.float32, q.shape)
    ref = orc.paged_decode_batched(q, ks, vs, tables, lengths, H, Hkv, d, bs, scale_for(d))
    check_fp32(got, ref)
    # Each member equals a standalone single-sequence run (within tolerance:
    # the split partition may differ with the batch's total work).
    for b in (0, 3, 6):
        single = run_single(gctx, q[b], ks, vs, tables[b], lengths[b], H, Hkv, d, bs,
                            scale_for(d))
        assert rel_norm(got[b], single) <= FP32_REL


@pytest.mark.parametrize("kernel", ["mfma", "valu"])
@pytest.mark.parametrize("bs", [16, 64, 8])
def test_batched_decode_bf16_kv(orc, kernel, bs, tctx):
    # Both bf16 kernels (QK^T on MFMA, or all-VALU); bs = 8 always takes the
    # VALU kernel.
    gctx = tctx(EHIP_DECODE_KERNEL=kernel)
    rng = np.random.default_rng(77 + bs)
    lengths = list(rng.integers(1, 3000, 24))
    H, Hkv, d = 32, 8, 128
    q, ks, vs, tables = batched_case(orc, rng, lengths, H, Hkv, d, bs)
    ks_b, vs_b = orc.to_bf16_bits(ks), orc.to_bf16_bits(vs)
    out = gctx.alloc(q.nbytes)
    rc = gctx.paged_decode_batched(gctx.to_device(q), gctx.to_device(ks_b), gctx.to_device(vs_b),
                                   tables, lengths, H, Hkv, d, bs, 0, ks.shape[0],
                                   scale_for(d), out, bf16=True)
    assert rc == 0, gctx.last_error()
    gctx.sync()
    got = out.download(np.float32, q.shape)
    ref32 = orc.paged_decode_batched(q, ks, vs, tables, lengths, H, Hkv, d, bs, scale_for(d))
    assert max_abs(got, ref32) <= BF16_ABS
    ref_r = orc.paged_decode_batched(q, orc.bf16_bits_to_f32(ks_b), orc.bf16_bits_to_f32(vs_b),
                                     tables, lengths, H, Hkv, d, bs, scale_for(d))
    check_fp32(got, ref_r)


@pytest.mark.parametrize("H,Hkv", [(8, 8), (8, 4), (32, 8), (64, 8), (14, 2)])
@pytest.mark.parametrize("d", [64, 128])
def test_bf16_decode_gqa_sweep(gctx, orc, H, Hkv, d):
    rng = np.random.default_rng(H * 100 + Hkv + d)
    lengths = [1, 15, 16, 17, 33, 700, 2049]
    q, ks, vs, tables = batched_case(orc, rng, lengths, H, Hkv, d, 16)
    ks_b, vs_b = orc.to_bf16_bits(ks), orc.to_bf16_bits(vs)
    out = gctx.alloc(q.nbytes)
    assert gctx.paged_decode_batched(gctx.to_device(q), gctx.to_device(ks_b),
                                     gctx.to_device(vs_b), tables, lengths, H, Hkv, d, 16, 0,
                                     ks.shape[0], scale_for(d), out, bf16=True) == 0
    gctx.sync()
    got = out.download(np.float32, q.shape)
    ref = orc.paged_decode_batched(q, orc.bf16_bits_to_f32(ks_b), orc.bf16_bits_to_f32(vs_b),
                                   tables, lengths, H, Hkv, d, 16, scale_for(d))
    check_fp32(got, ref)


@pytest.mark.parametrize("split", ["64", "128", "512", "1024", "2048"])
def test_split_count_independence(orc, split, tctx):
    # The merged result must not depend on how the keys were split (the
    # split-KV path: the workgroup-per-row kernel for small steps is off).
    gctx = tctx(EHIP_SPLIT_TOKENS=split, EHIP_DECODE_WG="0")
    rng = np.random.default_rng(3)
    lengths = [4000, 17, 1025, 2048, 64]
    H, Hkv, d, bs = 32, 8, 128, 16
    q, ks, vs, tables = batched_case(orc, rng, lengths, H, Hkv, d, bs)
    out = gctx.alloc(q.nbytes)
    assert gctx.paged_decode_batched(gctx.to_device(q), gctx.to_device(ks), gctx.to_device(vs),
                                     tables, lengths, H, Hkv, d, bs, 0, ks.shape[0],
                                     scale_for(d), out) == 0
    gctx.sync()
    got = out.download(np.float32, q.shape)
    ref = orc.paged_decode_batched(q, ks, vs, tables, lengths, H, Hkv, d, bs, scale_for(d))
    check_fp32(got, ref)


@pytest.mark.parametrize("H", [32, 64])
def test_merge_of_wide_groups(orc, H, tctx):
    # One kv head for all H query heads, and a row cut into the most splits a
    # row may have (64): 64 * 32 = 2048 (max, sum) pairs still fit the merge
    # workgroup's LDS; 64 * 64 = 4096 take the one-wavefront sequential merge.
    gctx = tctx(EHIP_SPLIT_TOKENS="128", EHIP_DECODE_WG="0")
    rng = np.random.default_rng(H)
    lengths = [8192, 300, 1, 2500]
    Hkv, d, bs = 1, 64, 16
    q, ks, vs, tables = batched_case(orc, rng, lengths, H, Hkv, d, bs)
    out = gctx.alloc(q.nbytes)
    assert gctx.paged_decode_batched(gctx.to_device(q), gctx.to_device(ks), gctx.to_device(vs),
                                     tables, lengths, H, Hkv, d, bs, 0, ks.shape[0],
                                     scale_for(d), out) == 0
    gctx.sync()
    got = out.download(np.float32, q.shape)
    ref = orc.paged_decode_batched(q, ks, vs, tables, lengths, H, Hkv, d, bs, scale_for(d))
    check_fp32(got, ref)


@pytest.mark.parametrize("split", ["128", "256"])
def test_large_merge_four_elements_per_thread(orc, split, tctx):
    # At least 32 split rows x 8 kv heads x 1024 elements = 2^18: the merge
    # takes four elements per thread; the 2049- and 4000-key rows have more
    # than the 16 splits whose partials are loaded before the weights are
    # formed.
    gctx = tctx(EHIP_SPLIT_TOKENS=split, EHIP_DECODE_WG="0")
    rng = np.random.default_rng(int(split))
    lengths = [int(x) for x in rng.integers(300, 900, size=40)] + [1, 2049, 4000]
    H, Hkv, d, bs = 64, 8, 128, 16
    q, ks, vs, tables = batched_case(orc, rng, lengths, H, Hkv, d, bs)
    out = gctx.alloc(q.nbytes)
    assert gctx.paged_decode_batched(gctx.to_device(q), gctx.to_device(ks), gctx.to_device(vs),
                                     tables, lengths, H, Hkv, d, bs, 0, ks.shape[0],
                                     scale_for(d), out) == 0
    gctx.sync()
    got = out.download(np.float32, q.shape)
    ref = orc.paged_decode_batched(q, ks, vs, tables, lengths, H, Hkv, d, bs, scale_for(d))
    check_fp32(got, ref)


# ------------------------------------------------------------------ step path
def run_step(gctx, ehip_mod, orc, w, seed, layers=1):
    """Upload one step, then per layer append + attend on the GPU; the oracle
    does the same with its scatter and varlen reference."""
    H, Hkv, d, bs = w.heads, w.kv_heads, w.head_dim, w.block_size
    bf16 = w.kv_dtype == ehip_mod.KV_BF16
    g = ehip_mod.geometry(H, Hkv, d, bs, w.kv_dtype, w.pool_blocks, w.scale)
    st = ehip_mod.StepArrays(w.query_lens, w.context_lens, w.tables, w.slot_mapping)
    assert gctx.step_upload(g, st) == 0, gctx.last_error()
    results = []
    for layer in range(layers):
        kpool, vpool = seeded_pool(orc, w, seed + 1000 * layer)
        kn, vn, q = new_rows(orc, w, seed + 1000 * layer + 500)
        if bf16:
            dk = gctx.to_device(orc.to_bf16_bits(kpool))
            dv = gctx.to_device(orc.to_bf16_bits(vpool))
        else:
            dk, dv = gctx.to_device(kpool), gctx.to_device(vpool)
        dq = gctx.to_device(q)
        out = gctx.alloc(q.nbytes)
        assert gctx.step_kv_append(gctx.to_device(kn), gctx.to_device(vn), dk, dv) == 0
        assert gctx.step_attention(dq, dk, dv, out) == 0, gctx.last_error()
        gctx.sync()
        got = out.download(np.float32, q.shape)
        # Oracle: the same append (bit-exact check of the whole slab), then
        # the reference attention over the post-append cache.
        if bf16:
            kb, vb = orc.to_bf16_bits(kpool), orc.to_bf16_bits(vpool)
            orc.kv_scatter(kn, vn, w.slot_mapping, Hkv, d, bs, kb, vb)
            assert np.array_equal(dk.download(np.uint16, kb.shape), kb)
            assert np.array_equal(dv.download(np.uint16, vb.shape), vb)
            kref, vref = orc.bf16_bits_to_f32(kb), orc.bf16_bits_to_f32(vb)
            orc.kv_scatter(kn, vn, w.slot_mapping, Hkv, d, bs, kpool, vpool)
        else:
            orc.kv_scatter(kn, vn, w.slot_mapping, Hkv, d, bs, kpool, vpool)
            assert np.array_equal(dk.download(np.float32, kpool.shape).view(np.uint32),
                                  kpool.view(np.uint32))
            kref, vref = kpool, vpool
        cu = np.concatenate([[0], np.cumsum(w.query_lens)]).astype(np.int32)
        kseq = [orc.paged_to_contig(kref, t, int(L), Hkv, d, bs) for t, L in
                zip(w.tables, w.context_lens)]
        vseq = [orc.paged_to_contig(vref, t, int(L), Hkv, d, bs) for t, L in
                zip(w.tables, w.context_lens)]
        ref = orc.prefill_varlen(q, cu, kseq, vseq, H, Hkv, d, w.scale, isa=1)
        results.append((got, ref, kpool, vpool, q, cu))
        for b in (dk, dv, dq, out):
            b.free()
    return results


@pytest.mark.parametrize("wg", ["1", "0"])
def test_step_c2_ragged_decode(ehip_mod, orc, wg, tctx):
    """C2 shape (B=32, L~U[64,2048]+1, fp32 pool 1.25x need): two layers of
    append + attention through the per-step descriptor."""
    gctx = tctx(EHIP_DECODE_WG=wg)  # workgroup per (row, kv head), or split-KV
    from ehip import workloads
    w = workloads.c2()
    for got, ref, *_ in run_step(gctx, ehip_mod, orc, w, 7, layers=2):
        check_fp32(got, ref)


PREFILL_REL = 1e-2  # MFMA prefill multiplies bf16 Q and bf16 P (fp32 accumulate)


def check_step_rows(w, got, ref, ref32):
    """Decode rows (T == 1) to the fp32 bar against the reference on the same
    bf16-rounded K/V; prefill-chunk rows (bf16 Q/P on MFMA) to the bf16-KV bar
    against the fp32 reference (2e-2 absolute) and to 1e-2 relative against
    the rounded one."""
    rows = np.repeat(w.query_lens, w.query_lens)
    dec = rows == 1
    if dec.any():
        check_fp32(got[dec], ref[dec])
    if (~dec).any():
        assert rel_norm(got[~dec], ref[~dec]) <= PREFILL_REL, rel_norm(got[~dec], ref[~dec])
    assert max_abs(got, ref32) <= BF16_ABS


def fp32_reference(orc, w, kpool, vpool, q, cu):
    H, Hkv, d, bs = w.heads, w.kv_heads, w.head_dim, w.block_size
    kseq = [orc.paged_to_contig(kpool, t, int(L), Hkv, d, bs) for t, L in
            zip(w.tables, w.context_lens)]
    vseq = [orc.paged_to_contig(vpool, t, int(L), Hkv, d, bs) for t, L in
            zip(w.tables, w.context_lens)]
    return orc.prefill_varlen(q, cu, kseq, vseq, H, Hkv, d, w.scale, isa=1)


@pytest.mark.parametrize("prefill", ["1", "0"])
def test_step_c3_mixed_prefill_and_decode(ehip_mod, orc, prefill, tctx):
    """C3 composition scaled down (2 causal chunks + 12 decodes, bf16 KV): the
    chunks run on the MFMA prefill kernel (or, with EHIP_PREFILL=0, on the
    decode kernels), the decodes on the decode kernel."""
    gctx = tctx(EHIP_PREFILL=prefill)
    from ehip import workloads
    w = workloads.c3()
    keep = [0, 1] + list(range(4, 16))
    w.query_lens = w.query_lens[keep].copy()
    w.context_lens = w.context_lens[keep].copy()
    w.tables = [w.tables[i] for i in keep]
    w.slot_mapping = workloads._append_slots(w.tables, w.query_lens, w.context_lens,
                                             w.block_size)
    (got, ref, kpool, vpool, q, cu), = run_step(gctx, ehip_mod, orc, w, 9)
    ref32 = fp32_reference(orc, w, kpool, vpool, q, cu)
    if prefill == "0":
        check_fp32(got, ref)
        assert max_abs(got, ref32) <= BF16_ABS
    else:
        check_step_rows(w, got, ref, ref32)


def chunk_workload(H, Hkv, T, P, extra_decodes=1, seed=0, std=0.5):
    """One causal chunk of T rows over P cached keys plus a few decode rows of
    other sequences, bf16 KV, d = 128, bs = 16, shuffled pool."""
    from ehip import workloads
    rng = np.random.default_rng(seed)
    qlens = [T] + [1] * extra_decodes
    L = [P + T] + list(rng.integers(20, 400, extra_decodes) + 1)
    need = [(x + 15) // 16 for x in L]
    pool = int(sum(need) * 1.3) + 2
    tables, _ = workloads._tables_from_pool(np.array(need), pool, rng)
    return workloads._finish("chunk", H, Hkv, 128, 16, ehip_mod_kv_bf16(), 1, qlens, L, tables,
                             pool, std)


def ehip_mod_kv_bf16():
    import ehip
    return ehip.KV_BF16


@pytest.mark.parametrize("H,Hkv", [(32, 8), (64, 8)])
@pytest.mark.parametrize("T,P", [(16, 0), (37, 0), (300, 0), (45, 100), (130, 515)])
def test_prefill_chunk_shapes(gctx, ehip_mod, orc, H, Hkv, T, P):
    """Causal chunks on the MFMA prefill kernel: ragged last query block,
    continuation chunks (P > 0), g = 4 and 8."""
    w = chunk_workload(H, Hkv, T, P, extra_decodes=2, seed=T + P + H)
    (got, ref, kpool, vpool, q, cu), = run_step(gctx, ehip_mod, orc, w, 31)
    ref32 = fp32_reference(orc, w, kpool, vpool, q, cu)
    check_step_rows(w, got, ref, ref32)


@pytest.mark.parametrize("H,Hkv", [(32, 8), (64, 8)])
@pytest.mark.parametrize("T,P", [(512, 1024), (700, 0), (96, 4000)])
def test_prefill_key_splits(ehip_mod, orc, H, Hkv, T, P, tctx):
    """Prefill blocks cut into key splits (the long ones relative to the
    step's prefill work) and merged by the split merge: against the
    references, and against the same step with every block whole."""
    w = chunk_workload(H, Hkv, T, P, extra_decodes=3, seed=T + P + H + 7)
    outs, partials = [], []
    for flag in ("1", "0"):
        gctx = tctx(EHIP_PREFILL_SPLIT=flag)
        (got, ref, kpool, vpool, q, cu), = run_step(gctx, ehip_mod, orc, w, 41)
        partials.append(gctx.step_info()[2])
        if flag == "1":
            ref32 = fp32_reference(orc, w, kpool, vpool, q, cu)
            check_step_rows(w, got, ref, ref32)
        outs.append(got)
    assert partials[0] > partials[1], f"expected key splits in the plan: {partials}"
    # Same bf16 products up to where P is rounded (each split keeps its own
    # softmax reference): within the prefill bar of each other.
    rows = np.repeat(w.query_lens, w.query_lens) > 1
    assert rel_norm(outs[0][rows], outs[1][rows]) <= PREFILL_REL


@pytest.mark.parametrize("slots", ["1", "7", "40", "64", "300"])
def test_persistent_decode_queue(ehip_mod, orc, slots, tctx):
    """The MFMA decode kernel's wavefronts take their later items from the
    launch's sub-queue counters (up to 32, one per wavefront index modulo
    their count). With the grid capped to a few wavefronts every one of them
    runs many items, over several launches in a row (each launch must leave
    the counters zero for the next); 40 leaves the sub-queues with unequal
    numbers of wavefronts. Outputs bit-identical to one workgroup per item,
    and within the bars of the oracle."""
    from ehip import workloads
    w = workloads.c4(num_seqs=24, share_frac=0.3)
    gctx = tctx(EHIP_DECODE_PERSIST="0")
    base = run_step(gctx, ehip_mod, orc, w, 17, layers=3)
    gctx = tctx(EHIP_DECODE_PERSIST="1", EHIP_DECODE_SLOTS=slots)
    got = run_step(gctx, ehip_mod, orc, w, 17, layers=3)
    for (g, ref, *_), (b, *_) in zip(got, base):
        assert np.array_equal(g.view(np.uint32), b.view(np.uint32))
        check_fp32(g, ref)


@pytest.mark.parametrize("kernel", ["mfma", "valu"])
def test_step_c4_shape_with_shared_prefix_blocks(ehip_mod, orc, kernel, tctx):
    """C4 construction (log-uniform lengths, pair-shared prefix blocks, bf16)
    at 24 sequences."""
    gctx = tctx(EHIP_DECODE_KERNEL=kernel)
    from ehip import workloads
    w = workloads.c4(num_seqs=24, share_frac=0.3)
    assert (w.refcount == 2).any()
    (got, ref, *_), = run_step(gctx, ehip_mod, orc, w, 13)
    check_fp32(got, ref)


@pytest.mark.parametrize("joint", ["1", "0"])
def test_step_shared_prefix_fp32_valu(ehip_mod, orc, joint, tctx):
    """Pair-shared prefix blocks through the fp32 VALU kernel, with and without
    joint work items (joint items are processed row by row there)."""
    # Joint items live in the split-KV path (no workgroup-per-row kernel).
    gctx = tctx(EHIP_DECODE_WG="0", EHIP_NO_JOINT="0" if joint == "1" else "1")
    from ehip import workloads
    w = workloads.c4(num_seqs=12, share_frac=0.4)
    w.kv_dtype = ehip_mod.KV_F32
    (got, ref, *_), = run_step(gctx, ehip_mod, orc, w, 17)
    check_fp32(got, ref)


def test_step_joint_items_match_plain_partition(ehip_mod, orc, tctx):
    """Joint items (one pass over shared blocks for two rows) against the plain
    per-row partition on the same bf16 step."""
    from ehip import workloads
    w = workloads.c4(num_seqs=16, share_frac=0.4)
    outs = []
    for flag in ("0", "1"):
        gctx = tctx(EHIP_NO_JOINT=flag)
        (got, ref, *_), = run_step(gctx, ehip_mod, orc, w, 21)
        check_fp32(got, ref)
        outs.append(got)
    assert rel_norm(outs[0], outs[1]) <= 1e-5


def test_step_requires_upload_and_validates(gctx, ehip_mod):
    g = ehip_mod.geometry(4, 2, 64, 16, 0, 8, 0.125)
    bad = ehip_mod.StepArrays([1], [40], [np.array([0, 1], np.int32)])  # needs 3 blocks
    assert gctx.step_upload(g, bad) == ehip_mod.INVALID_ARGUMENT
    bad = ehip_mod.StepArrays([1], [20], [np.array([0, 8], np.int32)])  # id 8 of 8 blocks
    assert gctx.step_upload(g, bad) == ehip_mod.INVALID_ARGUMENT
    bad = ehip_mod.StepArrays([1], [20], [np.array([0, 1], np.int32)], [8 * 16])
    assert gctx.step_upload(g, bad) == ehip_mod.INVALID_ARGUMENT


def test_bandwidth_probes(gctx, ehip_mod):
    """The benchmark's read-bandwidth probes (lib/libehip_probe.so, apart from
    the attention library) run and validate their arguments (ids out of range,
    bytes below one vector) without launching."""
    from ehip import probe
    nb, hkv, tile = 64, 2, 16 * 64 * 2
    k, v = gctx.alloc(nb * hkv * tile), gctx.alloc(nb * hkv * tile)
    g = probe.stream_read(k, nb * hkv * tile, nt=True, reps=2)
    assert np.isfinite(g) and g > 0
    blocks = np.random.default_rng(0).permutation(nb).astype(np.int32)
    for nt in (False, True):
        g = probe.tile_gather(k, v, nb, blocks, 8, hkv, hkv * tile, tile, nt=nt, reps=2)
        assert np.isfinite(g) and g > 0
    import ctypes as C
    out = C.c_float()
    bad = blocks.copy()
    bad[3] = nb
    rc = probe.plib().ehip_probe_tile_gather(k.ptr, v.ptr, nb, bad.ctypes.data, bad.size, 8, hkv,
                                             hkv * tile, tile, 1, 1, C.byref(out))
    assert rc == ehip_mod.INVALID_ARGUMENT
    assert probe.plib().ehip_probe_stream_read(k.ptr, 8, 0, 1,
                                               C.byref(out)) == ehip_mod.INVALID_ARGUMENT
    k.free()
    v.free()


def fork_group_case(rng, groups, Hkv, d, bs, H):
    """Rows forked from shared prefixes: groups of (shared_blocks, [lengths]).
    A group's members read the same physical blocks (the same K/V) over the
    shared prefix; every other block, the last included, is a member's own.
    Returns (q, k_slab, v_slab, tables, lengths)."""
    need = sum(sb + sum((L + bs - 1) // bs - sb for L in lens) for sb, lens in groups)
    nb = need + 9
    perm = rng.permutation(nb).astype(np.int32)
    k_slab = normal(rng, (nb, Hkv, bs, d))
    v_slab = normal(rng, (nb, Hkv, bs, d))
    tables, off = [], 0
    for sb, lens in groups:
        shared = perm[off:off + sb]
        off += sb
        for L in lens:
            own = (L + bs - 1) // bs - sb
            assert own >= 1
            tables.append(np.concatenate([shared, perm[off:off + own]]).astype(np.int32))
            off += own
    lengths = [L for _, ls in groups for L in ls]
    q = normal(rng, (len(lengths), H, d))
    return q, k_slab, v_slab, tables, lengths


FORK_GROUPS = [(20, [700, 530, 900, 400, 655]),  # five sharers of 320 keys
               (12, [300, 900, 260]),            # three sharers of 192 keys
               (30, [600, 610]),                 # a pair
               (0, [129, 77, 1])]                # no sharing


@pytest.mark.parametrize("H,Hkv,d,kv", [(32, 8, 128, "mfma"), (16, 8, 64, "mfma"),
                                        (8, 8, 128, "mfma"), (64, 8, 128, "mfma"),
                                        (32, 8, 128, "valu"), (14, 2, 64, "f32"),
                                        (8, 8, 64, "f32"), (14, 2, 64, "f32valu"),
                                        (16, 2, 128, "f32")])
def test_decode_fork_groups_beyond_pairs(ehip_mod, orc, H, Hkv, d, kv, tctx):
    """Joint work items of up to min(4, 16 / g) rows over fork groups' shared
    prefixes (groups of five and three sharers, a pair, unshared rows),
    through the MFMA kernel (its virtual heads: g per row, up to 16; bf16, and
    fp32 at head_dim 64), the bf16 and fp32 VALU kernels (rows one after the
    other; fp32 head_dim 128 always): against the oracle, and against the
    plain per-row partition."""
    kernel = "valu" if kv.endswith("valu") else "mfma"
    # Joint items live in the split-KV path (no workgroup-per-row kernel).
    gctx = tctx(EHIP_DECODE_KERNEL=kernel, EHIP_DECODE_WG="0")
    rng = np.random.default_rng(H + 3 * d)
    bs = 16
    q, ks, vs, tables, lengths = fork_group_case(rng, FORK_GROUPS, Hkv, d, bs, H)
    bf16 = not kv.startswith("f32")
    if bf16:
        ks_b, vs_b = orc.to_bf16_bits(ks), orc.to_bf16_bits(vs)
        kd, vd = gctx.to_device(ks_b), gctx.to_device(vs_b)
        ks_r, vs_r = orc.bf16_bits_to_f32(ks_b), orc.bf16_bits_to_f32(vs_b)
    else:
        kd, vd = gctx.to_device(ks), gctx.to_device(vs)
        ks_r, vs_r = ks, vs
    geo = ehip_mod.geometry(H, Hkv, d, bs, ehip_mod.KV_BF16 if bf16 else ehip_mod.KV_F32,
                            ks.shape[0], scale_for(d))
    st = ehip_mod.StepArrays(np.ones(len(lengths), np.int32), np.asarray(lengths, np.int64),
                             tables)
    _, items = ehip_mod.plan_items(geo, st)
    assert (items[:, :4] >= 0).sum(axis=1).max() == min(4, 16 // (H // Hkv))
    ref = orc.paged_decode_batched(q, ks_r, vs_r, tables, lengths, H, Hkv, d, bs, scale_for(d))
    qd = gctx.to_device(q)
    outs = []
    for flag in ("0", "1"):
        gctx = tctx(EHIP_NO_JOINT=flag)
        out = gctx.alloc(q.nbytes)
        assert gctx.paged_decode_batched(qd, kd, vd, tables, lengths, H, Hkv, d, bs, 0,
                                         ks.shape[0], scale_for(d), out, bf16=bf16) == 0, \
            gctx.last_error()
        gctx.sync()
        outs.append(out.download(np.float32, q.shape))
        out.free()
        check_fp32(outs[-1], ref)
    assert rel_norm(outs[0], outs[1]) <= FP32_REL
    for b in (qd, kd, vd):
        b.free()


@pytest.mark.parametrize("H,Hkv,reps", [(14, 2, 3), (8, 8, 1), (16, 4, 2)])
def test_fp32_joint_items_over_four_wavefronts(ehip_mod, orc, H, Hkv, reps, tctx):
    """fp32 fork groups (head_dim 64) in a step of 256..480 items: joint items
    of 2 (g = 7) and 4 (g = 1) rows over four wavefronts per item, and g = 4,
    whose 16 virtual heads keep Q in LDS and so stay one wavefront per item:
    against the oracle, and against one wavefront per item."""
    rng = np.random.default_rng(H + Hkv)
    bs, d = 16, 64
    q, ks, vs, tables, lengths = fork_group_case(rng, FORK_GROUPS * reps, Hkv, d, bs, H)
    geo = ehip_mod.geometry(H, Hkv, d, bs, ehip_mod.KV_F32, ks.shape[0], scale_for(d))
    st = ehip_mod.StepArrays(np.ones(len(lengths), np.int32), np.asarray(lengths, np.int64),
                             tables)
    rc, _, items, _, _, joint, _ = ehip_mod.plan_counts(geo, st, joint=True)
    assert rc == 0 and joint > 0 and 256 <= items <= 480, items
    ref = orc.paged_decode_batched(q, ks, vs, tables, lengths, H, Hkv, d, bs, scale_for(d))
    outs = []
    for split4 in ("1", "0"):
        gctx = tctx(EHIP_DECODE_SPLIT4=split4, EHIP_DECODE_WG="0")
        qd, kd, vd = gctx.to_device(q), gctx.to_device(ks), gctx.to_device(vs)
        out = gctx.alloc(q.nbytes)
        assert gctx.paged_decode_batched(qd, kd, vd, tables, lengths, H, Hkv, d, bs, 0,
                                         ks.shape[0], scale_for(d), out) == 0, gctx.last_error()
        gctx.sync()
        outs.append(out.download(np.float32, q.shape))
        check_fp32(outs[-1], ref)
        for b in (qd, kd, vd, out):
            b.free()
    assert rel_norm(outs[0], outs[1]) <= FP32_REL


@pytest.mark.parametrize("H,Hkv,d", [(14, 2, 64), (32, 8, 128), (8, 8, 128), (28, 4, 64),
                                     (8, 1, 128), (24, 3, 64)])
@pytest.mark.parametrize("lens", [[1, 17, 33, 1500, 513], [1024, 1536, 1], [32, 64, 96],
                                  [4000, 17]])
def test_small_step_workgroup_per_row(orc, H, Hkv, d, lens, tctx):
    """Small fp32 steps with short rows take one workgroup per (row, kv head),
    its wavefronts splitting the row's tiles and merging in LDS (a 4000-key
    row goes to the split-KV path instead): against the oracle, and against
    the split-KV path on the same inputs (both within the fp32 bar)."""
    rng = np.random.default_rng(H + 7 * d + len(lens))
    bs = 16
    q, ks, vs, tables = batched_case(orc, rng, lens, H, Hkv, d, bs)
    ref = orc.paged_decode_batched(q, ks, vs, tables, lens, H, Hkv, d, bs, scale_for(d))
    outs = []
    for wg in ("1", "0"):
        gctx = tctx(EHIP_DECODE_WG=wg)
        out = gctx.alloc(q.nbytes)
        assert gctx.paged_decode_batched(gctx.to_device(q), gctx.to_device(ks),
                                         gctx.to_device(vs), tables, lens, H, Hkv, d, bs, 0,
                                         ks.shape[0], scale_for(d), out) == 0
        gctx.sync()
        outs.append(out.download(np.float32, q.shape))
        check_fp32(outs[-1], ref)
    assert rel_norm(outs[0], outs[1]) <= FP32_REL


@pytest.mark.parametrize("kernel", ["mfma", "valu"])
def test_c2_layer_fp32_kernels(ehip_mod, orc, kernel, tctx):
    """One layer of the C2 step as drawn (32 rows, 14q/2kv, d = 64, fp32 slabs,
    split-KV) on the fp32 matrix-core kernel (Q and K in three bf16 parts,
    six products per chunk) and on the all-VALU kernel: both meet the fp32
    bar (1e-4 relative per output vector, the reference allclose) against the
    oracle on the same post-append cache."""
    from ehip import workloads
    gctx = tctx(EHIP_DECODE_KERNEL=kernel)
    w = workloads.c2()
    H, Hkv, d, bs = w.heads, w.kv_heads, w.head_dim, w.block_size
    kpool, vpool = seeded_pool(orc, w, 301)
    kn, vn, q = new_rows(orc, w, 401)
    g = ehip_mod.geometry(H, Hkv, d, bs, w.kv_dtype, w.pool_blocks, w.scale)
    st = ehip_mod.StepArrays(w.query_lens, w.context_lens, w.tables, w.slot_mapping)
    assert gctx.step_upload(g, st) == 0, gctx.last_error()
    dk, dv, dq = gctx.to_device(kpool), gctx.to_device(vpool), gctx.to_device(q)
    dkn, dvn = gctx.to_device(kn), gctx.to_device(vn)
    out = gctx.alloc(q.nbytes)
    assert gctx.step_append_attention(dkn, dvn, dq, dk, dv, out) == 0, gctx.last_error()
    gctx.sync()
    got = out.download(np.float32, q.shape)
    orc.kv_scatter(kn, vn, w.slot_mapping, Hkv, d, bs, kpool, vpool)
    assert np.array_equal(dk.download(np.float32, kpool.shape).view(np.uint32),
                          kpool.view(np.uint32))
    ref = orc.paged_decode_batched(q, kpool, vpool, w.tables, w.context_lens, H, Hkv, d, bs,
                                   w.scale)
    check_fp32(got, ref)
    for b in (dk, dv, dq, dkn, dvn, out):
        b.free()
