"""Pins the CPU oracle (oracle/) before anything is checked against it.

Each check is chosen so that a plausible restatement mistake (a dropped term,
a swapped index, a wrong rounding rule) fails: known-answer vectors, the
reference's own kernels compiled from its sources (oracle/_ref, bit-exact),
the HF goldens the reference's tests replay, closed forms and fp64 brute force.
"""
import math

import numpy as np
import pytest

from paged_util import (allclose_ref, brute_force_f64, normal, paged_layout, scale_for,
                        shared_pool_layout)

needs_ref = pytest.mark.skipif(
    not __import__("oracle.oracle", fromlist=["x"]).ref_available(),
    reason="oracle/_ref not built (needs /root/reference)")


# ------------------------------------------------------------------ generators
def test_mt19937_64_known_answer(orc):
    # The C++ standard fixes the 10000th output of a default-seeded (5489)
    # std::mt19937_64 ([rand.predef]).
    g = orc.Mt64(5489)
    for _ in range(9999):
        g.next()
    assert g.next() == 9981545732273789042


def test_fill_normal_moments_and_pairing(orc):
    x = orc.fill_normal(200001, 0.0, 0.5, 42).astype(np.float64)
    assert abs(x.mean()) < 5e-3 and abs(x.std() - 0.5) < 5e-3
    # Box-Muller pairs: (z0, z1) share a radius, so z0^2 + z1^2 = -2 ln u1 >= 0
    # and the odd tail element is the cosine branch of its pair only.
    y = orc.fill_normal(200000, 0.0, 1.0, 42)
    assert np.array_equal(y, orc.fill_normal(200001, 0.0, 1.0, 42)[:200000])
    g = orc.Mt64(42)
    u1 = ((g.next() >> 11) + 1) * 2.0 ** -53
    u2 = (g.next() >> 11) * 2.0 ** -53
    r = math.sqrt(-2.0 * math.log(u1))
    assert y[0] == np.float32(r * math.cos(2 * math.pi * u2))
    assert y[1] == np.float32(r * math.sin(2 * math.pi * u2))


# ------------------------------------------------------------------ bf16
def test_bf16_rne_matches_torch_on_finite_values(orc):
    import torch
    rng = np.random.default_rng(1)
    bits = rng.integers(0, 2 ** 32, 1 << 18, dtype=np.uint64).astype(np.uint32)
    x = bits.view(np.float32)
    x = x[np.isfinite(x)]
    ours = orc.to_bf16_bits(x)
    theirs = torch.from_numpy(x.copy()).to(torch.bfloat16).view(torch.int16).numpy().view(np.uint16)
    assert np.array_equal(ours, theirs)


def test_bf16_special_cases(orc):
    def nb(bits):  # narrow raw fp32 bit patterns (arrays keep signaling NaNs intact)
        return orc.to_bf16_bits(np.array([bits], np.uint32).view(np.float32))[0]
    # exact ties round to even: 1 + 2^-8 (0x3F808000) -> 0x3F80; 0x3F818000 -> 0x3F82
    assert nb(0x3F808000) == 0x3F80
    assert nb(0x3F818000) == 0x3F82
    # overflow to inf through the carry
    assert nb(0x7F7FFFFF) == 0x7F80
    # NaN keeps NaN-ness; a payload living only in the dropped bits is quieted
    assert nb(0x7F800001) == 0x7FC0
    assert nb(0xFFC00000) == 0xFFC0
    assert nb(0x7F810000) == 0x7F81
    # widening is exact
    b = np.arange(0, 1 << 16, dtype=np.uint16)
    assert np.array_equal(orc.bf16_bits_to_f32(b).view(np.uint32), b.astype(np.uint32) << 16)


# ------------------------------------------------------------------ exp
def test_exp_scalar_ulp_bound_and_domain(orc):
    xs = np.linspace(-87.33, 88.37, 200001, dtype=np.float32)
    ours = np.array([orc.exp_scalar(float(x)) for x in xs[::20]], np.float32)
    truth = np.exp(xs[::20].astype(np.float64)).astype(np.float32)
    ulp = np.abs(ours.view(np.int32).astype(np.int64) - truth.view(np.int32).astype(np.int64))
    assert ulp.max() <= 2
    assert orc.exp_scalar(-87.34) == 0.0 and orc.exp_scalar(float("-inf")) == 0.0
    assert orc.exp_scalar(0.0) == 1.0
    assert orc.exp_scalar(1000.0) == orc.exp_scalar(88.3762626647949)
    assert math.isnan(orc.exp_scalar(float("nan")))


def test_exp_avx2_ulp_bound(orc):
    xs = np.linspace(-87.33, 88.37, 80000, dtype=np.float32)
    ours = orc.exp_avx2(xs)
    truth = np.exp(xs.astype(np.float64)).astype(np.float32)
    ulp = np.abs(ours.view(np.int32).astype(np.int64) - truth.view(np.int32).astype(np.int64))
    assert ulp.max() <= 2
    assert orc.exp_avx2(np.full(8, -100.0, np.float32)).max() == 0.0


@needs_ref
def test_exp_scalar_bit_exact_vs_reference(orc):
    R = orc.ref()
    xs = np.linspace(-90.0, 90.0, 30001, dtype=np.float32)
    for x in xs:
        assert orc.exp_scalar(float(x)) == R.ref_exp_scalar(float(x)) or (
            math.isnan(orc.exp_scalar(float(x))))


# ------------------------------------------------------------------ attention vs HF goldens
CASES = ["l0_prefill_empty", "l1_prefill_empty", "l0_prefill_continue", "l1_prefill_continue",
         "l0_decode"]


@pytest.mark.parametrize("name", CASES)
def test_cpu_attention_matches_hf_goldens(orc, golden, name):
    # rtol/atol 1e-4 as tests/unit/attention_test.cpp:153-176 uses.
    q, k, v, ctx = (golden[f"{name}.{s}"] for s in ("q_rot", "k_all", "v_all", "ctx"))
    out = orc.cpu_attention(q, k, v, 4, 2, 16, 0.25)
    assert allclose_ref(out, ctx, 1e-4, 1e-4)


@pytest.mark.parametrize("name", CASES)
@pytest.mark.parametrize("isa", [0, 1])
def test_prefill_units_match_hf_goldens(orc, golden, name, isa):
    q, k, v, ctx = (golden[f"{name}.{s}"] for s in ("q_rot", "k_all", "v_all", "ctx"))
    out = orc.prefill(q, k, v, 4, 2, 16, 0.25, isa=isa)
    assert allclose_ref(out, ctx, 1e-4, 1e-5)


@pytest.mark.parametrize("name", CASES)
@pytest.mark.parametrize("isa", [0, 1])
def test_paged_decode_matches_hf_goldens(orc, golden, name, isa):
    # The last query row of each case is the decode of its final token
    # (tests/unit/paged_decode_attention_kernel_test.cpp:388-444, bs = 8).
    q, k, v, ctx = (golden[f"{name}.{s}"] for s in ("q_rot", "k_all", "v_all", "ctx"))
    ks, vs, table = paged_layout(k, v, 8, extra_blocks=1)
    out = orc.paged_decode(q[-1], ks, vs, table, k.shape[1], 4, 2, 16, 8, 0.25, isa=isa)
    assert allclose_ref(out, ctx[-1], 1e-4, 1e-4)


# ------------------------------------------------------------------ closed forms / brute force
def test_single_key_returns_v_row_of_group_head(orc):
    # L = 1: softmax over one key is 1, so out[h] = v[h // g, 0] exactly; a
    # head-to-kv-head mapping of h % Hkv instead of h // g fails this.
    rng = np.random.default_rng(3)
    H, Hkv, d = 8, 2, 16
    q = normal(rng, (1, H, d))
    k = normal(rng, (Hkv, 1, d))
    v = normal(rng, (Hkv, 1, d))
    out = orc.cpu_attention(q, k, v, H, Hkv, d, 0.25)
    for h in range(H):
        assert np.array_equal(out[0, h], v[h // 4, 0])
    ks, vs, table = paged_layout(k, v, 16)
    out2 = orc.paged_decode(q[0], ks, vs, table, 1, H, Hkv, d, 16, 0.25)
    for h in range(H):
        assert np.array_equal(out2[h], v[h // 4, 0])


def test_equal_keys_average_values(orc):
    rng = np.random.default_rng(4)
    H, Hkv, d, L = 4, 1, 32, 100
    q = normal(rng, (1, H, d))
    k = np.repeat(normal(rng, (Hkv, 1, d)), L, axis=1)
    v = normal(rng, (Hkv, L, d))
    ks, vs, table = paged_layout(k, v, 16, rng=rng)
    out = orc.paged_decode(q[0], ks, vs, table, L, H, Hkv, d, 16, scale_for(d))
    np.testing.assert_allclose(out, np.broadcast_to(v[0].mean(0), (H, d)), rtol=1e-5, atol=1e-6)


@pytest.mark.parametrize("H,Hkv,d,L", [(4, 4, 18, 70), (8, 1, 24, 129), (24, 2, 64, 300),
                                       (14, 2, 64, 513)])
def test_paged_decode_vs_fp64_brute_force(orc, H, Hkv, d, L):
    rng = np.random.default_rng(L)
    q = normal(rng, (1, H, d))
    k = normal(rng, (Hkv, L, d))
    v = normal(rng, (Hkv, L, d))
    truth = brute_force_f64(q, k, v, H, Hkv, scale_for(d))[0]
    for isa in (0, 1):
        ks, vs, table = paged_layout(k, v, 16, extra_blocks=3, rng=rng)
        out = orc.paged_decode(q[0], ks, vs, table, L, H, Hkv, d, 16, scale_for(d), isa=isa)
        assert allclose_ref(out, truth, 1e-4, 1e-5)
    assert allclose_ref(orc.cpu_attention(q, k, v, H, Hkv, d, scale_for(d))[0], truth,
                        1e-4, 1e-5)


def test_causal_mask_prefill_continue_vs_brute_force(orc):
    rng = np.random.default_rng(5)
    H, Hkv, d, P, T = 8, 2, 32, 37, 45
    q = normal(rng, (T, H, d))
    k = normal(rng, (Hkv, P + T, d))
    v = normal(rng, (Hkv, P + T, d))
    truth = brute_force_f64(q, k, v, H, Hkv, scale_for(d))
    assert allclose_ref(orc.cpu_attention(q, k, v, H, Hkv, d, scale_for(d)), truth, 1e-4, 1e-5)
    assert allclose_ref(orc.prefill(q, k, v, H, Hkv, d, scale_for(d)), truth, 1e-4, 1e-5)


def test_paged_rejects_block_size_not_dividing_64(orc):
    k = np.zeros((2, 40, 64), np.float32)
    ks, vs, table = paged_layout(k, k, 24)
    with pytest.raises(ValueError):
        orc.paged_decode(np.zeros((4, 64), np.float32), ks, vs, table, 40, 4, 2, 64, 24, 0.125)


# ------------------------------------------------------------------ bitwise invariants
@pytest.mark.parametrize("bs", [8, 16, 32, 64])
@pytest.mark.parametrize("L", [1, 7, 63, 64, 65, 129, 511])
def test_paged_equals_contiguous_bitwise(orc, bs, L):
    rng = np.random.default_rng(bs * 1000 + L)
    H, Hkv, d = 4, 2, 64
    q = normal(rng, (H, d))
    k = normal(rng, (Hkv, L, d))
    v = normal(rng, (Hkv, L, d))
    ks, vs, table = paged_layout(k, v, bs)
    for isa in (0, 1):
        assert np.array_equal(orc.paged_decode(q, ks, vs, table, L, H, Hkv, d, bs, 0.125, isa=isa),
                              orc.decode_contig(q, k, v, H, Hkv, d, 0.125, isa=isa))


def test_batched_equals_per_member_and_threads_invariant(orc):
    rng = np.random.default_rng(9)
    H, Hkv, d, bs = 14, 2, 64, 16
    lens = [1, 16, 33, 63, 128, 300]
    ks = [normal(rng, (Hkv, L, d)) for L in lens]
    vs = [normal(rng, (Hkv, L, d)) for L in lens]
    kslab, vslab, tables = shared_pool_layout(ks, vs, bs, rng)
    q = normal(rng, (len(lens), H, d))
    for isa in (0, 1):
        orc.set_threads(1)
        a = orc.paged_decode_batched(q, kslab, vslab, tables, lens, H, Hkv, d, bs, 0.125, isa=isa)
        orc.set_threads(6)
        b = orc.paged_decode_batched(q, kslab, vslab, tables, lens, H, Hkv, d, bs, 0.125, isa=isa)
        assert np.array_equal(a, b)
        for i, L in enumerate(lens):
            assert np.array_equal(a[i], orc.paged_decode(q[i], kslab, vslab, tables[i], L, H, Hkv,
                                                         d, bs, 0.125, isa=isa))
    orc.set_threads(1)
    assert orc.paged_decode_batched(q[:0], kslab, vslab, [], [], H, Hkv, d, bs, 0.125).shape[0] == 0


# ------------------------------------------------------------------ vs the reference's own code
@needs_ref
@pytest.mark.parametrize("isa", [0, 1])
@pytest.mark.parametrize("H,Hkv,d,bs", [(14, 2, 64, 16), (32, 8, 128, 16), (4, 2, 16, 8),
                                        (24, 2, 24, 32), (8, 1, 18, 64)])
def test_paged_batched_bit_exact_vs_reference_build(orc, isa, H, Hkv, d, bs):
    rng = np.random.default_rng(H * d + bs)
    lens = [int(x) for x in rng.integers(1, 700, 7)]
    ks = [normal(rng, (Hkv, L, d)) for L in lens]
    vs = [normal(rng, (Hkv, L, d)) for L in lens]
    kslab, vslab, tables = shared_pool_layout(ks, vs, bs, rng)
    q = normal(rng, (len(lens), H, d))
    sc = scale_for(d)
    ours = orc.paged_decode_batched(q, kslab, vslab, tables, lens, H, Hkv, d, bs, sc, isa=isa)
    theirs = orc.paged_decode_batched(q, kslab, vslab, tables, lens, H, Hkv, d, bs, sc, isa=isa,
                                      use_ref=True)
    assert np.array_equal(ours.view(np.uint32), theirs.view(np.uint32))


@needs_ref
@pytest.mark.parametrize("isa", [0, 1])
def test_prefill_varlen_bit_exact_vs_reference_build(orc, isa):
    rng = np.random.default_rng(77)
    H, Hkv, d = 8, 2, 64
    Ts = [1, 33, 70, 5]
    Ps = [0, 17, 64, 200]
    qs = normal(rng, (sum(Ts), H, d))
    cu = np.concatenate([[0], np.cumsum(Ts)]).astype(np.int32)
    ks = [normal(rng, (Hkv, P + T, d)) for P, T in zip(Ps, Ts)]
    vs = [normal(rng, (Hkv, P + T, d)) for P, T in zip(Ps, Ts)]
    a = orc.prefill_varlen(qs, cu, ks, vs, H, Hkv, d, 0.125, isa=isa)
    b = orc.prefill_varlen(qs, cu, ks, vs, H, Hkv, d, 0.125, isa=isa, use_ref=True)
    assert np.array_equal(a.view(np.uint32), b.view(np.uint32))


@needs_ref
def test_scatter_gather_bit_exact_vs_reference_build(orc):
    rng = np.random.default_rng(11)
    Hkv, d, bs, nb = 3, 40, 16, 23
    T = 150
    slots = rng.permutation(nb * bs)[:T].astype(np.int64)
    sk = normal(rng, (T, Hkv, d))
    sv = normal(rng, (T, Hkv, d))
    a_k = np.full((nb, Hkv, bs, d), 7.0, np.float32)
    a_v = a_k.copy()
    b_k, b_v = a_k.copy(), a_k.copy()
    orc.kv_scatter(sk, sv, slots, Hkv, d, bs, a_k, a_v)
    orc.kv_scatter(sk, sv, slots, Hkv, d, bs, b_k, b_v, use_ref=True)
    assert np.array_equal(a_k, b_k) and np.array_equal(a_v, b_v)
    table = rng.permutation(nb).astype(np.int32)
    for L in (0, 1, 15, 16, 17, 200):
        g1 = orc.kv_gather(a_k, a_v, table, bs, L, Hkv, d)
        g2 = orc.kv_gather(a_k, a_v, table, bs, L, Hkv, d, use_ref=True)
        assert np.array_equal(g1[0], g2[0]) and np.array_equal(g1[1], g2[1])


# ------------------------------------------------------------------ scatter closed form
def test_scatter_closed_form_and_round_trip(orc):
    # dst = ((block * Hkv + h) * bs + p) * d with block = slot / bs, p = slot % bs
    # (src/kernels/kv_scatter.cpp:33-40); gather inverts it for a table walk.
    rng = np.random.default_rng(12)
    Hkv, d, bs, nb = 2, 8, 8, 9
    table = rng.permutation(nb)[:5].astype(np.int32)
    L = 37
    slots = np.array([table[p // bs] * bs + p % bs for p in range(L)], np.int64)
    sk = normal(rng, (L, Hkv, d))
    sv = normal(rng, (L, Hkv, d))
    ksl = np.zeros((nb, Hkv, bs, d), np.float32)
    vsl = np.zeros_like(ksl)
    orc.kv_scatter(sk, sv, slots, Hkv, d, bs, ksl, vsl)
    flat = ksl.reshape(-1)
    for t in range(L):
        for h in range(Hkv):
            blk, p = divmod(int(slots[t]), bs)
            off = ((blk * Hkv + h) * bs + p) * d
            assert np.array_equal(flat[off:off + d], sk[t, h])
    gk, gv = orc.kv_gather(ksl, vsl, table, bs, L, Hkv, d)
    assert np.array_equal(gk, sk.transpose(1, 0, 2)) and np.array_equal(gv, sv.transpose(1, 0, 2))
    # bf16 storage: same addressing, element-wise RNE narrowing
    kb = np.zeros((nb, Hkv, bs, d), np.uint16)
    vb = np.zeros_like(kb)
    orc.kv_scatter(sk, sv, slots, Hkv, d, bs, kb, vb)
    assert np.array_equal(kb, orc.to_bf16_bits(ksl) * (ksl != 0) + 0 * kb)


# ------------------------------------------------------------------ RoPE (src/kernels/rope.h)
@needs_ref
@pytest.mark.parametrize("isa", [0, 1])
@pytest.mark.parametrize("d", [10, 64, 72, 128, 130])
def test_rope_bit_exact_vs_reference_build(orc, isa, d):
    rng = np.random.default_rng(d + 100 * isa)
    x = normal(rng, (11, 3, d))
    c, s = orc.rope_tables(d, 4096, theta=500000.0)
    pos = rng.integers(0, 4096, 11).astype(np.int32)
    pos[3] = pos[4]  # repeated positions are allowed (rope.h:18-20)
    ours = orc.rope_apply(x, pos, c, s, isa=isa)
    theirs = orc.rope_apply(x, pos, c, s, isa=isa, use_ref=True)
    assert np.array_equal(ours.view(np.uint32), theirs.view(np.uint32))


@pytest.mark.parametrize("isa", [0, 1])
def test_rope_closed_forms(orc, isa):
    """Position 0 is the identity; each (j, j + d/2) pair is rotated by the
    table angle (fp64 rotation within fp32 rounding); pair norms are kept."""
    rng = np.random.default_rng(9)
    d = 64
    x = normal(rng, (6, 4, d))
    c, s = orc.rope_tables(d, 1000)
    pos = np.array([0, 1, 17, 999, 500, 0], np.int32)
    y = orc.rope_apply(x, pos, c, s, isa=isa)
    assert np.array_equal(y[0], x[0]) and np.array_equal(y[5], x[5])
    lo, hi = x[..., : d // 2].astype(np.float64), x[..., d // 2:].astype(np.float64)
    cc, ss = c[pos][:, None, :].astype(np.float64), s[pos][:, None, :].astype(np.float64)
    want = np.concatenate([lo * cc - hi * ss, hi * cc + lo * ss], axis=-1)
    assert np.abs(y - want).max() <= 4e-7 * max(1.0, np.abs(want).max())
    n0 = lo ** 2 + hi ** 2
    n1 = y[..., : d // 2].astype(np.float64) ** 2 + y[..., d // 2:].astype(np.float64) ** 2
    assert np.allclose(n0, n1, rtol=2e-6, atol=1e-7)
    # The FMA (AVX2) and two-rounding (scalar) forms differ by at most an ulp or so.
    other = orc.rope_apply(x, pos, c, s, isa=1 - isa)
    assert np.abs(y - other).max() <= 4e-7 * max(1.0, np.abs(y).max())


# ------------------------------------------------------------ INT8 KV append
def int8_case(rng, nb=6, hkv=2, bs=16, d=8):
    k = np.zeros((nb, hkv, bs, d), np.int8)
    v = np.zeros((nb, hkv, bs, d), np.int8)
    return k, v, np.zeros((nb, hkv), np.float32), np.zeros((nb, hkv), np.float32)


def test_int8_fresh_block_closed_form(orc):
    """One call filling rows 0..n-1 of a fresh block: scale = max|x| / 127 in
    fp32, the max element maps to +-127, every element is within half a step
    of its value, and zero rows of a zero block give scale 0 and q = 0."""
    rng = np.random.default_rng(1)
    hkv, bs, d = 2, 16, 8
    k, v, ks, vs = int8_case(rng, hkv=hkv, bs=bs, d=d)
    n = 11
    src_k = (rng.standard_normal((n, hkv, d)) * 3).astype(np.float32)
    src_v = np.zeros((n, hkv, d), np.float32)
    slots = 3 * bs + np.arange(n)
    orc.kv_append_int8(src_k, src_v, slots, hkv, d, bs, k, v, ks, vs)
    for h in range(hkv):
        m = np.abs(src_k[:, h]).max()
        assert ks[3, h] == np.float32(m) / np.float32(127)
        q = k[3, h, :n]
        assert np.abs(q).max() == 127
        x = q.astype(np.float32) * ks[3, h]
        assert np.abs(x - src_k[:, h]).max() <= 0.5 * ks[3, h] * (1 + 1e-6)
        assert vs[3, h] == 0 and not v[3, h].any()
    untouched = np.ones(6, bool)
    untouched[3] = False
    assert not k[untouched].any() and not ks[untouched].any()


def test_int8_incremental_appends_requantise(orc):
    """Decode-style appends one row at a time: the scale never decreases,
    rises exactly when a row exceeds 127 * scale, and every stored value stays
    within one step of its input (double rounding after requantisation)."""
    rng = np.random.default_rng(2)
    hkv, bs, d = 1, 16, 16
    k, v, ks, vs = int8_case(rng, hkv=hkv, bs=bs, d=d)
    amps = [0.5, 0.2, 2.0, 1.0, 7.5, 7.4, 0.1]
    rows = []
    prev = np.float32(0)
    for off, a in enumerate(amps):
        x = (rng.uniform(-1, 1, (1, hkv, d)) * a).astype(np.float32)
        rows.append(x[0, 0])
        orc.kv_append_int8(x, x, np.array([2 * bs + off]), hkv, d, bs, k, v, ks, vs)
        m = np.abs(x).max()
        if m > prev * np.float32(127):
            assert ks[2, 0] == np.float32(m) / np.float32(127)
        else:
            assert ks[2, 0] == prev
        assert ks[2, 0] >= prev
        prev = ks[2, 0]
    x = k[2, 0, :len(amps)].astype(np.float32) * ks[2, 0]
    assert np.abs(x - np.array(rows)).max() <= ks[2, 0] * (1 + 1e-6)
    assert np.array_equal(k, v) and np.array_equal(ks, vs)


def test_int8_batched_equals_ordered_when_first_row_holds_the_max(orc):
    """When the first appended row carries the block's maximum, the scale is
    set once, no requantisation happens, and appending the rows one by one
    stores exactly what one batched call stores."""
    rng = np.random.default_rng(3)
    hkv, bs, d = 2, 8, 8
    x = rng.uniform(-1, 1, (bs, hkv, d)).astype(np.float32)
    x[0] *= 4  # row 0 holds the max of every head
    slots = 5 * bs + np.arange(bs)
    a = int8_case(rng, hkv=hkv, bs=bs, d=d)
    orc.kv_append_int8(x, x, slots, hkv, d, bs, *a)
    b = int8_case(rng, hkv=hkv, bs=bs, d=d)
    for i in range(bs):
        orc.kv_append_int8(x[i:i + 1], x[i:i + 1], slots[i:i + 1], hkv, d, bs, *b)
    for u, w in zip(a, b):
        assert np.array_equal(u, w)


def test_int8_fresh_block_ignores_a_stale_scale(orc):
    """A block reused after release starts at offset 0: its old scale (and
    rows) must not leak into the new contents."""
    rng = np.random.default_rng(4)
    hkv, bs, d = 2, 16, 8
    x = rng.standard_normal((5, hkv, d)).astype(np.float32)
    slots = 1 * bs + np.arange(5)
    a = int8_case(rng, hkv=hkv, bs=bs, d=d)
    b = int8_case(rng, hkv=hkv, bs=bs, d=d)
    b[0][1] = 99
    b[2][1] = 1e30  # stale state from a previous owner
    orc.kv_append_int8(x, x, slots, hkv, d, bs, *a)
    orc.kv_append_int8(x, x, slots, hkv, d, bs, *b)
    assert np.array_equal(a[0][1, :, :5], b[0][1, :, :5])
    assert np.array_equal(a[2][1], b[2][1])


def test_int8_dequant_matches_closed_form(orc):
    rng = np.random.default_rng(5)
    q = rng.integers(-127, 128, (3, 2, 4, 8)).astype(np.int8)
    s = rng.uniform(0.01, 1, (3, 2)).astype(np.float32)
    x = orc.int8_dequant(q, s)
    assert np.array_equal(x, q.astype(np.float32) * s[:, :, None, None])


# ------------------------------------------------------------ FP8 (E4M3) KV
def _torch_e4m3():
    torch = pytest.importorskip("torch")
    return torch


def test_e4m3_decode_every_code_matches_torch(orc):
    """The oracle's E4M3 decoder against torch.float8_e4m3fn on all 256 codes
    (two independent implementations of the OCP format), and its closed form:
    bias 7, 3 mantissa bits, subnormals m * 2^-9, 0x7F / 0xFF NaN, 448 max."""
    torch = _torch_e4m3()
    codes = np.arange(256, dtype=np.uint8)
    got = orc.e4m3_to_f32(codes)
    ref = torch.from_numpy(codes.copy()).view(torch.float8_e4m3fn).to(torch.float32).numpy()
    nan = np.isnan(ref)
    assert np.array_equal(np.isnan(got), nan) and set(np.where(nan)[0]) == {0x7F, 0xFF}
    assert np.array_equal(got[~nan].view(np.uint32), ref[~nan].view(np.uint32))
    assert got[0x7E] == 448.0 and got[0x01] == 2.0 ** -9 and got[0x08] == 2.0 ** -6
    assert got[0x38] == 1.0 and got[0xB8] == -1.0


def test_e4m3_encode_matches_torch_on_codes_midpoints_and_samples(orc):
    """Round to nearest, ties to even: every finite code's value encodes to
    itself, every midpoint between neighbouring codes goes to the even one,
    and 20000 log-uniform samples in (2^-12, 464] agree with torch bit for
    bit; beyond 448 the oracle saturates (torch gives NaN from 480 on)."""
    torch = _torch_e4m3()
    codes = np.array([c for c in range(256) if c & 0x7F != 0x7F], np.uint8)
    vals = orc.e4m3_to_f32(codes)
    assert np.array_equal(orc.f32_to_e4m3(vals), codes)
    pos = np.sort(vals[vals > 0])
    mids = ((pos[:-1].astype(np.float64) + pos[1:]) / 2).astype(np.float32)
    rng = np.random.default_rng(8)
    samp = (np.exp2(rng.uniform(-12, np.log2(464), 20000)) *
            rng.choice([-1, 1], 20000)).astype(np.float32)
    x = np.concatenate([mids, -mids, samp, np.float32([0.0, -0.0, 448.0, 460.0, 464.0])])
    ref = torch.from_numpy(x.copy()).to(torch.float8_e4m3fn).view(torch.uint8).numpy()
    assert np.array_equal(orc.f32_to_e4m3(x), ref)
    # ties to even at a midpoint: 1 + 1/16 lies between codes 0x38 (1.0) and 0x39
    assert orc.f32_to_e4m3(np.float32([1.0625]))[0] == 0x38
    assert orc.f32_to_e4m3(np.float32([1.1875]))[0] == 0x3A
    assert list(orc.f32_to_e4m3(np.float32([1000.0, -1e30, np.nan]))) == [0x7E, 0xFE, 0x7F]


def fp8_case(nb=6, hkv=2, bs=16, d=8):
    return (np.zeros((nb, hkv, bs, d), np.uint8), np.zeros((nb, hkv, bs, d), np.uint8),
            np.zeros((nb, hkv), np.float32), np.zeros((nb, hkv), np.float32))


def test_fp8_fresh_block_closed_form(orc):
    """A fresh block: scale = max|x| / 448 in fp32, the max element maps to
    +-448, each element is its value to within half an E4M3 step (relative
    2^-4 of the element, or 2^-10 of the scale below the normal range), and
    a zero V block gives scale 0 and zero codes."""
    rng = np.random.default_rng(11)
    hkv, bs, d = 2, 16, 8
    k, v, ks, vs = fp8_case(hkv=hkv, bs=bs, d=d)
    n = 11
    src_k = (rng.standard_normal((n, hkv, d)) * 3).astype(np.float32)
    src_v = np.zeros((n, hkv, d), np.float32)
    orc.kv_append_fp8(src_k, src_v, 3 * bs + np.arange(n), hkv, d, bs, k, v, ks, vs)
    for h in range(hkv):
        m = np.abs(src_k[:, h]).max()
        assert ks[3, h] == np.float32(m) / np.float32(448)
        y = orc.e4m3_to_f32(k[3, h, :n])
        assert np.abs(y).max() == 448.0
        x = y * ks[3, h]
        tol = np.maximum(np.abs(src_k[:, h]) * 2.0 ** -4, ks[3, h] * 2.0 ** -10) * (1 + 1e-6)
        assert (np.abs(x - src_k[:, h]) <= tol).all()
        assert vs[3, h] == 0 and not v[3, h].any()


def test_fp8_incremental_appends_requantise(orc):
    """One row at a time: the scale never decreases and rises exactly when a
    row exceeds 448 * scale; older rows are requantised to the new scale."""
    rng = np.random.default_rng(12)
    hkv, bs, d = 1, 16, 16
    k, v, ks, vs = fp8_case(hkv=hkv, bs=bs, d=d)
    amps = [0.5, 0.2, 2.0, 1.0, 7.5, 7.4, 0.1]
    rows, prev = [], np.float32(0)
    for off, a in enumerate(amps):
        x = (rng.uniform(-1, 1, (1, hkv, d)) * a).astype(np.float32)
        rows.append(x[0, 0])
        orc.kv_append_fp8(x, x, np.array([2 * bs + off]), hkv, d, bs, k, v, ks, vs)
        m = np.abs(x).max()
        exp = np.float32(m) / np.float32(448) if m > prev * np.float32(448) else prev
        assert ks[2, 0] == exp and ks[2, 0] >= prev
        prev = ks[2, 0]
    x = orc.e4m3_to_f32(k[2, 0, :len(amps)]) * ks[2, 0]
    r = np.array(rows)
    # two roundings at most (the row's own, then a requantisation)
    tol = np.maximum(np.abs(r) * 2.0 ** -3, ks[2, 0] * 2.0 ** -9) * (1 + 1e-6)
    assert (np.abs(x - r) <= tol).all()
    assert np.array_equal(k, v) and np.array_equal(ks, vs)


def test_fp8_batched_equals_ordered_and_ignores_stale_state(orc):
    """With the max in the first row, one batched call equals row-by-row
    appends; a block reused at offset 0 ignores its stale scale and rows."""
    rng = np.random.default_rng(13)
    hkv, bs, d = 2, 8, 8
    x = rng.uniform(-1, 1, (bs, hkv, d)).astype(np.float32)
    x[0] *= 4
    slots = 5 * bs + np.arange(bs)
    a = fp8_case(hkv=hkv, bs=bs, d=d)
    orc.kv_append_fp8(x, x, slots, hkv, d, bs, *a)
    b = fp8_case(hkv=hkv, bs=bs, d=d)
    b[0][5] = 77
    b[2][5] = 1e30  # stale state from a previous owner
    for i in range(bs):
        orc.kv_append_fp8(x[i:i + 1], x[i:i + 1], slots[i:i + 1], hkv, d, bs, *b)
    for u, w in zip(a, b):
        assert np.array_equal(u, w)


def test_fp8_dequant_matches_closed_form(orc):
    rng = np.random.default_rng(14)
    q = rng.integers(0, 256, (3, 2, 4, 8)).astype(np.uint8)
    q[(q & 0x7F) == 0x7F] = 0x10
    s = rng.uniform(0.01, 1, (3, 2)).astype(np.float32)
    x = orc.fp8_dequant(q, s)
    assert np.array_equal(x, orc.e4m3_to_f32(q) * s[:, :, None, None])


# ---- packed linear layer (o_proj): kernels::PackWeightPanels / PackedGemm ----
GEMM_SHAPES = [(16, 64, 64), (16, 64, 96), (16, 176, 64), (8, 64, 512), (1, 64, 64),
               (1, 2048, 512), (130, 300, 70), (7, 1, 33), (65, 129, 1000), (5, 40, 17)]


def _gemm_weights(orc, n, k, dtype, seed):
    wf = orc.fill_normal(n * k, 0.0, 1.0, seed).reshape(n, k)
    if dtype == 0:
        return wf
    if dtype == 1:
        return orc.to_bf16_bits(wf)
    return wf.astype(np.float16).view(np.uint16)


def test_pack_weight_panels_closed_form(orc):
    """Wp[p, k, r] = W[p*16 + r, k], zero past n (packed_gemm_test.cpp:96-121)."""
    rng = np.random.default_rng(3)
    for n, k in [(17, 5), (16, 3), (40, 9), (1, 1)]:
        w = rng.standard_normal((n, k)).astype(np.float32)
        wp = orc.pack_weight_panels(w)
        want = np.zeros(((n + 15) // 16 * 16, k), np.float32)
        want[:n] = w
        want = want.reshape(-1, 16, k).transpose(0, 2, 1)
        assert np.array_equal(wp, want)


def test_fp16_widening_exhaustive(orc):
    """Every binary16 pattern (normals, subnormals, +-0, inf, NaN payloads)
    against numpy's float16 -> float32 (src/tensor/half.h:84-109)."""
    bits = np.arange(65536, dtype=np.uint16)
    want = bits.view(np.float16).astype(np.float32)
    got = np.array([orc.fp16_bits_to_f32(int(b)) for b in bits], np.float32)
    nan = np.isnan(want)
    assert np.array_equal(np.isnan(got), nan)
    assert np.array_equal(got[~nan].view(np.uint32), want[~nan].view(np.uint32))


@pytest.mark.parametrize("dtype", [0, 1, 2])
def test_packed_gemm_fp64_brute_force(orc, dtype):
    """Independent of the restatement's loop: the fp64 product of the widened
    weights, within fp32 accumulation rounding (k * 2^-23 of sum |x w|)."""
    rng = np.random.default_rng(10 + dtype)
    for m, k, n in [(3, 50, 20), (1, 7, 33), (9, 129, 16)]:
        x = rng.standard_normal((m, k)).astype(np.float32)
        w = _gemm_weights(orc, n, k, dtype, 20 + m)
        wf = (w if dtype == 0 else orc.bf16_bits_to_f32(w) if dtype == 1
              else w.view(np.float16).astype(np.float32)).astype(np.float64)
        bias = rng.standard_normal(n).astype(np.float32)
        y = orc.packed_gemm(x, orc.pack_weight_panels(w), dtype, n, bias)
        exact = x.astype(np.float64) @ wf.T + bias
        bound = k * 2.0 ** -23 * (np.abs(x).astype(np.float64) @ np.abs(wf).T + np.abs(bias))
        assert (np.abs(y - exact) <= bound + 1e-30).all()


@needs_ref
@pytest.mark.parametrize("dtype", [0, 1, 2])
def test_packed_gemm_bit_exact_vs_reference_scalar(orc, dtype):
    """The restatement against the reference's own scalar GemmTile and
    PackWeightPanels, compiled from its sources: same bits."""
    for i, (m, k, n) in enumerate(GEMM_SHAPES):
        x = orc.fill_normal(m * k, 0.0, 1.0, 300 + i).reshape(m, k)
        w = _gemm_weights(orc, n, k, dtype, 400 + i)
        wp = orc.pack_weight_panels(w)
        assert np.array_equal(wp.view(np.uint8), orc.pack_weight_panels(w, use_ref=True).view(np.uint8))
        bias = orc.fill_normal(n, 0.0, 1.0, 500 + i) if i % 2 else None
        y = orc.packed_gemm(x, wp, dtype, n, bias)
        r = orc.packed_gemm(x, wp, dtype, n, bias, isa=0, use_ref=True)
        assert np.array_equal(y.view(np.uint32), r.view(np.uint32)), (m, k, n)
